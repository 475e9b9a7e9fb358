// C[m][n] = A_hi B_hi^T + A_hi B_lo^T + A_lo B_hi^T: the three products of
// fp16 operands split into hi and lo parts (pqa_batch.hip), fp32 accumulation
// and output, on v_mfma_f32_32x32x16_f16, each operand loaded once. A row of
// A holds hi at halfs [0, kh) and lo at [kh, 2 kh), likewise B; kh is a
// multiple of 32 (the callers pad with zeros). The batched Q/K/V and output
// projections use it with A = the split inputs (tokens) and B = the split
// weights (rows).
//
// Workgroup tile 256 (m) x 192 (n): at 2048 x 6144 that is 256 tiles, one per
// CU. 4 waves in a 2 x 2 grid, each wave 128 x 96 = 4 x 3 accumulators of
// 32 x 32 (192 AGPRs). K runs in 32-wide tiles through 2 LDS stages of 56 KB:
// A_hi and A_lo (256 rows of 64 bytes each), B_hi and B_lo (192 rows), filled
// by direct global->LDS loads (global_load_lds_dwordx4). Within a row, 16-byte
// chunk c sits at position c ^ ((r >> 2) & 3), so the 16 rows one pass of an
// MFMA operand read touches fall on distinct banks.
//
// Per tile, 2 k-steps of 16, each 36 MFMAs (3 products x 12 blocks; an
// accumulator is reused every 12 MFMAs) on 14 operand reads: two thirds of the
// load and LDS-read bytes per MFMA of one GEMM over the concatenated
// [hi | hi | lo] . [hi | lo | hi] rows (measured 3-4 % faster than that form
// at 2048 x 6144 x 3 x 2560, where it replaced it). Between the MFMAs of a
// k-step go the operand reads of the next k-step. The workgroup barrier sits
// after k-step 0 (every read of the tile has been issued and has completed by
// then); after it, k-step 1's MFMAs carry the reads of the next tile's k-step
// 0 and, spread evenly, the loads of the tile after next into the stage just
// freed.
//
// Tiles are ordered n-major (t = tn * mb + tm) and dealt to the 8 XCDs in
// contiguous runs: workgroup i runs on XCD i mod 8, so the tiles that run
// together on one XCD share their A and B row blocks in that XCD's L2
// (at 2048 x 6144: 8 m-blocks x 4 n-blocks per XCD).
//
// Rows past m (n) load the last row (clamped, never stored).
#include <algorithm>

#include "pqa_device.h"
#include "pqa_internal.h"

namespace pqa {

constexpr int kGemmBM = 256;
constexpr int kGemmBN = 192;
constexpr int kGemmWaves = 4;
constexpr int kGemmThreads = 64 * kGemmWaves;
constexpr int kG3BK = 32;
constexpr int kG3RowB = kG3BK * 2;                 // 64 bytes per tile row
constexpr int kG3ASub = kGemmBM * kG3RowB;          // 16 KB: A_hi or A_lo
constexpr int kG3BSub = kGemmBN * kG3RowB;          // 12 KB: B_hi or B_lo
constexpr int kG3Stage = 2 * kG3ASub + 2 * kG3BSub;  // 56 KB
constexpr int kG3Loads = kG3Stage / 1024 / kGemmWaves;  // 1 KB DMA pieces per wave and tile (14)
constexpr int kG3Frags = 14;                        // operand reads per k-step
constexpr int kG3Mfmas = 36;                        // MFMAs per k-step
static_assert(kG3Stage % (1024 * kGemmWaves) == 0, "whole 1 KB DMA pieces per wave");
static_assert(kG3Loads <= kG3Mfmas, "the loads of a tile fit between one k-step's MFMAs");

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ int g3_swz(int r) { return (r >> 2) & 3; }

struct Gemm3Args {
    const _Float16* a;
    const _Float16* b;
    float* c;
    int m, n, kh, lda, ldb, ldc;
    int mb, nb;
};

__global__ __launch_bounds__(kGemmThreads, 1) void gemm_f16x3_nt_kernel(const Gemm3Args g) {
    __shared__ __attribute__((aligned(1024))) char lds[2][kG3Stage];

    const int T = g.mb * g.nb;
    const int xcd = blockIdx.x & 7, jx = blockIdx.x >> 3;
    const int q8 = T >> 3, r8 = T & 7;
    if (jx >= q8 + (xcd < r8 ? 1 : 0)) return;  // whole workgroup, before any barrier
    const int t = xcd * q8 + min(xcd, r8) + jx;
    const int tn = t / g.mb, tm = t - tn * g.mb;
    const int m0 = tm * kGemmBM, n0 = tn * kGemmBN;

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int KT = g.kh / kG3BK;

    // ---- loads: the stage is A_hi (pieces 0-15), A_lo (16-31), B_hi (32-43),
    // B_lo (44-55), each piece 16 rows of 64 B; wave w fills pieces w, w + 4,
    // ...; lane l lands at row l / 4, position l % 4 ----
    unsigned goff[kG3Loads];
    const _Float16* gbase[kG3Loads];
    unsigned ldst[kG3Loads];
#pragma unroll
    for (int ii = 0; ii < kG3Loads; ii++) {
        const int piece = w + kGemmWaves * ii;
        const int part = piece < 16 ? 0 : piece < 32 ? 1 : piece < 44 ? 2 : 3;
        const int first = part == 0 ? 0 : part == 1 ? 16 : part == 2 ? 32 : 44;
        const int row = 16 * (piece - first) + (lane >> 2);
        const int chunk = (lane & 3) ^ g3_swz(row);
        if (part < 2) {
            const int gr = min(m0 + row, g.m - 1) - m0;
            gbase[ii] = g.a + (size_t)m0 * g.lda + (part == 1 ? g.kh : 0);
            goff[ii] = (unsigned)(((size_t)gr * g.lda + 8 * chunk) * 2);
        } else {
            const int gr = min(n0 + row, g.n - 1) - n0;
            gbase[ii] = g.b + (size_t)n0 * g.ldb + (part == 3 ? g.kh : 0);
            goff[ii] = (unsigned)(((size_t)gr * g.ldb + 8 * chunk) * 2);
        }
        ldst[ii] = (unsigned)(piece * 1024);
    }
    auto load = [&](int kt, int ii) {
        lds_dma_b128(gbase[ii] + (size_t)kt * kG3BK, goff[ii], lds_addr(&lds[kt & 1][0]) + ldst[ii]);
    };

    // ---- operand reads: wave (wm, wn) = (w & 1, w >> 1); k-step s reads
    // chunk 2 s + l / 32 of its rows ----
    const int wm = w & 1, wn = w >> 1;
    const int l32 = lane & 31, hk = lane >> 5;
    int offa[4][2], offb[3][2];
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++) {
        const int c = 2 * s2 + hk;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = wm * 128 + 32 * i + l32;
            offa[i][s2] = r * kG3RowB + 16 * (c ^ g3_swz(r));
        }
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const int r = wn * 96 + 32 * j + l32;
            offb[j][s2] = 2 * kG3ASub + r * kG3RowB + 16 * (c ^ g3_swz(r));
        }
    }
    // fragments: [slot][0 hi / 1 lo][block]
    half8 fa[2][2][4], fb[2][2][3];
    auto read = [&](int kt, int s2, int slot, int idx) {
        const char* st = &lds[kt & 1][0];
        if (idx < 8) {
            const int lo = idx >> 2, i = idx & 3;
            fa[slot][lo][i] = *(const half8*)(st + offa[i][s2] + lo * kG3ASub);
        } else {
            const int lo = idx >= 11, j = idx - (lo ? 11 : 8);
            fb[slot][lo][j] = *(const half8*)(st + offb[j][s2] + lo * kG3BSub);
        }
    };
    floatx16 acc[4][3];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 3; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;
    // MFMA q of a k-step: product q / 12 (hi.hi, hi.lo, lo.hi), block q % 12;
    // an accumulator is reused every 12 MFMAs
    auto mfma = [&](int slot, int q) {
        const int p = q / 12, idx = q % 12;
        const int i = idx / 3, j = idx % 3;
        const half8 av = fa[slot][p == 2 ? 1 : 0][i];
        const half8 bv = fb[slot][p == 1 ? 1 : 0][j];
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc[i][j], 0, 0, 0);
    };

    // ---- prologue: tiles 0 and 1 in flight, tile 0 landed everywhere ----
#pragma unroll
    for (int ii = 0; ii < kG3Loads; ii++) load(0, ii);
    if (KT > 1) {
#pragma unroll
        for (int ii = 0; ii < kG3Loads; ii++) load(1, ii);
        wait_vm<kG3Loads>();
    } else {
        wait_vm<0>();
    }
    __syncthreads();
#pragma unroll
    for (int idx = 0; idx < kG3Frags; idx++) read(0, 0, 0, idx);

    for (int kt = 0; kt < KT; kt++) {
        const bool next = kt + 1 < KT;
        // k-step 0, with the reads of k-step 1 between its MFMAs
#pragma unroll
        for (int q = 0; q < kG3Mfmas; q++) {
            mfma(0, q);
            __builtin_amdgcn_sched_barrier(0);
            if (q < kG3Frags) read(kt, 1, 1, q);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (next) {
            wait_vm<0>();     // this wave's loads of tile kt + 1
            __syncthreads();  // everyone's; every read of tile kt has completed
        }
        // k-step 1: the reads of tile kt + 1's k-step 0 (the last tile re-reads
        // its own stage, unused) and the loads of tile kt + 2 into stage kt % 2
        const int kn = next ? kt + 1 : kt;
        const bool more = kt + 2 < KT;
#pragma unroll
        for (int q = 0; q < kG3Mfmas; q++) {
            mfma(1, q);
            __builtin_amdgcn_sched_barrier(0);
            if (more) {
#pragma unroll
                for (int ii = 0; ii < kG3Loads; ii++)
                    if (q == (ii * kG3Mfmas) / kG3Loads) load(kt + 2, ii);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (q < kG3Frags) read(kn, 0, 0, q);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const int col = n0 + wn * 96 + 32 * j + l32;
            if (col >= g.n) continue;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int row = m0 + wm * 128 + 32 * i + 8 * (e >> 2) + 4 * hk + (e & 3);
                if (row < g.m) g.c[(size_t)row * g.ldc + col] = acc[i][j][e];
            }
        }
    }
}

hipError_t launch_gemm_f16x3_nt(const _Float16* a, int lda, const _Float16* b, int ldb, float* c, int ldc, int m,
                                int n, int kh, hipStream_t stream) {
    if (m <= 0 || n <= 0 || kh <= 0 || kh % kG3BK != 0 || lda < 2 * kh || ldb < 2 * kh || ldc < n || lda % 8 ||
        ldb % 8)
        return hipErrorInvalidValue;
    if ((size_t)kGemmBM * lda * 2 >= (1ull << 31) || (size_t)kGemmBN * ldb * 2 >= (1ull << 31))
        return hipErrorInvalidValue;
    Gemm3Args g;
    g.a = a;
    g.b = b;
    g.c = c;
    g.m = m;
    g.n = n;
    g.kh = kh;
    g.lda = lda;
    g.ldb = ldb;
    g.ldc = ldc;
    g.mb = (m + kGemmBM - 1) / kGemmBM;
    g.nb = (n + kGemmBN - 1) / kGemmBN;
    const long long tiles = (long long)g.mb * g.nb;
    const long long groups = (tiles + 7) / 8 * 8;
    if (groups > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gemm_f16x3_nt_kernel, dim3((unsigned)groups), dim3(kGemmThreads), 0, stream, g);
    return hipGetLastError();
}

}  // namespace pqa
