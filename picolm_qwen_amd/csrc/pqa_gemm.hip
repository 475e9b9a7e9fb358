// C[m][n] = sum_k A[m][k] B[n][k]: fp16 operands, both k-contiguous, fp32
// accumulation and output, on v_mfma_f32_32x32x16_f16. The batched Q/K/V
// projections (pqa_batch.hip) use it with A = X' (tokens x 3n, the split
// inputs) and B = W' (q, k and v rows x 3n, the split weights).
//
// Workgroup tile 256 (m) x 192 (n): at 2048 x 6144 that is 256 tiles, one per
// CU. 4 waves in a 2 x 2 grid, each wave 128 x 96 = 4 x 3 accumulators of
// 32 x 32 (192 AGPRs). K runs in 64-wide tiles through 2 LDS stages of 56 KB
// (256 + 192 rows of 128 bytes), filled by direct global->LDS loads
// (global_load_lds_dwordx4): a tile's rows are whole 128-byte cache lines.
// Within a row, 16-byte chunk c sits at position c ^ ((r >> 1) & 7), so the 16
// rows one pass of an MFMA operand read touches cover all 64 LDS banks once.
//
// Per tile, 4 k-steps of 12 MFMAs. Between the MFMAs of a k-step go the
// operand reads of the next k-step (one per MFMA), so no MFMA waits on LDS.
// The workgroup barrier sits after k-step 2 (every read of the tile has been
// issued and has completed by then); after it, k-step 3's MFMAs carry the
// reads of the next tile's k-step 0 and the loads of the tile after next,
// into the stage just freed: loads get 48 MFMAs (~1500 cycles) to land.
//
// Tiles are ordered n-major (t = tn * mb + tm) and dealt to the 8 XCDs in
// contiguous runs: workgroup i runs on XCD i mod 8, so the tiles that run
// together on one XCD share their A and B row blocks in that XCD's L2
// (at 2048 x 6144: 8 m-blocks x 4 n-blocks per XCD).
//
// Rows past m (n) load the last row (clamped, never stored); k must be a
// multiple of 64 (the callers pad with zeros).
#include <algorithm>

#include "pqa_device.h"
#include "pqa_internal.h"

namespace pqa {

constexpr int kGemmBM = 256;
constexpr int kGemmBN = 192;
constexpr int kGemmBK = 64;
constexpr int kGemmWaves = 4;
constexpr int kGemmThreads = 64 * kGemmWaves;
constexpr int kGemmRowB = kGemmBK * 2;                          // 128 bytes per tile row
constexpr int kGemmABytes = kGemmBM * kGemmRowB;                // 32 KB
constexpr int kGemmStage = kGemmABytes + kGemmBN * kGemmRowB;   // 56 KB
constexpr int kGemmLoads = kGemmStage / 1024 / kGemmWaves;      // 1 KB DMA pieces per wave and tile (14)
constexpr int kGemmFrags = 7;                                   // operand reads per k-step (4 A + 3 B)
constexpr int kGemmMfmas = 12;                                  // MFMAs per k-step
static_assert(kGemmStage % (1024 * kGemmWaves) == 0, "whole 1 KB DMA pieces per wave");
static_assert(kGemmABytes % 1024 == 0, "A and B parts of a stage start on 1 KB boundaries");
static_assert(kGemmLoads <= kGemmMfmas + 2, "the loads of a tile fit between k-step 3's MFMAs");

__device__ __forceinline__ int gemm_swz(int r) { return (r >> 1) & 7; }

struct GemmArgs {
    const _Float16* a;
    const _Float16* b;
    float* c;
    int m, n, k, lda, ldb, ldc;
    int mb, nb;  // tile counts
};

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__global__ __launch_bounds__(kGemmThreads, 1) void gemm_f16_nt_kernel(const GemmArgs g) {
    __shared__ __attribute__((aligned(1024))) char lds[2][kGemmStage];

    // ---- tile of this workgroup ----
    const int T = g.mb * g.nb;
    const int xcd = blockIdx.x & 7, jx = blockIdx.x >> 3;
    const int q8 = T >> 3, r8 = T & 7;
    if (jx >= q8 + (xcd < r8 ? 1 : 0)) return;  // whole workgroup, before any barrier
    const int t = xcd * q8 + min(xcd, r8) + jx;
    const int tn = t / g.mb, tm = t - tn * g.mb;
    const int m0 = tm * kGemmBM, n0 = tn * kGemmBN;

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int KT = g.k / kGemmBK;

    // ---- loads: wave w fills the stage's 1 KB pieces w, w + 4, ...; a piece
    // is 8 tile rows; lane l lands at row l / 8, chunk position l % 8 and
    // fetches the chunk that belongs there ----
    unsigned goff[kGemmLoads];
    const _Float16* gbase[kGemmLoads];
    unsigned ldst[kGemmLoads];
#pragma unroll
    for (int ii = 0; ii < kGemmLoads; ii++) {
        const int piece = w + kGemmWaves * ii;
        const bool isa = piece < kGemmABytes / 1024;
        const int row = (isa ? 8 * piece : 8 * (piece - kGemmABytes / 1024)) + (lane >> 3);
        const int chunk = (lane & 7) ^ gemm_swz(row);
        if (isa) {
            const int gr = min(m0 + row, g.m - 1) - m0;
            gbase[ii] = g.a + (size_t)m0 * g.lda;
            goff[ii] = (unsigned)(((size_t)gr * g.lda + 8 * chunk) * 2);
        } else {
            const int gr = min(n0 + row, g.n - 1) - n0;
            gbase[ii] = g.b + (size_t)n0 * g.ldb;
            goff[ii] = (unsigned)(((size_t)gr * g.ldb + 8 * chunk) * 2);
        }
        ldst[ii] = (unsigned)(piece * 1024);
    }
    auto load = [&](int kt, int ii) {
        lds_dma_b128(gbase[ii] + (size_t)kt * kGemmBK, goff[ii], lds_addr(&lds[kt & 1][0]) + ldst[ii]);
    };

    // ---- operand reads: wave (wm, wn) = (w & 1, w >> 1); k-step s reads
    // chunk 2 s + l / 32 of its rows ----
    const int wm = w & 1, wn = w >> 1;
    const int l32 = lane & 31, hk = lane >> 5;
    int offa[4][4], offb[3][4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int c = 2 * s + hk;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = wm * 128 + 32 * i + l32;
            offa[i][s] = r * kGemmRowB + 16 * (c ^ gemm_swz(r));
        }
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const int r = wn * 96 + 32 * j + l32;
            offb[j][s] = kGemmABytes + r * kGemmRowB + 16 * (c ^ gemm_swz(r));
        }
    }
    half8 fa[2][4], fb[2][3];
    auto read = [&](int kt, int s, int slot, int idx) {
        const char* st = &lds[kt & 1][0];
        if (idx < 4) fa[slot][idx] = *(const half8*)(st + offa[idx][s]);
        else fb[slot][idx - 4] = *(const half8*)(st + offb[idx - 4][s]);
    };
    floatx16 acc[4][3];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 3; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;
    auto mfma = [&](int slot, int idx) {
        const int i = idx / 3, j = idx % 3;
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[slot][i], fb[slot][j], acc[i][j], 0, 0, 0);
    };
    // one k-step's MFMAs with the next k-step's reads between them
    auto kstep = [&](int slot, int rkt, int rs) {
#pragma unroll
        for (int idx = 0; idx < kGemmMfmas; idx++) {
            mfma(slot, idx);
            __builtin_amdgcn_sched_barrier(0);
            if (idx < kGemmFrags) read(rkt, rs, slot ^ 1, idx);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // ---- prologue: tiles 0 and 1 in flight, tile 0 landed everywhere ----
#pragma unroll
    for (int ii = 0; ii < kGemmLoads; ii++) load(0, ii);
    if (KT > 1) {
#pragma unroll
        for (int ii = 0; ii < kGemmLoads; ii++) load(1, ii);
        wait_vm<kGemmLoads>();
    } else {
        wait_vm<0>();
    }
    __syncthreads();
#pragma unroll
    for (int idx = 0; idx < kGemmFrags; idx++) read(0, 0, 0, idx);

    // Straight-line body (uniform branches only around the barrier, loads and
    // reads): a separate last-tile path made the compiler copy the
    // accumulators between AGPRs and VGPRs around every MFMA.
    for (int kt = 0; kt < KT; kt++) {
        const bool next = kt + 1 < KT;
        kstep(0, kt, 1);
        kstep(1, kt, 2);
        kstep(0, kt, 3);
        if (next) {
            wait_vm<0>();     // this wave's loads of tile kt + 1
            __syncthreads();  // everyone's; every read of tile kt has completed
        }
        // k-step 3: the reads of tile kt + 1's k-step 0 (the last tile re-reads
        // its own stage, unused) and the loads of tile kt + 2 into stage kt % 2
        const int kn = next ? kt + 1 : kt;
        const bool more = kt + 2 < KT;
#pragma unroll
        for (int idx = 0; idx < kGemmMfmas; idx++) {
            mfma(1, idx);
            __builtin_amdgcn_sched_barrier(0);
            if (more) {
                load(kt + 2, idx);
                if (idx < kGemmLoads - kGemmMfmas) load(kt + 2, kGemmMfmas + idx);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (idx < kGemmFrags) read(kn, 0, 0, idx);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // ---- store: lane l, register e of a 32 x 32 block holds row
    // 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32 ----
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

hipError_t launch_gemm_f16_nt(const _Float16* a, int lda, const _Float16* b, int ldb, float* c, int ldc, int m,
                              int n, int k, hipStream_t stream) {
    if (m <= 0 || n <= 0 || k <= 0 || k % kGemmBK != 0 || lda < k || ldb < k || ldc < n || lda % 8 || ldb % 8)
        return hipErrorInvalidValue;
    // the loads' per-workgroup byte offsets are 32-bit
    if ((size_t)kGemmBM * lda * 2 >= (1ull << 31) || (size_t)kGemmBN * ldb * 2 >= (1ull << 31))
        return hipErrorInvalidValue;
    GemmArgs g;
    g.a = a;
    g.b = b;
    g.c = c;
    g.m = m;
    g.n = n;
    g.k = k;
    g.lda = lda;
    g.ldb = ldb;
    g.ldc = ldc;
    g.mb = (m + kGemmBM - 1) / kGemmBM;
    g.nb = (n + kGemmBN - 1) / kGemmBN;
    const long long tiles = (long long)g.mb * g.nb;
    const long long groups = (tiles + 7) / 8 * 8;
    if (groups > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gemm_f16_nt_kernel, dim3((unsigned)groups), dim3(kGemmThreads), 0, stream, g);
    return hipGetLastError();
}

}  // namespace pqa
