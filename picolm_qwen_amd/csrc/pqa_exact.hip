// The K and V projections of a whole prompt in the reference's own summation
// order, so that the cache rows a prompt writes are the reference's bits.
//
// Model::forward_batch projects each prompt token with TensorOps::matmul_bias
// (cpp/model.hpp:503-546 -> cpp/tensor.hpp:134-143), and vec_dot
// (cpp/quant.hpp:342-356) fixes the order of every sum:
//   F32 rows, and F16 / Q4_0 / Q4_K / Q6_K rows after dequantize_row
//   (cpp/quant.hpp:176-281): vec_dot_f32_f32's SSE2 loop (:297-319), two
//   4-lane accumulators over groups of 8, i.e. 8 chains (element i goes to
//   chain i mod 8, in increasing i), every product and sum rounded on its
//   own; then t_l = chain l + chain l+4 and (t0 + t2) + (t1 + t3) (:288-294);
//   Q8_0 rows (:321-340): per 32-element block sum += q * x in order, then
//   sumf += d * sum in block order;
//   then out + bias (vec_add).
// Nothing here reorders a sum: each kernel is a register-tiled VALU GEMM whose
// lanes each own one chain (or, for Q8_0, whole rows of blocks) of 64 (token,
// row) pairs and walk that chain's elements in increasing order, with
// separate multiply and add instructions (built with -ffp-contract=off). MFMA
// and tree reductions would round differently. The outputs are bit-identical
// to the reference's matmul_bias built without FMA contraction, like
// pqa_qkv_project for one token.
//
// ordered_dot_kernel (every type but Q8_0): workgroup = 64 tokens x 64 rows,
// 8 waves. Wave w owns tokens 8w .. 8w+7; lane = 8 rg + p owns rows
// 8 rg .. 8 rg+7 and chain c(p) (p < 4: chain p; p >= 4: chain 11 - p, so
// that chain l+4 sits at lane p ^ 7, DPP row_half_mirror). Per 64-element k
// tile the operands are staged in LDS with chain c's 8 elements at columns
// 4c .. 4c+3 (first 32) and 32 + 4c .. +3 (second 32), so a lane reads its
// chain as two 16-byte words per row. 64 products and 64 sums per lane per
// element of the chain: the kernel is bound by VALU issue.
//
// ordered_q8_kernel: workgroup = 64 tokens x 64 rows, 4 waves; thread (tg,
// rg) owns tokens tg + 16 i and rows rg + 16 j (i, j < 4) over every element
// in order, one 32-element block per LDS stage.
#include <algorithm>

#include "pqa_device.h"
#include "pqa_internal.h"

namespace pqa {

constexpr int kOrdTile = 64;                      // tokens and rows per workgroup, k elements per stage
constexpr int kOrdThreads = 512;                  // ordered_dot_kernel
constexpr int kOrdRowF = kOrdTile + 4;            // LDS row stride in floats (272 bytes: staging writes spread over banks)
constexpr int kQ8Threads = 256;                   // ordered_q8_kernel
constexpr int kQ8RowF = 36;                       // LDS row stride of one 32-element block row (+4 floats)

struct OrderedArgs {
    const float* x;  // [n_tok][ldx] fp32 inputs
    const float* w;  // [rows][n]: fp32 rows (dequantized), or for Q8_0 the int8 values as floats
    const float* d;  // Q8_0: [rows][n / 32] block scales; else unused
    int n_tok, rows, n, ldx;
    const uint8_t* b;  // bias [rows] (F32 or F16) or null
    int bt;
    float* out;  // out[t * ldo + r]
    int ldo;
};

__device__ __forceinline__ float ord_bias(const uint8_t* b, int bt, int r) {
    return bt == GG_F32 ? ((const float*)b)[r] : f16_bits_to_f32(((const uint16_t*)b)[r]);
}

// 16 bytes of row `row` at element k (k + 4 <= n, or zeros past n; n is a
// multiple of 4). ALIGNED: the row base is 16-byte aligned.
template <bool ALIGNED>
__device__ __forceinline__ float4 ord_load4(const float* base, size_t ld, int row, int k, int n) {
    if (k >= n) return float4{0.0f, 0.0f, 0.0f, 0.0f};
    const float* p = base + (size_t)row * ld + k;
    if constexpr (ALIGNED) return *(const float4*)p;
    return float4{p[0], p[1], p[2], p[3]};
}

// chain of lane position p within its 8 lanes (see the file comment)
__device__ __forceinline__ int ord_chain(int p) { return p < 4 ? p : 11 - p; }

// Natural element k (0..63) of a tile -> LDS column: chain c = k & 7, its
// element j = k >> 3 at column 32 (j >> 2) + 4 c + (j & 3).
__device__ __forceinline__ int ord_col(int k) { return 32 * (k >> 5) + 4 * (k & 7) + ((k >> 3) & 3); }

template <bool XALIGNED>
__global__ __launch_bounds__(kOrdThreads) void ordered_dot_kernel(const OrderedArgs a) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float xs[2][kOrdTile * kOrdRowF];
    __shared__ __attribute__((aligned(16))) float ws[2][kOrdTile * kOrdRowF];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int p = lane & 7, rg = lane >> 3;
    const int c = ord_chain(p);
    const int t0 = blockIdx.y * kOrdTile, r0 = blockIdx.x * kOrdTile;
    const int ntile = (a.n + kOrdTile - 1) / kOrdTile;

    // staging: thread tid moves float4 s = tid + 512 i (i < 2) of each
    // operand tile: tile row s / 16 (clamped to the last token / row), natural
    // elements 4 (s % 16) .. +3, written to their chain columns
    int srow[2], sk[2], scol[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int s = tid + kOrdThreads * i;
        srow[i] = s >> 4;
        sk[i] = 4 * (s & 15);
        scol[i] = ord_col(sk[i]);  // elements sk .. sk+3 share chain-element j, chains c .. c+3
    }
    auto load = [&](int tile, float4* xr, float4* wr) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int k = tile * kOrdTile + sk[i];
            xr[i] = ord_load4<XALIGNED>(a.x, a.ldx, min(t0 + srow[i], a.n_tok - 1), k, a.n);
            wr[i] = ord_load4<true>(a.w, a.n, min(r0 + srow[i], a.rows - 1), k, a.n);
        }
    };
    auto store = [&](int buf, const float4* xr, const float4* wr) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            float* xd = &xs[buf][srow[i] * kOrdRowF + scol[i]];
            float* wd = &ws[buf][srow[i] * kOrdRowF + scol[i]];
            xd[0] = xr[i].x, xd[4] = xr[i].y, xd[8] = xr[i].z, xd[12] = xr[i].w;
            wd[0] = wr[i].x, wd[4] = wr[i].y, wd[8] = wr[i].z, wd[12] = wr[i].w;
        }
    };

    float acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[i][j] = 0.0f;

    float4 xr[2], wr[2];
    load(0, xr, wr);
    store(0, xr, wr);
    __syncthreads();
    for (int tile = 0; tile < ntile; tile++) {
        const int buf = tile & 1;
        const bool more = tile + 1 < ntile;
        if (more) load(tile + 1, xr, wr);
        const float* xb = &xs[buf][(8 * w) * kOrdRowF + 4 * c];
        const float* wb = &ws[buf][(8 * rg) * kOrdRowF + 4 * c];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float4 xv[8], wv[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                xv[i] = *(const float4*)(xb + i * kOrdRowF + 32 * h);
                wv[i] = *(const float4*)(wb + i * kOrdRowF + 32 * h);
            }
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int i = 0; i < 8; i++)
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const float xe = e == 0 ? xv[i].x : e == 1 ? xv[i].y : e == 2 ? xv[i].z : xv[i].w;
                        const float we = e == 0 ? wv[j].x : e == 1 ? wv[j].y : e == 2 ? wv[j].z : wv[j].w;
                        acc[i][j] = acc[i][j] + we * xe;
                    }
        }
        if (more) store(buf ^ 1, xr, wr);
        __syncthreads();
    }

    // t = chain l + chain l+4 (lane p ^ 7), then (t0 + t2) + (t1 + t3): the
    // partners are symmetric, so all 8 lanes of a group end with the same bits
    // (a + b == b + a). Lane p then stores token 8w + p's 8 rows.
    const int tok = t0 + 8 * w + p;
    float res[8];
#pragma unroll
    for (int j = 0; j < 8; j++) res[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float v = acc[i][j];
            v = v + dpp_f<kDppXor7>(v);
            v = v + dpp_f<kDppXor2>(v);
            v = v + dpp_f<kDppXor1>(v);
            if (i == p) res[j] = v;
        }
    if (tok < a.n_tok) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int r = r0 + 8 * rg + j;
            if (r < a.rows) a.out[(size_t)tok * a.ldo + r] = a.b ? res[j] + ord_bias(a.b, a.bt, r) : res[j];
        }
    }
}

template <bool XALIGNED>
__global__ __launch_bounds__(kQ8Threads) void ordered_q8_kernel(const OrderedArgs a) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float xs[2][kOrdTile * kQ8RowF];
    __shared__ __attribute__((aligned(16))) float ws[2][kOrdTile * kQ8RowF];
    __shared__ float ds[2][kOrdTile];
    const int tid = threadIdx.x;
    const int tg = tid >> 4, rg = tid & 15;
    const int t0 = blockIdx.y * kOrdTile, r0 = blockIdx.x * kOrdTile;
    const int nblk = a.n / 32;

    // staging: 64 rows x 8 float4 per operand; thread tid moves float4 s = tid
    // + 256 i (i < 2): row s / 8, elements 4 (s % 8) .. +3 of the block
    auto load = [&](int blk, float4* xr, float4* wr, float& dr) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int s = tid + kQ8Threads * i;
            const int k = 32 * blk + 4 * (s & 7);
            xr[i] = ord_load4<XALIGNED>(a.x, a.ldx, min(t0 + (s >> 3), a.n_tok - 1), k, a.n);
            wr[i] = ord_load4<true>(a.w, a.n, min(r0 + (s >> 3), a.rows - 1), k, a.n);
        }
        dr = tid < kOrdTile ? a.d[(size_t)min(r0 + tid, a.rows - 1) * nblk + blk] : 0.0f;
    };
    auto store = [&](int buf, const float4* xr, const float4* wr, float dr) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int s = tid + kQ8Threads * i;
            *(float4*)&xs[buf][(s >> 3) * kQ8RowF + 4 * (s & 7)] = xr[i];
            *(float4*)&ws[buf][(s >> 3) * kQ8RowF + 4 * (s & 7)] = wr[i];
        }
        if (tid < kOrdTile) ds[buf][tid] = dr;
    };

    float sumf[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) sumf[i][j] = 0.0f;

    float4 xr[2], wr[2];
    float dr;
    load(0, xr, wr, dr);
    store(0, xr, wr, dr);
    __syncthreads();
    for (int blk = 0; blk < nblk; blk++) {
        const int buf = blk & 1;
        const bool more = blk + 1 < nblk;
        if (more) load(blk + 1, xr, wr, dr);
        float sum[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) sum[i][j] = 0.0f;
#pragma unroll 2
        for (int k4 = 0; k4 < 8; k4++) {
            float4 xv[4], wv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                xv[i] = *(const float4*)&xs[buf][(tg + 16 * i) * kQ8RowF + 4 * k4];
                wv[i] = *(const float4*)&ws[buf][(rg + 16 * i) * kQ8RowF + 4 * k4];
            }
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float xe = e == 0 ? xv[i].x : e == 1 ? xv[i].y : e == 2 ? xv[i].z : xv[i].w;
                        const float qe = e == 0 ? wv[j].x : e == 1 ? wv[j].y : e == 2 ? wv[j].z : wv[j].w;
                        sum[i][j] = sum[i][j] + qe * xe;
                    }
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float dj = ds[buf][rg + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; i++) sumf[i][j] = sumf[i][j] + dj * sum[i][j];
        }
        if (more) store(buf ^ 1, xr, wr, dr);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int tok = t0 + tg + 16 * i;
        if (tok >= a.n_tok) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = r0 + rg + 16 * j;
            if (r < a.rows) a.out[(size_t)tok * a.ldo + r] = a.b ? sumf[i][j] + ord_bias(a.b, a.bt, r) : sumf[i][j];
        }
    }
}

// Q8_0 rows -> the int8 values as floats [rows][n] and the block scales
// [rows][n / 32] (fp16 d widened exactly). One thread per 32-element block.
__global__ __launch_bounds__(256) void q8_unpack_kernel(const uint8_t* __restrict__ w, int stride, int rows, int n,
                                                        float* __restrict__ q, float* __restrict__ d) {
    const int nblk = n / 32;
    const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (long long)rows * nblk) return;
    const int row = (int)(gid / nblk), blk = (int)(gid % nblk);
    const uint8_t* b = w + (size_t)row * stride + 34 * blk;
    d[gid] = f16_bits_to_f32((uint16_t)(b[0] | (b[1] << 8)));
    float* o = q + (size_t)row * n + 32 * blk;
    for (int j = 0; j < 32; j++) o[j] = (float)(int8_t)b[2 + j];
}

// Floats of a matrix's prepared copy: [rows][n] (+ [rows][n / 32] for Q8_0).
size_t exact_matrix_floats(int type, int rows, int n) {
    return (size_t)rows * n + (type == GG_Q8_0 ? (size_t)rows * (n / 32) : 0);
}

hipError_t prepare_exact_matrix(int type, const void* w, int stride, int rows, int n, float* dst, hipStream_t s) {
    if (type == GG_Q8_0) {
        const long long items = (long long)rows * (n / 32);
        hipLaunchKernelGGL(q8_unpack_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, s,
                           (const uint8_t*)w, stride, rows, n, dst, dst + (size_t)rows * n);
        return hipGetLastError();
    }
    return launch_dequant_rows(type, w, stride, rows, n, dst, s);
}

hipError_t launch_ordered_project(int type, const float* prepared, int rows, int n, const float* x, int ldx, int n_tok,
                                  const void* bias, int btype, float* out, int ldo, hipStream_t s) {
    if (rows <= 0 || n_tok <= 0 || n <= 0 || n % 8 || ldx < n) return hipErrorInvalidValue;
    OrderedArgs a;
    a.x = x;
    a.w = prepared;
    a.d = type == GG_Q8_0 ? prepared + (size_t)rows * n : nullptr;
    a.n_tok = n_tok;
    a.rows = rows;
    a.n = n;
    a.ldx = ldx;
    a.b = (const uint8_t*)bias;
    a.bt = btype;
    a.out = out;
    a.ldo = ldo;
    const dim3 grid((unsigned)((rows + kOrdTile - 1) / kOrdTile), (unsigned)((n_tok + kOrdTile - 1) / kOrdTile));
    const bool xal = ((uintptr_t)x & 15) == 0 && ldx % 4 == 0;
    if (type == GG_Q8_0) {
        if (n % 32) return hipErrorInvalidValue;
        if (xal)
            hipLaunchKernelGGL(ordered_q8_kernel<true>, grid, dim3(kQ8Threads), 0, s, a);
        else
            hipLaunchKernelGGL(ordered_q8_kernel<false>, grid, dim3(kQ8Threads), 0, s, a);
    } else {
        if (xal)
            hipLaunchKernelGGL(ordered_dot_kernel<true>, grid, dim3(kOrdThreads), 0, s, a);
        else
            hipLaunchKernelGGL(ordered_dot_kernel<false>, grid, dim3(kOrdThreads), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace pqa
