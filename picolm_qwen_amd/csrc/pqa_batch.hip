// Q/K/V projections of a whole prompt: the per-token matmul_bias calls of
// Model::forward_batch (cpp/model.hpp:493-530) as one GEMM per matrix over
// all tokens, feeding the MFMA prefill.
//
// Each GGUF matrix is first dequantized into an fp32 workspace by the
// expressions of dequantize_row_* (cpp/quant.hpp:176-281), exactly. Then
// Y[n_tok][rows] = X[n_tok][n] W^T runs on the fp16 MFMA path with fp32
// accumulation (gemm_f16x3_nt_kernel, pqa_gemm.hip):
//   every row a of W and of X is scaled by a power of two 2^s (exact) so that
//   max |a 2^s| lies in [2^14, 2^15), and split into hi = fp16(a 2^s) and
//   lo = fp16(a 2^s - hi), which carry 22 of its 24 significand bits;
//   rows are stored as [hi | lo], each half padded with zeros to a multiple
//   of 32, and the GEMM sums w_hi x_hi + w_hi x_lo + w_lo x_hi, dropping
//   w_lo x_lo (about 2^-22 of |w x|); fp16 products are exact in fp32;
//   the result is scaled back by 2^-(s_w + s_x) (exact), then the bias is
//   added (vec_add: out + b).
// The error stays within (3n + 12) 2^-24 sum |w x| for any summation order
// the GEMM takes over its 3n products, so q/k/v agree with the reference to
// fp32 rounding (about 1e-6 relative) rather than bit for bit.
// pqa_qkv_project keeps the reference's order for one token.
#include <hip/hip_fp16.h>

#include <algorithm>
#include <string>

#include "pqa_device.h"
#include "pqa_internal.h"

namespace pqa {

__device__ __forceinline__ float bh2f(unsigned h) { return (float)__builtin_bit_cast(_Float16, (unsigned short)h); }
__device__ __forceinline__ unsigned bld16(const uint8_t* p) { return p[0] | ((unsigned)p[1] << 8); }

// One thread per 32 elements of a row: dst[row][32 g .. 32 g + 31]. F32 and
// F16 rows (block size 1) may end in a partial group; every other type's row
// is whole 32-element groups.
template <int T>
__global__ __launch_bounds__(256) void dequant_rows_kernel(const uint8_t* __restrict__ w, int stride, int rows, int n,
                                                           float* __restrict__ dst) {
    const int groups = (n + 31) / 32;
    const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (long long)rows * groups) return;
    const int row = (int)(gid / groups), g = (int)(gid % groups);
    const uint8_t* r = w + (size_t)row * stride;
    float* y = dst + (size_t)row * n + 32 * g;
    if constexpr (T == GG_F32) {
        const float* s = (const float*)(r + 128 * g);
        const int cnt = min(32, n - 32 * g);
        for (int j = 0; j < cnt; j++) y[j] = s[j];
    } else if constexpr (T == GG_F16) {
        const int cnt = min(32, n - 32 * g);
        for (int j = 0; j < cnt; j++) y[j] = bh2f(bld16(r + 64 * g + 2 * j));
    } else if constexpr (T == GG_Q4_0) {  // d * ((float)nibble - 8)
        const uint8_t* b = r + 18 * g;
        const float d = bh2f(bld16(b));
        for (int j = 0; j < 32; j++) {
            const unsigned nib = j < 16 ? (b[2 + j] & 0xF) : (b[2 + j - 16] >> 4);
            y[j] = d * ((float)nib - 8.0f);
        }
    } else if constexpr (T == GG_Q8_0) {  // d * q
        const uint8_t* b = r + 34 * g;
        const float d = bh2f(bld16(b));
        for (int j = 0; j < 32; j++) y[j] = d * (float)(int8_t)b[2 + j];
    } else if constexpr (T == GG_Q4_K) {  // sub-block is = g % 8 of block g / 8: d1 * q - m1
        const uint8_t* b = r + 144 * (g >> 3);
        const int is = g & 7, jj = is >> 1, hi = is & 1;
        const uint8_t* q = b + 16 + 32 * jj;
        unsigned sc, mn;
        if (is < 4) {
            sc = b[4 + is] & 63;
            mn = b[8 + is] & 63;
        } else {
            sc = (b[8 + is] & 0xF) | ((b[is] >> 6) << 4);
            mn = (b[8 + is] >> 4) | ((b[4 + is] >> 6) << 4);
        }
        const float d1 = bh2f(bld16(b)) * (float)sc, m1 = bh2f(bld16(b + 2)) * (float)mn;
        for (int l = 0; l < 32; l++) y[l] = d1 * (float)(hi ? (q[l] >> 4) : (q[l] & 0xF)) - m1;
    } else if constexpr (T == GG_Q6_K) {  // element e of a block: (d * sc) * q
        const uint8_t* b = r + 210 * (g >> 3);
        const float d = bh2f(bld16(b + 208));
        for (int j = 0; j < 32; j++) {
            const int e = 32 * (g & 7) + j, h = e >> 7, quad = (e >> 5) & 3, l = e & 31;
            const unsigned lb = b[64 * h + l + 32 * (quad & 1)];
            const unsigned lo = quad < 2 ? (lb & 0xF) : (lb >> 4);
            const unsigned hb = (b[128 + 32 * h + l] >> (2 * quad)) & 3;
            const int qv = (int)(lo | (hb << 4)) - 32;
            y[j] = d * (float)(int)(int8_t)b[192 + 8 * h + (l >> 4) + 2 * quad] * (float)qv;
        }
    }
}

// One workgroup per row of n floats: max |a| over the row, the power of two
// 2^s that takes it into [2^14, 2^15), dst row = the hi and lo fp16 halves of
// a 2^s as [hi | lo], each kh halfs wide (kh >= n, zeros past n), and
// inv_scale[row] = 2^-s.
__device__ __forceinline__ float split_max(float mx, float* s_max) {
    mx = group_max<64>(mx);
    if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = mx;
    __syncthreads();
    return fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
}

// mx in [2^e, 2^(e+1)): s = 14 - e; an all-zero row keeps s = 0
__device__ __forceinline__ int split_shift(float mx) { return mx > 0.0f ? min(126, max(-126, 14 - ilogbf(mx))) : 0; }

__global__ __launch_bounds__(256) void split2_kernel(const float* __restrict__ src, int n, _Float16* __restrict__ dst,
                                                     int kh, float* __restrict__ inv_scale) {
    __shared__ float s_max[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float* a = src + (size_t)row * n;
    _Float16* d = dst + (size_t)row * 2 * kh;
    for (int i = n + tid; i < kh; i += 256) {
        d[i] = (_Float16)0.0f;
        d[kh + i] = (_Float16)0.0f;
    }
    float mx = 0.0f;
    for (int i = tid; i < n; i += 256) mx = fmaxf(mx, fabsf(a[i]));
    mx = split_max(mx, s_max);
    const int s = split_shift(mx);
    const float sc = ldexpf(1.0f, s);
    if (tid == 0) inv_scale[row] = ldexpf(1.0f, -s);
    for (int i = tid; i < n; i += 256) {
        const float v = a[i] * sc;
        const _Float16 hi = (_Float16)v;
        d[i] = hi;
        d[kh + i] = (_Float16)(v - (float)hi);
    }
}

// The same split for rows of n % 4 == 0, n <= 256 * 4 * kSplitVec floats, 16-byte
// aligned: the row is read once into registers as float4s and written as
// half4s (same arithmetic, same bits).
constexpr int kSplitVec = 8;
__global__ __launch_bounds__(256) void split2_vec_kernel(const float* __restrict__ src, int n,
                                                         _Float16* __restrict__ dst, int kh,
                                                         float* __restrict__ inv_scale) {
    __shared__ float s_max[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    const int n4 = n >> 2;
    const float4* a = (const float4*)(src + (size_t)row * n);
    _Float16* d = dst + (size_t)row * 2 * kh;
    for (int i = n + tid; i < kh; i += 256) {
        d[i] = (_Float16)0.0f;
        d[kh + i] = (_Float16)0.0f;
    }
    float4 v[kSplitVec];
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < kSplitVec; j++) {
        const int i = tid + 256 * j;
        v[j] = i < n4 ? a[i] : float4{0.0f, 0.0f, 0.0f, 0.0f};
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    }
    mx = split_max(mx, s_max);
    const int s = split_shift(mx);
    const float sc = ldexpf(1.0f, s);
    if (tid == 0) inv_scale[row] = ldexpf(1.0f, -s);
#pragma unroll
    for (int j = 0; j < kSplitVec; j++) {
        const int i = tid + 256 * j;
        if (i >= n4) break;
        const float x[4] = {v[j].x * sc, v[j].y * sc, v[j].z * sc, v[j].w * sc};
        half4 hi, lo;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            hi[e] = (_Float16)x[e];
            lo[e] = (_Float16)(x[e] - (float)hi[e]);
        }
        *(half4*)(d + 4 * i) = hi;
        *(half4*)(d + kh + 4 * i) = lo;
    }
}

// one workgroup per row of src [rows][n] into dst [rows][2 kh], kh = k_half(n)
static void launch_split2(const float* src, int rows, int n, _Float16* dst, int kh, float* inv_scale,
                          hipStream_t stream) {
    const bool vec = n % 4 == 0 && n <= 256 * 4 * kSplitVec && ((uintptr_t)src & 15) == 0;
    if (vec)
        hipLaunchKernelGGL(split2_vec_kernel, dim3(rows), dim3(256), 0, stream, src, n, dst, kh, inv_scale);
    else
        hipLaunchKernelGGL(split2_kernel, dim3(rows), dim3(256), 0, stream, src, n, dst, kh, inv_scale);
}

// each half of a split row: n rounded up to the GEMM's 32-wide k tiles
static int k_half(int n) { return (n + 31) / 32 * 32; }

// The three outputs of the batched GEMM and their biases.
struct ScatterArgs {
    float* out[3];
    const uint8_t* b[3];
    int btype[3];
    int rows[3];
};

// Y [n_tok][ld] holds q|k|v of every token scaled by 2^(s_w + s_x):
// out_m[t][r] = Y[t][off_m + r] * 2^-(s_w + s_x), an exact rescale, then
// out + b[r] (vec_add, cpp/tensor.hpp:410-420), for the first ncols columns.
// Thread: 4 consecutive rows of one token (rows of q and kv are multiples of 4).
__global__ __launch_bounds__(256) void unscale_scatter_kernel(const float* __restrict__ Y, int ld, int ncols,
                                                              const float* __restrict__ w_inv,
                                                              const float* __restrict__ x_inv, const ScatterArgs a) {
    const int t = blockIdx.y;
    const int r = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (r >= ncols) return;
    const int m = r < a.rows[0] ? 0 : (r < a.rows[0] + a.rows[1] ? 1 : 2);
    const int rr = r - (m > 0 ? a.rows[0] : 0) - (m > 1 ? a.rows[1] : 0);
    const floatx4 y = *(const floatx4*)(Y + (size_t)t * ld + r);
    const floatx4 wi = *(const floatx4*)(w_inv + r);
    const float xi = x_inv[t];
    floatx4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        float v = y[e] * (wi[e] * xi);
        if (a.b[m]) v = v + (a.btype[m] == GG_F32 ? ((const float*)a.b[m])[rr + e] : bh2f(bld16(a.b[m] + 2 * (rr + e))));
        o[e] = v;
    }
    *(floatx4*)(a.out[m] + (size_t)t * a.rows[m] + rr) = o;
}

// The output projection of a prompt: Y [n_tok][rows] holds attn W_o^T scaled
// by 2^(s_w + s_x); x[t][r] = x[t][r] + (Y[t][r] * 2^-(s_w + s_x) + b[r]),
// the reference's matmul_bias then vec_add (cpp/model.hpp:595-600). Thread: 4
// consecutive rows of one token (rows a multiple of 4).
__global__ __launch_bounds__(256) void unscale_residual_kernel(const float* __restrict__ Y, int rows,
                                                               const float* __restrict__ w_inv,
                                                               const float* __restrict__ x_inv,
                                                               const uint8_t* __restrict__ b, int btype,
                                                               float* __restrict__ x) {
    const int t = blockIdx.y;
    const int r = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (r >= rows) return;
    const floatx4 y = *(const floatx4*)(Y + (size_t)t * rows + r);
    const floatx4 wi = *(const floatx4*)(w_inv + r);
    const float xi = x_inv[t];
    floatx4* xp = (floatx4*)(x + (size_t)t * rows + r);
    floatx4 o = *xp;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        float v = y[e] * (wi[e] * xi);
        if (b) v = v + (btype == GG_F32 ? ((const float*)b)[r + e] : bh2f(bld16(b + 2 * (r + e))));
        o[e] = o[e] + v;
    }
    *xp = o;
}

hipError_t launch_dequant_rows(int type, const void* w, int stride, int rows, int n, float* dst, hipStream_t s) {
    const long long items = (long long)rows * ((n + 31) / 32);
    const dim3 grid((unsigned)((items + 255) / 256));
    switch (type) {
#define PQA_DQ(T) \
    case T: hipLaunchKernelGGL(dequant_rows_kernel<T>, grid, dim3(256), 0, s, (const uint8_t*)w, stride, rows, n, dst); break;
        PQA_DQ(GG_F32) PQA_DQ(GG_F16) PQA_DQ(GG_Q4_0) PQA_DQ(GG_Q8_0) PQA_DQ(GG_Q4_K) PQA_DQ(GG_Q6_K)
#undef PQA_DQ
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace pqa

using pqa::hip_check;
using pqa::set_err;

// The fp32 weight workspace of a context, made on the first batched call.
static int ensure_batch(pqa_ctx* ctx, size_t wfloats, const char* fn) {
    if (wfloats > ctx->wf32_floats) {
        // earlier dequantizations on the stream may still write the old one
        if (int rc = hip_check(ctx, hipStreamSynchronize(ctx->stream), fn)) return rc;
        if (ctx->wf32) (void)hipFree(ctx->wf32);
        ctx->wf32 = nullptr;
        ctx->wf32_floats = 0;
        if (int rc = hip_check(ctx, hipMalloc(&ctx->wf32, wfloats * 4), fn)) return rc;
        ctx->wf32_floats = wfloats;
    }
    return PQA_OK;
}

void pqa_free_batch(pqa_ctx* c) {
    if (c->wf32) (void)hipFree(c->wf32);
    c->wf32 = nullptr;
    if (c->bsplit) (void)hipFree(c->bsplit);
    c->bsplit = nullptr;
    c->bsplit_bytes = 0;
    if (c->battn) (void)hipFree(c->battn);
    c->battn = nullptr;
    c->battn_floats = 0;
}

static size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

// A layer's W' = [hi | lo] rows of attn_q, attn_k and attn_v, one after the
// other ([total][2 k_half(n)] halfs), then their inverse scales: made once, on
// the first batched call for the layer (dequantized through the fp32 workspace).
// The attn_output rows get the same form in out_split ([n_embd][2 k_half(q_dim)]).
static int ensure_layer_split(pqa_ctx* ctx, int layer, const char* fn) {
    auto& p = ctx->proj[layer];
    if (p.split) return PQA_OK;
    const int n = p.n_embd;
    const int rows[3] = {(int)ctx->q_dim, (int)ctx->kv_dim, (int)ctx->kv_dim};
    const size_t total = ctx->q_dim + 2 * ctx->kv_dim;
    const int kh = pqa::k_half(n);
    const size_t wb = up256(total * 2 * kh * 2);
    if (int rc = ensure_batch(ctx, ctx->q_dim * (size_t)n, fn)) return rc;
    void* buf = nullptr;
    if (int rc = hip_check(ctx, hipMalloc(&buf, wb + up256(total * 4)), fn)) return rc;
    _Float16* w3 = (_Float16*)buf;
    float* w_inv = (float*)((char*)buf + wb);
    size_t off = 0;
    for (int i = 0; i < 3; i++) {
        hipError_t e = pqa::launch_dequant_rows(p.wtype[i], p.w[i], p.stride[i], rows[i], n, ctx->wf32, ctx->stream);
        if (e == hipSuccess) {
            pqa::launch_split2((const float*)ctx->wf32, rows[i], n, w3 + off * 2 * kh, kh, w_inv + off, ctx->stream);
            e = hipGetLastError();
        }
        if (int rc = hip_check(ctx, e, fn)) {
            (void)hipFree(buf);
            return rc;
        }
        off += rows[i];
    }
    p.split = buf;
    return PQA_OK;
}

static int ensure_layer_out_split(pqa_ctx* ctx, int layer, const char* fn) {
    auto& p = ctx->proj[layer];
    if (p.out_split) return PQA_OK;
    const int n = (int)ctx->q_dim, rows = p.out_rows;
    const int kh = pqa::k_half(n);
    const size_t wb = up256((size_t)rows * 2 * kh * 2);
    if (int rc = ensure_batch(ctx, (size_t)rows * n, fn)) return rc;
    void* buf = nullptr;
    if (int rc = hip_check(ctx, hipMalloc(&buf, wb + up256((size_t)rows * 4)), fn)) return rc;
    hipError_t e = pqa::launch_dequant_rows(p.wtype[3], p.w[3], p.stride[3], rows, n, ctx->wf32, ctx->stream);
    if (e == hipSuccess) {
        pqa::launch_split2((const float*)ctx->wf32, rows, n, (_Float16*)buf, kh, (float*)((char*)buf + wb),
                           ctx->stream);
        e = hipGetLastError();
    }
    if (int rc = hip_check(ctx, e, fn)) {
        (void)hipFree(buf);
        return rc;
    }
    p.out_split = buf;
    return PQA_OK;
}

// The layer's attn_k and attn_v rows prepared for the reference-order
// projection (pqa_exact.hip), made on the first call that needs them.
static int ensure_layer_exact(pqa_ctx* ctx, int layer, const char* fn) {
    auto& p = ctx->proj[layer];
    if (p.exact) return PQA_OK;
    const int n = p.n_embd, rows = (int)ctx->kv_dim;
    const size_t fk = pqa::exact_matrix_floats(p.wtype[1], rows, n);
    const size_t fv = pqa::exact_matrix_floats(p.wtype[2], rows, n);
    float* buf = nullptr;
    if (int rc = hip_check(ctx, hipMalloc(&buf, (fk + fv) * 4), fn)) return rc;
    hipError_t e = pqa::prepare_exact_matrix(p.wtype[1], p.w[1], p.stride[1], rows, n, buf, ctx->stream);
    if (e == hipSuccess) e = pqa::prepare_exact_matrix(p.wtype[2], p.w[2], p.stride[2], rows, n, buf + fk, ctx->stream);
    if (int rc = hip_check(ctx, e, fn)) {
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipFree(buf);
        return rc;
    }
    p.exact = buf;
    return PQA_OK;
}

// k[t * ldo + r] and v[t * ldo + r] = the attn_k / attn_v matmul_bias of token
// t in the reference's order (pqa_exact.hip), bit-exact.
static int exact_kv(pqa_ctx* ctx, int layer, int n_tok, const float* xb, float* k, float* v, int ldo, const char* fn) {
    if (int rc = ensure_layer_exact(ctx, layer, fn)) return rc;
    const auto& p = ctx->proj[layer];
    const int n = p.n_embd, rows = (int)ctx->kv_dim;
    const float* wk = p.exact;
    const float* wv = p.exact + pqa::exact_matrix_floats(p.wtype[1], rows, n);
    hipError_t e = pqa::launch_ordered_project(p.wtype[1], wk, rows, n, xb, n, n_tok, p.b[1], p.btype[1], k, ldo,
                                               ctx->stream);
    if (e == hipSuccess)
        e = pqa::launch_ordered_project(p.wtype[2], wv, rows, n, xb, n, n_tok, p.b[2], p.btype[2], v, ldo, ctx->stream);
    return hip_check(ctx, e, fn);
}

// Per call: X' [n_tok][2 k_half(n)] halfs, the inverse scales of X's rows, and
// the GEMM result Y [n_tok][total] floats. The workspace grows on demand; work
// queued earlier on the stream may still read the old one, so the stream is
// drained before it is freed.
static int grow_split(pqa_ctx* ctx, size_t need, const char* fn) {
    if (need <= ctx->bsplit_bytes) return PQA_OK;
    if (int rc = hip_check(ctx, hipStreamSynchronize(ctx->stream), fn)) return rc;
    if (ctx->bsplit) (void)hipFree(ctx->bsplit);
    ctx->bsplit = nullptr;
    ctx->bsplit_bytes = 0;
    if (int rc = hip_check(ctx, hipMalloc(&ctx->bsplit, need), fn)) return rc;
    ctx->bsplit_bytes = need;
    return PQA_OK;
}
struct SplitBufs {
    _Float16* x3;
    float* x_inv;
    float* y;
};

static size_t split_need(int n_tok, int n, size_t total) {
    return up256((size_t)n_tok * 2 * pqa::k_half(n) * 2) + up256((size_t)n_tok * 4) + (size_t)n_tok * total * 4;
}

static int ensure_split(pqa_ctx* ctx, int n_tok, int n, size_t total, SplitBufs* sb, const char* fn) {
    const size_t xb = up256((size_t)n_tok * 2 * pqa::k_half(n) * 2), xs = up256((size_t)n_tok * 4);
    if (int rc = grow_split(ctx, split_need(n_tok, n, total), fn)) return rc;
    char* base = (char*)ctx->bsplit;
    sb->x3 = (_Float16*)base;
    sb->x_inv = (float*)(base + xb);
    sb->y = (float*)(base + xb + xs);
    return PQA_OK;
}

// X' and the GEMM of one call: sb->y [n_tok][q_dim + 2 kv_dim] = X W^T, every
// element scaled by 2^(s_w[c] + s_x[t]); *w_inv = the inverse column scales.
// q_only: the GEMM covers the q columns alone (the reference-order projection
// fills the k and v columns).
static int batch_gemm(pqa_ctx* ctx, int layer, int n_tok, const float* xb, SplitBufs* sb, const float** w_inv,
                      const char* fn, bool q_only = false) {
    const int n = ctx->proj[layer].n_embd;
    if (int rc = ensure_layer_split(ctx, layer, fn)) return rc;
    const auto& p = ctx->proj[layer];
    const size_t total = ctx->q_dim + 2 * ctx->kv_dim;
    const int kh = pqa::k_half(n);
    const _Float16* w3 = (const _Float16*)p.split;
    *w_inv = (const float*)((const char*)p.split + up256(total * 2 * kh * 2));
    if (int rc = ensure_split(ctx, n_tok, n, total, sb, fn)) return rc;
    pqa::launch_split2(xb, n_tok, n, sb->x3, kh, sb->x_inv, ctx->stream);
    if (int rc = hip_check(ctx, hipGetLastError(), fn)) return rc;
    // Y[n_tok][total] = X_hi W_hi^T + X_hi W_lo^T + X_lo W_hi^T (the q rows come first)
    const int ncols = q_only ? (int)ctx->q_dim : (int)total;
    return hip_check(ctx,
                     pqa::launch_gemm_f16x3_nt(sb->x3, 2 * kh, w3, 2 * kh, sb->y, (int)total, n_tok, ncols, kh,
                                                        ctx->stream),
                     fn);
}

static int check_batch(pqa_ctx* ctx, int layer, int n_tok, const char* fn) {
    if (layer < 0 || layer >= ctx->n_layers) return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": bad layer");
    if (ctx->proj.empty() || !ctx->proj[layer].n_embd)
        return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": no projection weights for this layer");
    if (n_tok <= 0) return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": n_tok must be positive");
    return PQA_OK;
}

extern "C" int pqa_qkv_project_batch(pqa_ctx* ctx, int layer, int n_tok, const float* xb, float* q, float* k,
                                     float* v) {
    static const char* fn = "pqa_qkv_project_batch";
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_qkv_project_batch: ctx is NULL");
    if (int rc = check_batch(ctx, layer, n_tok, fn)) return rc;
    if (!xb || !q || !k || !v) return set_err(ctx, PQA_ERR_ARG, "pqa_qkv_project_batch: NULL buffer");
    // q/k/v are written as float4s
    if (ctx->q_dim % 4 || ctx->kv_dim % 4)
        return set_err(ctx, PQA_ERR_UNSUPPORTED,
                       "pqa_qkv_project_batch: n_heads * head_dim and n_kv_heads * head_dim must be multiples of 4");
    if ((((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) & 15u) != 0)
        return set_err(ctx, PQA_ERR_ARG, "pqa_qkv_project_batch: q, k and v must be 16-byte aligned");
    const bool exact = ctx->batch_exact_kv != 0;
    if (exact)  // the prepared K/V rows exist before any kernel of the call is queued
        if (int rc = ensure_layer_exact(ctx, layer, fn)) return rc;
    SplitBufs sb;
    const float* w_inv = nullptr;
    if (int rc = batch_gemm(ctx, layer, n_tok, xb, &sb, &w_inv, fn, exact)) return rc;
    const auto& p = ctx->proj[layer];
    const size_t total = ctx->q_dim + 2 * ctx->kv_dim;
    pqa::ScatterArgs sa;
    float* outs[3] = {q, k, v};
    for (int i = 0; i < 3; i++) {
        sa.out[i] = outs[i];
        sa.b[i] = (const uint8_t*)p.b[i];
        sa.btype[i] = p.btype[i];
        sa.rows[i] = i == 0 ? (int)ctx->q_dim : (int)ctx->kv_dim;
    }
    const int ncols = exact ? (int)ctx->q_dim : (int)total;
    const unsigned gx = (unsigned)((ncols / 4 + 255) / 256);
    hipLaunchKernelGGL(pqa::unscale_scatter_kernel, dim3(gx, n_tok), dim3(256), 0, ctx->stream, (const float*)sb.y,
                       (int)total, ncols, w_inv, (const float*)sb.x_inv, sa);
    if (int rc = hip_check(ctx, hipGetLastError(), fn)) return rc;
    return exact ? exact_kv(ctx, layer, n_tok, xb, k, v, (int)ctx->kv_dim, fn) : PQA_OK;
}

// The prompt path from the normed inputs: the GEMM result goes to the prefill
// kernels as it is (they undo the scales and add the biases as they read q, k
// and v), without a q/k/v copy.
extern "C" int pqa_prefill_x(pqa_ctx* ctx, int layer, int start_pos, int n_tok, const float* xb, float* out) {
    static const char* fn = "pqa_prefill_x";
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_prefill_x: ctx is NULL");
    if (int rc = check_batch(ctx, layer, n_tok, fn)) return rc;
    if (!xb || !out) return set_err(ctx, PQA_ERR_ARG, "pqa_prefill_x: NULL buffer");
    if (((uintptr_t)out & 15) != 0) return set_err(ctx, PQA_ERR_ARG, "pqa_prefill_x: out must be 16-byte aligned");
    if (start_pos < 0 || (long long)start_pos + n_tok > ctx->max_seq_len)
        return set_err(ctx, PQA_ERR_RANGE, "pqa_prefill_x: positions past max_seq_len");
    const bool exact = ctx->batch_exact_kv != 0;
    if (exact)
        if (int rc = ensure_layer_exact(ctx, layer, fn)) return rc;
    SplitBufs sb;
    const float* w_inv = nullptr;
    if (int rc = batch_gemm(ctx, layer, n_tok, xb, &sb, &w_inv, fn, exact)) return rc;
    const auto& p = ctx->proj[layer];
    const int ld = (int)(ctx->q_dim + 2 * ctx->kv_dim);
    if (exact)  // the k and v columns of the GEMM result, in the reference's order
        if (int rc = exact_kv(ctx, layer, n_tok, xb, sb.y + ctx->q_dim, sb.y + ctx->q_dim + ctx->kv_dim, ld, fn))
            return rc;
    pqa::PrefillScaled ys;
    ys.y = sb.y;
    ys.ld = ld;
    ys.w_inv = w_inv;
    ys.x_inv = sb.x_inv;
    for (int i = 0; i < 3; i++) {
        ys.b[i] = (const uint8_t*)p.b[i];
        ys.bt[i] = p.btype[i];
    }
    ys.kv_plain = exact;
    return hip_check(ctx, pqa::launch_prefill_scaled(ctx, layer, start_pos, n_tok, ys, out), fn);
}

// The output projection of a whole prompt with the residual add, x[t] +=
// attn[t] W_o^T + b for every token (the per-token matmul_bias + vec_add of
// Model::forward_batch, cpp/model.hpp:595-600), on the same split fp16 GEMM as
// the Q/K/V rows and within the same bound.
static int out_project_batch(pqa_ctx* ctx, int layer, int n_tok, const float* attn, float* x, const char* fn) {
    if (int rc = ensure_layer_out_split(ctx, layer, fn)) return rc;
    const auto& p = ctx->proj[layer];
    const int n = (int)ctx->q_dim, rows = p.out_rows;
    const int kh = pqa::k_half(n);
    SplitBufs sb;
    if (int rc = ensure_split(ctx, n_tok, n, (size_t)rows, &sb, fn)) return rc;
    pqa::launch_split2(attn, n_tok, n, sb.x3, kh, sb.x_inv, ctx->stream);
    if (int rc = hip_check(ctx, hipGetLastError(), fn)) return rc;
    const _Float16* w3 = (const _Float16*)p.out_split;
    const float* w_inv = (const float*)((const char*)p.out_split + up256((size_t)rows * 2 * kh * 2));
    if (int rc = hip_check(ctx,
                           pqa::launch_gemm_f16x3_nt(sb.x3, 2 * kh, w3, 2 * kh, sb.y, rows, n_tok, rows, kh,
                                                     ctx->stream),
                           fn))
        return rc;
    const unsigned gx = (unsigned)((rows / 4 + 255) / 256);
    hipLaunchKernelGGL(pqa::unscale_residual_kernel, dim3(gx, n_tok), dim3(256), 0, ctx->stream, (const float*)sb.y,
                       rows, w_inv, (const float*)sb.x_inv, (const uint8_t*)p.b[3], p.btype[3], x);
    return hip_check(ctx, hipGetLastError(), fn);
}

static int check_out_batch(pqa_ctx* ctx, int layer, int n_tok, const char* fn) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, std::string(fn) + ": ctx is NULL");
    if (layer < 0 || layer >= ctx->n_layers) return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": bad layer");
    if (ctx->proj.empty() || !ctx->proj[layer].out_rows)
        return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": no attn_output weights for this layer");
    if (n_tok <= 0) return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": n_tok must be positive");
    if (ctx->proj[layer].out_rows % 4)
        return set_err(ctx, PQA_ERR_UNSUPPORTED, std::string(fn) + ": n_embd must be a multiple of 4");
    return PQA_OK;
}

extern "C" int pqa_out_project_batch(pqa_ctx* ctx, int layer, int n_tok, const float* attn, float* x) {
    static const char* fn = "pqa_out_project_batch";
    if (int rc = check_out_batch(ctx, layer, n_tok, fn)) return rc;
    if (!attn || !x) return set_err(ctx, PQA_ERR_ARG, "pqa_out_project_batch: NULL buffer");
    if (((uintptr_t)x & 15) != 0) return set_err(ctx, PQA_ERR_ARG, "pqa_out_project_batch: x must be 16-byte aligned");
    return out_project_batch(ctx, layer, n_tok, attn, x, fn);
}

// The attention half of Model::forward_batch for one layer and a prompt chunk
// (cpp/model.hpp:493-600 without the FFN): pqa_prefill_x into the context's
// attention workspace, then pqa_out_project_batch into x.
extern "C" int pqa_prefill_block(pqa_ctx* ctx, int layer, int start_pos, int n_tok, const float* xb, float* x) {
    static const char* fn = "pqa_prefill_block";
    if (int rc = check_out_batch(ctx, layer, n_tok, fn)) return rc;
    if (int rc = check_batch(ctx, layer, n_tok, fn)) return rc;
    if (!xb || !x) return set_err(ctx, PQA_ERR_ARG, "pqa_prefill_block: NULL buffer");
    if (((uintptr_t)x & 15) != 0) return set_err(ctx, PQA_ERR_ARG, "pqa_prefill_block: x must be 16-byte aligned");
    if (start_pos < 0 || (long long)start_pos + n_tok > ctx->max_seq_len)
        return set_err(ctx, PQA_ERR_RANGE, "pqa_prefill_block: positions past max_seq_len");
    // every buffer of both GEMMs exists before the first kernel is queued
    const auto& p = ctx->proj[layer];
    const size_t total = ctx->q_dim + 2 * ctx->kv_dim;
    const size_t need = std::max(split_need(n_tok, p.n_embd, total), split_need(n_tok, (int)ctx->q_dim, p.out_rows));
    if (int rc = grow_split(ctx, need, fn)) return rc;
    const size_t af = (size_t)n_tok * ctx->q_dim;
    if (af > ctx->battn_floats) {
        if (int rc = hip_check(ctx, hipStreamSynchronize(ctx->stream), fn)) return rc;
        if (ctx->battn) (void)hipFree(ctx->battn);
        ctx->battn = nullptr;
        ctx->battn_floats = 0;
        if (int rc = hip_check(ctx, hipMalloc(&ctx->battn, af * 4), fn)) return rc;
        ctx->battn_floats = af;
    }
    if (int rc = ensure_layer_split(ctx, layer, fn)) return rc;
    if (int rc = ensure_layer_out_split(ctx, layer, fn)) return rc;
    if (ctx->batch_exact_kv)
        if (int rc = ensure_layer_exact(ctx, layer, fn)) return rc;
    if (int rc = pqa_prefill_x(ctx, layer, start_pos, n_tok, xb, ctx->battn)) return rc;
    return out_project_batch(ctx, layer, n_tok, ctx->battn, x, fn);
}

extern "C" int pqa_set_batch_projection(pqa_ctx* ctx, int exact_kv) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_set_batch_projection: ctx is NULL");
    if (exact_kv != 0 && exact_kv != 1) return set_err(ctx, PQA_ERR_ARG, "pqa_set_batch_projection: 0 or 1");
    ctx->batch_exact_kv = exact_kv;
    return PQA_OK;
}
