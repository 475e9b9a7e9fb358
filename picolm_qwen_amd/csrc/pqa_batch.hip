// Q/K/V projections of a whole prompt: the per-token matmul_bias calls of
// Model::forward_batch (cpp/model.hpp:493-530) as one GEMM per matrix over
// all tokens, feeding the MFMA prefill.
//
// Each GGUF matrix is first dequantized into an fp32 workspace by the
// expressions of dequantize_row_* (cpp/quant.hpp:176-281), exactly, then
// Y[n_tok][rows] = X[n_tok][n] W^T runs as a plain fp32 GEMM (rocBLAS sgemm on
// the context stream), then the bias is added (vec_add: out + b). The weights
// and the inputs are exact; only the summation order of each dot product
// differs from the reference's, so q/k/v agree to fp32 rounding (about 1e-6
// relative) rather than bit for bit. pqa_qkv_project keeps the reference's
// order for one token.
#include <rocblas/rocblas.h>

#include <string>

#include "pqa_device.h"
#include "pqa_internal.h"

namespace pqa {

__device__ __forceinline__ float bh2f(unsigned h) { return (float)__builtin_bit_cast(_Float16, (unsigned short)h); }
__device__ __forceinline__ unsigned bld16(const uint8_t* p) { return p[0] | ((unsigned)p[1] << 8); }

// One thread per 32 elements of a row: dst[row][32 g .. 32 g + 31].
template <int T>
__global__ __launch_bounds__(256) void dequant_rows_kernel(const uint8_t* __restrict__ w, int stride, int rows, int n,
                                                           float* __restrict__ dst) {
    const int groups = n / 32;
    const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (long long)rows * groups) return;
    const int row = (int)(gid / groups), g = (int)(gid % groups);
    const uint8_t* r = w + (size_t)row * stride;
    float* y = dst + (size_t)row * n + 32 * g;
    if constexpr (T == GG_F32) {
        const float* s = (const float*)(r + 128 * g);
        for (int j = 0; j < 32; j++) y[j] = s[j];
    } else if constexpr (T == GG_F16) {
        for (int j = 0; j < 32; j++) y[j] = bh2f(bld16(r + 64 * g + 2 * j));
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

// out[t][r] = out[t][r] + b[r] (vec_add, cpp/tensor.hpp:410-420)
__global__ __launch_bounds__(256) void add_bias_kernel(float* out, const uint8_t* b, int btype, int rows, int n_tok) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long long)rows * n_tok) return;
    const int r = (int)(i % rows);
    const float bv = btype == GG_F32 ? ((const float*)b)[r] : bh2f(bld16(b + 2 * r));
    out[i] = out[i] + bv;
}

static hipError_t launch_dequant(int type, const void* w, int stride, int rows, int n, float* dst, hipStream_t s) {
    const long long items = (long long)rows * (n / 32);
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

// The rocBLAS handle and the fp32 weight workspace of a context, made on the
// first batched call.
static int ensure_batch(pqa_ctx* ctx, size_t wfloats, const char* fn) {
    if (!ctx->blas) {
        rocblas_handle h = nullptr;
        if (rocblas_create_handle(&h) != rocblas_status_success)
            return set_err(ctx, PQA_ERR_HIP, std::string(fn) + ": rocblas_create_handle failed");
        if (rocblas_set_stream(h, ctx->stream) != rocblas_status_success) {
            rocblas_destroy_handle(h);
            return set_err(ctx, PQA_ERR_HIP, std::string(fn) + ": rocblas_set_stream failed");
        }
        ctx->blas = h;
    }
    if (wfloats > ctx->wf32_floats) {
        if (ctx->wf32) (void)hipFree(ctx->wf32);
        ctx->wf32 = nullptr;
        ctx->wf32_floats = 0;
        if (int rc = hip_check(ctx, hipMalloc(&ctx->wf32, wfloats * 4), fn)) return rc;
        ctx->wf32_floats = wfloats;
    }
    return PQA_OK;
}

void pqa_free_batch(pqa_ctx* c) {
    if (c->blas) rocblas_destroy_handle((rocblas_handle)c->blas);
    c->blas = nullptr;
    if (c->wf32) (void)hipFree(c->wf32);
    c->wf32 = nullptr;
}

extern "C" int pqa_qkv_project_batch(pqa_ctx* ctx, int layer, int n_tok, const float* xb, float* q, float* k,
                                     float* v) {
    static const char* fn = "pqa_qkv_project_batch";
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_qkv_project_batch: ctx is NULL");
    if (layer < 0 || layer >= ctx->n_layers) return set_err(ctx, PQA_ERR_ARG, "pqa_qkv_project_batch: bad layer");
    if (ctx->proj.empty() || !ctx->proj[layer].n_embd)
        return set_err(ctx, PQA_ERR_ARG, "pqa_qkv_project_batch: no projection weights for this layer");
    if (n_tok <= 0 || !xb || !q || !k || !v) return set_err(ctx, PQA_ERR_ARG, "pqa_qkv_project_batch: bad arguments");
    const auto& p = ctx->proj[layer];
    const int n = p.n_embd;
    const int rows[3] = {(int)ctx->q_dim, (int)ctx->kv_dim, (int)ctx->kv_dim};
    float* outs[3] = {q, k, v};
    if (int rc = ensure_batch(ctx, (size_t)ctx->q_dim * n, fn)) return rc;
    const float one = 1.0f, zero = 0.0f;
    for (int i = 0; i < 3; i++) {
        if (int rc = hip_check(ctx, pqa::launch_dequant(p.wtype[i], p.w[i], p.stride[i], rows[i], n, ctx->wf32, ctx->stream),
                               fn))
            return rc;
        // row-major Y[n_tok][rows] = X[n_tok][n] W[rows][n]^T, i.e. column-major
        // C (rows x n_tok) = W^T (rows x n) * X^T (n x n_tok)
        if (rocblas_sgemm((rocblas_handle)ctx->blas, rocblas_operation_transpose, rocblas_operation_none, rows[i],
                          n_tok, n, &one, ctx->wf32, n, xb, n, &zero, outs[i], rows[i]) != rocblas_status_success)
            return set_err(ctx, PQA_ERR_HIP, "pqa_qkv_project_batch: rocblas_sgemm failed");
        if (p.b[i]) {
            const long long items = (long long)rows[i] * n_tok;
            hipLaunchKernelGGL(pqa::add_bias_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, ctx->stream,
                               outs[i], (const uint8_t*)p.b[i], p.btype[i], rows[i], n_tok);
            if (int rc = hip_check(ctx, hipGetLastError(), fn)) return rc;
        }
    }
    return PQA_OK;
}

extern "C" int pqa_prefill_x(pqa_ctx* ctx, int layer, int start_pos, int n_tok, const float* xb, float* out) {
    static const char* fn = "pqa_prefill_x";
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_prefill_x: ctx is NULL");
    if (n_tok <= 0 || !xb || !out) return set_err(ctx, PQA_ERR_ARG, "pqa_prefill_x: bad arguments");
    if (start_pos < 0 || (long long)start_pos + n_tok > ctx->max_seq_len)
        return set_err(ctx, PQA_ERR_RANGE, "pqa_prefill_x: positions past max_seq_len");
    const size_t need = (size_t)n_tok * (ctx->q_dim + 2 * ctx->kv_dim);
    if (need > ctx->bqkv_floats) {
        if (ctx->bqkv) (void)hipFree(ctx->bqkv);
        ctx->bqkv = nullptr;
        ctx->bqkv_floats = 0;
        if (int rc = hip_check(ctx, hipMalloc(&ctx->bqkv, need * 4), fn)) return rc;
        ctx->bqkv_floats = need;
    }
    float* q = ctx->bqkv;
    float* k = q + (size_t)n_tok * ctx->q_dim;
    float* v = k + (size_t)n_tok * ctx->kv_dim;
    if (int rc = pqa_qkv_project_batch(ctx, layer, n_tok, xb, q, k, v)) return rc;
    return pqa_prefill(ctx, layer, start_pos, n_tok, q, k, v, out);
}
