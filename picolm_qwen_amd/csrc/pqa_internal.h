// Context layout and kernel launchers of the attention backend (host side).
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "pqa.h"

#define PQA_MAX_EMBD 8192  // longest projection input row (x and the chunk rings share the LDS)

namespace pqa {
// GGUF tensor types as the reference numbers them (cpp/quant.hpp:16-31)
enum : int { GG_NONE = 0, GG_F32 = 1, GG_F16 = 2, GG_Q4_0 = 3, GG_Q8_0 = 9, GG_Q4_K = 13, GG_Q6_K = 15 };
}

// One layer's projection weights in HBM: GGUF rows at a 16-byte stride,
// biases (F32 or F16) or null. Matrices 0-2: attn_q/k/v ([q_dim or kv_dim]
// rows of n_embd); 3: attn_output ([n_embd] rows of q_dim).
struct pqa_proj_weights {
    void* w[4] = {nullptr, nullptr, nullptr, nullptr};
    void* b[4] = {nullptr, nullptr, nullptr, nullptr};
    int wtype[4] = {0, 0, 0, 0}, btype[4] = {0, 0, 0, 0}, stride[4] = {0, 0, 0, 0};
    int n_embd = 0;   // q/k/v set (row width); 0: not set
    int out_rows = 0; // attn_output set (its row count, = n_embd); 0: not set
    // the batched path's fp16 hi/lo copy of the attn_q, attn_k and attn_v rows
    // and their row scales; made on the first batched call, dropped with the weights
    void* split = nullptr;
    // the same for the attn_output rows (pqa_out_project_batch)
    void* out_split = nullptr;
    // the batched path's attn_k and attn_v rows for the reference-order
    // projection (pqa_exact.hip): fp32 [kv_dim][n_embd] each (Q8_0: the int8
    // values as floats, then the block scales); made on the first call that
    // needs them, dropped with the weights
    float* exact = nullptr;
};

namespace pqa {
struct CopyPool;  // pqa_copy_pool.h
}

struct pqa_ctx {
    int n_layers = 0, max_seq_len = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0, rope_style = 0;
    int kv_mul = 1;            // query heads per KV head (cpp/model.hpp:295)
    int n_chunk = 1, chunk_heads = 1;  // query heads of one KV head split into chunks of <= 8
    size_t q_dim = 0, kv_dim = 0;
    size_t layer_elems = 0;    // max_seq_len * kv_dim

    uint16_t* key_cache = nullptr;  // [n_layers][max_seq_len][kv_dim]
    uint16_t* val_cache = nullptr;
    float* rope_cos = nullptr;      // [max_seq_len][head_dim/2]
    float* rope_sin = nullptr;
    float* qk_norm = nullptr;       // [n_layers][2][head_dim]
    std::vector<char> has_qk_norm;

    // decode split-K workspace
    float* part_acc = nullptr;      // [n_kv*n_chunk][max_splits][chunk_heads][head_dim]
    float* part_ml = nullptr;       // [n_kv*n_chunk][max_splits][chunk_heads][2]
    int max_splits = 0;
    int split_override = 0;
    int cu_count = 256;

    // prefill: q = fp16 hi + lo in the score products (outlier-heavy caches)
    // prefill q: 1 (default) fp16 hi + lo, fp32-level scores; 0 one fp16 q,
    // whose score error grows with |q| |k|
    int prefill_split_q = 1;

    // one-token projections (pqa_qkv_project and the entries built on it): 0
    // (default) q rows of F32, F16 and Q4_K summed in any order on a
    // bandwidth-bound path, k and v in the reference's order; 1 all three in
    // the reference's order
    int token_exact_q = 0;
    // attn_output of one token (pqa_out_project, pqa_attention_block): 1
    // (default) the reference's order; 0 rows of F32, F16 and Q4_K in any order
    int out_exact = 1;

    // batched projections: 1 (default) the K and V columns in the reference's
    // summation order (bit-exact cache rows), q on the split fp16 GEMM; 0 all
    // three on the split GEMM
    int batch_exact_kv = 1;

    // projections (pqa_set_qkv_weights) and the q/k/v of pqa_decode_x
    std::vector<pqa_proj_weights> proj;
    float* qkv = nullptr;  // [q_dim + 2 kv_dim + q_dim]: q, k, v and the attention output

    // batched projections (pqa_batch.hip): fp32 weights of one matrix while a
    // layer's split copy is made, and the per-call operands; made on first use
    float* wf32 = nullptr;
    size_t wf32_floats = 0;
    void* bsplit = nullptr;  // fp16 hi/lo operands of the batched GEMMs and their row scales
    size_t bsplit_bytes = 0;
    float* battn = nullptr;  // pqa_prefill_block's attention rows [n_tok][q_dim]
    size_t battn_floats = 0;

    // head sizes other than 64 and 128 (pqa_general.hip): the prepared q rows,
    // one token's worth from context creation on, grown by prompts
    float* gen_q = nullptr;
    size_t gen_q_floats = 0;

    // staging for the _host entry points: device buffers for q, k, v and out,
    // and a pinned host buffer that carries payloads up to kHostStageBytes in
    // one copy each way
    float* stage = nullptr;
    size_t stage_floats = 0;
    float* hstage = nullptr;
    size_t hstage_floats = 0;

    // .kvc file streaming: two pinned host buffers and their copy events,
    // made on the first pqa_kvc_save / pqa_kvc_load
    void* kvc_buf[2] = {nullptr, nullptr};
    hipEvent_t kvc_ev[2] = {nullptr, nullptr};

    // host entries with payloads past the one-copy staging (prompts): two
    // pinned slots, their copy events and the CPU threads that fill and drain
    // them; made on the first such call
    void* hpipe_buf[2] = {nullptr, nullptr};
    hipEvent_t hpipe_ev[2] = {nullptr, nullptr};
    pqa::CopyPool* copy_pool = nullptr;

    hipStream_t stream = nullptr;
    int device = 0;
    std::string err;
};

namespace pqa {

// head sizes with MFMA kernels; other even sizes up to 512 take pqa_general.hip
inline bool mfma_head_dim(int hd) { return hd == 64 || hd == 128; }
constexpr int kMaxHeadDim = 512;

int set_err(pqa_ctx* ctx, int code, const std::string& msg);
int hip_check(pqa_ctx* ctx, hipError_t e, const char* what);

// Rows per decode workgroup, the number of splits (at most max_splits), the
// columns (KV head, chunk) per workgroup and the 16-row tiles per
// wave for `hist` history rows.
void decode_split(const pqa_ctx* ctx, int hist, int max_splits, int* rows_per_split, int* nsplit, int* cols_per_wg,
                  int* tiles);

// Where a decode's split partials go: part_acc [ny][splits][G][hd] and
// part_ml [ny][splits][G][2] floats, for at most max_splits splits.
struct DecodeWorkspace {
    float* part_acc;
    float* part_ml;
    int max_splits;
};

hipError_t launch_decode(pqa_ctx* ctx, int layer, int pos, const float* q, const float* k,
                         const float* v, float* out, const DecodeWorkspace& ws);

// The no-allocation decode (pqa_decode_noalloc): its split partials live in a
// file-scope device array of pqa_decode.hip, one per GPU.
// scratch_init takes that array's address on the current device (once per
// device, at context creation); scratch_workspace gives the workspace on the
// context's device, or an error code with ctx->err set.
int scratch_init(int device);
int scratch_workspace(pqa_ctx* ctx, DecodeWorkspace* ws, const char* fn);
// C[m][n] = A_hi B_hi^T + A_hi B_lo^T + A_lo B_hi^T with rows of A (B) holding
// hi at [0, kh) and lo at [kh, 2 kh) halfs (fp16 operands, fp32 result; kh a
// multiple of 32; pqa_gemm.hip).
hipError_t launch_gemm_f16x3_nt(const _Float16* a, int lda, const _Float16* b, int ldb, float* c, int ldc, int m,
                                int n, int kh, hipStream_t stream);
hipError_t launch_prefill(pqa_ctx* ctx, int layer, int start, int n_tok, const float* q,
                          const float* k, const float* v, float* out);
// q/k/v of a prompt as the columns of one GEMM result y [n_tok][ld] (q at
// column 0, k at q_dim, v at q_dim + kv_dim), scaled by powers of two: the
// value of column c of token t is y * (w_inv[c] * x_inv[t]) + b_m[c]
// With kv_plain, the k and v columns hold final values (the reference-order
// projection wrote them, biases included) and are read as they are.
struct PrefillScaled {
    const float* y;
    int ld;
    const float* w_inv;
    const float* x_inv;
    const uint8_t* b[3];  // q, k, v biases or null
    int bt[3];
    bool kv_plain;
};
hipError_t launch_prefill_scaled(pqa_ctx* ctx, int layer, int start, int n_tok, const PrefillScaled& ys, float* out);
// The general-head_dim path (pqa_general.hip): the same contracts as
// launch_decode and launch_prefill / launch_prefill_scaled (ys non-null: q, k
// and v read from the scaled GEMM result, q/k/v pointers unused).
hipError_t launch_decode_general(pqa_ctx* ctx, int layer, int pos, const float* q, const float* k, const float* v,
                                 float* out, const DecodeWorkspace& ws);
hipError_t launch_prefill_general(pqa_ctx* ctx, int layer, int start, int n_tok, const float* q, const float* k,
                                  const float* v, const PrefillScaled* ys, float* out);
hipError_t launch_synth_kv(pqa_ctx* ctx, int layer, int pos0, int n, uint64_t seed, float prob);
hipError_t launch_f32_to_f16(pqa_ctx* ctx, const float* src, uint16_t* dst, size_t n);
hipError_t launch_qkv_project(pqa_ctx* ctx, int layer, const float* xb, float* q, float* k, float* v);
// GGUF rows [rows][n] -> fp32 [rows][n] by the dequantize_row_* expressions
// (pqa_batch.hip).
hipError_t launch_dequant_rows(int type, const void* w, int stride, int rows, int n, float* dst, hipStream_t s);
// The reference-order projection of a prompt (pqa_exact.hip):
// exact_matrix_floats / prepare_exact_matrix make a matrix's prepared copy
// from its GGUF rows; launch_ordered_project writes out[t * ldo + r] =
// matmul_bias of token t's input x[t * ldx ..] for rows r < rows, bit-exact.
size_t exact_matrix_floats(int type, int rows, int n);
hipError_t prepare_exact_matrix(int type, const void* w, int stride, int rows, int n, float* dst, hipStream_t s);
hipError_t launch_ordered_project(int type, const float* prepared, int rows, int n, const float* x, int ldx, int n_tok,
                                  const void* bias, int btype, float* out, int ldo, hipStream_t s);
hipError_t launch_out_project(pqa_ctx* ctx, int layer, const float* attn, float* x);

}  // namespace pqa

// Frees every layer's projection weights (pqa_proj.hip).
void pqa_free_projections(pqa_ctx* c);

// Releases the fp32 weight workspace and the batched operands (pqa_batch.hip).
void pqa_free_batch(pqa_ctx* c);
