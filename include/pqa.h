/*
 * pqa.h -- C ABI of the MI355X (gfx950) attention backend for the
 * rain1201/picolm_qwen C++ forward pass.
 *
 * The reference has no plugin or FFI API for this path: the attention is
 * inline code in Model::forward (cpp/model.hpp:326-418) and
 * Model::forward_batch (cpp/model.hpp:507-593). This header defines the
 * boundary as that block's live-ins and live-outs: q/k/v of the layer,
 * the position, the QK-norm weights, the RoPE rows and the KV cache in,
 * the attention output xb out.
 *
 * Memory: the context owns the KV cache in HBM in the reference's layout
 *   key_cache/val_cache: uint16 fp16 [n_layers][max_seq_len][n_kv_heads][head_dim]
 * (cpp/model.hpp:160, allocated :1003-1006, indexed :355-356,:369-370,:388-389),
 * the RoPE tables, the QK-norm weights, a workspace and one HIP stream.
 * Every call is asynchronous on that stream unless its name ends in _host.
 *
 * Errors: every int function returns PQA_OK (0) or a negative PQA_ERR_*;
 * pqa_last_error() gives the message. Nothing throws across the ABI.
 * Threading: a context is used by one host thread at a time.
 */
#ifndef PQA_H
#define PQA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PQA_OK 0
#define PQA_ERR_ARG (-1)         /* bad pointer, shape or layer index */
#define PQA_ERR_RANGE (-2)       /* position outside [0, max_seq_len) */
#define PQA_ERR_UNSUPPORTED (-3) /* a size the kernels do not take (head_dim odd or above 512, ...) */
#define PQA_ERR_HIP (-4)         /* a HIP runtime call failed */
#define PQA_ERR_NOMEM (-5)       /* device allocation failed */
#define PQA_ERR_IO (-6)          /* a .kvc file could not be opened, read or written */
#define PQA_ERR_FORMAT (-7)      /* a .kvc file has a bad magic or another model's shape */

typedef struct pqa_ctx pqa_ctx;

/* RopeFn choices (cpp/model.hpp:176, picked by cpp/picolm.cpp:179-186). */
typedef enum {
    PQA_ROPE_NEOX_HALF = 0,         /* TensorOps::rope_qwen, cpp/tensor.hpp:201-283: pairs (i, i+hd/2) */
    PQA_ROPE_LLAMA_X86_BLOCK8 = 1,  /* TensorOps::rope_llama on x86 (SSE2 path), cpp/tensor.hpp:290-346:
                                       pairs (8b+j, 8b+4+j) at angle 4b+j -- what the reference runs */
    PQA_ROPE_LLAMA_INTERLEAVED = 2  /* rope_llama scalar branch, cpp/tensor.hpp:347-368: pairs (2i, 2i+1) */
} pqa_rope_t;

/*
 * Allocates the cache and uploads the RoPE tables. Replaces
 * Model::allocate_run_state's KV/RoPE part (cpp/model.hpp:1003-1017).
 * rope_cos/rope_sin: host, [max_seq_len][head_dim/2] (state.rope_cos/sin).
 * head_dim must be even and at most 512 (the reference's acc[512],
 * cpp/model.hpp:172) and n_heads a multiple of n_kv_heads (kv_mul,
 * cpp/model.hpp:295). 64 and 128 run on the MFMA kernels; other sizes on
 * plain VALU kernels with the same results contract (bit-exact K/V rows,
 * outputs within max-abs 2e-3 / rel 1e-2), where q, k and v need only 4-byte
 * and out 8-byte alignment. The cache starts zeroed, as the reference's
 * std::vector does.
 */
int pqa_create(pqa_ctx** out, int n_layers, int max_seq_len, int n_heads, int n_kv_heads,
               int head_dim, int rope_style, const float* rope_cos, const float* rope_sin);

/* QK-RMSNorm weights of one layer (state.attn_q_norm_w/attn_k_norm_w,
 * cpp/model.hpp:170, :984-1001). Host [head_dim] each; NULL for both turns the
 * norm off for that layer, as when the GGUF lacks attn_q_norm (:327-328). */
int pqa_set_qk_norm(pqa_ctx* ctx, int layer, const float* q_norm_w, const float* k_norm_w);

/*
 * One decode step of one layer: the block of cpp/model.hpp:326-418.
 * Q/K RMSNorm (if set), RoPE at pos, K and V rounded to fp16 (the reference's
 * ties-away-from-zero rounding, cpp/quant.hpp:102-135) and written at row pos,
 * then attention of every query head over rows 0..pos.
 * q [n_heads*head_dim], k/v [n_kv_heads*head_dim], out [n_heads*head_dim]:
 * fp32 DEVICE pointers, 16-byte aligned, ready when the context stream
 * reaches the call (produce them on that stream or synchronise first).
 * q/k/v are not modified (the reference normalises in place; the caller
 * never reads them afterwards).
 */
int pqa_decode(pqa_ctx* ctx, int layer, int pos, const float* q, const float* k, const float* v,
               float* out);

/*
 * Prompt of n_tok tokens at positions start_pos..start_pos+n_tok-1: the token
 * loop of cpp/model.hpp:493-593 for one layer. Token-major fp32 DEVICE
 * pointers q [n_tok][n_heads*hd], k/v [n_tok][n_kv*hd], out [n_tok][n_heads*hd].
 * Rows are appended first and attention is causal (token i reads rows
 * 0..start_pos+i), which is what the reference's serial loop computes.
 * Same alignment and readiness rules as pqa_decode.
 */
int pqa_prefill(pqa_ctx* ctx, int layer, int start_pos, int n_tok, const float* q, const float* k,
                const float* v, float* out);

/*
 * pqa_decode that allocates nothing: the same kernels, with the split
 * partials in a static device array of the library (8 MiB per GPU, held until
 * the process ends; its address is taken once per device by pqa_create)
 * instead of the context's split workspace. Head sizes other than 64 and 128
 * also use the prepared-q buffer that pqa_create allocates (one token's q,
 * read and written, never grown by this call). No counterpart in the
 * reference: this entry point is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Same arguments, results and errors as pqa_decode. The
 * split count is capped at what fits in the 8 MiB (each split's partials take
 * n_kv_heads * ceil(g / 8) * chunk heads * (head_dim + 2) * 4 bytes); when
 * not even two fit (about 8000 query heads), every call runs as one split,
 * which needs no scratch. Every call on one GPU shares the array: calls that
 * overlap on one GPU (other streams or threads) race and must be ordered by
 * the caller.
 */
int pqa_decode_noalloc(pqa_ctx* ctx, int layer, int pos, const float* q, const float* k, const float* v,
                       float* out);

/* Host-pointer forms of the two calls above for a forward loop whose q/k/v
 * live in host std::vectors (cpp/model.hpp state.q / xb2): copy in, run,
 * copy out, synchronise. */
int pqa_decode_host(pqa_ctx* ctx, int layer, int pos, const float* q, const float* k,
                    const float* v, float* out);
int pqa_prefill_host(pqa_ctx* ctx, int layer, int start_pos, int n_tok, const float* q,
                     const float* k, const float* v, float* out);

/* Copy cache rows [pos0, pos0+n) of one layer between host and HBM, in the
 * reference row layout (kv_dim uint16 per row). Synchronous. Either row
 * pointer may be NULL to skip that half. */
int pqa_kv_upload(pqa_ctx* ctx, int layer, int pos0, int n, const uint16_t* k_rows,
                  const uint16_t* v_rows);
int pqa_kv_download(pqa_ctx* ctx, int layer, int pos0, int n, uint16_t* k_rows, uint16_t* v_rows);

/* Device base pointers of the whole cache ([n_layers][max_seq_len][kv_dim]). */
int pqa_kv_cache(pqa_ctx* ctx, uint16_t** key_cache, uint16_t** val_cache);

/*
 * KV-cache persistence in the reference's .kvc format, so files written by
 * either side load in the other (picolm/model.c:870-983, declared
 * picolm/model.h:156-164, called picolm/picolm.c:266-293,:364-367):
 *   uint32 {0x4B564350 "KVCP", n_pos, n_layers, kv_dim} in host byte order,
 *   then K rows [0, n_pos) of layer 0, 1, ..., then V rows the same way,
 *   kv_dim fp16 per row.
 * Both stream the HBM cache through two pinned host buffers (16 MiB each,
 * made on first use) and are synchronous: the cache state is the one the
 * context stream has reached when the call is made.
 *
 * pqa_kvc_save replaces kvcache_save (picolm/model.c:882-921). Returns PQA_OK,
 * PQA_ERR_RANGE for n_pos outside [1, max_seq_len] (no file is created, the
 * reference's -1 case), PQA_ERR_IO when the file cannot be opened or a write
 * fails (the reference does not check its writes). Prints nothing.
 */
int pqa_kvc_save(pqa_ctx* ctx, const char* path, int n_pos);

/*
 * pqa_kvc_load replaces kvcache_load (picolm/model.c:923-983) with its
 * return contract: the header's position count on success, 0 on any failure
 * (missing file, short header, bad magic, n_layers or kv_dim other than the
 * context's, more positions than max_seq_len, a file that ends early), with
 * the reason in pqa_last_error. As in the reference, a file that ends early
 * leaves the bytes it did hold in the cache, and a header count of 2^31 or
 * more comes back negative with nothing loaded.
 */
int pqa_kvc_load(pqa_ctx* ctx, const char* path);

/*
 * Q/K/V projections of the decode step: TensorOps::matmul_bias
 * (cpp/tensor.hpp:110-143) for ATTN_Q, ATTN_K and ATTN_V as Model::forward
 * calls it (cpp/model.hpp:320-366), on the GPU and in the reference's own
 * summation order (the x86 SSE2 path of vec_dot, cpp/quant.hpp:297-356), so
 * q, k and v are bit-identical to the reference built without FMA contraction.
 *
 * Weight and bias types are the reference's GGUFType numbers
 * (cpp/quant.hpp:16-31), as the caller holds them in its tensor entries.
 */
#define PQA_GGUF_NONE 0
#define PQA_GGUF_F32 1
#define PQA_GGUF_F16 2
#define PQA_GGUF_Q4_0 3
#define PQA_GGUF_Q8_0 9
#define PQA_GGUF_Q4_K 13
#define PQA_GGUF_Q6_K 15

/* Uploads one layer's attn_q/attn_k/attn_v weights: HOST pointers to GGUF
 * rows, [q_dim][row] for wq and [kv_dim][row] for wk/wv, row = n_embd
 * elements in the type's blocks (the tensor data as the reference maps it).
 * Biases: HOST [rows] in F32 or F16, or NULL / PQA_GGUF_NONE for none
 * (the attn_*_b entries). Types: F32, F16, Q4_0, Q8_0, Q4_K, Q6_K;
 * PQA_ERR_UNSUPPORTED for other types, n_embd > 8192, rows that are not
 * whole blocks, F32/F16 rows not a multiple of 8, Q4_0/Q8_0 rows not a
 * multiple of 64 or Q6_K rows not a multiple of 512 elements. Synchronous;
 * replaces earlier weights of the layer. */
int pqa_set_qkv_weights(pqa_ctx* ctx, int layer, int n_embd, const void* wq, int wq_type, const void* bq,
                        int bq_type, const void* wk, int wk_type, const void* bk, int bk_type, const void* wv,
                        int wv_type, const void* bv, int bv_type);

/* q = Wq xb + bq, k = Wk xb + bk, v = Wv xb + bv for one token (the
 * matmul_bias calls of cpp/model.hpp:320-323, :337-340, :362-365). DEVICE
 * pointers xb [n_embd], q [n_heads*head_dim], k and v [n_kv_heads*head_dim];
 * asynchronous on the context stream. k and v are the reference's bits (its
 * summation order, cpp/quant.hpp:297-356); q follows
 * pqa_set_token_projection. */
int pqa_qkv_project(pqa_ctx* ctx, int layer, const float* xb, float* q, float* k, float* v);

/*
 * How pqa_qkv_project (and pqa_decode_x, pqa_attention_block and their host
 * forms, which call it) computes q.
 * 0 (default): q rows of type F32, F16 or Q4_K are summed in any order on a
 *    bandwidth-bound path (one row per wave), within (n_embd + 12) 2^-24
 *    sum_i |w_i x_i| of the reference's sum; q only feeds the attention
 *    scores, so no cache row depends on its bits. Other q types, and k and v
 *    always, keep the reference's order.
 * 1: q in the reference's order too, bit-identical to matmul_bias.
 * No counterpart in the reference, which has one order only.
 */
int pqa_set_token_projection(pqa_ctx* ctx, int exact_q);

/* The attention block of Model::forward from the normed input on
 * (cpp/model.hpp:320-418): pqa_qkv_project into a context workspace, then
 * pqa_decode. DEVICE pointers xb [n_embd], out [n_heads*head_dim]. */
int pqa_decode_x(pqa_ctx* ctx, int layer, int pos, const float* xb, float* out);

/*
 * Attention output projection and residual add (cpp/model.hpp:420-427):
 * xb2 = Wo attn + bo (TensorOps::matmul_bias, same order and types as above),
 * then x = x + xb2 (TensorOps::vec_add, cpp/tensor.hpp:410-420).
 * pqa_set_out_weights: attn_output as HOST GGUF rows [n_embd][q_dim elements]
 * (q_dim = n_heads*head_dim) and an optional F32/F16 bias [n_embd]; the same
 * type and width limits as pqa_set_qkv_weights, applied to q_dim.
 */
int pqa_set_out_weights(pqa_ctx* ctx, int layer, int n_embd, const void* wo, int wo_type, const void* bo,
                        int bo_type);

/* How pqa_out_project and pqa_attention_block (and its host form) sum the
 * attn_output rows.
 * 1 (default): the reference's order; x is bit-identical to matmul_bias then
 *    vec_add.
 * 0: rows of type F32, F16 or Q4_K on the any-order path of
 *    pqa_set_token_projection (one row per wave), within (q_dim + 12) 2^-24
 *    sum_i |w_i a_i| (Q4_K: |d q_i| + |m| in place of |w_i|) of the
 *    reference's sum before the residual add; other types keep the order.
 * No counterpart in the reference, which has one order only.
 */
int pqa_set_out_projection(pqa_ctx* ctx, int exact);

/* x[n_embd] += Wo attn + bo, DEVICE pointers attn [q_dim] and x (updated in
 * place); asynchronous on the context stream. */
int pqa_out_project(pqa_ctx* ctx, int layer, const float* attn, float* x);

/* The attention half of a decode layer, cpp/model.hpp:320-427: from the
 * normed input xb [n_embd] to the residual stream x [n_embd] (updated in
 * place): Q/K/V projections, norms, RoPE, K/V append and attention at pos,
 * output projection, x += result. Needs both weight sets of the layer. */
int pqa_attention_block(pqa_ctx* ctx, int layer, int pos, const float* xb, float* x);

/*
 * Q/K/V projections of a whole prompt (the per-token matmul_bias calls of
 * Model::forward_batch, cpp/model.hpp:493-530) as one GEMM over all tokens
 * and all q/k/v rows: the GGUF weights are dequantized exactly
 * (dequantize_row_*); weights and inputs, each row scaled by a power of two,
 * are split into fp16 hi + lo parts (22 significand bits); the GEMM (this
 * library's gemm_f16x3_nt_kernel, fp16 MFMA, fp32 accumulation) sums
 * w_hi x_hi + w_hi x_lo + w_lo x_hi; the
 * scale is undone exactly and the bias added. The error stays within
 * (3 n_embd + 12) 2^-24 sum |w x|, so q agrees with the reference to fp32
 * rounding (about 1e-6 relative), not bit for bit (pqa_qkv_project keeps the
 * order for one token). k and v follow pqa_set_batch_projection: by default
 * in the reference's own order, bit-identical to pqa_qkv_project's, so the
 * cache rows a prompt writes are the reference's; with exact_kv = 0 on the
 * same GEMM as q. DEVICE pointers xb [n_tok][n_embd], q [n_tok][q_dim],
 * k and v [n_tok][kv_dim]; asynchronous on the context stream.
 * Memory: the first call for a layer keeps that layer's split weights,
 * about (q_dim + 2 kv_dim) * (4 n_embd + 4) bytes, until its weights are
 * replaced or the context is destroyed; the first call also allocates a
 * q_dim * n_embd float workspace, and each call needs a workspace of about
 * n_tok * (4 n_embd + 4 (q_dim + 2 kv_dim) + 4) bytes (the hi and lo halves
 * of a row each padded to 32 halfs), grown on demand.
 */
int pqa_qkv_project_batch(pqa_ctx* ctx, int layer, int n_tok, const float* xb, float* q, float* k, float* v);

/* The prompt path of one layer from the normed inputs: pqa_qkv_project_batch
 * into a context workspace (grown on demand), then pqa_prefill. DEVICE
 * pointers xb [n_tok][n_embd], out [n_tok][n_heads*head_dim]. */
int pqa_prefill_x(pqa_ctx* ctx, int layer, int start_pos, int n_tok, const float* xb, float* out);

/* Output projection and residual for a whole prompt: x[t] += Wo attn[t] + bo
 * for t < n_tok (the per-token matmul_bias + vec_add of Model::forward_batch,
 * cpp/model.hpp:595-600), on the split fp16 GEMM of pqa_qkv_project_batch:
 * the same error bound, (3 q_dim + 12) 2^-24 sum |w a|, not bit for bit
 * (pqa_out_project keeps the order for one token). DEVICE pointers attn
 * [n_tok][q_dim] and x [n_tok][n_embd] (16-byte aligned, n_embd a multiple of
 * 4); asynchronous. The first call for a layer keeps its split attn_output
 * rows, about n_embd * (4 q_dim + 4) bytes, until they are replaced. */
int pqa_out_project_batch(pqa_ctx* ctx, int layer, int n_tok, const float* attn, float* x);

/* The attention half of one layer of Model::forward_batch for a prompt chunk,
 * cpp/model.hpp:493-600 without the FFN: from the attention norm's output xb
 * [n_tok][n_embd] to the residual stream x [n_tok][n_embd] (read and written),
 * token i at position start_pos + i: pqa_prefill_x into a context workspace,
 * then pqa_out_project_batch. Token i's attention reads only rows written by
 * tokens <= i of the same layer, so the reference's token loop (norm, block,
 * FFN per token) and this layer-at-once order give the same values. DEVICE
 * pointers (x 16-byte aligned); asynchronous. */
int pqa_prefill_block(pqa_ctx* ctx, int layer, int start_pos, int n_tok, const float* xb, float* x);

/* pqa_attention_block (cpp/model.hpp:320-427) and pqa_prefill_block for HOST
 * pointers, as a CPU forward loop holds xb and x in its RunState vectors: xb
 * and x are copied in, x is copied back, the call synchronises. */
int pqa_attention_block_host(pqa_ctx* ctx, int layer, int pos, const float* xb, float* x);
int pqa_prefill_block_host(pqa_ctx* ctx, int layer, int start_pos, int n_tok, const float* xb, float* x);

/* The context's HIP stream (a hipStream_t), for event timing or ordering. */
void* pqa_stream(pqa_ctx* ctx);
int pqa_sync(pqa_ctx* ctx);

/* Message of the last failed call on ctx; ctx == NULL gives the calling
 * thread's last pqa_create failure. */
const char* pqa_last_error(const pqa_ctx* ctx);
void pqa_destroy(pqa_ctx* ctx);

/* RoPE table exactly as the reference builds it (cpp/model.hpp:1008-1017):
 * theta = (float)pos / powf(base, (float)(2i)/(float)hd), cosf, sinf, on the
 * host. cos_tab/sin_tab: [max_seq_len][head_dim/2]. */
void pqa_rope_table(float rope_base, int head_dim, int max_seq_len, float* cos_tab, float* sin_tab);

/* fp32 -> fp16 with the reference's rounding (cpp/quant.hpp:102-135) as a
 * device op on n elements, on the context stream. DEVICE pointers. */
int pqa_fp32_to_fp16(pqa_ctx* ctx, const float* src, uint16_t* dst, size_t n);

/*
 * Benchmark and test helper with no counterpart in the reference: fills cache
 * rows [pos0, pos0+n) of `layer` with seeded synthetic history on the device.
 * K and V ~N(0,1) from SplitMix64 + Box-Muller (the same generator as the
 * CPU oracle's pqo_synth_kv_rows), rows with uniform < outlier_prob scaled by
 * 8, then fp16 by the reference rounding.
 */
int pqa_synth_kv(pqa_ctx* ctx, int layer, int pos0, int n, uint64_t seed, float outlier_prob);

/* Decode split size in cache rows per workgroup (a multiple of 64; 0 = the
 * automatic choice). For tuning sweeps; results do not depend on it beyond
 * fp32 summation order. */
int pqa_set_decode_split(pqa_ctx* ctx, int rows_per_split);

/*
 * How the batched entry points (pqa_qkv_project_batch, pqa_prefill_x,
 * pqa_prefill_block) project K and V.
 * 1 (default): the attn_k and attn_v columns are computed in the reference's
 *    own summation order (vec_dot, cpp/quant.hpp:297-356, as forward_batch
 *    calls matmul_bias per token, cpp/model.hpp:503-546) on a VALU GEMM, so k
 *    and v are bit-identical to pqa_qkv_project's and the cache rows a prompt
 *    writes are the reference's bits (built without FMA contraction); q stays
 *    on the split fp16 GEMM, within its error bound (q only feeds scores).
 *    The first such call for a layer keeps its K/V rows as fp32, about
 *    2 * kv_dim * n_embd * 4 bytes (plus n_embd / 8 floats per row for Q8_0),
 *    until the weights are replaced.
 * 0: all three on the split fp16 GEMM: faster, but a K or V element can land
 *    one fp16 step away from the reference's.
 * No counterpart in the reference, which has one order only.
 */
int pqa_set_batch_projection(pqa_ctx* ctx, int exact_kv);

/* Prefill score precision.
 * 1 (default): q is carried as fp16 hi + lo (two MFMAs per k-step),
 *    fp32-level scores.
 * 0: q is rounded once to fp16 for the QK^T MFMA: about 13 % faster on a
 *    Qwen3-4B prefill, but the score error grows with |q| |k| (QK-norm
 *    weights of 2 already put outputs past max-abs 2e-3 / rel 1e-2). */
int pqa_set_prefill_precision(pqa_ctx* ctx, int split_q);

#ifdef __cplusplus
}
#endif

#endif /* PQA_H */
