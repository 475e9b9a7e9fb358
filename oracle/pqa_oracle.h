/*
 * CPU oracle for the picolm_qwen attention path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a loop-for-loop restatement of the
 * reference CPU algorithm (rain1201/picolm_qwen, cpp/model.hpp:326-418 for
 * decode and :507-593 for prefill, with the helpers it calls in
 * cpp/tensor.hpp and cpp/quant.hpp). It is the checker for the HIP library:
 * only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py
 * may load it. No product code path may call it.
 *
 * Bit-exactness contract: built with -ffp-contract=off (no FMA contraction),
 * every fp32 operation below rounds exactly as the reference compiled with
 * `-O3 -std=c++17 -march=native -ffp-contract=off`. libm expf/sqrtf/powf/
 * cosf/sinf are the host glibc ones, as in the reference.
 *
 * Parity pins (see tests/test_oracle_*.py):
 *   fp16 widen            exhaustive 65536-value KAT against IEEE widening
 *   fp16 narrow           closed-form spec (nearest, ties away from zero)
 *                         over every exponent/sign/top-mantissa pattern and
 *                         the whole fp16-subnormal band; golden K/V rows
 *   rmsnorm, rope         golden K rows written by the compiled reference;
 *                         closed forms (pos 0 identity, pair-norm invariance,
 *                         rms(out/w) == 1, block8 permutation KAT)
 *   attention             golden outputs of the compiled reference (bit-exact);
 *                         float64 brute-force softmax; ctx=1, equal-key and
 *                         dominant-key closed forms
 *   rng                   SplitMix64 published test vector; N(0,1) moments
 *   projections           the reference's own dequantize_row, vec_dot and
 *                         matmul_bias compiled from its sources (bit-exact);
 *                         closed forms per GGUF type; a summation-order case
 *                         that only the reference's order passes
 *   .kvc format           (oracle/__init__.py) the reference's compiled
 *                         kvcache_save / kvcache_load: identical files and
 *                         cache bytes, short and malformed files included
 */
#ifndef PQA_ORACLE_H
#define PQA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { PQO_ROPE_NEOX_HALF = 0, PQO_ROPE_LLAMA_X86_BLOCK8 = 1, PQO_ROPE_LLAMA_INTERLEAVED = 2 };

/* ---- fp16 <-> fp32 (cpp/quant.hpp:73-100, :102-135) ---- */
float    pqo_fp16_to_fp32(uint16_t h);
uint16_t pqo_fp32_to_fp16(float f);
void     pqo_fp16_to_fp32_array(const uint16_t* src, float* dst, size_t n);
void     pqo_fp32_to_fp16_array(const float* src, uint16_t* dst, size_t n);
/* Converts every fp32 bit pattern in [first, first+n) (as uint32) to fp16. */
void     pqo_fp32_bits_to_fp16_range(uint32_t first, size_t n, uint16_t* dst, int n_threads);

/* ---- per-head RMSNorm with the SSE lane order (cpp/tensor.hpp:146-176) ---- */
void pqo_rmsnorm(float* out, const float* x, const float* w, int n);

/* ---- RoPE (cpp/tensor.hpp:201-283 qwen, :286-369 llama) ---- */
void pqo_rope(int style, float* q, float* k, int head_dim, int n_heads, int n_kv_heads,
              const float* cos_pos, const float* sin_pos);
/* RoPE table (cpp/model.hpp:1008-1017): rows [max_seq_len][head_dim/2]. */
void pqo_rope_table(float base, int head_dim, int max_seq_len, float* cos_tab, float* sin_tab);
/* Rows [pos0, pos0+n) only, same values as the full table. */
void pqo_rope_rows(float base, int head_dim, int pos0, int n, float* cos_rows, float* sin_rows);

typedef struct {
    int n_heads, n_kv_heads, head_dim, max_seq_len, rope_style;
} pqo_shape;

/*
 * One attention block at position `pos` (cpp/model.hpp:326-418): optional
 * Q/K per-head RMSNorm, RoPE, K and V fp16 append into the layer's cache
 * slice, then online-softmax GQA attention over t = 0..pos.
 * q[n_heads*hd], k[kv_dim], v[kv_dim] are inputs (not modified).
 * q_norm_w / k_norm_w: [hd] or NULL. cos_pos/sin_pos: the table rows at pos.
 * kc/vc: the layer slice [max_seq_len][kv_dim]. out[n_heads*hd].
 * n_threads > 1 splits query heads across threads; the per-head loop is the
 * same, so the result is bit-identical to n_threads == 1.
 */
void pqo_attn_step(const pqo_shape* s, int pos, const float* q, const float* k, const float* v,
                   const float* q_norm_w, const float* k_norm_w,
                   const float* cos_pos, const float* sin_pos,
                   uint16_t* kc, uint16_t* vc, float* out, int n_threads);

/* Attention only (cpp/model.hpp:375-418) over the cache as it stands, for a
 * query that is already normed and roped. q[n_heads*hd]. */
void pqo_attend(const pqo_shape* s, int pos, const float* q, const uint16_t* kc,
                const uint16_t* vc, float* out, int n_threads);

/* Norm + RoPE + fp16 append only (cpp/model.hpp:326-373); q is normed and
 * roped in place, the K/V rows are written at pos. */
void pqo_append(const pqo_shape* s, int pos, float* q, const float* k, const float* v,
                const float* q_norm_w, const float* k_norm_w,
                const float* cos_pos, const float* sin_pos, uint16_t* kc, uint16_t* vc);

/*
 * Prefill of n_tok tokens at positions start..start+n_tok-1
 * (cpp/model.hpp:493-593): token-major q[n_tok][n_heads*hd],
 * k/v[n_tok][kv_dim], out[n_tok][n_heads*hd]. cos_tab/sin_tab are full
 * tables [max_seq_len][hd/2].
 * serial != 0 runs the reference's own order (append i, attend i, next i).
 * serial == 0 appends every row first and then attends all (token, head)
 * pairs across n_threads; token i only reads rows <= i, so both orders give
 * identical bits.
 */
void pqo_prefill(const pqo_shape* s, int start, int n_tok, const float* q, const float* k,
                 const float* v, const float* q_norm_w, const float* k_norm_w,
                 const float* cos_tab, const float* sin_tab, uint16_t* kc, uint16_t* vc,
                 float* out, int serial, int n_threads);

/* ---- float64 brute-force softmax attention (independent closed form) ---- */
void pqo_attend_f64(const pqo_shape* s, int pos, const float* q, const uint16_t* kc,
                    const uint16_t* vc, double* out);

/* ---- deterministic synthetic inputs ----
 * SplitMix64 (Steele, Lea, Flood 2014) evaluated counter-style:
 * value i of key K is mix(K + (i+1)*0x9E3779B97F4A7C15).
 * Normal i of a stream: Box-Muller in double on uniforms 2i and 2i+1,
 * u = ((r >> 11) + 0.5) * 2^-53, z = sqrt(-2 ln u1) * cos(2 pi u2), rounded to fp32.
 */
uint64_t pqo_splitmix64(uint64_t key, uint64_t i);
uint64_t pqo_stream_key(uint64_t seed, uint32_t kind, uint32_t layer);
float    pqo_normal(uint64_t key, uint64_t i);
void     pqo_fill_normal(uint64_t key, uint64_t first, size_t n, float mean, float stddev, float* out);
/* Outlier flag of cache row `pos`: uniform < outlier_prob. */
int      pqo_is_outlier(uint64_t seed, uint32_t layer, uint64_t pos, float outlier_prob);
/* Cache history rows [pos0, pos0+n) of one layer, fp16 by the reference
 * rounding, K and V ~N(0,1), rows flagged as outliers scaled by 8 first. */
void     pqo_synth_kv_rows(uint64_t seed, uint32_t layer, int kv_dim, int pos0, int n,
                           float outlier_prob, uint16_t* k_rows, uint16_t* v_rows, int n_threads);

enum {
    PQO_KIND_Q = 1, PQO_KIND_K = 2, PQO_KIND_V = 3, PQO_KIND_KHIST = 4, PQO_KIND_VHIST = 5,
    PQO_KIND_QNORM = 6, PQO_KIND_KNORM = 7, PQO_KIND_OUTLIER = 8
};

/* ---- Q/K/V projections (cpp/tensor.hpp:110-143, cpp/quant.hpp:176-358),
 *      pqa_oracle_proj.c; pinned against the reference's own dequantize_row,
 *      vec_dot and matmul_bias (tests/test_oracle_proj.py) ---- */
enum {
    PQO_GGUF_NONE = 0, PQO_GGUF_F32 = 1, PQO_GGUF_F16 = 2, PQO_GGUF_Q4_0 = 3,
    PQO_GGUF_Q8_0 = 9, PQO_GGUF_Q4_K = 13, PQO_GGUF_Q6_K = 15
};  /* the reference's GGUFType numbers (cpp/quant.hpp:16-31) */
size_t pqo_row_bytes(int type, int n);
int    pqo_dequant_row(int type, const void* src, float* dst, int n);
float  pqo_vec_dot(int type, const void* row, const float* x, int n);
int    pqo_matmul_bias(float* out, const float* x, const void* w, int wtype, const void* b, int btype,
                       int n, int d);
/* pqo_matmul_bias for each of n_tok inputs x [n_tok][n] -> out [n_tok][d],
 * rows split over n_threads (same bits per token). */
int    pqo_matmul_bias_tokens(float* out, const float* x, int n_tok, const void* w, int wtype, const void* b,
                              int btype, int n, int d, int n_threads);

#ifdef __cplusplus
}
#endif
#endif
