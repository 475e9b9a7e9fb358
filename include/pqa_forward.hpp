/*
 * pqa_forward.hpp -- the attention path of picolm_qwen's forward loops on the
 * MI355X backend, as a header-only C++17 adapter over pqa.h.
 *
 * It mirrors the layer loops of Model::forward (cpp/model.hpp:311-451) and
 * Model::forward_batch (cpp/model.hpp:489-626) with their attention block --
 * the Q/K/V projections, QK-norm, RoPE, the fp16 K/V append, attention, the
 * output projection and the residual add (:320-427 and :493-600) -- replaced
 * by the backend. What the loop does besides (the RMSNorms, the FFN, the
 * logits) stays with the caller and is passed in as callables, so a
 * maintainer swaps the block and keeps the rest of Model as it is.
 *
 * Host pointers throughout, as the reference holds its RunState vectors; the
 * KV cache lives in HBM in the reference's byte layout. Build: add
 * -I<repo>/include, link -L<repo>/picolm_qwen_amd -lpqa. Needs no HIP header.
 */
#ifndef PQA_FORWARD_HPP
#define PQA_FORWARD_HPP

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "pqa.h"

namespace pqa_fwd {

// A failed backend call: the pqa_* return code and pqa_last_error's message.
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& msg) : std::runtime_error(msg), code(c) {}
};

inline void check(int rc, const pqa_ctx* ctx) {
    if (rc != PQA_OK) {
        const char* m = pqa_last_error(ctx);
        throw Error(rc, m ? m : "pqa error");
    }
}

// One GGUF matrix as the model file stores it ([rows][row bytes]) and its
// optional bias (F32 or F16, PQA_GGUF_NONE for none): the LayerWeights entries
// the block reads (cpp/model.hpp:320-366, :420-425).
struct Matrix {
    const void* w = nullptr;
    int type = PQA_GGUF_NONE;
    const void* b = nullptr;
    int btype = PQA_GGUF_NONE;
};

struct LayerWeights {
    Matrix q, k, v, o;              // attn_q, attn_k, attn_v, attn_output
    const float* q_norm = nullptr;  // attn_q_norm / attn_k_norm [head_dim], or null
    const float* k_norm = nullptr;
};

// The model dimensions the block needs (cpp/model.hpp:288-300).
struct Dims {
    int n_layers = 0, n_embd = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0, max_seq_len = 0;
    int rope_style = PQA_ROPE_NEOX_HALF;  // the RopeFn picked at cpp/picolm.cpp:179-186
    float rope_base = 10000.0f;
};

class Attention {
  public:
    // allocate_run_state's attention part (cpp/model.hpp:1003-1017): the RoPE
    // table with the reference's formula and the HBM KV cache.
    explicit Attention(const Dims& d) : d_(d) {
        const size_t half = (size_t)d.head_dim / 2;
        std::vector<float> cos_tab((size_t)d.max_seq_len * half), sin_tab(cos_tab.size());
        pqa_rope_table(d.rope_base, d.head_dim, d.max_seq_len, cos_tab.data(), sin_tab.data());
        check(pqa_create(&ctx_, d.n_layers, d.max_seq_len, d.n_heads, d.n_kv_heads, d.head_dim, d.rope_style,
                         cos_tab.data(), sin_tab.data()),
              nullptr);
    }
    ~Attention() { pqa_destroy(ctx_); }
    Attention(const Attention&) = delete;
    Attention& operator=(const Attention&) = delete;

    const Dims& dims() const { return d_; }
    pqa_ctx* ctx() const { return ctx_; }

    // The layer's weights as the GGUF stores them (uploaded once).
    void set_layer(int layer, const LayerWeights& w) {
        check(pqa_set_qk_norm(ctx_, layer, w.q_norm, w.k_norm), ctx_);
        check(pqa_set_qkv_weights(ctx_, layer, d_.n_embd, w.q.w, w.q.type, w.q.b, w.q.btype, w.k.w, w.k.type, w.k.b,
                                  w.k.btype, w.v.w, w.v.type, w.v.b, w.v.btype),
              ctx_);
        check(pqa_set_out_weights(ctx_, layer, d_.n_embd, w.o.w, w.o.type, w.o.b, w.o.btype), ctx_);
    }

    // cpp/model.hpp:320-427 for one token: xb [n_embd] (the attention norm's
    // output) in, the residual stream x [n_embd] updated in place.
    void decode(int layer, int pos, const float* xb, float* x) {
        check(pqa_attention_block_host(ctx_, layer, pos, xb, x), ctx_);
    }

    // cpp/model.hpp:493-600 for a prompt chunk, without the FFN: xb and x
    // [n_tok][n_embd], token i at position start + i.
    void prefill(int layer, int start, int n_tok, const float* xb, float* x) {
        check(pqa_prefill_block_host(ctx_, layer, start, n_tok, xb, x), ctx_);
    }

    // The attention alone (cpp/model.hpp:326-418) for a loop that keeps its own
    // projections: q [q_dim], k and v [kv_dim] as matmul_bias left them; out
    // [q_dim] is what the block leaves in xb.
    void attend(int layer, int pos, const float* q, const float* k, const float* v, float* out) {
        check(pqa_decode_host(ctx_, layer, pos, q, k, v, out), ctx_);
    }

    // The cache rows the reference would hold in state.key_cache/val_cache.
    void kv_rows(int layer, int pos0, int n, uint16_t* k_rows, uint16_t* v_rows) {
        check(pqa_kv_download(ctx_, layer, pos0, n, k_rows, v_rows), ctx_);
    }

  private:
    Dims d_;
    pqa_ctx* ctx_ = nullptr;
};

// Model::forward's layer loop (cpp/model.hpp:311-451) for the token at pos,
// with the block on the backend:
//   for each layer: attn_norm(layer, xb, x)  -- rmsnorm(xb, x, attn_norm_w[l]) (:314)
//                   the block                 -- :320-427
//                   ffn(layer, x)             -- :428-450, x updated in place
// xb is caller scratch of n_embd floats; x is the residual stream.
template <class AttnNorm, class Ffn>
void forward_layers(Attention& a, int pos, float* x, float* xb, AttnNorm&& attn_norm, Ffn&& ffn) {
    for (int l = 0; l < a.dims().n_layers; l++) {
        attn_norm(l, xb, (const float*)x);
        a.decode(l, pos, xb, x);
        ffn(l, x);
    }
}

// Model::forward_batch's layer loop (cpp/model.hpp:489-626) over a prompt
// chunk of n_tok tokens from start: per layer, the attention norm of every
// token, the block for all of them at once, then each token's FFN. Token i's
// attention reads only rows written by tokens <= i of the same layer, so this
// order gives the values of the reference's token-by-token loop. x and xb are
// [n_tok][n_embd].
template <class AttnNorm, class Ffn>
void forward_batch_layers(Attention& a, int start, int n_tok, float* x, float* xb, AttnNorm&& attn_norm, Ffn&& ffn) {
    const size_t n = (size_t)a.dims().n_embd;
    for (int l = 0; l < a.dims().n_layers; l++) {
        for (int i = 0; i < n_tok; i++) attn_norm(l, xb + i * n, (const float*)(x + i * n));
        a.prefill(l, start, n_tok, xb, x);
        for (int i = 0; i < n_tok; i++) ffn(l, x + i * n);
    }
}

}  // namespace pqa_fwd

#endif  // PQA_FORWARD_HPP
