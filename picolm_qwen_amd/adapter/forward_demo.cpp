// The drop-in adapter (include/pqa_forward.hpp) driven the way picolm_qwen's
// Model drives its layers: a prompt through Model::forward_batch's loop
// (cpp/model.hpp:489-626), then tokens one at a time through Model::forward's
// (cpp/model.hpp:311-451), with the attention block on the MI355X backend.
// The parts the reference keeps (the attention RMSNorm, the FFN) come in as
// callbacks, as a maintainer would pass the Model's own. Built as a small
// shared library with one C entry point so the tests can drive it.
#include <cstring>
#include <string>
#include <vector>

#include "pqa_forward.hpp"

extern "C" {

// attn_norm(layer, xb, x, user): xb [n_embd] = rmsnorm(x, attn_norm_w[layer])
typedef void (*pqaf_norm_fn)(int layer, float* xb, const float* x, void* user);
// ffn(layer, x, user): the FFN of one token, x [n_embd] updated in place
typedef void (*pqaf_ffn_fn)(int layer, float* x, void* user);

// F32 GGUF weights, per layer: wq [q_dim][n_embd], wk and wv [kv_dim][n_embd],
// wo [n_embd][q_dim], biases bq [q_dim], bk and bv [kv_dim], bo [n_embd] (any
// may be NULL), QK-norm weights qn and kn [head_dim] (both NULL: none); all
// layers back to back. x_prompt [n_prompt][n_embd] and x_decode
// [n_decode][n_embd] are the token embeddings, updated in place to the
// residual stream after the last layer. Returns 0, or the pqa error code with
// its message in err.
int pqaf_demo_run(int n_layers, int n_embd, int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
                  int rope_style, float rope_base, const float* wq, const float* wk, const float* wv,
                  const float* wo, const float* bq, const float* bk, const float* bv, const float* bo,
                  const float* qn, const float* kn, int n_prompt, float* x_prompt, int n_decode, float* x_decode,
                  pqaf_norm_fn attn_norm, pqaf_ffn_fn ffn, void* user, char* err, int err_len) {
    try {
        pqa_fwd::Dims d;
        d.n_layers = n_layers;
        d.n_embd = n_embd;
        d.n_heads = n_heads;
        d.n_kv_heads = n_kv_heads;
        d.head_dim = head_dim;
        d.max_seq_len = max_seq_len;
        d.rope_style = rope_style;
        d.rope_base = rope_base;
        pqa_fwd::Attention attn(d);
        const size_t q_dim = (size_t)n_heads * head_dim, kv_dim = (size_t)n_kv_heads * head_dim;
        const size_t n = (size_t)n_embd;
        auto mat = [](const float* base, size_t per_layer, int l, const float* b, size_t b_per_layer) {
            pqa_fwd::Matrix m;
            m.w = base + (size_t)l * per_layer;
            m.type = PQA_GGUF_F32;
            if (b) {
                m.b = b + (size_t)l * b_per_layer;
                m.btype = PQA_GGUF_F32;
            }
            return m;
        };
        for (int l = 0; l < n_layers; l++) {
            pqa_fwd::LayerWeights w;
            w.q = mat(wq, q_dim * n, l, bq, q_dim);
            w.k = mat(wk, kv_dim * n, l, bk, kv_dim);
            w.v = mat(wv, kv_dim * n, l, bv, kv_dim);
            w.o = mat(wo, n * q_dim, l, bo, n);
            if (qn && kn) {
                w.q_norm = qn + (size_t)l * head_dim;
                w.k_norm = kn + (size_t)l * head_dim;
            }
            attn.set_layer(l, w);
        }
        auto norm = [&](int l, float* xb, const float* x) { attn_norm(l, xb, x, user); };
        auto feed = [&](int l, float* x) { ffn(l, x, user); };
        std::vector<float> xb((size_t)(n_prompt > 1 ? n_prompt : 1) * n);
        if (n_prompt > 0) pqa_fwd::forward_batch_layers(attn, 0, n_prompt, x_prompt, xb.data(), norm, feed);
        for (int t = 0; t < n_decode; t++)
            pqa_fwd::forward_layers(attn, n_prompt + t, x_decode + (size_t)t * n, xb.data(), norm, feed);
        return PQA_OK;
    } catch (const pqa_fwd::Error& e) {
        if (err && err_len > 0) {
            std::strncpy(err, e.what(), (size_t)err_len - 1);
            err[err_len - 1] = 0;
        }
        return e.code;
    }
}

}  // extern "C"
