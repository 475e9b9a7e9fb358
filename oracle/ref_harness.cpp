// Driver around the reference's own attention code (rain1201/picolm_qwen,
// cpp/model.hpp), used only to produce golden vectors and to pin the oracle.
// TEST INFRASTRUCTURE: built from the reference headers where they lie by
// oracle/Makefile into oracle/_ref/, never shipped as product code.
//
// Method: a one-layer F32 GGUF whose projections are all zero and whose
// attention output projection is the identity. With a zero token embedding
// the attention RMSNorm output is exactly 0, so Q/K/V equal their bias
// vectors bit for bit (cpp/model.hpp:319-366, matmul_bias adds the bias to an
// exact 0). The harness writes the wanted q/k/v into the public per-layer bias
// vectors of RunState before every Model::forward(token, pos) call. After the
// call the residual stream x[0:q_dim] holds the attention output xb exactly:
// x = 0 + I*xb, and the FFN adds exact zeros because ffn_norm is 0
// (cpp/model.hpp:420-450). The appended K/V rows are read from the public
// key_cache/val_cache vectors.
//
// Bias tensors are named blk.0.attn_{q,k,v}_b.weight: parse_gguf strips
// ".weight" (cpp/model.hpp:866-869) and matmul_bias looks the bias up as
// "attn_q_b" (cpp/model.hpp:321).
//
// Context lengths above the reference's 2048 clamp (cpp/model.hpp:823-828)
// are reached by enlarging the public cache and RoPE vectors after load and
// refilling the table with the reference formula (cpp/model.hpp:1008-1017).
#include "model.hpp"

#include <cstdio>
#include <string>
#include <vector>

namespace {

struct Blob {
    std::vector<uint8_t> b;
    void u32(uint32_t v) { put(&v, 4); }
    void u64(uint64_t v) { put(&v, 8); }
    void f32(float v) { put(&v, 4); }
    void str(const std::string& s) { u64(s.size()); put(s.data(), s.size()); }
    void put(const void* p, size_t n) {
        const uint8_t* c = (const uint8_t*)p;
        b.insert(b.end(), c, c + n);
    }
};

struct TensorSpec {
    std::string name;
    std::vector<uint64_t> dims;
    std::vector<float> data;
};

// Writes a GGUF v3 file: header, metadata, tensor infos, 32-byte aligned data.
bool write_gguf(const char* path, const std::vector<std::pair<std::string, int32_t>>& ints,
                const std::vector<std::pair<std::string, float>>& floats,
                const std::vector<TensorSpec>& tensors) {
    Blob h;
    h.u32(0x46554747u);
    h.u32(3);
    h.u64(tensors.size());
    h.u64(ints.size() + floats.size());
    for (auto& kv : ints) { h.str(kv.first); h.u32(5); h.put(&kv.second, 4); }
    for (auto& kv : floats) { h.str(kv.first); h.u32(6); h.f32(kv.second); }
    uint64_t off = 0;
    std::vector<uint64_t> offs;
    for (auto& t : tensors) {
        h.str(t.name);
        h.u32((uint32_t)t.dims.size());
        for (auto d : t.dims) h.u64(d);
        h.u32(0);  // GGUF F32
        h.u64(off);
        offs.push_back(off);
        off += ((t.data.size() * 4 + 31) / 32) * 32;
    }
    while (h.b.size() % 32) h.b.push_back(0);
    FILE* f = fopen(path, "wb");
    if (!f) return false;
    bool ok = fwrite(h.b.data(), 1, h.b.size(), f) == h.b.size();
    std::vector<uint8_t> pad(32, 0);
    for (size_t i = 0; i < tensors.size() && ok; i++) {
        size_t n = tensors[i].data.size() * 4;
        ok = fwrite(tensors[i].data.data(), 1, n, f) == n;
        size_t p = ((n + 31) / 32) * 32 - n;
        if (ok && p) ok = fwrite(pad.data(), 1, p, f) == p;
    }
    fclose(f);
    return ok;
}

struct RefModel {
    Model m;
    int nh, nkv, hd, smax;
};

}  // namespace

extern "C" {

void* ref_open(const char* gguf_path, int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
               float rope_base, int rope_qwen, int qk_norm) {
    const int q_dim = n_heads * head_dim, kv_dim = n_kv_heads * head_dim;
    const int dim = q_dim, n_ffn = 4, vocab = 2;
    const int ctx_file = max_seq_len > 2048 ? 2048 : max_seq_len;
    std::vector<std::pair<std::string, int32_t>> ints = {
        {"llama.embedding_length", dim},       {"llama.feed_forward_length", n_ffn},
        {"llama.attention.head_count", n_heads}, {"llama.attention.head_count_kv", n_kv_heads},
        {"llama.block_count", 1},              {"llama.context_length", ctx_file},
        {"llama.attention.key_length", head_dim}, {"general.alignment", 32},
    };
    std::vector<std::pair<std::string, float>> floats = {{"llama.rope.freq_base", rope_base}};
    auto zeros = [](std::string name, std::vector<uint64_t> dims) {
        size_t n = 1;
        for (auto d : dims) n *= d;
        return TensorSpec{std::move(name), std::move(dims), std::vector<float>(n, 0.0f)};
    };
    std::vector<TensorSpec> t;
    t.push_back(zeros("token_embd.weight", {(uint64_t)dim, (uint64_t)vocab}));
    t.push_back(zeros("output_norm.weight", {(uint64_t)dim}));
    t.push_back(zeros("blk.0.attn_norm.weight", {(uint64_t)dim}));
    t.push_back(zeros("blk.0.attn_q.weight", {(uint64_t)dim, (uint64_t)q_dim}));
    t.push_back(zeros("blk.0.attn_k.weight", {(uint64_t)dim, (uint64_t)kv_dim}));
    t.push_back(zeros("blk.0.attn_v.weight", {(uint64_t)dim, (uint64_t)kv_dim}));
    TensorSpec wo = zeros("blk.0.attn_output.weight", {(uint64_t)q_dim, (uint64_t)dim});
    for (int i = 0; i < dim; i++) wo.data[(size_t)i * q_dim + i] = 1.0f;
    t.push_back(std::move(wo));
    t.push_back(zeros("blk.0.attn_q_b.weight", {(uint64_t)q_dim}));
    t.push_back(zeros("blk.0.attn_k_b.weight", {(uint64_t)kv_dim}));
    t.push_back(zeros("blk.0.attn_v_b.weight", {(uint64_t)kv_dim}));
    if (qk_norm) {
        TensorSpec qn = zeros("blk.0.attn_q_norm.weight", {(uint64_t)head_dim});
        TensorSpec kn = zeros("blk.0.attn_k_norm.weight", {(uint64_t)head_dim});
        for (auto& x : qn.data) x = 1.0f;
        for (auto& x : kn.data) x = 1.0f;
        t.push_back(std::move(qn));
        t.push_back(std::move(kn));
    }
    t.push_back(zeros("blk.0.ffn_norm.weight", {(uint64_t)dim}));
    t.push_back(zeros("blk.0.ffn_gate.weight", {(uint64_t)dim, (uint64_t)n_ffn}));
    t.push_back(zeros("blk.0.ffn_up.weight", {(uint64_t)dim, (uint64_t)n_ffn}));
    t.push_back(zeros("blk.0.ffn_down.weight", {(uint64_t)n_ffn, (uint64_t)dim}));
    if (!write_gguf(gguf_path, ints, floats, t)) return nullptr;
    t.clear();

    RefModel* r = new RefModel();
    r->nh = n_heads; r->nkv = n_kv_heads; r->hd = head_dim; r->smax = max_seq_len;
    if (r->m.load(gguf_path, 0, false, false) != 0) { delete r; return nullptr; }
    // cpp/picolm.cpp:179-186 picks the RoPE function by model name.
    r->m.rope_fn = rope_qwen ? TensorOps::rope_qwen : TensorOps::rope_llama;
    if (max_seq_len > ctx_file) {
        auto& st = r->m.state;
        r->m.config.ints()[cfg::MAX_SEQ_LEN] = max_seq_len;
        st.key_cache.assign((size_t)max_seq_len * kv_dim, 0);
        st.val_cache.assign((size_t)max_seq_len * kv_dim, 0);
        const int half = head_dim / 2;
        st.rope_cos.assign((size_t)max_seq_len * half, 0.0f);
        st.rope_sin.assign((size_t)max_seq_len * half, 0.0f);
        for (int pos = 0; pos < max_seq_len; pos++) {
            for (int i = 0; i < half; i++) {
                float theta = (float)pos / std::pow(rope_base, (float)(2 * i) / (float)head_dim);
                st.rope_cos[(size_t)pos * half + i] = std::cos(theta);
                st.rope_sin[(size_t)pos * half + i] = std::sin(theta);
            }
        }
    }
    return r;
}

int ref_set_qk_norm(void* h, const float* q_w, const float* k_w) {
    RefModel* r = (RefModel*)h;
    std::copy(q_w, q_w + r->hd, r->m.state.attn_q_norm_w[0].begin());
    std::copy(k_w, k_w + r->hd, r->m.state.attn_k_norm_w[0].begin());
    return 0;
}

int ref_set_cache_rows(void* h, int pos0, int n, const uint16_t* k, const uint16_t* v) {
    RefModel* r = (RefModel*)h;
    size_t kv_dim = (size_t)r->nkv * r->hd;
    std::copy(k, k + (size_t)n * kv_dim, r->m.state.key_cache.begin() + (size_t)pos0 * kv_dim);
    std::copy(v, v + (size_t)n * kv_dim, r->m.state.val_cache.begin() + (size_t)pos0 * kv_dim);
    return 0;
}

int ref_get_cache_rows(void* h, int pos0, int n, uint16_t* k, uint16_t* v) {
    RefModel* r = (RefModel*)h;
    size_t kv_dim = (size_t)r->nkv * r->hd;
    auto kb = r->m.state.key_cache.begin() + (size_t)pos0 * kv_dim;
    auto vb = r->m.state.val_cache.begin() + (size_t)pos0 * kv_dim;
    std::copy(kb, kb + (size_t)n * kv_dim, k);
    std::copy(vb, vb + (size_t)n * kv_dim, v);
    return 0;
}

int ref_get_rope_rows(void* h, int pos0, int n, float* c, float* s) {
    RefModel* r = (RefModel*)h;
    size_t half = (size_t)r->hd / 2;
    auto cb = r->m.state.rope_cos.begin() + (size_t)pos0 * half;
    auto sb = r->m.state.rope_sin.begin() + (size_t)pos0 * half;
    std::copy(cb, cb + (size_t)n * half, c);
    std::copy(sb, sb + (size_t)n * half, s);
    return 0;
}

// One Model::forward(0, pos) with q/k/v injected; out[q_dim] = attention output.
int ref_step(void* h, int pos, const float* q, const float* k, const float* v, float* out) {
    RefModel* r = (RefModel*)h;
    size_t q_dim = (size_t)r->nh * r->hd, kv_dim = (size_t)r->nkv * r->hd;
    auto& st = r->m.state;
    std::copy(q, q + q_dim, st.attn_q_bias[0].begin());
    std::copy(k, k + kv_dim, st.attn_k_bias[0].begin());
    std::copy(v, v + kv_dim, st.attn_v_bias[0].begin());
    r->m.forward(0, pos);
    std::copy(st.x.begin(), st.x.begin() + q_dim, out);
    return 0;
}

void ref_close(void* h) { delete (RefModel*)h; }

// The reference's own sub-operations, for direct pinning of the oracle.
void ref_fp32_bits_to_fp16_range(uint32_t first, size_t n, uint16_t* dst) {
    for (size_t i = 0; i < n; i++) {
        uint32_t u = first + (uint32_t)i;
        float f;
        std::memcpy(&f, &u, 4);
        dst[i] = fp32_to_fp16(f);
    }
}

void ref_fp16_to_fp32_all(float* dst) {
    for (uint32_t i = 0; i < 65536u; i++) dst[i] = fp16_to_fp32((uint16_t)i);
}

void ref_rmsnorm(float* out, const float* x, const float* w, int n) { TensorOps::rmsnorm(out, x, w, n); }

void ref_rope(int qwen, float* q, float* k, int hd, int nh, int nkv, const float* c, const float* s) {
    if (qwen) TensorOps::rope_qwen(q, k, hd, nh, nkv, c, s);
    else TensorOps::rope_llama(q, k, hd, nh, nkv, c, s);
}

// The projection path of Model::forward as the reference computes it
// (cpp/model.hpp:320-366): dequantize_row, vec_dot and TensorOps::matmul_bias
// themselves, for the oracle's projection pins.
void ref_dequantize_row(const void* src, float* dst, int n, int type) { dequantize_row(src, dst, n, (GGUFType)type); }
float ref_vec_dot(const void* row, const float* x, int n, int type) { return vec_dot(row, x, n, (GGUFType)type); }
void ref_matmul_bias(float* out, const float* x, const void* w, const void* b, int n, int d, int wtype, int btype) {
    std::vector<float> scratch((size_t)d);
    TensorOps::matmul_bias(out, x, w, b, n, d, (GGUFType)wtype, (GGUFType)btype, scratch.data());
}

}  // extern "C"
