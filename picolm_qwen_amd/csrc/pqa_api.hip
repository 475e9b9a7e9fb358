// The extern "C" boundary (include/pqa.h): argument checks, HBM ownership,
// host staging, error reporting. Kernels live in pqa_decode.hip,
// pqa_prefill.hip and pqa_util.hip.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <thread>

#include "pqa_copy_pool.h"
#include "pqa_internal.h"

static thread_local std::string g_create_err;

namespace pqa {

int set_err(pqa_ctx* ctx, int code, const std::string& msg) {
    if (ctx) ctx->err = msg;
    else g_create_err = msg;
    return code;
}

int hip_check(pqa_ctx* ctx, hipError_t e, const char* what) {
    if (e == hipSuccess) return PQA_OK;
    const int code = e == hipErrorOutOfMemory ? PQA_ERR_NOMEM : PQA_ERR_HIP;
    return set_err(ctx, code, std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace pqa

using pqa::hip_check;
using pqa::set_err;

static void free_ctx(pqa_ctx* c) {
    if (!c) return;
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    pqa_free_projections(c);
    pqa_free_batch(c);
    void* bufs[] = {c->key_cache, c->val_cache, c->rope_cos, c->rope_sin, c->qk_norm, c->part_acc,
                    c->part_ml,   c->stage,     c->qkv,      c->gen_q};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    if (c->hstage) (void)hipHostFree(c->hstage);
    for (int i = 0; i < 2; ++i) {
        if (c->kvc_buf[i]) (void)hipHostFree(c->kvc_buf[i]);
        if (c->kvc_ev[i]) (void)hipEventDestroy(c->kvc_ev[i]);
        if (c->hpipe_buf[i]) (void)hipHostFree(c->hpipe_buf[i]);
        if (c->hpipe_ev[i]) (void)hipEventDestroy(c->hpipe_ev[i]);
    }
    delete c->copy_pool;
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

template <typename T>
static hipError_t dev_alloc(T** p, size_t count) {
    return hipMalloc((void**)p, std::max<size_t>(count, 1) * sizeof(T));
}

extern "C" int pqa_create(pqa_ctx** out, int n_layers, int max_seq_len, int n_heads, int n_kv_heads,
                          int head_dim, int rope_style, const float* rope_cos, const float* rope_sin) {
    if (!out) return set_err(nullptr, PQA_ERR_ARG, "pqa_create: out is NULL");
    *out = nullptr;
    if (n_layers <= 0 || max_seq_len <= 0 || n_heads <= 0 || n_kv_heads <= 0)
        return set_err(nullptr, PQA_ERR_ARG, "pqa_create: sizes must be positive");
    if (n_heads % n_kv_heads != 0)
        return set_err(nullptr, PQA_ERR_ARG, "pqa_create: n_heads must be a multiple of n_kv_heads");
    if (head_dim <= 0 || head_dim > pqa::kMaxHeadDim || head_dim % 2 != 0)
        return set_err(nullptr, PQA_ERR_UNSUPPORTED, "pqa_create: head_dim must be even and at most 512");
    if (n_heads / n_kv_heads > 0xFFFF)  // the decode launch packs it in 16 bits
        return set_err(nullptr, PQA_ERR_UNSUPPORTED, "pqa_create: more than 65535 query heads per KV head");
    if (rope_style < 0 || rope_style > 2) return set_err(nullptr, PQA_ERR_ARG, "pqa_create: bad rope_style");
    if (!rope_cos || !rope_sin) return set_err(nullptr, PQA_ERR_ARG, "pqa_create: RoPE tables are NULL");

    pqa_ctx* c = new pqa_ctx();
    c->n_layers = n_layers;
    c->max_seq_len = max_seq_len;
    c->n_heads = n_heads;
    c->n_kv_heads = n_kv_heads;
    c->head_dim = head_dim;
    c->rope_style = rope_style;
    c->kv_mul = n_heads / n_kv_heads;
    c->n_chunk = (c->kv_mul + 7) / 8;
    c->chunk_heads = (c->kv_mul + c->n_chunk - 1) / c->n_chunk;
    c->q_dim = (size_t)n_heads * head_dim;
    c->kv_dim = (size_t)n_kv_heads * head_dim;
    c->layer_elems = (size_t)max_seq_len * c->kv_dim;
    c->has_qk_norm.assign(n_layers, 0);

    int rc = PQA_OK;
    auto chk = [&](hipError_t e, const char* what) {
        if (rc == PQA_OK && e != hipSuccess) {
            const int code = e == hipErrorOutOfMemory ? PQA_ERR_NOMEM : PQA_ERR_HIP;
            rc = set_err(nullptr, code, std::string("pqa_create: ") + what + ": " + hipGetErrorString(e));
        }
        return rc == PQA_OK;
    };
    if (chk(hipGetDevice(&c->device), "hipGetDevice")) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, c->device) == hipSuccess && cus > 0)
            c->cu_count = cus;
    }
    chk(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "stream");
    const size_t cache = (size_t)n_layers * c->layer_elems;
    const size_t half = (size_t)head_dim / 2;
    const int ny = n_kv_heads * c->n_chunk;
    c->max_splits = 256;  // the split merge holds one (max, weight) per split in LDS
    if (chk(dev_alloc(&c->key_cache, cache), "key cache") && chk(dev_alloc(&c->val_cache, cache), "value cache")) {
        chk(hipMemset(c->key_cache, 0, cache * 2), "memset");
        chk(hipMemset(c->val_cache, 0, cache * 2), "memset");
    }
    if (chk(dev_alloc(&c->rope_cos, (size_t)max_seq_len * half), "rope") &&
        chk(dev_alloc(&c->rope_sin, (size_t)max_seq_len * half), "rope")) {
        chk(hipMemcpy(c->rope_cos, rope_cos, (size_t)max_seq_len * half * 4, hipMemcpyHostToDevice), "rope copy");
        chk(hipMemcpy(c->rope_sin, rope_sin, (size_t)max_seq_len * half * 4, hipMemcpyHostToDevice), "rope copy");
    }
    chk(dev_alloc(&c->qk_norm, (size_t)n_layers * 2 * head_dim), "qk norm");
    chk(dev_alloc(&c->part_acc, (size_t)ny * c->max_splits * c->chunk_heads * head_dim), "workspace");
    chk(dev_alloc(&c->part_ml, (size_t)ny * c->max_splits * c->chunk_heads * 2), "workspace");
    chk(dev_alloc(&c->qkv, 2 * c->q_dim + 2 * c->kv_dim), "workspace");
    if (!pqa::mfma_head_dim(head_dim) && chk(dev_alloc(&c->gen_q, c->q_dim), "workspace")) c->gen_q_floats = c->q_dim;
    if (rc == PQA_OK) {
        // the no-allocation decode's scratch address on this device
        const int src = pqa::scratch_init(c->device);
        if (src != PQA_OK) rc = src;
    }
    if (rc == PQA_OK) chk(hipDeviceSynchronize(), "sync");
    if (rc != PQA_OK) {
        free_ctx(c);
        return rc;
    }
    *out = c;
    return PQA_OK;
}

extern "C" void pqa_destroy(pqa_ctx* ctx) { free_ctx(ctx); }

extern "C" const char* pqa_last_error(const pqa_ctx* ctx) {
    return ctx ? ctx->err.c_str() : g_create_err.c_str();
}

// The MFMA kernels move q, k, v and out as 16-byte vectors; the general
// head_dim kernels read q, k and v as floats and write out as float pairs.
static bool misaligned(const pqa_ctx* ctx, const void* a, const void* b, const void* c, const void* out) {
    if (!pqa::mfma_head_dim(ctx->head_dim)) return (((uintptr_t)a | (uintptr_t)b | (uintptr_t)c) & 3u) != 0 ||
                                                   ((uintptr_t)out & 7u) != 0;
    return (((uintptr_t)a | (uintptr_t)b | (uintptr_t)c | (uintptr_t)out) & 15u) != 0;
}

static int check_layer(pqa_ctx* ctx, int layer, const char* fn) {
    if (layer < 0 || layer >= ctx->n_layers)
        return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": layer out of range");
    return PQA_OK;
}

extern "C" int pqa_set_qk_norm(pqa_ctx* ctx, int layer, const float* q_norm_w, const float* k_norm_w) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_set_qk_norm: ctx is NULL");
    if (int rc = check_layer(ctx, layer, "pqa_set_qk_norm")) return rc;
    if (!q_norm_w && !k_norm_w) {
        ctx->has_qk_norm[layer] = 0;
        return PQA_OK;
    }
    if (!q_norm_w || !k_norm_w)
        return set_err(ctx, PQA_ERR_ARG, "pqa_set_qk_norm: give both weights or neither");
    const size_t hd = (size_t)ctx->head_dim;
    float* dst = ctx->qk_norm + (size_t)layer * 2 * hd;
    if (int rc = hip_check(ctx, hipStreamSynchronize(ctx->stream), "pqa_set_qk_norm")) return rc;
    if (int rc = hip_check(ctx, hipMemcpy(dst, q_norm_w, hd * 4, hipMemcpyHostToDevice), "pqa_set_qk_norm"))
        return rc;
    if (int rc = hip_check(ctx, hipMemcpy(dst + hd, k_norm_w, hd * 4, hipMemcpyHostToDevice), "pqa_set_qk_norm"))
        return rc;
    ctx->has_qk_norm[layer] = 1;
    return PQA_OK;
}

extern "C" int pqa_decode(pqa_ctx* ctx, int layer, int pos, const float* q, const float* k, const float* v,
                          float* out) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_decode: ctx is NULL");
    if (int rc = check_layer(ctx, layer, "pqa_decode")) return rc;
    if (pos < 0 || pos >= ctx->max_seq_len) return set_err(ctx, PQA_ERR_RANGE, "pqa_decode: pos out of range");
    if (!q || !k || !v || !out) return set_err(ctx, PQA_ERR_ARG, "pqa_decode: NULL buffer");
    if (misaligned(ctx, q, k, v, out))
        return set_err(ctx, PQA_ERR_ARG,
                       "pqa_decode: misaligned buffer (16 bytes for head_dim 64/128; else q/k/v 4, out 8)");
    const pqa::DecodeWorkspace ws{ctx->part_acc, ctx->part_ml, ctx->max_splits};
    return hip_check(ctx, pqa::launch_decode(ctx, layer, pos, q, k, v, out, ws), "pqa_decode");
}

// pqa_decode with its split partials in the library's static device scratch
// (pqa_decode.hip) instead of the context's workspace; calls nothing that
// allocates.
extern "C" int pqa_decode_noalloc(pqa_ctx* ctx, int layer, int pos, const float* q, const float* k,
                                  const float* v, float* out) {
    static const char* fn = "pqa_decode_noalloc";
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_decode_noalloc: ctx is NULL");
    if (int rc = check_layer(ctx, layer, fn)) return rc;
    if (pos < 0 || pos >= ctx->max_seq_len) return set_err(ctx, PQA_ERR_RANGE, "pqa_decode_noalloc: pos out of range");
    if (!q || !k || !v || !out) return set_err(ctx, PQA_ERR_ARG, "pqa_decode_noalloc: NULL buffer");
    if (misaligned(ctx, q, k, v, out))
        return set_err(ctx, PQA_ERR_ARG,
                       "pqa_decode_noalloc: misaligned buffer (16 bytes for head_dim 64/128; else q/k/v 4, out 8)");
    pqa::DecodeWorkspace ws;
    if (int rc = pqa::scratch_workspace(ctx, &ws, fn)) return rc;
    return hip_check(ctx, pqa::launch_decode(ctx, layer, pos, q, k, v, out, ws), fn);
}

extern "C" int pqa_prefill(pqa_ctx* ctx, int layer, int start_pos, int n_tok, const float* q, const float* k,
                           const float* v, float* out) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_prefill: ctx is NULL");
    if (int rc = check_layer(ctx, layer, "pqa_prefill")) return rc;
    if (n_tok <= 0) return set_err(ctx, PQA_ERR_ARG, "pqa_prefill: n_tok must be positive");
    if (start_pos < 0 || (long long)start_pos + n_tok > ctx->max_seq_len)
        return set_err(ctx, PQA_ERR_RANGE, "pqa_prefill: positions out of range");
    if (!q || !k || !v || !out) return set_err(ctx, PQA_ERR_ARG, "pqa_prefill: NULL buffer");
    if (misaligned(ctx, q, k, v, out))
        return set_err(ctx, PQA_ERR_ARG,
                       "pqa_prefill: misaligned buffer (16 bytes for head_dim 64/128; else q/k/v 4, out 8)");
    return hip_check(ctx, pqa::launch_prefill(ctx, layer, start_pos, n_tok, q, k, v, out), "pqa_prefill");
}

static int ensure_stage(pqa_ctx* ctx, size_t floats) {
    if (floats <= ctx->stage_floats) return PQA_OK;
    if (int rc = hip_check(ctx, hipStreamSynchronize(ctx->stream), "staging")) return rc;
    if (ctx->stage) (void)hipFree(ctx->stage);
    ctx->stage = nullptr;
    ctx->stage_floats = 0;
    if (int rc = hip_check(ctx, dev_alloc(&ctx->stage, floats), "staging")) return rc;
    ctx->stage_floats = floats;
    return PQA_OK;
}

// Payloads (q, k, v in and out back) up to this size go through one pinned
// host buffer: a CPU copy into it, one host-to-device copy, the kernels, one
// device-to-host copy. A decode call moves 2 (q_dim + kv_dim) floats, 80 KB at
// 32 query heads of 128; every pageable copy would cost a staged transfer of
// its own. Larger payloads (prompts) stream through two pinned slots (below).
constexpr size_t kHostStageBytes = size_t(4) << 20;

// The pinned staging buffer of the host entries: hipHostMallocDefault, i.e.
// mapped host memory whose coherence kind follows HIP_HOST_COHERENT (fine-
// grained when it is set, coarse-grained otherwise). Either kind is correct
// here because every use is bracketed the same way: the CPU writes the inputs
// before the launch that reads them (a kernel start acquires at system scope)
// and reads the outputs only after hipStreamSynchronize (a kernel end
// releases at system scope); no kernel and CPU touch the buffer at once.
static int ensure_hstage(pqa_ctx* ctx, size_t floats) {
    if (floats <= ctx->hstage_floats) return PQA_OK;
    if (ctx->hstage) (void)hipHostFree(ctx->hstage);
    ctx->hstage = nullptr;
    ctx->hstage_floats = 0;
    if (int rc = hip_check(ctx, hipHostMalloc((void**)&ctx->hstage, floats * sizeof(float), hipHostMallocDefault),
                           "pinned staging"))
        return rc;
    ctx->hstage_floats = floats;
    return PQA_OK;
}

// Larger payloads move through two pinned slots of kPipeBytes: the CPU
// threads fill one slot from the caller's memory while the DMA engine copies
// the other to HBM (and the reverse for the results), so the PCIe copies run
// at DMA speed instead of at the runtime's single-threaded staging of
// pageable memory.
constexpr size_t kPipeBytes = size_t(8) << 20;

static int ensure_pipe(pqa_ctx* ctx, const char* fn) {
    for (int i = 0; i < 2; ++i) {
        if (!ctx->hpipe_buf[i]) {
            if (int rc = hip_check(ctx, hipHostMalloc(&ctx->hpipe_buf[i], kPipeBytes, hipHostMallocDefault), fn)) {
                ctx->hpipe_buf[i] = nullptr;
                return rc;
            }
        }
        if (!ctx->hpipe_ev[i]) {
            if (int rc = hip_check(ctx, hipEventCreateWithFlags(&ctx->hpipe_ev[i], hipEventDisableTiming), fn)) {
                ctx->hpipe_ev[i] = nullptr;
                return rc;
            }
        }
    }
    if (!ctx->copy_pool) {
        const unsigned hw = std::thread::hardware_concurrency();
        const int workers = (int)std::min(7u, std::max(1u, hw / 2) - 1u);
        try {
            ctx->copy_pool = new pqa::CopyPool(workers);
        } catch (...) {
            return set_err(ctx, PQA_ERR_NOMEM, std::string(fn) + ": cannot start the copy threads");
        }
    }
    return PQA_OK;
}

struct HostSpan {
    const char* p;
    size_t n;
};

// dev[0, total) = the concatenation of spans, queued on the context stream;
// returns once every slot is refilled for the last time (the last copies may
// still be in flight; the caller's later stream work orders after them).
static int pipe_to_device(pqa_ctx* ctx, char* dev, const HostSpan* spans, int nspans, const char* fn) {
    size_t total = 0;
    for (int i = 0; i < nspans; ++i) total += spans[i].n;
    int si = 0;
    size_t soff = 0;
    for (size_t off = 0, c = 0; off < total; off += kPipeBytes, ++c) {
        const int b = (int)(c & 1);
        if (c >= 2)
            if (int rc = hip_check(ctx, hipEventSynchronize(ctx->hpipe_ev[b]), fn)) return rc;
        const size_t len = std::min(kPipeBytes, total - off);
        char* slot = (char*)ctx->hpipe_buf[b];
        for (size_t done = 0; done < len;) {  // gather [off, off + len) from the spans
            const size_t m = std::min(len - done, spans[si].n - soff);
            ctx->copy_pool->copy(slot + done, spans[si].p + soff, m);
            done += m;
            soff += m;
            if (soff == spans[si].n) {
                ++si;
                soff = 0;
            }
        }
        if (int rc = hip_check(ctx, hipMemcpyAsync(dev + off, slot, len, hipMemcpyHostToDevice, ctx->stream), fn))
            return rc;
        if (int rc = hip_check(ctx, hipEventRecord(ctx->hpipe_ev[b], ctx->stream), fn)) return rc;
    }
    return PQA_OK;
}

// host[0, total) = dev[0, total) after the work queued so far; returns when
// every byte is in host memory.
static int pipe_to_host(pqa_ctx* ctx, char* host, const char* dev, size_t total, const char* fn) {
    const size_t nc = (total + kPipeBytes - 1) / kPipeBytes;
    auto queue = [&](size_t c) {
        const int b = (int)(c & 1);
        const size_t off = c * kPipeBytes, len = std::min(kPipeBytes, total - off);
        int rc = hip_check(ctx, hipMemcpyAsync(ctx->hpipe_buf[b], dev + off, len, hipMemcpyDeviceToHost, ctx->stream), fn);
        if (!rc) rc = hip_check(ctx, hipEventRecord(ctx->hpipe_ev[b], ctx->stream), fn);
        return rc;
    };
    for (size_t c = 0; c < std::min<size_t>(2, nc); ++c)
        if (int rc = queue(c)) return rc;
    for (size_t c = 0; c < nc; ++c) {
        const int b = (int)(c & 1);
        if (int rc = hip_check(ctx, hipEventSynchronize(ctx->hpipe_ev[b]), fn)) return rc;
        const size_t off = c * kPipeBytes, len = std::min(kPipeBytes, total - off);
        ctx->copy_pool->copy(host + off, (const char*)ctx->hpipe_buf[b], len);
        if (c + 2 < nc)
            if (int rc = queue(c + 2)) return rc;
    }
    return PQA_OK;
}

static int run_host(pqa_ctx* ctx, int layer, int pos, int n_tok, bool prefill, const float* q, const float* k,
                    const float* v, float* out, const char* fn) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, std::string(fn) + ": ctx is NULL");
    if (!q || !k || !v || !out) return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": NULL buffer");
    if (n_tok <= 0) return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": n_tok must be positive");
    const size_t nq = (size_t)n_tok * ctx->q_dim, nkv = (size_t)n_tok * ctx->kv_dim;
    const size_t in_floats = nq + 2 * nkv;
    if (int rc = ensure_stage(ctx, in_floats + nq)) return rc;
    float* dq = ctx->stage;  // q, k, v contiguous, then out
    float* dk = dq + nq;
    float* dv = dk + nkv;
    float* dout = dv + nkv;
    hipStream_t st = ctx->stream;
    const bool pinned = (in_floats + nq) * sizeof(float) <= kHostStageBytes;
    int rc = PQA_OK;
    if (pinned && !prefill) {
        // Decode reads q, k, v and writes out in the pinned staging buffer
        // itself (host memory the device addresses directly): no DMA copies,
        // the launches and one stream sync. The previous call ended with a
        // stream sync, so the buffer is free.
        if ((rc = ensure_hstage(ctx, in_floats + nq))) return rc;
        float* h = ctx->hstage;
        std::memcpy(h, q, nq * sizeof(float));
        std::memcpy(h + nq, k, nkv * sizeof(float));
        std::memcpy(h + nq + nkv, v, nkv * sizeof(float));
        float* hd = nullptr;
        rc = hip_check(ctx, hipHostGetDevicePointer((void**)&hd, h, 0), fn);
        if (!rc) rc = pqa_decode(ctx, layer, pos, hd, hd + nq, hd + nq + nkv, hd + in_floats);
        if (!rc) rc = hip_check(ctx, hipStreamSynchronize(st), fn);
        else (void)hipStreamSynchronize(st);  // a failed call leaves no kernel using the buffer
        if (!rc) std::memcpy(out, h + in_floats, nq * sizeof(float));
        return rc;
    }
    if (pinned) {
        // the previous call ended with a stream sync, so the buffer is free
        if ((rc = ensure_hstage(ctx, in_floats + nq))) return rc;
        float* h = ctx->hstage;
        std::memcpy(h, q, nq * sizeof(float));
        std::memcpy(h + nq, k, nkv * sizeof(float));
        std::memcpy(h + nq + nkv, v, nkv * sizeof(float));
        rc = hip_check(ctx, hipMemcpyAsync(dq, h, in_floats * sizeof(float), hipMemcpyHostToDevice, st), fn);
    } else {
        // q, k and v are contiguous in the device staging
        const HostSpan spans[3] = {{(const char*)q, nq * 4}, {(const char*)k, nkv * 4}, {(const char*)v, nkv * 4}};
        rc = ensure_pipe(ctx, fn);
        if (!rc) rc = pipe_to_device(ctx, (char*)dq, spans, 3, fn);
        if (!rc)
            rc = prefill ? pqa_prefill(ctx, layer, pos, n_tok, dq, dk, dv, dout)
                         : pqa_decode(ctx, layer, pos, dq, dk, dv, dout);
        if (!rc) rc = pipe_to_host(ctx, (char*)out, (const char*)dout, nq * 4, fn);
        (void)hipStreamSynchronize(st);  // also after a failure: no copy still uses the slots
        return rc;
    }
    if (!rc)
        rc = prefill ? pqa_prefill(ctx, layer, pos, n_tok, dq, dk, dv, dout)
                     : pqa_decode(ctx, layer, pos, dq, dk, dv, dout);
    float* back = ctx->hstage + in_floats;
    if (!rc) rc = hip_check(ctx, hipMemcpyAsync(back, dout, nq * 4, hipMemcpyDeviceToHost, st), fn);
    if (!rc) rc = hip_check(ctx, hipStreamSynchronize(st), fn);
    else (void)hipStreamSynchronize(st);  // a failed call leaves no copy reading the buffer
    if (!rc) std::memcpy(out, back, nq * sizeof(float));
    return rc;
}

// Host-pointer forms of pqa_attention_block and pqa_prefill_block: xb and x
// (read and written) copied in, the block, x copied back, a stream sync; the
// same pinned staging as run_host for payloads up to kHostStageBytes.
static int run_block_host(pqa_ctx* ctx, int layer, int pos, int n_tok, bool prefill, const float* xb, float* x,
                          const char* fn) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, std::string(fn) + ": ctx is NULL");
    if (int rc = check_layer(ctx, layer, fn)) return rc;
    if (ctx->proj.empty() || !ctx->proj[layer].n_embd || !ctx->proj[layer].out_rows)
        return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": the layer needs q/k/v and attn_output weights");
    if (ctx->proj[layer].n_embd != ctx->proj[layer].out_rows)
        return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": attn_q/k/v width and attn_output rows differ");
    if (!xb || !x) return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": NULL buffer");
    if (n_tok <= 0) return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": n_tok must be positive");
    const size_t n = (size_t)n_tok * ctx->proj[layer].out_rows;
    const size_t n4 = (n + 3) & ~(size_t)3;  // x starts 16-byte aligned in the staging
    if (int rc = ensure_stage(ctx, n4 + n)) return rc;
    float* dxb = ctx->stage;
    float* dx = dxb + n4;
    hipStream_t st = ctx->stream;
    const bool pinned = (n4 + n + n) * sizeof(float) <= kHostStageBytes;
    int rc = PQA_OK;
    if (pinned) {
        if ((rc = ensure_hstage(ctx, n4 + n + n))) return rc;
        float* h = ctx->hstage;
        std::memcpy(h, xb, n * sizeof(float));
        std::memcpy(h + n4, x, n * sizeof(float));
        rc = hip_check(ctx, hipMemcpyAsync(dxb, h, (n4 + n) * sizeof(float), hipMemcpyHostToDevice, st), fn);
    } else {
        // xb, then x at its 16-byte aligned offset n4
        static const float zero_pad[3] = {0.0f, 0.0f, 0.0f};
        const HostSpan spans[3] = {{(const char*)xb, n * 4}, {(const char*)zero_pad, (n4 - n) * 4}, {(const char*)x, n * 4}};
        rc = ensure_pipe(ctx, fn);
        if (!rc) rc = pipe_to_device(ctx, (char*)dxb, spans, 3, fn);
        if (!rc)
            rc = prefill ? pqa_prefill_block(ctx, layer, pos, n_tok, dxb, dx)
                         : pqa_attention_block(ctx, layer, pos, dxb, dx);
        if (!rc) rc = pipe_to_host(ctx, (char*)x, (const char*)dx, n * 4, fn);
        (void)hipStreamSynchronize(st);  // also after a failure: no copy still uses the slots
        return rc;
    }
    if (!rc)
        rc = prefill ? pqa_prefill_block(ctx, layer, pos, n_tok, dxb, dx) : pqa_attention_block(ctx, layer, pos, dxb, dx);
    float* back = ctx->hstage + n4 + n;
    if (!rc) rc = hip_check(ctx, hipMemcpyAsync(back, dx, n * sizeof(float), hipMemcpyDeviceToHost, st), fn);
    if (!rc) rc = hip_check(ctx, hipStreamSynchronize(st), fn);
    else (void)hipStreamSynchronize(st);  // a failed call leaves no copy reading the buffers
    if (!rc) std::memcpy(x, back, n * sizeof(float));
    return rc;
}

extern "C" int pqa_attention_block_host(pqa_ctx* ctx, int layer, int pos, const float* xb, float* x) {
    return run_block_host(ctx, layer, pos, 1, false, xb, x, "pqa_attention_block_host");
}

extern "C" int pqa_prefill_block_host(pqa_ctx* ctx, int layer, int start_pos, int n_tok, const float* xb,
                                      float* x) {
    return run_block_host(ctx, layer, start_pos, n_tok, true, xb, x, "pqa_prefill_block_host");
}

extern "C" int pqa_decode_host(pqa_ctx* ctx, int layer, int pos, const float* q, const float* k, const float* v,
                               float* out) {
    return run_host(ctx, layer, pos, 1, false, q, k, v, out, "pqa_decode_host");
}

extern "C" int pqa_prefill_host(pqa_ctx* ctx, int layer, int start_pos, int n_tok, const float* q,
                                const float* k, const float* v, float* out) {
    return run_host(ctx, layer, start_pos, n_tok, true, q, k, v, out, "pqa_prefill_host");
}

static int kv_rows_check(pqa_ctx* ctx, int layer, int pos0, int n, const char* fn) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, std::string(fn) + ": ctx is NULL");
    if (int rc = check_layer(ctx, layer, fn)) return rc;
    if (n < 0 || pos0 < 0 || (long long)pos0 + n > ctx->max_seq_len)
        return set_err(ctx, PQA_ERR_RANGE, std::string(fn) + ": rows out of range");
    return PQA_OK;
}

extern "C" int pqa_kv_upload(pqa_ctx* ctx, int layer, int pos0, int n, const uint16_t* k_rows,
                             const uint16_t* v_rows) {
    if (int rc = kv_rows_check(ctx, layer, pos0, n, "pqa_kv_upload")) return rc;
    const size_t off = (size_t)layer * ctx->layer_elems + (size_t)pos0 * ctx->kv_dim;
    const size_t bytes = (size_t)n * ctx->kv_dim * 2;
    int rc = PQA_OK;
    if (k_rows && bytes)
        rc = hip_check(ctx, hipMemcpyAsync(ctx->key_cache + off, k_rows, bytes, hipMemcpyHostToDevice, ctx->stream),
                       "pqa_kv_upload");
    if (!rc && v_rows && bytes)
        rc = hip_check(ctx, hipMemcpyAsync(ctx->val_cache + off, v_rows, bytes, hipMemcpyHostToDevice, ctx->stream),
                       "pqa_kv_upload");
    if (!rc) rc = hip_check(ctx, hipStreamSynchronize(ctx->stream), "pqa_kv_upload");
    return rc;
}

extern "C" int pqa_kv_download(pqa_ctx* ctx, int layer, int pos0, int n, uint16_t* k_rows, uint16_t* v_rows) {
    if (int rc = kv_rows_check(ctx, layer, pos0, n, "pqa_kv_download")) return rc;
    const size_t off = (size_t)layer * ctx->layer_elems + (size_t)pos0 * ctx->kv_dim;
    const size_t bytes = (size_t)n * ctx->kv_dim * 2;
    int rc = PQA_OK;
    if (k_rows && bytes)
        rc = hip_check(ctx, hipMemcpyAsync(k_rows, ctx->key_cache + off, bytes, hipMemcpyDeviceToHost, ctx->stream),
                       "pqa_kv_download");
    if (!rc && v_rows && bytes)
        rc = hip_check(ctx, hipMemcpyAsync(v_rows, ctx->val_cache + off, bytes, hipMemcpyDeviceToHost, ctx->stream),
                       "pqa_kv_download");
    if (!rc) rc = hip_check(ctx, hipStreamSynchronize(ctx->stream), "pqa_kv_download");
    return rc;
}

extern "C" int pqa_kv_cache(pqa_ctx* ctx, uint16_t** key_cache, uint16_t** val_cache) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_kv_cache: ctx is NULL");
    if (key_cache) *key_cache = ctx->key_cache;
    if (val_cache) *val_cache = ctx->val_cache;
    return PQA_OK;
}

extern "C" void* pqa_stream(pqa_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

extern "C" int pqa_sync(pqa_ctx* ctx) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_sync: ctx is NULL");
    return hip_check(ctx, hipStreamSynchronize(ctx->stream), "pqa_sync");
}

extern "C" void pqa_rope_table(float rope_base, int head_dim, int max_seq_len, float* cos_tab, float* sin_tab) {
    const int half = head_dim / 2;
    for (int pos = 0; pos < max_seq_len; pos++)
        for (int i = 0; i < half; i++) {
            const float theta = (float)pos / powf(rope_base, (float)(2 * i) / (float)head_dim);
            cos_tab[(size_t)pos * half + i] = cosf(theta);
            sin_tab[(size_t)pos * half + i] = sinf(theta);
        }
}

extern "C" int pqa_fp32_to_fp16(pqa_ctx* ctx, const float* src, uint16_t* dst, size_t n) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_fp32_to_fp16: ctx is NULL");
    if (n && (!src || !dst)) return set_err(ctx, PQA_ERR_ARG, "pqa_fp32_to_fp16: NULL buffer");
    return hip_check(ctx, pqa::launch_f32_to_f16(ctx, src, dst, n), "pqa_fp32_to_fp16");
}

extern "C" int pqa_synth_kv(pqa_ctx* ctx, int layer, int pos0, int n, uint64_t seed, float outlier_prob) {
    if (int rc = kv_rows_check(ctx, layer, pos0, n, "pqa_synth_kv")) return rc;
    return hip_check(ctx, pqa::launch_synth_kv(ctx, layer, pos0, n, seed, outlier_prob), "pqa_synth_kv");
}

extern "C" int pqa_set_decode_split(pqa_ctx* ctx, int rows_per_split) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_set_decode_split: ctx is NULL");
    if (rows_per_split < 0 || (rows_per_split % 64) != 0)
        return set_err(ctx, PQA_ERR_ARG, "pqa_set_decode_split: must be 0 or a positive multiple of 64");
    ctx->split_override = rows_per_split;
    return PQA_OK;
}

extern "C" int pqa_set_prefill_precision(pqa_ctx* ctx, int split_q) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_set_prefill_precision: ctx is NULL");
    if (split_q != 0 && split_q != 1) return set_err(ctx, PQA_ERR_ARG, "pqa_set_prefill_precision: 0 or 1");
    ctx->prefill_split_q = split_q;
    return PQA_OK;
}
