// .kvc persistence of the HBM KV cache, in the file format of the reference's
// kvcache_save / kvcache_load (picolm/model.c:870-983):
//   uint32 header {magic 0x4B564350 "KVCP", n_pos, n_layers, kv_dim}, host order,
//   then rows [0, n_pos) of the K cache of layer 0, 1, ..., then the same of V.
// Rows [0, n_pos) of one layer are one contiguous run of the cache in HBM
// ([n_layers][max_seq_len][kv_dim] fp16), so the file body is 2*n_layers runs
// of n_pos*kv_dim*2 bytes. The body is streamed in chunks through two pinned
// host buffers: the PCIe copy of one chunk overlaps the file write (save) or
// read (load) of the other, and a chunk may span several runs.
#include <errno.h>
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <string>

#include "pqa_internal.h"

using pqa::hip_check;
using pqa::set_err;

namespace {

constexpr uint32_t kKvcMagic = 0x4B564350u;  // picolm/model.h:12
constexpr size_t kChunk = size_t(16) << 20;  // bytes per staging buffer

// Position in the file body: run r < n_layers is layer r of the K cache, run
// n_layers + l is layer l of the V cache.
struct BodyCursor {
    const pqa_ctx* c;
    size_t run_bytes;
    int run = 0;
    size_t off = 0;

    char* run_base() const {
        const uint16_t* cache = run < c->n_layers ? c->key_cache : c->val_cache;
        return (char*)(cache + (size_t)(run % c->n_layers) * c->layer_elems);
    }

    // Queues the copies of the next `bytes` bytes of the body between HBM and
    // host[0, bytes).
    hipError_t copy(char* host, size_t bytes, bool to_host, hipStream_t s) {
        size_t done = 0;
        while (done < bytes) {
            const size_t n = std::min(bytes - done, run_bytes - off);
            char* dev = run_base() + off;
            const hipError_t e = to_host ? hipMemcpyAsync(host + done, dev, n, hipMemcpyDeviceToHost, s)
                                         : hipMemcpyAsync(dev, host + done, n, hipMemcpyHostToDevice, s);
            if (e != hipSuccess) return e;
            done += n;
            off += n;
            if (off == run_bytes) {
                ++run;
                off = 0;
            }
        }
        return hipSuccess;
    }
};

int ensure_staging(pqa_ctx* c, const char* fn) {
    for (int i = 0; i < 2; ++i) {
        if (!c->kvc_buf[i]) {
            if (int rc = hip_check(c, hipHostMalloc(&c->kvc_buf[i], kChunk, hipHostMallocDefault), fn)) {
                c->kvc_buf[i] = nullptr;
                return rc;
            }
        }
        if (!c->kvc_ev[i]) {
            if (int rc = hip_check(c, hipEventCreateWithFlags(&c->kvc_ev[i], hipEventDisableTiming), fn)) {
                c->kvc_ev[i] = nullptr;
                return rc;
            }
        }
    }
    return PQA_OK;
}

bool write_full(int fd, const void* p, size_t n) {
    const char* b = (const char*)p;
    while (n) {
        const ssize_t w = write(fd, b, n);
        if (w < 0) {
            if (errno == EINTR) continue;
            return false;
        }
        b += w;
        n -= (size_t)w;
    }
    return true;
}

// Bytes read (fewer than n only at end of file), or -1 on a read error.
ssize_t read_full(int fd, void* p, size_t n) {
    char* b = (char*)p;
    size_t got = 0;
    while (got < n) {
        const ssize_t r = read(fd, b + got, n - got);
        if (r < 0) {
            if (errno == EINTR) continue;
            return -1;
        }
        if (r == 0) break;
        got += (size_t)r;
    }
    return (ssize_t)got;
}

std::string sys_err(const char* fn, const char* what, const char* path) {
    return std::string(fn) + ": " + what + " " + path + ": " + strerror(errno);
}

}  // namespace

extern "C" int pqa_kvc_save(pqa_ctx* ctx, const char* path, int n_pos) {
    static const char* fn = "pqa_kvc_save";
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_kvc_save: ctx is NULL");
    if (!path) return set_err(ctx, PQA_ERR_ARG, "pqa_kvc_save: path is NULL");
    if (n_pos <= 0 || n_pos > ctx->max_seq_len)
        return set_err(ctx, PQA_ERR_RANGE, "pqa_kvc_save: n_pos outside [1, max_seq_len]");
    if (int rc = ensure_staging(ctx, fn)) return rc;
    const int fd = open(path, O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0666);
    if (fd < 0) return set_err(ctx, PQA_ERR_IO, sys_err(fn, "cannot open", path));

    const uint32_t header[4] = {kKvcMagic, (uint32_t)n_pos, (uint32_t)ctx->n_layers, (uint32_t)ctx->kv_dim};
    BodyCursor cur{ctx, (size_t)n_pos * ctx->kv_dim * sizeof(uint16_t)};
    size_t left = 2 * (size_t)ctx->n_layers * cur.run_bytes;
    int rc = PQA_OK;
    if (!write_full(fd, header, sizeof header)) rc = set_err(ctx, PQA_ERR_IO, sys_err(fn, "write failed on", path));

    // Chunk i is copied into buffer i&1 while chunk i-1 is written from the
    // other; the copies queue behind the work already on the context stream.
    size_t len[2] = {0, 0};
    auto issue = [&](int b) -> int {
        len[b] = std::min(kChunk, left);
        left -= len[b];
        if (!len[b]) return PQA_OK;
        if (int r = hip_check(ctx, cur.copy((char*)ctx->kvc_buf[b], len[b], true, ctx->stream), fn)) return r;
        return hip_check(ctx, hipEventRecord(ctx->kvc_ev[b], ctx->stream), fn);
    };
    if (!rc) rc = issue(0);
    for (int b = 0; !rc && len[b]; b ^= 1) {
        if ((rc = issue(b ^ 1))) break;
        if ((rc = hip_check(ctx, hipEventSynchronize(ctx->kvc_ev[b]), fn))) break;
        if (!write_full(fd, ctx->kvc_buf[b], len[b])) rc = set_err(ctx, PQA_ERR_IO, sys_err(fn, "write failed on", path));
    }
    if (rc) (void)hipStreamSynchronize(ctx->stream);  // no copy may still target a staging buffer
    if (close(fd) != 0 && !rc) rc = set_err(ctx, PQA_ERR_IO, sys_err(fn, "close failed on", path));
    return rc;
}

extern "C" int pqa_kvc_load(pqa_ctx* ctx, const char* path) {
    static const char* fn = "pqa_kvc_load";
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_kvc_load: ctx is NULL"), 0;
    if (!path) return set_err(ctx, PQA_ERR_ARG, "pqa_kvc_load: path is NULL"), 0;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return set_err(ctx, PQA_ERR_IO, sys_err(fn, "cannot open", path)), 0;
    auto fail = [&](int code, const std::string& msg) {
        close(fd);
        return set_err(ctx, code, msg), 0;
    };

    uint32_t header[4];
    if (read_full(fd, header, sizeof header) != (ssize_t)sizeof header)
        return fail(PQA_ERR_IO, std::string(fn) + ": short header in " + path);
    if (header[0] != kKvcMagic) return fail(PQA_ERR_FORMAT, std::string(fn) + ": invalid magic in " + path);
    const int n_pos = (int)header[1];
    if ((int)header[2] != ctx->n_layers || (int)header[3] != (int)ctx->kv_dim)
        return fail(PQA_ERR_FORMAT, std::string(fn) + ": model mismatch (layers " + std::to_string((int)header[2]) +
                                        "/" + std::to_string(ctx->n_layers) + ", kv_dim " +
                                        std::to_string((int)header[3]) + "/" + std::to_string(ctx->kv_dim) + ")");
    if (n_pos > ctx->max_seq_len)
        return fail(PQA_ERR_FORMAT, std::string(fn) + ": " + std::to_string(n_pos) +
                                        " cached positions exceed max_seq_len");
    if (n_pos <= 0) {
        // Nothing to read; the header count comes back as it is, as in the
        // reference (a count of 2^31 or more reads as negative there too).
        close(fd);
        return n_pos;
    }
    if (ensure_staging(ctx, fn)) return close(fd), 0;

    BodyCursor cur{ctx, (size_t)n_pos * ctx->kv_dim * sizeof(uint16_t)};
    size_t left = 2 * (size_t)ctx->n_layers * cur.run_bytes;
    bool pending[2] = {false, false};
    int rc = PQA_OK;
    bool short_file = false;
    // Chunk i is read into buffer i&1 while the copy of chunk i-1 runs. On a
    // short file the bytes that were read are still placed, so the cache ends
    // as the reference's row-by-row fread leaves it.
    for (int b = 0; left && !rc && !short_file; b ^= 1) {
        const size_t want = std::min(kChunk, left);
        if (pending[b] && (rc = hip_check(ctx, hipEventSynchronize(ctx->kvc_ev[b]), fn))) break;
        const ssize_t got = read_full(fd, ctx->kvc_buf[b], want);
        if (got < 0) {
            rc = set_err(ctx, PQA_ERR_IO, sys_err(fn, "read failed on", path));
            break;
        }
        if ((rc = hip_check(ctx, cur.copy((char*)ctx->kvc_buf[b], (size_t)got, false, ctx->stream), fn))) break;
        if ((rc = hip_check(ctx, hipEventRecord(ctx->kvc_ev[b], ctx->stream), fn))) break;
        pending[b] = true;
        left -= (size_t)got;
        short_file = (size_t)got < want;
    }
    const int sync_rc = hip_check(ctx, hipStreamSynchronize(ctx->stream), fn);
    close(fd);
    if (rc || sync_rc) return 0;
    if (short_file) return set_err(ctx, PQA_ERR_IO, std::string(fn) + ": " + path + " ends early"), 0;
    return n_pos;
}
