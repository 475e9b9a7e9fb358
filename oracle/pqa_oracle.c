/*
 * CPU oracle for the picolm_qwen attention path -- TEST INFRASTRUCTURE ONLY.
 * Restates rain1201/picolm_qwen cpp/model.hpp:326-418 (decode block),
 * :493-593 (prefill token loop), cpp/tensor.hpp:146-176 (rmsnorm),
 * :201-369 (RoPE), cpp/quant.hpp:73-135 (fp16), :296-302 (hsum_sse),
 * cpp/model.hpp:1008-1017 (RoPE table). Must be compiled with
 * -ffp-contract=off; see pqa_oracle.h for the pins.
 */
#include "pqa_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* cpp/quant.hpp:73-100: exact widening, fp16 subnormals renormalised. */
float pqo_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0x1Fu) return u2f(sign | 0x7F800000u | (m << 13));
    if (e != 0) return u2f(sign | ((e + 112u) << 23) | (m << 13));
    if (m == 0) return u2f(sign);
    /* subnormal: shift the leading one up to bit 10 */
    int ex = 1;
    while (!(m & 0x400u)) { m <<= 1; ex--; }
    return u2f(sign | ((uint32_t)(ex + 112) << 23) | ((m & 0x3FFu) << 13));
}

/*
 * cpp/quant.hpp:102-135. Rounding is "add half an fp16 ulp to the magnitude
 * and truncate", i.e. nearest with ties away from zero. fp32 zero/subnormal
 * inputs give a signed zero; inf stays inf; NaN becomes sign|0x7E00; a
 * magnitude that rounds past 65504 becomes inf.
 */
uint16_t pqo_fp32_to_fp16(float f) {
    uint32_t bits = f2u(f);
    uint32_t sign = (bits >> 16) & 0x8000u;
    uint32_t be = (bits >> 23) & 0xFFu;
    uint32_t mant = bits & 0x7FFFFFu;
    int e = (int)be - 112; /* fp16 biased exponent */
    if (be == 0) return (uint16_t)sign;
    if (be == 0xFFu) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t m = (mant | 0x800000u) + (1u << (shift - 1));
        return (uint16_t)(sign | (m >> shift));
    }
    mant += 0x1000u;
    if (mant & 0x800000u) {
        mant = 0;
        e++;
        if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | (mant >> 13));
}

void pqo_fp16_to_fp32_array(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = pqo_fp16_to_fp32(src[i]);
}

void pqo_fp32_to_fp16_array(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = pqo_fp32_to_fp16(src[i]);
}

typedef struct { uint32_t first; size_t n; uint16_t* dst; } bits_job;

static void* bits_worker(void* arg) {
    bits_job* j = (bits_job*)arg;
    for (size_t i = 0; i < j->n; i++) j->dst[i] = pqo_fp32_to_fp16(u2f(j->first + (uint32_t)i));
    return NULL;
}

void pqo_fp32_bits_to_fp16_range(uint32_t first, size_t n, uint16_t* dst, int n_threads) {
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    pthread_t th[64];
    bits_job jobs[64];
    size_t per = (n + (size_t)n_threads - 1) / (size_t)n_threads;
    int started = 0;
    for (int t = 0; t < n_threads; t++) {
        size_t a = (size_t)t * per;
        if (a >= n) break;
        size_t b = a + per < n ? a + per : n;
        jobs[t].first = first + (uint32_t)a;
        jobs[t].n = b - a;
        jobs[t].dst = dst + a;
        if (n_threads == 1) { bits_worker(&jobs[t]); continue; }
        pthread_create(&th[t], NULL, bits_worker, &jobs[t]);
        started = t + 1;
    }
    for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
}

/*
 * cpp/tensor.hpp:146-176 on the SSE2 path (always taken on x86-64):
 * four lane accumulators (lane j sums x[i]^2 for i = j mod 4 while i+3 < n),
 * horizontal sum (l0+l2)+(l1+l3) (cpp/quant.hpp:296-302), scalar tail,
 * s = 1/sqrt(ss/n + 1e-6), out = (x*s)*w.
 */
void pqo_rmsnorm(float* out, const float* x, const float* w, int n) {
    float l0 = 0.0f, l1 = 0.0f, l2 = 0.0f, l3 = 0.0f;
    int i = 0;
    for (; i + 3 < n; i += 4) {
        l0 = l0 + x[i] * x[i];
        l1 = l1 + x[i + 1] * x[i + 1];
        l2 = l2 + x[i + 2] * x[i + 2];
        l3 = l3 + x[i + 3] * x[i + 3];
    }
    float ss = (l0 + l2) + (l1 + l3);
    for (; i < n; i++) ss += x[i] * x[i];
    ss = 1.0f / sqrtf(ss / (float)n + 1e-6f);
    for (int j = 0; j < n; j++) out[j] = (x[j] * ss) * w[j];
}

/* One head of rope_qwen (cpp/tensor.hpp:201-283): pairs (i, i+half). */
static void rope_neox_head(float* x, int hd, const float* c, const float* s) {
    int half = hd / 2;
    for (int i = 0; i < half; i++) {
        float a = x[i], b = x[i + half];
        x[i] = a * c[i] - b * s[i];
        x[i + half] = a * s[i] + b * c[i];
    }
}

/*
 * One head of rope_llama on its SSE2 path (cpp/tensor.hpp:290-346): blocks
 * of 8 elements; element 8b+j pairs with 8b+4+j at angle 4b+j, j = 0..3.
 * Pairs left over when half is not a multiple of 4 use the interleaved
 * scalar tail (:316-323).
 */
static void rope_block8_head(float* x, int hd, const float* c, const float* s) {
    int half = hd / 2;
    int i = 0;
    for (; i + 3 < half; i += 4) {
        float e[4], o[4];
        for (int j = 0; j < 4; j++) { e[j] = x[2 * i + j]; o[j] = x[2 * i + 4 + j]; }
        for (int j = 0; j < 4; j++) {
            x[2 * i + j] = e[j] * c[i + j] - o[j] * s[i + j];
            x[2 * i + 4 + j] = e[j] * s[i + j] + o[j] * c[i + j];
        }
    }
    for (; i < half; i++) {
        float a = x[2 * i], b = x[2 * i + 1];
        x[2 * i] = a * c[i] - b * s[i];
        x[2 * i + 1] = a * s[i] + b * c[i];
    }
}

/* rope_llama scalar branch (cpp/tensor.hpp:347-368): pairs (2i, 2i+1). */
static void rope_interleaved_head(float* x, int hd, const float* c, const float* s) {
    int half = hd / 2;
    for (int i = 0; i < half; i++) {
        float a = x[2 * i], b = x[2 * i + 1];
        x[2 * i] = a * c[i] - b * s[i];
        x[2 * i + 1] = a * s[i] + b * c[i];
    }
}

static void rope_head(int style, float* x, int hd, const float* c, const float* s) {
    if (style == PQO_ROPE_NEOX_HALF) rope_neox_head(x, hd, c, s);
    else if (style == PQO_ROPE_LLAMA_X86_BLOCK8) rope_block8_head(x, hd, c, s);
    else rope_interleaved_head(x, hd, c, s);
}

void pqo_rope(int style, float* q, float* k, int hd, int n_heads, int n_kv_heads,
              const float* cos_pos, const float* sin_pos) {
    for (int h = 0; h < n_heads; h++) rope_head(style, q + (size_t)h * hd, hd, cos_pos, sin_pos);
    for (int h = 0; h < n_kv_heads; h++) rope_head(style, k + (size_t)h * hd, hd, cos_pos, sin_pos);
}

/* cpp/model.hpp:1008-1017: theta = pos / base^(2i/hd) in float (powf), cosf, sinf. */
void pqo_rope_rows(float base, int hd, int pos0, int n, float* cos_rows, float* sin_rows) {
    int half = hd / 2;
    for (int r = 0; r < n; r++) {
        int pos = pos0 + r;
        for (int i = 0; i < half; i++) {
            float theta = (float)pos / powf(base, (float)(2 * i) / (float)hd);
            cos_rows[(size_t)r * half + i] = cosf(theta);
            sin_rows[(size_t)r * half + i] = sinf(theta);
        }
    }
}

void pqo_rope_table(float base, int hd, int max_seq_len, float* cos_tab, float* sin_tab) {
    pqo_rope_rows(base, hd, 0, max_seq_len, cos_tab, sin_tab);
}

/*
 * The per-head attention loop of cpp/model.hpp:378-418: running max starts
 * at -1e30, a new maximum rescales sum and acc by exp(old-new) and adds the
 * row with weight 1, otherwise the row is added with weight exp(s-max).
 * Score is a sequential fp32 dot product divided by sqrt(hd).
 */
static void attend_head(const pqo_shape* s, int pos, int h, const float* qh, const uint16_t* kc,
                        const uint16_t* vc, float* out_h, float* acc) {
    int hd = s->head_dim;
    int kv_dim = s->n_kv_heads * hd;
    int kv_mul = s->n_heads / s->n_kv_heads;
    int kv_h = h / kv_mul;
    float max_score = -1e30f;
    float sum_exp = 0.0f;
    for (int d = 0; d < hd; d++) acc[d] = 0.0f;
    for (int t = 0; t <= pos; t++) {
        const uint16_t* kt = kc + (size_t)t * kv_dim + (size_t)kv_h * hd;
        const uint16_t* vt = vc + (size_t)t * kv_dim + (size_t)kv_h * hd;
        float score = 0.0f;
        for (int d = 0; d < hd; d++) score += qh[d] * pqo_fp16_to_fp32(kt[d]);
        score /= sqrtf((float)hd);
        if (score > max_score) {
            float corr = expf(max_score - score);
            sum_exp *= corr;
            for (int d = 0; d < hd; d++) acc[d] *= corr;
            sum_exp += 1.0f;
            for (int d = 0; d < hd; d++) acc[d] += pqo_fp16_to_fp32(vt[d]);
            max_score = score;
        } else {
            float w = expf(score - max_score);
            sum_exp += w;
            for (int d = 0; d < hd; d++) acc[d] += w * pqo_fp16_to_fp32(vt[d]);
        }
    }
    for (int d = 0; d < hd; d++) out_h[d] = acc[d] / sum_exp;
}

typedef struct {
    const pqo_shape* s;
    const int* pos_of;      /* per work item: position */
    const float* const* q_of;
    float* const* out_of;
    const int* head_of;
    const uint16_t* kc;
    const uint16_t* vc;
    int n_items;
    int t, nt;
} attend_job;

static void* attend_worker(void* arg) {
    attend_job* j = (attend_job*)arg;
    float* acc = (float*)malloc(sizeof(float) * (size_t)j->s->head_dim);
    for (int it = j->t; it < j->n_items; it += j->nt)
        attend_head(j->s, j->pos_of[it], j->head_of[it], j->q_of[it], j->kc, j->vc, j->out_of[it], acc);
    free(acc);
    return NULL;
}

/* Runs n_items independent (pos, head) attention loops over n_threads. */
static void attend_items(const pqo_shape* s, int n_items, const int* pos_of, const int* head_of,
                         const float* const* q_of, float* const* out_of, const uint16_t* kc,
                         const uint16_t* vc, int n_threads) {
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    if (n_threads > n_items) n_threads = n_items > 0 ? n_items : 1;
    attend_job jobs[256];
    pthread_t th[256];
    for (int t = 0; t < n_threads; t++) {
        jobs[t] = (attend_job){s, pos_of, q_of, out_of, head_of, kc, vc, n_items, t, n_threads};
    }
    if (n_threads == 1) { attend_worker(&jobs[0]); return; }
    for (int t = 0; t < n_threads; t++) pthread_create(&th[t], NULL, attend_worker, &jobs[t]);
    for (int t = 0; t < n_threads; t++) pthread_join(th[t], NULL);
}

void pqo_attend(const pqo_shape* s, int pos, const float* q, const uint16_t* kc,
                const uint16_t* vc, float* out, int n_threads) {
    int nh = s->n_heads, hd = s->head_dim;
    int* pos_of = (int*)malloc(sizeof(int) * (size_t)nh);
    int* head_of = (int*)malloc(sizeof(int) * (size_t)nh);
    const float** q_of = (const float**)malloc(sizeof(float*) * (size_t)nh);
    float** out_of = (float**)malloc(sizeof(float*) * (size_t)nh);
    for (int h = 0; h < nh; h++) {
        pos_of[h] = pos;
        head_of[h] = h;
        q_of[h] = q + (size_t)h * hd;
        out_of[h] = out + (size_t)h * hd;
    }
    attend_items(s, nh, pos_of, head_of, (const float* const*)q_of, out_of, kc, vc, n_threads);
    free(pos_of); free(head_of); free(q_of); free(out_of);
}

/* cpp/model.hpp:326-373: Q norm, K norm, RoPE(q, k), K append, V append. */
void pqo_append(const pqo_shape* s, int pos, float* q, const float* k, const float* v,
                const float* q_norm_w, const float* k_norm_w,
                const float* cos_pos, const float* sin_pos, uint16_t* kc, uint16_t* vc) {
    int hd = s->head_dim, nh = s->n_heads, nkv = s->n_kv_heads;
    int kv_dim = nkv * hd;
    float* kb = (float*)malloc(sizeof(float) * (size_t)kv_dim);
    memcpy(kb, k, sizeof(float) * (size_t)kv_dim);
    if (q_norm_w)
        for (int h = 0; h < nh; h++) pqo_rmsnorm(q + (size_t)h * hd, q + (size_t)h * hd, q_norm_w, hd);
    if (k_norm_w)
        for (int h = 0; h < nkv; h++) pqo_rmsnorm(kb + (size_t)h * hd, kb + (size_t)h * hd, k_norm_w, hd);
    pqo_rope(s->rope_style, q, kb, hd, nh, nkv, cos_pos, sin_pos);
    uint16_t* krow = kc + (size_t)pos * kv_dim;
    uint16_t* vrow = vc + (size_t)pos * kv_dim;
    for (int d = 0; d < kv_dim; d++) krow[d] = pqo_fp32_to_fp16(kb[d]);
    for (int d = 0; d < kv_dim; d++) vrow[d] = pqo_fp32_to_fp16(v[d]);
    free(kb);
}

void pqo_attn_step(const pqo_shape* s, int pos, const float* q, const float* k, const float* v,
                   const float* q_norm_w, const float* k_norm_w,
                   const float* cos_pos, const float* sin_pos,
                   uint16_t* kc, uint16_t* vc, float* out, int n_threads) {
    size_t q_dim = (size_t)s->n_heads * s->head_dim;
    float* qb = (float*)malloc(sizeof(float) * q_dim);
    memcpy(qb, q, sizeof(float) * q_dim);
    pqo_append(s, pos, qb, k, v, q_norm_w, k_norm_w, cos_pos, sin_pos, kc, vc);
    pqo_attend(s, pos, qb, kc, vc, out, n_threads);
    free(qb);
}

void pqo_prefill(const pqo_shape* s, int start, int n_tok, const float* q, const float* k,
                 const float* v, const float* q_norm_w, const float* k_norm_w,
                 const float* cos_tab, const float* sin_tab, uint16_t* kc, uint16_t* vc,
                 float* out, int serial, int n_threads) {
    int hd = s->head_dim, nh = s->n_heads;
    size_t q_dim = (size_t)nh * hd, kv_dim = (size_t)s->n_kv_heads * hd, half = (size_t)hd / 2;
    if (serial) {
        for (int i = 0; i < n_tok; i++) {
            int pos = start + i;
            pqo_attn_step(s, pos, q + i * q_dim, k + i * kv_dim, v + i * kv_dim, q_norm_w, k_norm_w,
                          cos_tab + (size_t)pos * half, sin_tab + (size_t)pos * half, kc, vc,
                          out + i * q_dim, n_threads);
        }
        return;
    }
    float* qb = (float*)malloc(sizeof(float) * q_dim * (size_t)n_tok);
    memcpy(qb, q, sizeof(float) * q_dim * (size_t)n_tok);
    for (int i = 0; i < n_tok; i++) {
        int pos = start + i;
        pqo_append(s, pos, qb + i * q_dim, k + i * kv_dim, v + i * kv_dim, q_norm_w, k_norm_w,
                   cos_tab + (size_t)pos * half, sin_tab + (size_t)pos * half, kc, vc);
    }
    size_t n_items = (size_t)n_tok * nh;
    int* pos_of = (int*)malloc(sizeof(int) * n_items);
    int* head_of = (int*)malloc(sizeof(int) * n_items);
    const float** q_of = (const float**)malloc(sizeof(float*) * n_items);
    float** out_of = (float**)malloc(sizeof(float*) * n_items);
    /* longest rows first so threads finish together */
    size_t it = 0;
    for (int i = n_tok - 1; i >= 0; i--)
        for (int h = 0; h < nh; h++, it++) {
            pos_of[it] = start + i;
            head_of[it] = h;
            q_of[it] = qb + i * q_dim + (size_t)h * hd;
            out_of[it] = out + i * q_dim + (size_t)h * hd;
        }
    attend_items(s, (int)n_items, pos_of, head_of, (const float* const*)q_of, out_of, kc, vc, n_threads);
    free(pos_of); free(head_of); free(q_of); free(out_of); free(qb);
}

/* Plain softmax(q.k/sqrt(hd)) . V in double: two-pass, no online rescaling. */
void pqo_attend_f64(const pqo_shape* s, int pos, const float* q, const uint16_t* kc,
                    const uint16_t* vc, double* out) {
    int hd = s->head_dim, nh = s->n_heads;
    int kv_dim = s->n_kv_heads * hd, g = nh / s->n_kv_heads;
    double* sc = (double*)malloc(sizeof(double) * (size_t)(pos + 1));
    for (int h = 0; h < nh; h++) {
        int kvh = h / g;
        double mx = -INFINITY;
        for (int t = 0; t <= pos; t++) {
            double acc = 0.0;
            for (int d = 0; d < hd; d++)
                acc += (double)q[(size_t)h * hd + d] *
                       (double)pqo_fp16_to_fp32(kc[(size_t)t * kv_dim + (size_t)kvh * hd + d]);
            sc[t] = acc / sqrt((double)hd);
            if (sc[t] > mx) mx = sc[t];
        }
        double den = 0.0;
        for (int t = 0; t <= pos; t++) { sc[t] = exp(sc[t] - mx); den += sc[t]; }
        for (int d = 0; d < hd; d++) {
            double num = 0.0;
            for (int t = 0; t <= pos; t++)
                num += sc[t] * (double)pqo_fp16_to_fp32(vc[(size_t)t * kv_dim + (size_t)kvh * hd + d]);
            out[(size_t)h * hd + d] = num / den;
        }
    }
    free(sc);
}

/* ---- synthetic inputs ---- */
uint64_t pqo_splitmix64(uint64_t key, uint64_t i) {
    uint64_t z = key + (i + 1u) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t pqo_stream_key(uint64_t seed, uint32_t kind, uint32_t layer) {
    return pqo_splitmix64(seed, ((uint64_t)kind << 32) | (uint64_t)layer);
}

static inline double u01(uint64_t r) { return ((double)(r >> 11) + 0.5) * 0x1.0p-53; }

float pqo_normal(uint64_t key, uint64_t i) {
    double u1 = u01(pqo_splitmix64(key, 2 * i));
    double u2 = u01(pqo_splitmix64(key, 2 * i + 1));
    return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

void pqo_fill_normal(uint64_t key, uint64_t first, size_t n, float mean, float stddev, float* out) {
    for (size_t i = 0; i < n; i++) {
        float z = pqo_normal(key, first + i);
        out[i] = (mean == 0.0f && stddev == 1.0f) ? z : mean + stddev * z;
    }
}

int pqo_is_outlier(uint64_t seed, uint32_t layer, uint64_t pos, float outlier_prob) {
    if (outlier_prob <= 0.0f) return 0;
    uint64_t key = pqo_stream_key(seed, PQO_KIND_OUTLIER, layer);
    return u01(pqo_splitmix64(key, pos)) < (double)outlier_prob;
}

typedef struct {
    uint64_t seed; uint32_t layer; int kv_dim, pos0, n; float prob;
    uint16_t* k; uint16_t* v; int t, nt;
} synth_job;

static void* synth_worker(void* arg) {
    synth_job* j = (synth_job*)arg;
    uint64_t kk = pqo_stream_key(j->seed, PQO_KIND_KHIST, j->layer);
    uint64_t vk = pqo_stream_key(j->seed, PQO_KIND_VHIST, j->layer);
    for (int r = j->t; r < j->n; r += j->nt) {
        uint64_t pos = (uint64_t)(j->pos0 + r);
        float scale = pqo_is_outlier(j->seed, j->layer, pos, j->prob) ? 8.0f : 1.0f;
        for (int d = 0; d < j->kv_dim; d++) {
            uint64_t idx = pos * (uint64_t)j->kv_dim + (uint64_t)d;
            j->k[(size_t)r * j->kv_dim + d] = pqo_fp32_to_fp16(pqo_normal(kk, idx) * scale);
            j->v[(size_t)r * j->kv_dim + d] = pqo_fp32_to_fp16(pqo_normal(vk, idx) * scale);
        }
    }
    return NULL;
}

void pqo_synth_kv_rows(uint64_t seed, uint32_t layer, int kv_dim, int pos0, int n,
                       float outlier_prob, uint16_t* k_rows, uint16_t* v_rows, int n_threads) {
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    synth_job jobs[256];
    pthread_t th[256];
    for (int t = 0; t < n_threads; t++)
        jobs[t] = (synth_job){seed, layer, kv_dim, pos0, n, outlier_prob, k_rows, v_rows, t, n_threads};
    if (n_threads == 1) { synth_worker(&jobs[0]); return; }
    for (int t = 0; t < n_threads; t++) pthread_create(&th[t], NULL, synth_worker, &jobs[t]);
    for (int t = 0; t < n_threads; t++) pthread_join(th[t], NULL);
}
