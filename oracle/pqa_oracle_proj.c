/*
 * CPU oracle for the Q/K/V projections: TensorOps::matmul_bias
 * (cpp/tensor.hpp:110-143) over GGUF-quantized rows, with the dequantizers
 * and dot products of cpp/quant.hpp:176-358 and vec_add (cpp/tensor.hpp:410-420).
 *
 * TEST INFRASTRUCTURE ONLY (see pqa_oracle.h). Built with -ffp-contract=off:
 * every product and sum rounds separately, in the reference's order on x86
 * (the SSE2 path of vec_dot_f32_f32).
 */
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "pqa_oracle.h"

static int block_elems(int t) {
    switch (t) {
        case PQO_GGUF_F32: case PQO_GGUF_F16: return 1;
        case PQO_GGUF_Q4_0: case PQO_GGUF_Q8_0: return 32;
        case PQO_GGUF_Q4_K: case PQO_GGUF_Q6_K: return 256;
        default: return 0;
    }
}

static int block_bytes(int t) {
    switch (t) {
        case PQO_GGUF_F32: return 4;
        case PQO_GGUF_F16: return 2;
        case PQO_GGUF_Q4_0: return 18;
        case PQO_GGUF_Q8_0: return 34;
        case PQO_GGUF_Q4_K: return 144;
        case PQO_GGUF_Q6_K: return 210;
        default: return 0;
    }
}

/* gguf_type_row_size (cpp/quant.hpp:168-174); 0 for an unsupported type or a
 * row that is not a whole number of blocks. */
size_t pqo_row_bytes(int type, int n) {
    const int be = block_elems(type);
    if (!be || n <= 0 || n % be) return 0;
    return (size_t)(n / be) * (size_t)block_bytes(type);
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* get_scale_min_k4 (cpp/quant.hpp:210-218): 6-bit scale and min of sub-block j. */
static void scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* dequantize_row (cpp/quant.hpp:176-281, dispatch :283-294). */
int pqo_dequant_row(int type, const void* src, float* y, int n) {
    const uint8_t* b = (const uint8_t*)src;
    if (!pqo_row_bytes(type, n)) return -1;
    switch (type) {
        case PQO_GGUF_F32:
            memcpy(y, src, (size_t)n * 4);
            return 0;
        case PQO_GGUF_F16:
            for (int i = 0; i < n; i++) y[i] = pqo_fp16_to_fp32(rd16(b + 2 * i));
            return 0;
        case PQO_GGUF_Q8_0:  /* {fp16 d, int8 qs[32]} */
            for (int i = 0; i < n / 32; i++, b += 34) {
                const float d = pqo_fp16_to_fp32(rd16(b));
                for (int j = 0; j < 32; j++) y[32 * i + j] = d * (float)(int8_t)b[2 + j];
            }
            return 0;
        case PQO_GGUF_Q4_0:  /* {fp16 d, uint8 qs[16]}: low nibbles are elements 0..15 */
            for (int i = 0; i < n / 32; i++, b += 18) {
                const float d = pqo_fp16_to_fp32(rd16(b));
                for (int j = 0; j < 32; j++) {
                    const uint8_t nib = j < 16 ? (b[2 + j] & 0xF) : (b[2 + j - 16] >> 4);
                    y[32 * i + j] = d * ((float)nib - 8.0f);
                }
            }
            return 0;
        case PQO_GGUF_Q4_K:  /* {fp16 d, fp16 dmin, uint8 scales[12], uint8 qs[128]} */
            for (int i = 0; i < n / 256; i++, b += 144) {
                const float d = pqo_fp16_to_fp32(rd16(b));
                const float dmin = pqo_fp16_to_fp32(rd16(b + 2));
                const uint8_t* sc12 = b + 4;
                const uint8_t* q = b + 16;
                float* o = y + 256 * i;
                for (int j = 0; j < 4; j++, o += 64, q += 32) {
                    uint8_t sc, mn;
                    scale_min_k4(2 * j, sc12, &sc, &mn);
                    const float d1 = d * (float)sc, m1 = dmin * (float)mn;
                    scale_min_k4(2 * j + 1, sc12, &sc, &mn);
                    const float d2 = d * (float)sc, m2 = dmin * (float)mn;
                    for (int l = 0; l < 32; l++) o[l] = d1 * (float)(q[l] & 0xF) - m1;
                    for (int l = 0; l < 32; l++) o[l + 32] = d2 * (float)(q[l] >> 4) - m2;
                }
            }
            return 0;
        case PQO_GGUF_Q6_K:  /* {uint8 ql[128], uint8 qh[64], int8 scales[16], fp16 d} */
            for (int i = 0; i < n / 256; i++, b += 210) {
                const float d = pqo_fp16_to_fp32(rd16(b + 208));
                const uint8_t* ql = b;
                const uint8_t* qh = b + 128;
                const int8_t* sc = (const int8_t*)(b + 192);
                float* o = y + 256 * i;
                for (int half = 0; half < 2; half++, o += 128, ql += 64, qh += 32) {
                    const int is = 8 * half;
                    for (int l = 0; l < 32; l++) {
                        const int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                        const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                        const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                        const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                        const int il = is + l / 16;
                        o[l] = d * (float)sc[il + 0] * (float)q1;
                        o[l + 32] = d * (float)sc[il + 2] * (float)q2;
                        o[l + 64] = d * (float)sc[il + 4] * (float)q3;
                        o[l + 96] = d * (float)sc[il + 6] * (float)q4;
                    }
                }
            }
            return 0;
        default:
            return -1;
    }
}

/* vec_dot_f32_f32, SSE2 path (cpp/quant.hpp:297-319): two 4-lane
 * accumulators over groups of 8, hsum (:288-294) = (t0 + t2) + (t1 + t3) of
 * t = acc0 + acc1, then the tail in order. */
static float dot_f32(const float* w, const float* x, int n) {
    float a0[4] = {0.0f, 0.0f, 0.0f, 0.0f}, a1[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int i = 0;
    for (; i + 7 < n; i += 8)
        for (int l = 0; l < 4; l++) {
            a0[l] = a0[l] + w[i + l] * x[i + l];
            a1[l] = a1[l] + w[i + 4 + l] * x[i + 4 + l];
        }
    float t[4];
    for (int l = 0; l < 4; l++) t[l] = a0[l] + a1[l];
    float s = (t[0] + t[2]) + (t[1] + t[3]);
    for (; i < n; i++) s += w[i] * x[i];
    return s;
}

/* vec_dot (cpp/quant.hpp:342-356): F32 direct, Q8_0 per-block sums
 * (:321-340), the rest dequantized and then vec_dot_f32_f32. */
float pqo_vec_dot(int type, const void* row, const float* x, int n) {
    if (type == PQO_GGUF_F32) return dot_f32((const float*)row, x, n);
    if (type == PQO_GGUF_Q8_0) {
        const uint8_t* b = (const uint8_t*)row;
        float sumf = 0.0f;
        for (int i = 0; i < n / 32; i++, b += 34) {
            const float d = pqo_fp16_to_fp32(rd16(b));
            float sum = 0.0f;
            for (int j = 0; j < 32; j++) sum += (float)(int8_t)b[2 + j] * x[32 * i + j];
            sumf += d * sum;
        }
        return sumf;
    }
    float buf[16384];
    if (n > 16384 || pqo_dequant_row(type, row, buf, n)) return 0.0f;
    return dot_f32(buf, x, n);
}

/* matmul_bias (cpp/tensor.hpp:134-143): out[i] = vec_dot(row i) then, with a
 * bias, out[i] + bias[i]. Returns -1 for an unsupported type or shape. */
int pqo_matmul_bias(float* out, const float* x, const void* w, int wtype, const void* b, int btype, int n,
                    int d) {
    const size_t rb = pqo_row_bytes(wtype, n);
    if (!rb || n > 16384) return -1;
    for (int i = 0; i < d; i++) out[i] = pqo_vec_dot(wtype, (const uint8_t*)w + (size_t)i * rb, x, n);
    if (btype != PQO_GGUF_NONE && b) {
        float bias[16384];
        if (d > 16384 || pqo_dequant_row(btype, b, bias, d)) return -1;
        for (int i = 0; i < d; i++) out[i] = out[i] + bias[i];
    }
    return 0;
}

/* matmul_bias for n_tok inputs x [n_tok][n] -> out [n_tok][d]: per token the
 * same arithmetic as pqo_matmul_bias (forward_batch calls matmul_bias per
 * token, cpp/model.hpp:503-546); a row is dequantized once for all tokens
 * (dequantize_row is exact and does not depend on x), and rows are split over
 * n_threads. */
typedef struct {
    float* out;
    const float* x;
    const uint8_t* w;
    const float* bias;
    size_t rb;
    int n_tok, wtype, n, d, r0, r1;
} mm_job;

static void* mm_worker(void* arg) {
    const mm_job* j = (const mm_job*)arg;
    float* buf = (float*)malloc((size_t)j->n * sizeof(float));
    for (int r = j->r0; r < j->r1 && buf; r++) {
        const uint8_t* row = j->w + (size_t)r * j->rb;
        const int direct = j->wtype == PQO_GGUF_F32 || j->wtype == PQO_GGUF_Q8_0;
        if (!direct) pqo_dequant_row(j->wtype, row, buf, j->n);
        for (int t = 0; t < j->n_tok; t++) {
            const float* xt = j->x + (size_t)t * j->n;
            float v = direct ? pqo_vec_dot(j->wtype, row, xt, j->n) : dot_f32(buf, xt, j->n);
            if (j->bias) v = v + j->bias[r];
            j->out[(size_t)t * j->d + r] = v;
        }
    }
    free(buf);
    return NULL;
}

int pqo_matmul_bias_tokens(float* out, const float* x, int n_tok, const void* w, int wtype, const void* b, int btype,
                           int n, int d, int n_threads) {
    const size_t rb = pqo_row_bytes(wtype, n);
    if (!rb || n > 16384 || n_tok <= 0 || d <= 0) return -1;
    float* bias = NULL;
    if (btype != PQO_GGUF_NONE && b) {
        bias = (float*)malloc((size_t)d * sizeof(float));
        if (!bias || pqo_dequant_row(btype, b, bias, d)) {
            free(bias);
            return -1;
        }
    }
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    if (n_threads > d) n_threads = d;
    mm_job jobs[64];
    pthread_t th[64];
    const int per = (d + n_threads - 1) / n_threads;
    for (int t = 0; t < n_threads; t++) {
        const int r0 = t * per, r1 = r0 + per < d ? r0 + per : d;
        jobs[t] = (mm_job){out, x, (const uint8_t*)w, bias, rb, n_tok, wtype, n, d, r0, r1};
        if (n_threads > 1) pthread_create(&th[t], NULL, mm_worker, &jobs[t]);
    }
    if (n_threads == 1) mm_worker(&jobs[0]);
    else
        for (int t = 0; t < n_threads; t++) pthread_join(th[t], NULL);
    free(bias);
    return 0;
}
