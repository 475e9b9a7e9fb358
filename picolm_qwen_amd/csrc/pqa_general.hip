// Attention for the head sizes the MFMA kernels are not built for: any even
// head_dim up to 512 (cpp/model.hpp:172 sizes its accumulator for 512), for
// decode and prefill alike.
//
// Two launches (three with splits):
//   gen_prep_kernel  one wave per (token, head): the head's q or k through
//                    RMSNorm in the reference's lane order and RoPE of any of
//                    the three pairings (block8's interleaved tail included),
//                    K and V rounded to fp16 into the cache (bit-exact, like
//                    the MFMA path's prologues), q scaled by log2(e)/sqrt(hd)
//                    into a workspace;
//   gen_attn8_kernel one wave per (token, KV head chunk, key range): 64 keys
//                    per tile, one key per lane for the scores (each lane
//                    walks its key's row), online softmax per query head, then
//                    the tile's V rows in 16-byte chunks (head_dim a multiple
//                    of 8; gen_attn_kernel, with 4-byte loads, takes the rest);
//   gen_combine_kernel  merges the key ranges of a long decode.
// These are plain VALU kernels: they stream the cache and have no MFMA or
// LDS-tiled operand path, which is what the 64/128 kernels add.
#include <algorithm>

#include "pqa_device.h"
#include "pqa_internal.h"

namespace pqa {

constexpr int kGenMaxHd = 512;
constexpr int kMaxGenSplits = 256;  // the combine keeps one weight per key range in LDS
constexpr int kGenWaves = 4;
constexpr int kGenMaxG = 8;  // query heads per wave (a KV head's chunk)

// One q/k/v operand: column c of token t at p[t * ld + c]; with w_inv the
// value is the batched GEMM's scaled result, p * (w_inv[c] * x_inv[t]) + b[c].
struct GenSrc {
    const float* p;
    int ld;
    const float* w_inv;
    const float* x_inv;
    const uint8_t* b;
    int bt;
};

__device__ __forceinline__ float gen_load(const GenSrc& s, int t, int c) {
    float v = s.p[(size_t)t * s.ld + c];
    if (s.w_inv) {
        v = v * (s.w_inv[c] * s.x_inv[t]);
        if (s.b) v = v + (s.bt == GG_F32 ? ((const float*)s.b)[c] : f16_bits_to_f32(((const uint16_t*)s.b)[c]));
    }
    return v;
}

struct GenPrepArgs {
    GenSrc q, k, v;
    const float* qn;  // [hd] or null
    const float* kn;
    const float* cos_tab;  // [S][hd / 2]
    const float* sin_tab;
    uint16_t* kc;  // the layer's cache
    uint16_t* vc;
    float* qp;  // [n_tok][nh * hd]
    int start, n_tok, nh, nkv, hd, rope;
    float qscale;
};

// grid (ceil((nh + nkv) / 4), n_tok); wave -> one head of one token (query
// heads first, then KV heads, which also write their V row).
__global__ __launch_bounds__(64 * kGenWaves) void gen_prep_kernel(const GenPrepArgs a) {
    __shared__ float s_row[kGenWaves][kGenMaxHd];
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int t = blockIdx.y;
    const int head = blockIdx.x * kGenWaves + w;
    if (head >= a.nh + a.nkv) return;  // whole wave; the kernel has no workgroup barrier
    const bool isq = head < a.nh;
    const int h = isq ? head : head - a.nh;
    const int hd = a.hd, half = hd >> 1;
    const int pos = a.start + t;
    const int c0 = h * hd;
    float* r = s_row[w];
    const GenSrc& src = isq ? a.q : a.k;
    for (int e = lane; e < hd; e += 64) r[e] = gen_load(src, t, c0 + e);
    wave_sync();
    const float* nw = isq ? a.qn : a.kn;
    if (nw) {
        // every quad computes the scale in the reference's order (the same
        // LDS words for all quads, read as broadcasts)
        const float s = rms_scale_ref_quad(r, hd, lane & 3);
        wave_sync();
        for (int e = lane; e < hd; e += 64) r[e] = rms_apply(r[e], s, nw[e]);
        wave_sync();
    }
    const float* cr = a.cos_tab + (size_t)pos * half;
    const float* sr = a.sin_tab + (size_t)pos * half;
    const size_t kv_dim = (size_t)a.nkv * hd;
    for (int p = lane; p < half; p += 64) {
        int e0, e1;
        rope_pair(a.rope, p, hd, e0, e1);
        float x0 = r[e0], x1 = r[e1];
        rope_rotate(x0, x1, cr[p], sr[p]);
        if (isq) {
            float* qo = a.qp + (size_t)t * a.nh * hd + c0;
            qo[e0] = x0 * a.qscale;
            qo[e1] = x1 * a.qscale;
        } else {
            uint16_t* ko = a.kc + (size_t)pos * kv_dim + c0;
            ko[e0] = f32_to_f16_ref(x0);
            ko[e1] = f32_to_f16_ref(x1);
        }
    }
    if (!isq) {
        uint16_t* vo = a.vc + (size_t)pos * kv_dim + c0;
        for (int e = lane; e < hd; e += 64) vo[e] = f32_to_f16_ref(gen_load(a.v, t, c0 + e));
    }
}

struct GenAttnArgs {
    const float* qp;  // [n_tok][nh * hd], scaled by log2(e) / sqrt(hd)
    const uint16_t* kc;
    const uint16_t* vc;
    float* out;       // [n_tok][nh * hd] when nsplit == 1
    float* part_acc;  // [ny][nsplit][G][hd] when nsplit > 1 (one token)
    float* part_ml;   // [ny][nsplit][G][2]
    int start, n_tok, nh, hd, kv_dim, g, nchunk, G, ny, rps, nsplit;
};

// Keys of a tile (head_dim not a multiple of 8): lane j takes key k0 + j and
// walks its K row in fp16 pairs.
template <int QW>
__device__ __forceinline__ void gen_scores2(const uint16_t* krow, const float (*q)[QW], int hd, int Gc,
                                            float (&sc)[kGenMaxG]) {
#pragma unroll
    for (int h = 0; h < kGenMaxG; h++) sc[h] = 0.0f;
    const uint32_t* kr = (const uint32_t*)krow;
#pragma unroll 4
    for (int d2 = 0; d2 < hd / 2; d2++) {
        const uint32_t u = kr[d2];
        const float k0 = f16_bits_to_f32((uint16_t)(u & 0xFFFFu)), k1 = f16_bits_to_f32((uint16_t)(u >> 16));
#pragma unroll
        for (int h = 0; h < kGenMaxG; h++) {
            if (h < Gc) {
                const float2 qq = *(const float2*)&q[h][2 * d2];
                sc[h] = fmaf(qq.y, k1, fmaf(qq.x, k0, sc[h]));
            }
        }
    }
}

// Head sizes that are not a multiple of 8 (4-byte loads). NS: fp16 pairs per
// lane in the PV product (hd / 2 <= 64 NS); the q rows in LDS are 128 NS
// floats wide (24 KB per workgroup for NS = 1).
template <int NS>
__global__ __launch_bounds__(64 * kGenWaves) void gen_attn_kernel(const GenAttnArgs a) {
    constexpr int QW = 128 * NS;
    __shared__ __attribute__((aligned(16))) float s_q[kGenWaves][kGenMaxG][QW];
    __shared__ float s_p[kGenWaves][kGenMaxG][64];
    constexpr float NEG_INF = -__builtin_huge_valf();
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int item = blockIdx.x * kGenWaves + w;
    if (item >= a.ny * a.n_tok * a.nsplit) return;  // whole wave; no workgroup barrier below
    const int split = item % a.nsplit;
    const int rest = item / a.nsplit;
    const int t = rest % a.n_tok;
    const int y = rest / a.n_tok;
    const int kvh = y / a.nchunk, hc = y - kvh * a.nchunk;
    const int Gc = min(a.G, a.g - hc * a.G);
    const int h0 = kvh * a.g + hc * a.G;
    const int hd = a.hd, hd2 = hd >> 1;
    const int pos = a.start + t;
    const int kbeg = split * a.rps;
    const int kend = min(kbeg + a.rps, pos + 1);

    float(*q)[QW] = s_q[w];
    for (int h = 0; h < Gc; h++)
        for (int e = lane; e < hd; e += 64) q[h][e] = a.qp[((size_t)t * a.nh + h0 + h) * hd + e];
    wave_sync();

    float m[kGenMaxG], l[kGenMaxG];
    float2 acc[kGenMaxG][NS];
#pragma unroll
    for (int h = 0; h < kGenMaxG; h++) {
        m[h] = NEG_INF;
        l[h] = 0.0f;
#pragma unroll
        for (int i = 0; i < NS; i++) acc[h][i] = float2{0.0f, 0.0f};
    }
    const uint16_t* kbase = a.kc + (size_t)kvh * hd;
    const uint16_t* vbase = a.vc + (size_t)kvh * hd;
    for (int k0 = kbeg; k0 < kend; k0 += 64) {
        const int key = k0 + lane;
        const bool valid = key < kend;
        float sc[kGenMaxG];
        gen_scores2<QW>(kbase + (size_t)(valid ? key : kbeg) * a.kv_dim, q, hd, Gc, sc);
#pragma unroll
        for (int h = 0; h < kGenMaxG; h++) {
            if (h < Gc) {
                const float s = valid ? sc[h] : NEG_INF;
                const float mn = fmaxf(m[h], group_max<64>(s));  // finite: the tile has a key
                const float alpha = fast_exp2(m[h] - mn);         // 0 on the first tile
                const float p = valid ? fast_exp2(s - mn) : 0.0f;
                l[h] = l[h] * alpha + group_sum<64>(p);
                m[h] = mn;
#pragma unroll
                for (int i = 0; i < NS; i++) acc[h][i] = float2{acc[h][i].x * alpha, acc[h][i].y * alpha};
                s_p[w][h][lane] = p;
            }
        }
        wave_sync();
        const int nk = min(64, kend - k0);
        for (int j = 0; j < nk; j++) {
            const uint32_t* vrow = (const uint32_t*)(vbase + (size_t)(k0 + j) * a.kv_dim);
            float2 vv[NS];
#pragma unroll
            for (int i = 0; i < NS; i++) {
                const int pi = lane + 64 * i;
                const uint32_t u = pi < hd2 ? vrow[pi] : 0u;
                vv[i] = float2{f16_bits_to_f32((uint16_t)(u & 0xFFFFu)), f16_bits_to_f32((uint16_t)(u >> 16))};
            }
#pragma unroll
            for (int h = 0; h < kGenMaxG; h++) {
                if (h < Gc) {
                    const float pj = s_p[w][h][j];
#pragma unroll
                    for (int i = 0; i < NS; i++)
                        acc[h][i] = float2{fmaf(pj, vv[i].x, acc[h][i].x), fmaf(pj, vv[i].y, acc[h][i].y)};
                }
            }
        }
        wave_sync();  // every lane has read this tile's P before the next tile writes it
    }

#pragma unroll
    for (int h = 0; h < kGenMaxG; h++) {
        if (h < Gc) {
            if (a.nsplit == 1) {
                const float inv = 1.0f / l[h];
                float* o = a.out + ((size_t)t * a.nh + h0 + h) * hd;
#pragma unroll
                for (int i = 0; i < NS; i++) {
                    const int pi = lane + 64 * i;
                    if (pi < hd2) *(float2*)(o + 2 * pi) = float2{acc[h][i].x * inv, acc[h][i].y * inv};
                }
            } else {
                const size_t slot = ((size_t)y * a.nsplit + split) * a.G + h;
                float* o = a.part_acc + slot * hd;
#pragma unroll
                for (int i = 0; i < NS; i++) {
                    const int pi = lane + 64 * i;
                    if (pi < hd2) *(float2*)(o + 2 * pi) = acc[h][i];
                }
                if (lane == 0) *(float2*)(a.part_ml + slot * 2) = float2{m[h], l[h]};
            }
        }
    }
}

// head_dim a multiple of 8: 16-byte loads in both phases, more of them in
// flight. Scores: lane = key, its row read 4 chunks at a time with the next 4
// requested before the current ones are summed. PV: lane = (sub, chunk), sub
// = lane / (hd / 8): each pass covers 64 / (hd / 8) keys, one 16-byte chunk of
// a V row per lane, 4 passes requested at once; the subs' partial sums meet
// in LDS after the last tile (in sub order).
template <int QW>
__global__ __launch_bounds__(64 * kGenWaves) void gen_attn8_kernel(const GenAttnArgs a) {
    __shared__ __attribute__((aligned(16))) float s_q[kGenWaves][kGenMaxG][QW];
    __shared__ float s_p[kGenWaves][kGenMaxG][64];
    constexpr float NEG_INF = -__builtin_huge_valf();
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int item = blockIdx.x * kGenWaves + w;
    if (item >= a.ny * a.n_tok * a.nsplit) return;  // whole wave; no workgroup barrier below
    const int split = item % a.nsplit;
    const int rest = item / a.nsplit;
    const int t = rest % a.n_tok;
    const int y = rest / a.n_tok;
    const int kvh = y / a.nchunk, hc = y - kvh * a.nchunk;
    const int Gc = min(a.G, a.g - hc * a.G);
    const int h0 = kvh * a.g + hc * a.G;
    const int hd = a.hd, nc = hd >> 3;
    const int pos = a.start + t;
    const int kbeg = split * a.rps;
    const int kend = min(kbeg + a.rps, pos + 1);
    const int kps = 64 / nc;                 // keys per PV pass
    const int sub = lane / nc, ch = lane - sub * nc;
    const bool pv_lane = sub < kps;
    const int passes = (64 + kps - 1) / kps;

    float(*q)[QW] = s_q[w];
    for (int h = 0; h < Gc; h++)
        for (int e = lane; e < hd; e += 64) q[h][e] = a.qp[((size_t)t * a.nh + h0 + h) * hd + e];
    wave_sync();

    float m[kGenMaxG], l[kGenMaxG], acc[kGenMaxG][8];
#pragma unroll
    for (int h = 0; h < kGenMaxG; h++) {
        m[h] = NEG_INF;
        l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[h][e] = 0.0f;
    }
    const uint16_t* kbase = a.kc + (size_t)kvh * hd;
    const uint16_t* vbase = a.vc + (size_t)kvh * hd;
    for (int k0 = kbeg; k0 < kend; k0 += 64) {
        const int key = k0 + lane;
        const bool valid = key < kend;
        const u32x4* kr = (const u32x4*)(kbase + (size_t)(valid ? key : kbeg) * a.kv_dim);
        float sc[kGenMaxG];
#pragma unroll
        for (int h = 0; h < kGenMaxG; h++) sc[h] = 0.0f;
        u32x4 nb[4];
#pragma unroll
        for (int i = 0; i < 4; i++) nb[i] = kr[min(i, nc - 1)];
        for (int c0 = 0; c0 < nc; c0 += 4) {
            u32x4 cb[4];
#pragma unroll
            for (int i = 0; i < 4; i++) cb[i] = nb[i];
            if (c0 + 4 < nc) {
#pragma unroll
                for (int i = 0; i < 4; i++) nb[i] = kr[min(c0 + 4 + i, nc - 1)];
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (c0 + i < nc) {
                    float kf[8];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        kf[2 * e] = f16_bits_to_f32((uint16_t)(cb[i][e] & 0xFFFFu));
                        kf[2 * e + 1] = f16_bits_to_f32((uint16_t)(cb[i][e] >> 16));
                    }
#pragma unroll
                    for (int h = 0; h < kGenMaxG; h++) {
                        if (h < Gc) {
                            const floatx4 q0 = *(const floatx4*)&q[h][8 * (c0 + i)];
                            const floatx4 q1 = *(const floatx4*)&q[h][8 * (c0 + i) + 4];
                            float s = sc[h];
#pragma unroll
                            for (int e = 0; e < 4; e++) s = fmaf(q0[e], kf[e], s);
#pragma unroll
                            for (int e = 0; e < 4; e++) s = fmaf(q1[e], kf[4 + e], s);
                            sc[h] = s;
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int h = 0; h < kGenMaxG; h++) {
            if (h < Gc) {
                const float sv = valid ? sc[h] : NEG_INF;
                const float mn = fmaxf(m[h], group_max<64>(sv));  // finite: the tile has a key
                const float alpha = fast_exp2(m[h] - mn);          // 0 on the first tile
                const float p = valid ? fast_exp2(sv - mn) : 0.0f;
                l[h] = l[h] * alpha + group_sum<64>(p);
                m[h] = mn;
#pragma unroll
                for (int e = 0; e < 8; e++) acc[h][e] *= alpha;
                s_p[w][h][lane] = p;
            }
        }
        wave_sync();
        if (pv_lane) {
            for (int p0 = 0; p0 < passes; p0 += 4) {
                u32x4 vb[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int j = min((p0 + u) * kps + sub, 63);
                    const int row = min(k0 + j, kend - 1);  // keys past kend have p = 0
                    vb[u] = ((const u32x4*)(vbase + (size_t)row * a.kv_dim))[ch];
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int j = (p0 + u) * kps + sub;
                    if (p0 + u < passes && j < 64) {
                        float vf[8];
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            vf[2 * e] = f16_bits_to_f32((uint16_t)(vb[u][e] & 0xFFFFu));
                            vf[2 * e + 1] = f16_bits_to_f32((uint16_t)(vb[u][e] >> 16));
                        }
#pragma unroll
                        for (int h = 0; h < kGenMaxG; h++) {
                            if (h < Gc) {
                                const float pj = s_p[w][h][j];
#pragma unroll
                                for (int e = 0; e < 8; e++) acc[h][e] = fmaf(pj, vf[e], acc[h][e]);
                            }
                        }
                    }
                }
            }
        }
        wave_sync();  // every lane has read this tile's P before the next tile writes it
    }

    // the subs' partial sums, in sub order, into the q rows (no longer read)
    for (int s2 = 0; s2 < kps; s2++) {
        if (sub == s2) {
#pragma unroll
            for (int h = 0; h < kGenMaxG; h++) {
                if (h < Gc) {
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        float* d = &q[h][8 * ch + e];
                        *d = s2 == 0 ? acc[h][e] : *d + acc[h][e];
                    }
                }
            }
        }
        wave_sync();
    }
#pragma unroll
    for (int h = 0; h < kGenMaxG; h++) {
        if (h < Gc) {
            if (a.nsplit == 1) {
                const float inv = 1.0f / l[h];
                float* o = a.out + ((size_t)t * a.nh + h0 + h) * hd;
                for (int e = lane; e < hd; e += 64) o[e] = q[h][e] * inv;
            } else {
                const size_t slot = ((size_t)y * a.nsplit + split) * a.G + h;
                float* o = a.part_acc + slot * hd;
                for (int e = lane; e < hd; e += 64) o[e] = q[h][e];
                if (lane == 0) *(float2*)(a.part_ml + slot * 2) = float2{m[h], l[h]};
            }
        }
    }
}

// out = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s over the key ranges of
// one query head; grid (G, ny). An empty range has m = -inf, weight 0.
__global__ __launch_bounds__(256) void gen_combine_kernel(const float* __restrict__ part_acc,
                                                          const float* __restrict__ part_ml, float* __restrict__ out,
                                                          int G, int g, int nchunk, int nsplit, int hd) {
    __shared__ float s_w[kMaxGenSplits];
    __shared__ float s_red[2][4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int h = blockIdx.x, y = blockIdx.y;
    const int kvh = y / nchunk, hc = y - kvh * nchunk;
    if (h >= min(G, g - hc * G)) return;  // whole workgroup
    const float* pml = part_ml + ((size_t)y * nsplit * G + h) * 2;
    // thread s holds key range s (nsplit <= 256)
    const float2 ml = tid < nsplit ? *(const float2*)(pml + (size_t)tid * G * 2)
                                   : float2{-__builtin_huge_valf(), 0.0f};
    float mx = group_max<64>(ml.x);
    if (lane == 0) s_red[0][wv] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(s_red[0][0], s_red[0][1]), fmaxf(s_red[0][2], s_red[0][3]));
    const float wt = tid < nsplit ? fast_exp2(ml.x - M) : 0.0f;
    if (tid < nsplit) s_w[tid] = wt;
    const float wl = group_sum<64>(wt * ml.y);
    if (lane == 0) s_red[1][wv] = wl;
    __syncthreads();
    const float inv = 1.0f / ((s_red[1][0] + s_red[1][1]) + (s_red[1][2] + s_red[1][3]));
    const float* pa = part_acc + ((size_t)y * nsplit * G + h) * hd;
    float* o = out + (size_t)(kvh * g + hc * G + h) * hd;
    for (int d = tid; d < hd; d += 256) {
        float acc = 0.0f;
#pragma unroll 8
        for (int s2 = 0; s2 < nsplit; s2++) acc = fmaf(s_w[s2], pa[(size_t)s2 * G * hd + d], acc);
        o[d] = acc * inv;
    }
}

// The workspace of prepared q rows, grown on demand (work queued earlier on
// the stream may still read the old one, so the stream drains first).
static hipError_t ensure_gen_q(pqa_ctx* ctx, size_t floats) {
    if (floats <= ctx->gen_q_floats) return hipSuccess;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return e;
    if (ctx->gen_q) (void)hipFree(ctx->gen_q);
    ctx->gen_q = nullptr;
    ctx->gen_q_floats = 0;
    e = hipMalloc((void**)&ctx->gen_q, floats * sizeof(float));
    if (e == hipSuccess) ctx->gen_q_floats = floats;
    return e;
}

static hipError_t launch_gen_prep(pqa_ctx* ctx, int layer, int start, int n_tok, const GenSrc& q, const GenSrc& k,
                                  const GenSrc& v) {
    const int hd = ctx->head_dim;
    GenPrepArgs p;
    p.q = q;
    p.k = k;
    p.v = v;
    const bool norm = ctx->has_qk_norm[layer] != 0;
    p.qn = norm ? ctx->qk_norm + (size_t)layer * 2 * hd : nullptr;
    p.kn = norm ? ctx->qk_norm + (size_t)layer * 2 * hd + hd : nullptr;
    p.cos_tab = ctx->rope_cos;
    p.sin_tab = ctx->rope_sin;
    p.kc = ctx->key_cache + (size_t)layer * ctx->layer_elems;
    p.vc = ctx->val_cache + (size_t)layer * ctx->layer_elems;
    p.qp = ctx->gen_q;
    p.start = start;
    p.n_tok = n_tok;
    p.nh = ctx->n_heads;
    p.nkv = ctx->n_kv_heads;
    p.hd = hd;
    p.rope = ctx->rope_style;
    p.qscale = 1.4426950408889634f / sqrtf((float)hd);
    const int heads = ctx->n_heads + ctx->n_kv_heads;
    hipLaunchKernelGGL(gen_prep_kernel, dim3((heads + kGenWaves - 1) / kGenWaves, n_tok), dim3(64 * kGenWaves), 0,
                       ctx->stream, p);
    return hipGetLastError();
}

template <int NS>
static hipError_t launch_gen_attn_ns(const GenAttnArgs& a, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL((gen_attn_kernel<NS>), grid, dim3(64 * kGenWaves), 0, st, a);
    return hipGetLastError();
}

static hipError_t launch_gen_attn(pqa_ctx* ctx, int layer, int start, int n_tok, float* out,
                                  const DecodeWorkspace* ws) {
    GenAttnArgs a;
    const int hd = ctx->head_dim;
    a.qp = ctx->gen_q;
    a.kc = ctx->key_cache + (size_t)layer * ctx->layer_elems;
    a.vc = ctx->val_cache + (size_t)layer * ctx->layer_elems;
    a.out = out;
    a.part_acc = ws ? ws->part_acc : nullptr;
    a.part_ml = ws ? ws->part_ml : nullptr;
    a.start = start;
    a.n_tok = n_tok;
    a.nh = ctx->n_heads;
    a.hd = hd;
    a.kv_dim = (int)ctx->kv_dim;
    a.g = ctx->kv_mul;
    a.nchunk = ctx->n_chunk;
    a.G = ctx->chunk_heads;
    a.ny = ctx->n_kv_heads * ctx->n_chunk;
    a.rps = ctx->max_seq_len;
    a.nsplit = 1;
    if (ws && n_tok == 1) {
        // a decode: key ranges of whole 64-key tiles, about 4 waves per CU in
        // all, at most the workspace's split count
        const int hist = start + 1;
        const int max_s = std::min(ws->max_splits, kMaxGenSplits);
        const int target = std::max(1, std::min(max_s, 8 * ctx->cu_count / a.ny));
        int rps = (hist + target - 1) / target;
        rps = std::max(64, (rps + 63) / 64 * 64);
        while ((hist + rps - 1) / rps > max_s) rps += 64;
        a.rps = rps;
        a.nsplit = (hist + rps - 1) / rps;
    }
    const long long items = (long long)a.ny * n_tok * a.nsplit;
    const dim3 grid((unsigned)((items + kGenWaves - 1) / kGenWaves));
    hipError_t e;
    if (hd % 8 == 0) {
        const dim3 blk(64 * kGenWaves);
        if (hd <= 128) hipLaunchKernelGGL(gen_attn8_kernel<128>, grid, blk, 0, ctx->stream, a);
        else if (hd <= 256) hipLaunchKernelGGL(gen_attn8_kernel<256>, grid, blk, 0, ctx->stream, a);
        else hipLaunchKernelGGL(gen_attn8_kernel<512>, grid, blk, 0, ctx->stream, a);
        e = hipGetLastError();
    } else {
        const int ns = (hd / 2 + 63) / 64;
        e = ns == 1 ? launch_gen_attn_ns<1>(a, grid, ctx->stream)
          : ns == 2 ? launch_gen_attn_ns<2>(a, grid, ctx->stream)
          : ns == 3 ? launch_gen_attn_ns<3>(a, grid, ctx->stream)
                    : launch_gen_attn_ns<4>(a, grid, ctx->stream);
    }
    if (e != hipSuccess || a.nsplit == 1) return e;
    hipLaunchKernelGGL(gen_combine_kernel, dim3(a.G, a.ny), dim3(256), 0, ctx->stream, (const float*)a.part_acc,
                       (const float*)a.part_ml, out, a.G, a.g, a.nchunk, a.nsplit, hd);
    return hipGetLastError();
}

static GenSrc plain_src(const float* p, size_t ld) { return GenSrc{p, (int)ld, nullptr, nullptr, nullptr, 0}; }

hipError_t launch_decode_general(pqa_ctx* ctx, int layer, int pos, const float* q, const float* k, const float* v,
                                 float* out, const DecodeWorkspace& ws) {
    // gen_q holds one token's q from context creation on: no allocation here
    if (ctx->gen_q_floats < ctx->q_dim) return hipErrorInvalidValue;
    hipError_t e = launch_gen_prep(ctx, layer, pos, 1, plain_src(q, ctx->q_dim), plain_src(k, ctx->kv_dim),
                                   plain_src(v, ctx->kv_dim));
    if (e != hipSuccess) return e;
    return launch_gen_attn(ctx, layer, pos, 1, out, &ws);
}

hipError_t launch_prefill_general(pqa_ctx* ctx, int layer, int start, int n_tok, const float* q, const float* k,
                                  const float* v, const PrefillScaled* ys, float* out) {
    hipError_t e = ensure_gen_q(ctx, (size_t)n_tok * ctx->q_dim);
    if (e != hipSuccess) return e;
    GenSrc sq, sk, sv;
    if (ys) {
        const size_t off[3] = {0, ctx->q_dim, ctx->q_dim + ctx->kv_dim};
        GenSrc* s[3] = {&sq, &sk, &sv};
        for (int i = 0; i < 3; i++)
            *s[i] = i > 0 && ys->kv_plain ? GenSrc{ys->y + off[i], ys->ld, nullptr, nullptr, nullptr, 0}
                                          : GenSrc{ys->y + off[i], ys->ld, ys->w_inv + off[i], ys->x_inv, ys->b[i], ys->bt[i]};
    } else {
        sq = plain_src(q, ctx->q_dim);
        sk = plain_src(k, ctx->kv_dim);
        sv = plain_src(v, ctx->kv_dim);
    }
    e = launch_gen_prep(ctx, layer, start, n_tok, sq, sk, sv);
    if (e != hipSuccess) return e;
    return launch_gen_attn(ctx, layer, start, n_tok, out, nullptr);
}

}  // namespace pqa
