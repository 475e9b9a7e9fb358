// Split-K flash decoding for one layer at one position: the decode block of
// cpp/model.hpp:326-418 as one kernel launch.
//
// Grid (nsplit, n_kv_heads * n_chunk), 256 threads (4 waves). Workgroup
// (split, kvh, chunk) owns cache rows [split*R, min(pos, (split+1)*R)) of KV
// head kvh and the G query heads of the chunk, so each K/V row is read from
// HBM once for the whole GQA group. The last split also owns the new row:
// it applies the QK-norm and RoPE, rounds K and V to fp16 with the
// reference's rounding, stores them at row pos and adds that row's softmax
// term itself, so no workgroup reads a row written in the same launch.
//
// Inside a wave, 16-row tiles:
//   scores  S[16 rows][16 cols] = K_tile (16x32 fp16 per MFMA step) x Q^T on
//           v_mfma_f32_16x16x32_f16; q is split into fp16 hi + lo parts
//           (two MFMAs into one accumulator) so the score keeps fp32
//           precision; the 1/sqrt(hd) and log2(e) factors are folded into q.
//   softmax each 16-lane group keeps its own running max / sum per head over
//           the 4 rows of every tile that land in its registers; exp2; the
//           accumulator is rescaled only when a maximum moves.
//   PV      VALU (v_fma_mix): the same lane group loads those 4 V rows, each
//           lane 8 head dims (one 16-byte load, HD/8 lanes per row), and
//           accumulates p[row][h] * v for the G heads; p comes from lane h of
//           the group by a DPP row broadcast.
// Loads run one tile ahead (two register sets, unconditional, row indices
// clamped to the wave's range) so every wait is for the tile being used.
// The lane groups are merged once per wave with log-sum-exp weights, the
// four waves' (max, sum, acc) are merged in LDS, and the workgroup writes
// either the output (one split) or its partial; decode_combine_kernel then
// merges the splits of each (kvh, chunk) with log-sum-exp weights.
#include "pqa_device.h"
#include "pqa_internal.h"

namespace pqa {

struct DecodeArgs {
    const float* q;
    const float* k;
    const float* v;
    const float* qn;  // [HD] or null
    const float* kn;
    const float* cosr;  // RoPE row at pos, [HD/2]
    const float* sinr;
    uint16_t* kc;  // layer slice [S][kv_dim]
    uint16_t* vc;
    float* out;
    float* part_acc;
    float* part_ml;
    int pos, g, nchunk, rope, kv_dim, nsplit, rows_per_split;
    float qscale;
};

constexpr int kDecodeThreads = 256;
constexpr int kMaxCombineSplits = 256;

template <int HD, int G>
__global__ __launch_bounds__(kDecodeThreads) void decode_kernel(const DecodeArgs a) {
    constexpr int KS = HD / 32;       // MFMA k-steps over the head dim
    constexpr int LPR = HD / 8;       // lanes per V row (8 fp16 each)
    constexpr int VL = 4 * LPR / 16;  // V loads per lane per 16-row tile
    constexpr float NEG_INF = -__builtin_huge_valf();

    __shared__ __attribute__((aligned(16))) float sq[G][HD];
    __shared__ __attribute__((aligned(16))) float sk[HD];
    __shared__ __attribute__((aligned(16))) float sv[HD];
    __shared__ __attribute__((aligned(16))) float s_qn[HD];
    __shared__ __attribute__((aligned(16))) float s_kn[HD];
    __shared__ __attribute__((aligned(16))) float s_cos[HD / 2];
    __shared__ __attribute__((aligned(16))) float s_sin[HD / 2];
    __shared__ float s_scale[G + 1];
    __shared__ float s_new[G];
    __shared__ float wm[4][G];
    __shared__ float wl[4][G];
    __shared__ float wacc[4][G][HD];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int y = blockIdx.y;
    const int split = blockIdx.x;
    const int kvh = y / a.nchunk;
    const int hc = y - kvh * a.nchunk;
    const int h0 = kvh * a.g + hc * G;
    const int Gc = min(G, a.g - hc * G);
    const bool owner = split == a.nsplit - 1;

    // ---------------- prologue: q heads (and the new K/V row) ----------------
    // Every global read of the prologue is issued before the first use, as
    // float4, so the prologue costs one memory round trip.
    {
        constexpr int H4 = HD / 4;
        float4 vq[(G * H4 + kDecodeThreads - 1) / kDecodeThreads];
#pragma unroll
        for (int r = 0; r < (G * H4 + kDecodeThreads - 1) / kDecodeThreads; r++) {
            const int i = tid + r * kDecodeThreads;
            vq[r] = (i < Gc * H4) ? ((const float4*)(a.q + (size_t)h0 * HD))[i] : float4{0.f, 0.f, 0.f, 0.f};
        }
        float4 vk = {0.f, 0.f, 0.f, 0.f}, vv = vk, wq = vk, wk = vk, cs = vk;
        if (owner && tid < H4) {
            vk = ((const float4*)(a.k + (size_t)kvh * HD))[tid];
            vv = ((const float4*)(a.v + (size_t)kvh * HD))[tid];
        }
        if (a.qn && tid < H4) {
            wq = ((const float4*)a.qn)[tid];
            wk = ((const float4*)a.kn)[tid];
        }
        // cos row in threads [0, HD/8), sin row in [HD/8, HD/4)
        if (tid < H4) cs = tid < H4 / 2 ? ((const float4*)a.cosr)[tid] : ((const float4*)a.sinr)[tid - H4 / 2];
#pragma unroll
        for (int r = 0; r < (G * H4 + kDecodeThreads - 1) / kDecodeThreads; r++) {
            const int i = tid + r * kDecodeThreads;
            if (i < G * H4) ((float4*)&sq[0][0])[i] = vq[r];
        }
        if (owner && tid < H4) {
            ((float4*)sk)[tid] = vk;
            ((float4*)sv)[tid] = vv;
        }
        if (a.qn && tid < H4) {
            ((float4*)s_qn)[tid] = wq;
            ((float4*)s_kn)[tid] = wk;
        }
        if (tid < H4) {
            if (tid < H4 / 2) ((float4*)s_cos)[tid] = cs;
            else ((float4*)s_sin)[tid - H4 / 2] = cs;
        }
    }
    __syncthreads();
    {
        // QK-RMSNorm scale, one quad per head (quad G is the K head).
        const int qd = tid >> 2, j = tid & 3;
        if (qd < Gc && a.qn) s_scale[qd] = rms_scale_ref_quad(sq[qd], HD, j);
        if (qd == G && owner && a.kn) s_scale[G] = rms_scale_ref_quad(sk, HD, j);
    }
    __syncthreads();
    if (a.qn)
        for (int i = tid; i < Gc * HD; i += kDecodeThreads) {
            const int h = i / HD, d = i - (i / HD) * HD;
            sq[h][d] = rms_apply(sq[h][d], s_scale[h], s_qn[d]);
        }
    if (owner && a.kn)
        for (int i = tid; i < HD; i += kDecodeThreads) sk[i] = rms_apply(sk[i], s_scale[G], s_kn[i]);
    __syncthreads();
    {
        constexpr int HALF = HD / 2;
        const int npairs = (Gc + (owner ? 1 : 0)) * HALF;
        for (int i = tid; i < npairs; i += kDecodeThreads) {
            const int h = i / HALF, p = i - (i / HALF) * HALF;
            float* x = h < Gc ? sq[h] : sk;
            int e0, e1;
            rope_pair(a.rope, p, HD, e0, e1);
            rope_rotate(x[e0], x[e1], s_cos[p], s_sin[p]);
        }
    }
    __syncthreads();
    if (owner) {
        for (int i = tid; i < HD; i += kDecodeThreads) {
            const uint16_t kb = f32_to_f16_ref(sk[i]);
            const uint16_t vb = f32_to_f16_ref(sv[i]);
            if (hc == 0) {
                const size_t off = (size_t)a.pos * a.kv_dim + (size_t)kvh * HD + i;
                a.kc[off] = kb;
                a.vc[off] = vb;
            }
            sk[i] = f16_bits_to_f32(kb);
            sv[i] = f16_bits_to_f32(vb);
        }
    }
    for (int i = tid; i < G * HD; i += kDecodeThreads) {
        const int h = i / HD, d = i - (i / HD) * HD;
        sq[h][d] *= a.qscale;
    }
    __syncthreads();
    if (owner && tid < Gc) {
        float s = 0.0f;
        for (int d = 0; d < HD; d++) s = fmaf(sq[tid][d], sk[d], s);
        s_new[tid] = s;
    }

    // ---------------- wave loop over history rows ----------------
    // Lane (g, n), g = lane/16, n = lane%16. The score MFMA reads K row n of the
    // tile and puts S[row 4g+i][head n] in register i of lane (g, n). The same
    // lane group g also loads V rows 4g..4g+3 (HD/8 lanes per row), so each
    // group runs its own online softmax over its rows: no cross-group traffic
    // per tile. p[row][h] reaches the V lanes of the group by a DPP row
    // broadcast from lane h. The four groups are merged once, at the end.
    const int n = lane & 15;
    const int grp = lane >> 4;
    half8 qh[KS], ql[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float x = n < G ? sq[n][32 * ks + 8 * grp + e] : 0.0f;
            const _Float16 hi = (_Float16)x;
            qh[ks][e] = hi;
            ql[ks][e] = (_Float16)(x - (float)hi);
        }
    }

    const int r0 = split * a.rows_per_split;
    const int rend = min(a.pos, r0 + a.rows_per_split);
    const int per_w = a.rows_per_split >> 2;
    const int w0 = r0 + w * per_w;
    const int w1 = min(rend, w0 + per_w);

    constexpr int RPG = 16 / LPR;  // V rows per lane group per load (1 for HD 128, 2 for HD 64)
    const int vsub = n / LPR;      // which of those rows this lane takes
    const int vdim = 8 * (n % LPR);

    float m_run = NEG_INF;
    float l_run = 0.0f;
    float acc[G][8];
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[h][e] = 0.0f;

    if (w0 < w1) {
        const uint16_t* kbase = a.kc + (size_t)kvh * HD + 8 * grp;
        const uint16_t* vbase = a.vc + (size_t)kvh * HD + vdim;
        const size_t stride = (size_t)a.kv_dim;
        const int rlast = w1 - 1;

        // Rows past the wave's range are clamped to its last row: the loads
        // stay in bounds and hit lines fetched a moment earlier.
        auto load_tile = [&](int tb, u32x4 (&kf)[KS], u32x4 (&vf)[VL]) {
            const int kr = min(tb + n, rlast);
            const uint16_t* kp = kbase + (size_t)kr * stride;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) kf[ks] = *(const u32x4*)(kp + 32 * ks);
#pragma unroll
            for (int j = 0; j < VL; j++) {
                const int vr = min(tb + 4 * grp + vsub + RPG * j, rlast);
                vf[j] = *(const u32x4*)(vbase + (size_t)vr * stride);
            }
        };

        auto process = [&](int tb, const u32x4 (&kf)[KS], const u32x4 (&vf)[VL]) {
            floatx4 S = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const half8 kh = __builtin_bit_cast(half8, kf[ks]);
                S = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[ks], S, 0, 0, 0);
                S = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[ks], S, 0, 0, 0);
            }
            float s[4];
#pragma unroll
            for (int i = 0; i < 4; i++) s[i] = (tb + 4 * grp + i < w1 && n < Gc) ? S[i] : NEG_INF;
            const float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
            const float m_new = fmaxf(m_run, mx);
            const bool moved = m_new > m_run;
            if (__any(moved)) {
                const float corr = moved ? fast_exp2(m_run - m_new) : 1.0f;
                l_run *= corr;
                m_run = m_new;
#pragma unroll
                for (int h = 0; h < G; h++) {
                    const float c = row_bcast(corr, h);
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[h][e] *= c;
                }
            }
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; i++) p[i] = s[i] == NEG_INF ? 0.0f : fast_exp2(s[i] - m_run);
            l_run += (p[0] + p[1]) + (p[2] + p[3]);
#pragma unroll
            for (int j = 0; j < VL; j++) {
                const half8 vh = __builtin_bit_cast(half8, vf[j]);
                float pr[G];
#pragma unroll
                for (int h = 0; h < G; h++) {
                    if constexpr (RPG == 1) {
                        pr[h] = row_bcast(p[j], h);
                    } else {
                        const float lo = row_bcast(p[RPG * j], h), hi = row_bcast(p[RPG * j + 1], h);
                        pr[h] = vsub ? hi : lo;
                    }
                }
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float ve = (float)vh[e];
#pragma unroll
                    for (int h = 0; h < G; h++) acc[h][e] = fmaf(pr[h], ve, acc[h][e]);
                }
            }
        };

        u32x4 kA[KS], vA[VL], kB[KS], vB[VL];
        load_tile(w0, kA, vA);
        load_tile(w0 + 16, kB, vB);
        for (int tb = w0; tb < w1; tb += 32) {
            process(tb, kA, vA);
            load_tile(tb + 32, kA, vA);
            if (tb + 16 >= w1) break;
            process(tb + 16, kB, vB);
            load_tile(tb + 48, kB, vB);
        }
    }

    // ---------------- merge the four lane groups, then write the wave partial ----------------
    {
        float M = fmaxf(m_run, __shfl_xor(m_run, 16));
        M = fmaxf(M, __shfl_xor(M, 32));
        const float e = (m_run == NEG_INF) ? 0.0f : fast_exp2(m_run - M);
        float l = l_run * e;
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float eh = row_bcast(e, h);
#pragma unroll
            for (int k = 0; k < 8; k++) {
                float x = acc[h][k] * eh;
#pragma unroll
                for (int off = LPR; off < 64; off <<= 1) x += __shfl_xor(x, off);
                acc[h][k] = x;
            }
        }
        if (lane < LPR) {
#pragma unroll
            for (int h = 0; h < G; h++)
#pragma unroll
                for (int k = 0; k < 8; k++) wacc[w][h][vdim + k] = acc[h][k];
        }
        if (lane < G) {
            wm[w][lane] = M;
            wl[w][lane] = l;
        }
    }
    __syncthreads();

    // ---------------- workgroup merge (+ the new row) ----------------
    const size_t part_base = ((size_t)y * a.nsplit + split) * G;
    for (int i = tid; i < Gc * HD; i += kDecodeThreads) {
        const int h = i / HD, d = i - (i / HD) * HD;
        float M = owner ? s_new[h] : NEG_INF;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) M = fmaxf(M, wm[ww][h]);
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) {
            const float e = fast_exp2(wm[ww][h] - M);
            L += e * wl[ww][h];
            A += e * wacc[ww][h][d];
        }
        if (owner) {
            const float e = fast_exp2(s_new[h] - M);
            L += e;
            A += e * sv[d];
        }
        if (a.nsplit == 1) {
            a.out[(size_t)(h0 + h) * HD + d] = A / L;
        } else {
            a.part_acc[(part_base + h) * HD + d] = A;
            if (d == 0) {
                a.part_ml[(part_base + h) * 2] = M;
                a.part_ml[(part_base + h) * 2 + 1] = L;
            }
        }
    }
}

// Merge of the split partials of one (KV head, chunk), one workgroup per query
// head: M = max_s m_s, w_s = exp2(m_s - M), out = sum_s w_s acc_s / sum_s w_s l_s.
// A separate launch: the kernel boundary makes every partial visible, so the
// split workgroups need no fences or atomics.
template <int HD>
__global__ __launch_bounds__(kDecodeThreads) void decode_combine_kernel(const float* __restrict__ part_acc,
                                                                        const float* __restrict__ part_ml,
                                                                        float* __restrict__ out, int G, int g,
                                                                        int nchunk, int nsplit) {
    constexpr int H4 = HD / 4;
    constexpr int P = kDecodeThreads / H4;  // split groups summed in parallel
    constexpr float NEG_INF = -__builtin_huge_valf();
    __shared__ float s_m[kMaxCombineSplits];
    __shared__ float s_w[kMaxCombineSplits];
    __shared__ float s_red[kDecodeThreads / 64];
    __shared__ __attribute__((aligned(16))) floatx4 s_acc[P][H4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int h = blockIdx.x, y = blockIdx.y;
    const int kvh = y / nchunk, hc = y - kvh * nchunk;
    const int Gc = min(G, g - hc * G);
    if (h >= Gc) return;
    const float* pml = part_ml + ((size_t)y * nsplit * G + h) * 2;
    float mloc = NEG_INF, lloc = 0.0f;
    if (tid < nsplit) {
        mloc = pml[(size_t)tid * G * 2];
        lloc = pml[(size_t)tid * G * 2 + 1];
        s_m[tid] = mloc;
    }
    float M = mloc;
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
    if (lane == 0) s_red[w] = M;
    __syncthreads();
    M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    float wl = 0.0f;
    if (tid < nsplit) {
        const float wt = fast_exp2(mloc - M);
        s_w[tid] = wt;
        wl = wt * lloc;
    }
    for (int off = 32; off > 0; off >>= 1) wl += __shfl_xor(wl, off);
    __syncthreads();
    if (lane == 0) s_red[w] = wl;
    __syncthreads();
    const float L = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
    const int d4 = tid % H4, pg = tid / H4;
    const floatx4* src = (const floatx4*)(part_acc + ((size_t)y * nsplit * G + h) * HD) + d4;
    const size_t sstride = (size_t)G * H4;
    floatx4 A = {0.f, 0.f, 0.f, 0.f};
    int sp = pg;
    for (; sp + 7 * P < nsplit; sp += 8 * P) {
        floatx4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = src[(size_t)(sp + u * P) * sstride];
#pragma unroll
        for (int u = 0; u < 8; u++) A += s_w[sp + u * P] * v[u];
    }
    for (; sp < nsplit; sp += P) A += s_w[sp] * src[(size_t)sp * sstride];
    s_acc[pg][d4] = A;
    __syncthreads();
    if (tid < H4) {
        floatx4 r = s_acc[0][tid];
#pragma unroll
        for (int q = 1; q < P; q++) r += s_acc[q][tid];
        const float inv = 1.0f / L;
        ((floatx4*)(out + (size_t)(kvh * g + hc * G + h) * HD))[tid] = r * inv;
    }
}

void decode_split(const pqa_ctx* ctx, int hist, int* rows_per_split, int* nsplit) {
    int rps;
    if (ctx->split_override > 0) {
        rps = ctx->split_override;
    } else {
        // Aim at about two workgroups per CU across all (kvh, chunk) columns,
        // never fewer than 64 rows (16 per wave) per workgroup.
        const int ny = ctx->n_kv_heads * ctx->n_chunk;
        const int per_y = max(1, (2 * ctx->cu_count) / ny);
        rps = (hist + per_y - 1) / per_y;
    }
    rps = max(64, (rps + 63) & ~63);
    int ns = max(1, (hist + rps - 1) / rps);
    while (ns > ctx->max_splits) {
        rps += 64;
        ns = max(1, (hist + rps - 1) / rps);
    }
    *rows_per_split = rps;
    *nsplit = ns;
}

template <int HD>
static hipError_t launch_decode_hd(const DecodeArgs& a, int G, dim3 grid, hipStream_t st) {
    switch (G) {
#define PQA_CASE(GG) \
    case GG: hipLaunchKernelGGL((decode_kernel<HD, GG>), grid, dim3(kDecodeThreads), 0, st, a); break;
        PQA_CASE(1) PQA_CASE(2) PQA_CASE(3) PQA_CASE(4) PQA_CASE(5) PQA_CASE(6) PQA_CASE(7) PQA_CASE(8)
#undef PQA_CASE
        default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit == 1) return e;
    hipLaunchKernelGGL(decode_combine_kernel<HD>, dim3(G, grid.y), dim3(kDecodeThreads), 0, st, a.part_acc,
                       a.part_ml, a.out, G, a.g, a.nchunk, a.nsplit);
    return hipGetLastError();
}

hipError_t launch_decode(pqa_ctx* ctx, int layer, int pos, const float* q, const float* k,
                         const float* v, float* out) {
    DecodeArgs a;
    const int hd = ctx->head_dim;
    a.q = q;
    a.k = k;
    a.v = v;
    const bool norm = ctx->has_qk_norm[layer] != 0;
    a.qn = norm ? ctx->qk_norm + (size_t)layer * 2 * hd : nullptr;
    a.kn = norm ? ctx->qk_norm + (size_t)layer * 2 * hd + hd : nullptr;
    a.cosr = ctx->rope_cos + (size_t)pos * (hd / 2);
    a.sinr = ctx->rope_sin + (size_t)pos * (hd / 2);
    a.kc = ctx->key_cache + (size_t)layer * ctx->layer_elems;
    a.vc = ctx->val_cache + (size_t)layer * ctx->layer_elems;
    a.out = out;
    a.part_acc = ctx->part_acc;
    a.part_ml = ctx->part_ml;
    a.pos = pos;
    a.g = ctx->kv_mul;
    a.nchunk = ctx->n_chunk;
    a.rope = ctx->rope_style;
    a.kv_dim = (int)ctx->kv_dim;
    decode_split(ctx, pos, &a.rows_per_split, &a.nsplit);
    a.qscale = 1.4426950408889634f / sqrtf((float)hd);
    dim3 grid(a.nsplit, ctx->n_kv_heads * ctx->n_chunk);
    if (hd == 64) return launch_decode_hd<64>(a, ctx->chunk_heads, grid, ctx->stream);
    if (hd == 128) return launch_decode_hd<128>(a, ctx->chunk_heads, grid, ctx->stream);
    return hipErrorInvalidValue;
}

}  // namespace pqa
