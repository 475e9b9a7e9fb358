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
//   softmax per-head running max over the tile (xor-shuffles across the four
//           lane groups), exp2, running sum; the accumulator is rescaled
//           only when a maximum moves.
//   PV      VALU: each lane holds 8 head dims of one V row (one 16-byte load,
//           HD/8 lanes per row) and accumulates p[row][h] * v for the G heads;
//           p reaches the V lanes through a 17x8 float LDS tile per wave.
// The four waves' (max, sum, acc) are merged in LDS, the workgroup's partial
// goes to the workspace, and the last workgroup of each (kvh, chunk) to
// finish (atomic counter) merges all splits with log-sum-exp weights and
// writes out[h][:] = acc / sum.
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
    unsigned* cnt;
    int pos, g, nchunk, rope, kv_dim, nsplit, rows_per_split;
    float qscale;
};

constexpr int kDecodeThreads = 256;
constexpr int kMaxCombineSplits = 256;

template <int HD, int G>
__global__ __launch_bounds__(kDecodeThreads) void decode_kernel(const DecodeArgs a) {
    constexpr int KS = HD / 32;       // MFMA k-steps over the head dim
    constexpr int LPR = HD / 8;       // lanes per V row (8 fp16 each)
    constexpr int RPL = 64 / LPR;     // V rows per wave-wide load
    constexpr int VL = 16 / RPL;      // V loads per 16-row tile
    constexpr int PS = 8;             // p-tile row stride (floats)
    constexpr float NEG_INF = -__builtin_huge_valf();

    __shared__ float sq[G][HD];
    __shared__ float sk[HD];
    __shared__ float sv[HD];
    __shared__ float s_scale[G + 1];
    __shared__ float s_new[G];
    __shared__ float sp[4][17 * PS];
    __shared__ float wm[4][G];
    __shared__ float wl[4][G];
    __shared__ float wacc[4][G][HD];
    __shared__ float sw[kMaxCombineSplits * G];
    __shared__ float sM[G], sL[G];
    __shared__ int s_last;

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
    for (int i = tid; i < G * HD; i += kDecodeThreads) {
        const int h = i / HD, d = i - (i / HD) * HD;
        sq[h][d] = h < Gc ? a.q[(size_t)(h0 + h) * HD + d] : 0.0f;
    }
    if (owner) {
        for (int i = tid; i < HD; i += kDecodeThreads) {
            sk[i] = a.k[(size_t)kvh * HD + i];
            sv[i] = a.v[(size_t)kvh * HD + i];
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
            sq[h][d] = rms_apply(sq[h][d], s_scale[h], a.qn[d]);
        }
    if (owner && a.kn)
        for (int i = tid; i < HD; i += kDecodeThreads) sk[i] = rms_apply(sk[i], s_scale[G], a.kn[i]);
    __syncthreads();
    {
        constexpr int HALF = HD / 2;
        const int npairs = (Gc + (owner ? 1 : 0)) * HALF;
        for (int i = tid; i < npairs; i += kDecodeThreads) {
            const int h = i / HALF, p = i - (i / HALF) * HALF;
            float* x = h < Gc ? sq[h] : sk;
            int e0, e1;
            rope_pair(a.rope, p, HD, e0, e1);
            rope_rotate(x[e0], x[e1], a.cosr[p], a.sinr[p]);
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
    const int n = lane & 15;   // MFMA row / column index
    const int grp = lane >> 4;  // MFMA k-group / output row group
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

    float m_run = NEG_INF;
    float l_run = 0.0f;
    float acc[G][8];
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[h][e] = 0.0f;

    float* p_tile = sp[w];
    const int vrow = lane / LPR;
    const int vdim = 8 * (lane % LPR);

    if (w0 < w1) {
        const uint16_t* kbase = a.kc + (size_t)kvh * HD + 8 * grp;
        const uint16_t* vbase = a.vc + (size_t)kvh * HD + vdim;
        const size_t stride = (size_t)a.kv_dim;
        const int rlast = w1 - 1;

        auto load_tile = [&](int tb, u32x4 (&kf)[KS], u32x4 (&vf)[VL]) {
            const int kr = min(tb + n, rlast);
            const uint16_t* kp = kbase + (size_t)kr * stride;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) kf[ks] = *(const u32x4*)(kp + 32 * ks);
#pragma unroll
            for (int j = 0; j < VL; j++) {
                const int vr = min(tb + vrow + RPL * j, rlast);
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
            // lane holds rows tb + 4*grp + i (i = 0..3) of head column n
            float s[4];
#pragma unroll
            for (int i = 0; i < 4; i++) s[i] = (tb + 4 * grp + i < w1 && n < Gc) ? S[i] : NEG_INF;
            float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float m_new = fmaxf(m_run, mx);
            const bool moved = m_new > m_run;
            const bool any_moved = __any(moved);
            if (any_moved) {
                const float corr = moved ? fast_exp2(m_run - m_new) : 1.0f;
                l_run *= corr;
                if (grp == 0 && n < PS) p_tile[16 * PS + n] = corr;
                m_run = m_new;
            }
            float psum = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float p = (n < Gc) ? fast_exp2(s[i] - m_run) : 0.0f;
                psum += p;
                if (n < PS) p_tile[(4 * grp + i) * PS + n] = p;
            }
            l_run += psum;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (any_moved) {
                float c[G];
#pragma unroll
                for (int h = 0; h < G; h++) c[h] = p_tile[16 * PS + h];
#pragma unroll
                for (int h = 0; h < G; h++)
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[h][e] *= c[h];
            }
#pragma unroll
            for (int j = 0; j < VL; j++) {
                const int r = vrow + RPL * j;
                float pr[G];
#pragma unroll
                for (int h = 0; h < G; h++) pr[h] = p_tile[r * PS + h];
                const half8 vh = __builtin_bit_cast(half8, vf[j]);
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float ve = (float)vh[e];
#pragma unroll
                    for (int h = 0; h < G; h++) acc[h][e] = fmaf(pr[h], ve, acc[h][e]);
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        };

        u32x4 kA[KS], vA[VL], kB[KS], vB[VL];
        load_tile(w0, kA, vA);
        for (int tb = w0; tb < w1; tb += 32) {
            const bool has_b = tb + 16 < w1;
            if (has_b) load_tile(tb + 16, kB, vB);
            process(tb, kA, vA);
            if (!has_b) break;
            if (tb + 32 < w1) load_tile(tb + 32, kA, vA);
            process(tb + 16, kB, vB);
        }
    }

    // ---------------- merge the wave's lane partials ----------------
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float x = acc[h][e];
#pragma unroll
            for (int off = LPR; off < 64; off <<= 1) x += __shfl_xor(x, off);
            acc[h][e] = x;
        }
    if (lane < LPR) {
#pragma unroll
        for (int h = 0; h < G; h++)
#pragma unroll
            for (int e = 0; e < 8; e++) wacc[w][h][vdim + e] = acc[h][e];
    }
    if (lane < G) {
        wm[w][lane] = m_run;
        wl[w][lane] = l_run;
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
    if (a.nsplit == 1) return;

    // ---------------- last workgroup of this (kvh, chunk) merges all splits ----------------
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = atomicAdd(&a.cnt[y], 1u);
        s_last = prev == (unsigned)(a.nsplit - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    const float* pml = a.part_ml + (size_t)y * a.nsplit * G * 2;
    const float* pacc = a.part_acc + (size_t)y * a.nsplit * G * HD;
    if (tid < Gc) {
        float M = NEG_INF;
        for (int s = 0; s < a.nsplit; s++) M = fmaxf(M, __builtin_nontemporal_load(pml + ((size_t)s * G + tid) * 2));
        sM[tid] = M;
    }
    __syncthreads();
    for (int i = tid; i < a.nsplit * Gc; i += kDecodeThreads) {
        const int s = i / Gc, h = i - (i / Gc) * Gc;
        sw[s * G + h] = fast_exp2(__builtin_nontemporal_load(pml + ((size_t)s * G + h) * 2) - sM[h]);
    }
    __syncthreads();
    if (tid < Gc) {
        float L = 0.0f;
        for (int s = 0; s < a.nsplit; s++)
            L += sw[s * G + tid] * __builtin_nontemporal_load(pml + ((size_t)s * G + tid) * 2 + 1);
        sL[tid] = L;
    }
    __syncthreads();
    for (int i = tid; i < Gc * HD; i += kDecodeThreads) {
        const int h = i / HD, d = i - (i / HD) * HD;
        float A = 0.0f;
        for (int s = 0; s < a.nsplit; s++)
            A += sw[s * G + h] * __builtin_nontemporal_load(pacc + ((size_t)s * G + h) * HD + d);
        a.out[(size_t)(h0 + h) * HD + d] = A / sL[h];
    }
    if (tid == 0) a.cnt[y] = 0u;
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
    a.cnt = ctx->counters;
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
