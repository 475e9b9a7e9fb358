// Split-K flash decoding for one layer at one position: the decode block of
// cpp/model.hpp:326-418 in two launches (split pass + merge).
//
// Columns: the query heads of one KV head form a column y = (kvh, chunk) of
// G <= 8 heads (a GQA group wider than 8 is cut into chunks), so each K/V row
// of the column is read from HBM once for all its query heads.
//
// Split pass, grid (nsplit, ceil(ny / 8)), 512 threads = 8 waves. Workgroup
// (split, column group) owns cache rows [split*R, min(pos, (split+1)*R)) of
// up to 8 columns, one wave per column; with fewer columns each column gets
// several waves on consecutive sub-ranges. The eight waves thus read the same
// rows, all KV heads of them: whole 2 KB cache rows stream from HBM together,
// which keeps DRAM pages open (reading one head's 256 B slice of every row
// per workgroup costs ~15 % of bandwidth). K/V loads are non-temporal (the
// cache is read once per step) and run two 16-row tiles ahead, with row
// indices clamped to the wave's range so no load sits behind a branch.
// The last split also owns the new row: it applies the QK-norm and RoPE,
// rounds K and V to fp16 with the reference's rounding, stores them at row
// pos and adds that row's softmax term itself, so no workgroup reads a row
// written in the same launch.
//
// Inside a wave, per 16-row tile:
//   scores  S[16 rows][16 cols] = K_tile x Q^T on v_mfma_f32_16x16x32_f16;
//           q is split into fp16 hi + lo parts (two MFMAs into one fp32
//           accumulator) so scores keep fp32 precision; 1/sqrt(hd) and
//           log2(e) are folded into q.
//   softmax each 16-lane group keeps its own running max / sum per head over
//           the 4 rows of every tile that land in its registers; exp2; the
//           accumulator is rescaled only when a maximum moves.
//   PV      VALU (v_fma_mix): the same lane group loads those 4 V rows, each
//           lane 8 head dims (HD/8 lanes per row), and accumulates
//           p[row][h] * v for the G heads; p comes from lane h of the group by
//           a DPP row broadcast.
// Lane groups are merged once per wave, waves of a column once per workgroup
// (log-sum-exp weights); the workgroup writes the output (one split) or its
// partial (max, sum, acc) per head, and decode_combine_kernel merges splits.
#include "pqa_device.h"
#include "pqa_internal.h"

namespace pqa {

struct DecodeArgs {
    const float* q;
    const float* k;
    const float* v;
    const float* qn;  // [HD] or null
    const float* kn;
    const float* wpad;  // 2*HD readable floats, loaded in place of absent norm weights
    const float* cosr;  // RoPE row at pos, [HD/2]
    const float* sinr;
    uint16_t* kc;  // layer slice [S][kv_dim]
    uint16_t* vc;
    float* out;
    float* part_acc;  // [ny][nsplit][G][HD]
    float* part_ml;   // [ny][nsplit][G][2]
    int pos, g, nchunk, ny, rope, kv_dim, nsplit, rows_per_split;
    float qscale;
};

constexpr int kDecodeWaves = 8;
constexpr int kDecodeThreads = 64 * kDecodeWaves;
constexpr int kCombineThreads = 256;
constexpr int kMaxCombineSplits = 256;

template <int HD, int G>
__global__ __launch_bounds__(kDecodeThreads) void decode_kernel(const DecodeArgs a) {
    constexpr int NW = kDecodeWaves;
    constexpr int KS = HD / 32;       // MFMA k-steps over the head dim
    constexpr int LPR = HD / 8;       // lanes per V row (8 fp16 each)
    constexpr int VL = 4 * LPR / 16;  // V loads per lane per 16-row tile
    constexpr int RPG = 16 / LPR;     // V rows per lane group per load (1 for HD 128, 2 for HD 64)
    constexpr int H4 = HD / 4;
    constexpr int HALF = HD / 2;
    constexpr int QR = (NW * G * H4 + kDecodeThreads - 1) / kDecodeThreads;  // q float4 loads per thread
    constexpr float NEG_INF = -__builtin_huge_valf();

    // q heads of every column ([NW][G][HD]); after the fragments are built the
    // same space holds the wave partials ([NW][G][HD]).
    __shared__ __attribute__((aligned(16))) float sqw[NW * G * HD];
    __shared__ __attribute__((aligned(16))) float sk[NW][HD];
    __shared__ __attribute__((aligned(16))) float sv[NW][HD];
    __shared__ __attribute__((aligned(16))) float s_qn[HD];
    __shared__ __attribute__((aligned(16))) float s_kn[HD];
    __shared__ __attribute__((aligned(16))) float s_cs[HD];  // cos row | sin row
    __shared__ float s_scale[NW * G + NW];
    __shared__ float s_new[NW][G];
    __shared__ float wm[NW][G];
    __shared__ float wl[NW][G];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int split = blockIdx.x;
    const int ybase = blockIdx.y * NW;
    const int cols = min(a.ny - ybase, NW);
    const int sub = NW / cols;
    const bool active = w < cols * sub;
    const int c = active ? w % cols : 0;
    const int sb = active ? w / cols : 0;
    const bool owner = split == a.nsplit - 1;

    // first query head, KV head, chunk index and head count of column cc
    auto col_h0 = [&](int cc, int& kvh_o, int& hc_o, int& gc_o) {
        const int yy = ybase + cc;
        kvh_o = yy / a.nchunk;
        hc_o = yy - kvh_o * a.nchunk;
        gc_o = min(G, a.g - hc_o * G);
        return kvh_o * a.g + hc_o * G;
    };
    int kvh, hc, Gc;
    const int h0 = col_h0(c, kvh, hc, Gc);
    (void)hc;

    // ---------------- this wave's history rows; first two tiles in flight ----------------
    // The first K/V tiles do not depend on q, so they are requested with the
    // prologue's loads. Loads are unconditional: an empty range (or pos == 0)
    // clamps to row 0, which is allocated and never used.
    const int n = lane & 15;    // MFMA row (K) / column (head) index
    const int grp = lane >> 4;  // MFMA k-group / output row group
    const int vsub = n / LPR;
    const int vdim = 8 * (n % LPR);
    const int r0 = split * a.rows_per_split;
    const int r1 = min(a.pos, r0 + a.rows_per_split);
    const int per_s = a.rows_per_split / sub;
    const int w0 = r0 + sb * per_s;
    const int w1 = active ? min(r1, w0 + per_s) : w0;
    const uint16_t* kbase = a.kc + (size_t)kvh * HD + 8 * grp;
    const uint16_t* vbase = a.vc + (size_t)kvh * HD + vdim;
    const size_t stride = (size_t)a.kv_dim;
    const int rlast = max(w1 - 1, 0);

    auto load_tile = [&](int tb, u32x4 (&kf)[KS], u32x4 (&vf)[VL]) {
        const int kr = min(tb + n, rlast);
        const u32x4* kp = (const u32x4*)(kbase + (size_t)kr * stride);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) kf[ks] = __builtin_nontemporal_load(kp + 4 * ks);
#pragma unroll
        for (int j = 0; j < VL; j++) {
            const int vr = min(tb + 4 * grp + vsub + RPG * j, rlast);
            vf[j] = __builtin_nontemporal_load((const u32x4*)(vbase + (size_t)vr * stride));
        }
    };
    u32x4 kA[KS], vA[VL], kB[KS], vB[VL];

    // ---------------- prologue: q heads of every column, the new K/V rows ----------------
    {
        float4 vq[QR];
#pragma unroll
        for (int r = 0; r < QR; r++) {
            const int i = min(tid + r * kDecodeThreads, cols * G * H4 - 1);
            const int cc = i / (G * H4), rem = i - cc * (G * H4), h = rem / H4, d4 = rem - h * H4;
            int kq, hq, gq;
            const int hb = col_h0(cc, kq, hq, gq);
            vq[r] = ((const float4*)(a.q + (size_t)(hb + min(h, gq - 1)) * HD))[d4];
        }
        const int t = tid % (NW * H4);
        int kk_, hk_, gk_;
        col_h0(min(t / H4, cols - 1), kk_, hk_, gk_);
        float4 vk = ((const float4*)(a.k + (size_t)kk_ * HD))[t % H4];
        float4 vv = ((const float4*)(a.v + (size_t)kk_ * HD))[t % H4];
        const int t4 = tid % H4;
        const float* qn = a.qn ? a.qn : a.wpad;  // loads stay unconditional without a norm
        const float* kn = a.kn ? a.kn : a.wpad + HD;
        float4 wq = ((const float4*)qn)[t4];
        float4 wk = ((const float4*)kn)[t4];
        float4 cs = t4 < H4 / 2 ? ((const float4*)a.cosr)[t4] : ((const float4*)a.sinr)[t4 - H4 / 2];
        load_tile(w0, kA, vA);
        load_tile(w0 + 16, kB, vB);
#pragma unroll
        for (int r = 0; r < QR; r++) pin(vq[r]);
        pin(vk);
        pin(vv);
        pin(wq);
        pin(wk);
        pin(cs);
#pragma unroll
        for (int r = 0; r < QR; r++) {
            const int i = tid + r * kDecodeThreads;
            if (i < NW * G * H4) {
                const int cc = i / (G * H4), h = (i - cc * (G * H4)) / H4;
                int kq, hq, gq;
                col_h0(min(cc, cols - 1), kq, hq, gq);
                ((float4*)sqw)[i] = (cc < cols && h < gq) ? vq[r] : float4{0.f, 0.f, 0.f, 0.f};
            }
        }
        if (tid < NW * H4) {
            ((float4*)&sk[0][0])[tid] = vk;
            ((float4*)&sv[0][0])[tid] = vv;
        }
        if (tid < H4) {
            ((float4*)s_qn)[tid] = wq;
            ((float4*)s_kn)[tid] = wk;
            ((float4*)s_cs)[tid] = cs;
        }
    }
    __syncthreads();
    {
        // QK-RMSNorm scales, one quad per head: q heads [0, NW*G), K rows after.
        const int qd = tid >> 2, j = tid & 3;
        if (a.qn && qd < cols * G) {
            int kq, hq, gq;
            col_h0(qd / G, kq, hq, gq);
            if (qd % G < gq) s_scale[qd] = rms_scale_ref_quad(sqw + (size_t)qd * HD, HD, j);
        } else if (a.kn && owner && qd >= NW * G && qd < NW * G + cols) {
            s_scale[qd] = rms_scale_ref_quad(sk[qd - NW * G], HD, j);
        }
    }
    __syncthreads();
    if (a.qn) {
        for (int i = tid; i < cols * G * HD; i += kDecodeThreads) {
            const int hh = i / HD, d = i - hh * HD;
            int kq, hq, gq;
            col_h0(hh / G, kq, hq, gq);
            if (hh % G < gq) sqw[i] = rms_apply(sqw[i], s_scale[hh], s_qn[d]);
        }
        if (owner)
            for (int i = tid; i < cols * HD; i += kDecodeThreads) {
                const int cc = i / HD, d = i - cc * HD;
                sk[cc][d] = rms_apply(sk[cc][d], s_scale[NW * G + cc], s_kn[d]);
            }
    }
    __syncthreads();
    {
        const int nq = cols * G * HALF;
        const int npairs = nq + (owner ? cols * HALF : 0);
        for (int i = tid; i < npairs; i += kDecodeThreads) {
            const int hh = i / HALF, p = i - hh * HALF;
            float* x = i < nq ? sqw + (size_t)hh * HD : sk[hh - cols * G];
            int e0, e1;
            rope_pair(a.rope, p, HD, e0, e1);
            rope_rotate(x[e0], x[e1], s_cs[p], s_cs[HALF + p]);
        }
    }
    __syncthreads();
    if (owner) {
        for (int i = tid; i < cols * HD; i += kDecodeThreads) {
            const int cc = i / HD, d = i - cc * HD;
            int kq, hq, gq;
            col_h0(cc, kq, hq, gq);
            const uint16_t kb = f32_to_f16_ref(sk[cc][d]);
            const uint16_t vb = f32_to_f16_ref(sv[cc][d]);
            if (hq == 0) {
                const size_t off = (size_t)a.pos * a.kv_dim + (size_t)kq * HD + d;
                a.kc[off] = kb;
                a.vc[off] = vb;
            }
            sk[cc][d] = f16_bits_to_f32(kb);
            sv[cc][d] = f16_bits_to_f32(vb);
        }
    }
    for (int i = tid; i < NW * G * HD; i += kDecodeThreads) sqw[i] *= a.qscale;
    __syncthreads();
    if (owner && tid < cols * G) {
        const int cc = tid / G, h = tid - cc * G;
        float s = 0.0f;
        for (int d = 0; d < HD; d++) s = fmaf(sqw[(size_t)tid * HD + d], sk[cc][d], s);
        s_new[cc][h] = s;
    }

    // ---------------- wave loop over history rows ----------------
    // Lane (g, n), g = lane/16, n = lane%16. The score MFMA reads K row n of the
    // tile and puts S[row 4g+i][head n] in register i of lane (g, n). The same
    // lane group g also loads V rows 4g..4g+3, so each group runs its own
    // online softmax over its rows: no cross-group traffic per tile.
    half8 qh[KS], ql[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float x = n < G ? sqw[(size_t)(c * G + n) * HD + 32 * ks + 8 * grp + e] : 0.0f;
            const _Float16 hi = (_Float16)x;
            qh[ks][e] = hi;
            ql[ks][e] = (_Float16)(x - (float)hi);
        }
    }
    __syncthreads();  // sqw is reused below for the wave partials

    float m_run = NEG_INF;
    float l_run = 0.0f;
    float acc[G][8];
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[h][e] = 0.0f;

    if (w0 < w1) {
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
                    const float cf = row_bcast(corr, h);
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[h][e] *= cf;
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
                for (int k = 0; k < 8; k++) sqw[(size_t)(w * G + h) * HD + vdim + k] = acc[h][k];
        }
        if (lane < G) {
            wm[w][lane] = M;
            wl[w][lane] = l;
        }
    }
    __syncthreads();

    // ---------------- workgroup merge per column (+ the new row) ----------------
    for (int i = tid; i < cols * G * HD; i += kDecodeThreads) {
        const int cc = i / (G * HD), h = (i / HD) - cc * G, d = i - (i / HD) * HD;
        int kq, hq, gq;
        const int hb = col_h0(cc, kq, hq, gq);
        if (h >= gq) continue;
        float M = owner ? s_new[cc][h] : NEG_INF;
        for (int s = 0; s < sub; s++) M = fmaxf(M, wm[cc + s * cols][h]);
        float L = 0.0f, A = 0.0f;
        for (int s = 0; s < sub; s++) {
            const int wv = cc + s * cols;
            const float e = fast_exp2(wm[wv][h] - M);
            L += e * wl[wv][h];
            A += e * sqw[(size_t)(wv * G + h) * HD + d];
        }
        if (owner) {
            const float e = fast_exp2(s_new[cc][h] - M);
            L += e;
            A += e * sv[cc][d];
        }
        if (a.nsplit == 1) {
            a.out[(size_t)(hb + h) * HD + d] = A / L;
        } else {
            const size_t pb = ((size_t)(ybase + cc) * a.nsplit + split) * G + h;
            a.part_acc[pb * HD + d] = A;
            if (d == 0) {
                a.part_ml[pb * 2] = M;
                a.part_ml[pb * 2 + 1] = L;
            }
        }
    }
    (void)h0;
}

// Merge of the split partials of one column, one workgroup per query head:
// M = max_s m_s, w_s = exp2(m_s - M), out = sum_s w_s acc_s / sum_s w_s l_s.
// A separate launch: the kernel boundary makes every partial visible, so the
// split workgroups need no fences or atomics. The first batch of partial
// loads is issued together with the (max, sum) loads: one round trip when
// nsplit <= 8 * P.
template <int HD>
__global__ __launch_bounds__(kCombineThreads) void decode_combine_kernel(const float* __restrict__ part_acc,
                                                                         const float* __restrict__ part_ml,
                                                                         float* __restrict__ out, int G, int g,
                                                                         int nchunk, int nsplit) {
    constexpr int H4 = HD / 4;
    constexpr int P = kCombineThreads / H4;  // split groups summed in parallel
    constexpr int U = 8;                     // loads per batch per thread
    constexpr float NEG_INF = -__builtin_huge_valf();
    __shared__ float s_w[kMaxCombineSplits];
    __shared__ float s_red[kCombineThreads / 64];
    __shared__ __attribute__((aligned(16))) floatx4 s_acc[P][H4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int h = blockIdx.x, y = blockIdx.y;
    const int kvh = y / nchunk, hc = y - kvh * nchunk;
    const int Gc = min(G, g - hc * G);
    if (h >= Gc) return;
    const float* pml = part_ml + ((size_t)y * nsplit * G + h) * 2;
    const int d4 = tid % H4, pg = tid / H4;
    const floatx4* src = (const floatx4*)(part_acc + ((size_t)y * nsplit * G + h) * HD) + d4;
    const size_t sstride = (size_t)G * H4;

    const int ts = min(tid, nsplit - 1);
    float mloc = pml[(size_t)ts * G * 2];
    float lloc = pml[(size_t)ts * G * 2 + 1];
    floatx4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = src[(size_t)min(pg + u * P, nsplit - 1) * sstride];
    if (tid >= nsplit) {
        mloc = NEG_INF;
        lloc = 0.0f;
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
    floatx4 A = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < U; u++)
        if (pg + u * P < nsplit) A += s_w[pg + u * P] * v[u];
    for (int sp = pg + U * P; sp < nsplit; sp += P) A += s_w[sp] * src[(size_t)sp * sstride];
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
        // About one workgroup (8 waves) per CU; a workgroup reads whole cache
        // rows of all its columns.
        rps = (hist + ctx->cu_count - 1) / ctx->cu_count;
    }
    rps = max(128, (rps + 127) & ~127);
    int ns = max(1, (hist + rps - 1) / rps);
    while (ns > ctx->max_splits) {
        rps += 128;
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
    hipLaunchKernelGGL(decode_combine_kernel<HD>, dim3(G, a.ny), dim3(kCombineThreads), 0, st, a.part_acc,
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
    a.wpad = ctx->qk_norm;
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
    a.ny = ctx->n_kv_heads * ctx->n_chunk;
    a.rope = ctx->rope_style;
    a.kv_dim = (int)ctx->kv_dim;
    decode_split(ctx, pos, &a.rows_per_split, &a.nsplit);
    a.qscale = 1.4426950408889634f / sqrtf((float)hd);
    dim3 grid(a.nsplit, (a.ny + kDecodeWaves - 1) / kDecodeWaves);
    if (hd == 64) return launch_decode_hd<64>(a, ctx->chunk_heads, grid, ctx->stream);
    if (hd == 128) return launch_decode_hd<128>(a, ctx->chunk_heads, grid, ctx->stream);
    return hipErrorInvalidValue;
}

}  // namespace pqa
