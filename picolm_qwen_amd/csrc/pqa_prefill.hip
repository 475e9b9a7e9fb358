// Causal prefill of one layer: the token loop of cpp/model.hpp:493-593 as two
// launches.
//
// 1. prefill_kv: the new cache rows. One wave per 64/(HD/4) (token, KV head)
//    rows: K gets the QK-RMSNorm in the reference's summation order, RoPE at
//    the token's position and the reference's fp16 rounding; V the rounding
//    only. Rows start..start+n-1 of the layer slice are written.
// 2. prefill_attn: flash attention over the fp16 cache on
//    v_mfma_f32_32x32x16_f16. The query heads of one KV head are packed as
//    rows R = token*g + h (g = query heads per KV head), so one K/V tile in
//    LDS serves the whole GQA group. A workgroup is 4 waves x 32 packed rows.
//    Each wave first builds its q fragments in registers from the fp32
//    projections: in the MFMA operand layout a lane holds 64 of its row's
//    dims and every RoPE pair of all three pairings lies inside the lane, so
//    norm (one exchange with the partner lane) and rotation need no LDS.
//    Per 64-key tile each wave computes S^T = K Q^T (keys x rows), the online
//    softmax per row (a lane owns one row: its 32 scores plus the partner
//    lane 32 apart), and O^T += V^T P^T. With S^T in the MFMA result layout
//    the lane's scores are already the B operand of the PV product, so P
//    never leaves registers. The running maximum is raised (and O, l
//    rescaled) only when a score exceeds it by more than 2^8, so most tiles
//    skip the rescale. K/V tiles arrive by direct global->LDS loads, double
//    buffered, one barrier per tile; V fragments are read with transposing
//    LDS reads. Tiles past the causal limit of every row in a wave are
//    skipped.
#include <type_traits>

#include "pqa_device.h"
#include "pqa_internal.h"

namespace pqa {

struct KvArgs {
    const float* k;  // [n_tok][kv_dim]
    const float* v;
    const float* kn;       // [HD] or null
    const float* wpad;     // 2*HD readable floats, loaded in place of absent norm weights
    const float* cos_tab;  // [S][HD/2]
    const float* sin_tab;
    uint16_t* kc;  // layer slice [S][kv_dim]
    uint16_t* vc;
    int start, n_tok, nkv, rope;
};

constexpr int kKvThreads = 256;

template <int HD>
__global__ __launch_bounds__(kKvThreads) void prefill_kv_kernel(const KvArgs a) {
    constexpr int H4 = HD / 4;
    constexpr int IPW = 64 / H4;  // rows per wave
    constexpr int NW = kKvThreads / 64;
    __shared__ __attribute__((aligned(16))) float sk[NW][IPW][HD];
    __shared__ float s_scale[NW][IPW];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t = lane % H4, hh = lane / H4;
    const int n_items = a.n_tok * a.nkv;
    const int item = (blockIdx.x * NW + w) * IPW + hh;
    const int it = min(item, n_items - 1);  // loads stay in bounds; stores are predicated
    const int tok = it / a.nkv, kvh = it - tok * a.nkv;
    const int pos = a.start + tok;
    const size_t kv_dim = (size_t)a.nkv * HD;
    const float4 kx = ((const float4*)(a.k + (size_t)tok * kv_dim + (size_t)kvh * HD))[t];
    const float4 vx = ((const float4*)(a.v + (size_t)tok * kv_dim + (size_t)kvh * HD))[t];
    const float4 wk = ((const float4*)(a.kn ? a.kn : a.wpad + HD))[t];
    const int ci = rope_angle_f4<HD>(a.rope, t);
    const float4 cs = ((const float4*)(a.cos_tab + (size_t)pos * (HD / 2)))[ci];
    const float4 sn = ((const float4*)(a.sin_tab + (size_t)pos * (HD / 2)))[ci];
    float4 x = kx;
    if (a.kn) {
        ((float4*)sk[w][hh])[t] = kx;
        wave_sync();
        const int qd = min(lane >> 2, IPW - 1);  // quad qd sums row qd in the reference's order
        const float s = rms_scale_ref_quad(sk[w][qd], HD, lane & 3);
        if ((lane & 3) == 0 && (lane >> 2) < IPW) s_scale[w][qd] = s;
        wave_sync();
        const float sc = s_scale[w][hh];
        x = float4{rms_apply(x.x, sc, wk.x), rms_apply(x.y, sc, wk.y), rms_apply(x.z, sc, wk.z),
                   rms_apply(x.w, sc, wk.w)};
    }
    x = rope_lanes<HD>(x, a.rope, t, cs, sn);
    if (item < n_items) {
        const size_t off = (size_t)pos * kv_dim + (size_t)kvh * HD + 4 * t;
        *(u32x2*)(a.kc + off) = u32x2{f32_to_f16_ref(x.x) | ((uint32_t)f32_to_f16_ref(x.y) << 16),
                                      f32_to_f16_ref(x.z) | ((uint32_t)f32_to_f16_ref(x.w) << 16)};
        *(u32x2*)(a.vc + off) = u32x2{f32_to_f16_ref(vx.x) | ((uint32_t)f32_to_f16_ref(vx.y) << 16),
                                      f32_to_f16_ref(vx.z) | ((uint32_t)f32_to_f16_ref(vx.w) << 16)};
    }
}

struct AttnArgs {
    const float* q;   // [n_tok][nh*HD] fp32 projections
    const float* qn;  // [HD] or null
    const float* wpad;
    const float* cos_tab;  // [S][HD/2]
    const float* sin_tab;
    const uint16_t* kc;
    const uint16_t* vc;
    float* out;
    int start, n_tok, nh, g, n_kv, kv_dim, rows, nblk, rope;
    float qscale;
};

constexpr int kAttnThreads = 256;
constexpr int kRowsPerBlock = 128;
constexpr int kKeysPerTile = 64;
constexpr float kRescaleSlack = 8.0f;  // log2 units: P stays <= 256 between rescales

// LDS tile layout: 64 rows of HD fp16 (row = one key), rows unpadded, the
// 16-byte chunks of row r stored at chunk index c ^ swz(r). The direct
// global->LDS loads pick, for each lane, the global chunk whose swizzled slot
// is the lane's LDS slot, so the tile is written already swizzled.
//   K: swz(r) = r mod chunks: the A-operand reads (32 rows, one chunk
//      column) hit 16 distinct chunk slots per 16 lanes.
//   V: swz(r) = 4 * (r mod 4): the transposed reads (8 rows x 4 chunks per
//      instruction) touch every chunk slot exactly twice (the 2-pass minimum).
template <int HD>
struct PrefillTile {
    static constexpr int CH = HD / 8;            // 16-byte chunks per row
    static constexpr int ROWB = HD * 2;          // bytes per row
    static constexpr int BYTES = kKeysPerTile * ROWB;
    static constexpr int RPI = 1024 / ROWB;      // rows per 1 KB wave-wide load
    static constexpr int NI = BYTES / 1024 / (kAttnThreads / 64);  // loads per wave per tile and operand
    __device__ static int swz_k(int r) { return r & (CH - 1); }
    __device__ static int swz_v(int r) { return (4 * (r & 3)) & (CH - 1); }
};

// SPLITQ: scores use q = hi + lo (two fp16 MFMAs into one fp32 accumulator),
// which keeps fp32-level score precision when keys carry large outliers.
template <int HD, bool SPLITQ>
__global__ __launch_bounds__(kAttnThreads, 2) void prefill_attn_kernel(const AttnArgs a) {
    using T = PrefillTile<HD>;
    constexpr int QK = HD / 16;  // k-steps of S^T = K Q^T
    constexpr int DT = HD / 32;  // 32-dim tiles of O^T
    constexpr float NEG_INF = -__builtin_huge_valf();
    __shared__ __attribute__((aligned(1024))) char lds[2][2][T::BYTES];  // [buffer][K, V]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31;  // q row within the wave / MFMA row index
    const int hk = lane >> 5;   // MFMA k-group
    // Work item: all blocks of one KV head run on the same XCD (workgroups go
    // round-robin over the 8 XCDs), keeping that head's K/V in one L2. Within a
    // head, the first half of the items are the long causal blocks in
    // decreasing length, the second half the short ones in increasing length,
    // so the two workgroups a CU receives add up to about the same work.
    const int kvh = (int)blockIdx.x % a.n_kv;
    const int jj = (int)blockIdx.x / a.n_kv;
    const int half = (a.nblk + 1) / 2;
    const int b = jj < half ? a.nblk - 1 - jj : jj - half;

    const char* kbase = (const char*)(a.kc + (size_t)kvh * HD);
    const char* vbase = (const char*)(a.vc + (size_t)kvh * HD);
    const size_t rowb = (size_t)a.kv_dim * 2;  // bytes per cache row

    const int R0 = b * kRowsPerBlock + w * 32;
    const int R = R0 + col;
    const bool rvalid = R < a.rows;
    const int tok = rvalid ? R / a.g : 0;
    const int hq = kvh * a.g + (rvalid ? R - (R / a.g) * a.g : 0);
    const int qpos = a.start + tok;
    const int last_row_blk = min(a.rows, (b + 1) * kRowsPerBlock) - 1;
    const int kend = a.start + last_row_blk / a.g + 1;
    const int ntiles = (kend + kKeysPerTile - 1) / kKeysPerTile;
    const int kend_w = R0 < a.rows ? a.start + (min(a.rows, R0 + 32) - 1) / a.g + 1 : 0;
    const int qpos_min_w = R0 < a.rows ? a.start + R0 / a.g : 0;

    // ---- per-lane offsets, fixed for the whole loop ----
    // global -> LDS: wave load i of an operand fills LDS bytes [1024 (w NI + i), +1024):
    // tile row r = (w NI + i) RPI + lane / CH, source chunk (lane % CH) ^ swz(r)
    unsigned gk[T::NI], gv[T::NI];
#pragma unroll
    for (int i = 0; i < T::NI; i++) {
        const int r = (w * T::NI + i) * T::RPI + lane / T::CH;
        const int p = lane % T::CH;
        gk[i] = (unsigned)(r * rowb) + 16u * (unsigned)(p ^ T::swz_k(r));
        gv[i] = (unsigned)(r * rowb) + 16u * (unsigned)(p ^ T::swz_v(r));
    }
    // K fragment reads: row 32 t2 + col, chunk (2 ks + hk) ^ swz_k(col)
    int koff[QK];
#pragma unroll
    for (int ks = 0; ks < QK; ks++) koff[ks] = col * T::ROWB + 16 * ((2 * ks + hk) ^ T::swz_k(col));
    // V^T fragment reads (transposing): row 16 s + 8 t + 4 hk + tr_e,
    // dims 32 dt + 16 (g16 & 1) + 4 tr_q .. +3
    const int j16 = lane & 15, g16 = lane >> 4;
    const int tr_e = j16 >> 2, tr_q = j16 & 3;
    int voff[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
        const int c = 4 * dt + 2 * (g16 & 1) + (tr_q >> 1);
        voff[dt] = (4 * hk + tr_e) * T::ROWB + 16 * (c ^ T::swz_v(tr_e)) + 8 * (tr_q & 1);
    }

    auto issue = [&](int kt, int buf) {
        const int key0 = kt * kKeysPerTile;
        if (key0 + kKeysPerTile <= kend) {
            const char* kb = kbase + (size_t)key0 * rowb;
            const char* vb = vbase + (size_t)key0 * rowb;
#pragma unroll
            for (int i = 0; i < T::NI; i++) {
                const int inst = w * T::NI + i;
                __builtin_amdgcn_global_load_lds((const void*)(kb + gk[i]),
                                                 (__attribute__((address_space(3))) void*)&lds[buf][0][inst * 1024], 16, 0, 0);
                __builtin_amdgcn_global_load_lds((const void*)(vb + gv[i]),
                                                 (__attribute__((address_space(3))) void*)&lds[buf][1][inst * 1024], 16, 0, 0);
            }
        } else {  // last tile: rows past kend (never read unmasked) clamp to kend - 1
#pragma unroll
            for (int i = 0; i < T::NI; i++) {
                const int inst = w * T::NI + i;
                const int r = inst * T::RPI + lane / T::CH;
                const int p = lane % T::CH;
                const size_t row = (size_t)min(key0 + r, kend - 1) * rowb;
                __builtin_amdgcn_global_load_lds((const void*)(kbase + row + 16 * (p ^ T::swz_k(r))),
                                                 (__attribute__((address_space(3))) void*)&lds[buf][0][inst * 1024], 16, 0, 0);
                __builtin_amdgcn_global_load_lds((const void*)(vbase + row + 16 * (p ^ T::swz_v(r))),
                                                 (__attribute__((address_space(3))) void*)&lds[buf][1][inst * 1024], 16, 0, 0);
            }
        }
    };

    issue(0, 0);

    // ---- q fragments: lane (col, hk) holds dims 16 ks + 8 hk + e of row col ----
    // One round trip: the q row slice, the RoPE cos/sin values it needs and
    // (direct to LDS) the norm weights are all requested with tile 0.
    __shared__ __attribute__((aligned(16))) float s_qw[HD];
    if (w == 0 && lane < HD / 4)
        __builtin_amdgcn_global_load_lds((const void*)((a.qn ? a.qn : a.wpad) + 4 * lane),
                                         (__attribute__((address_space(3))) void*)s_qw, 16, 0, 0);
    half8 qf[QK], qfl[SPLITQ ? QK : 1];
    {
        const float* qrow = a.q + ((size_t)tok * a.nh + hq) * HD + 8 * hk;
        float x[QK][8];
#pragma unroll
        for (int ks = 0; ks < QK; ks++) {
            const float4 u0 = *(const float4*)(qrow + 16 * ks);
            const float4 u1 = *(const float4*)(qrow + 16 * ks + 4);
            x[ks][0] = u0.x, x[ks][1] = u0.y, x[ks][2] = u0.z, x[ks][3] = u0.w;
            x[ks][4] = u1.x, x[ks][5] = u1.y, x[ks][6] = u1.z, x[ks][7] = u1.w;
        }
        // cos/sin float4 i: NeoX angles 16 (i/2) + 8 hk + 4 (i%2) (dims of ks = i/2 < QK/2);
        // block8 / interleaved angles 4 (2 i + hk) (8-dim chunk 2 i + hk)
        const float* crow = a.cos_tab + (size_t)qpos * (HD / 2);
        const float* srow = a.sin_tab + (size_t)qpos * (HD / 2);
        float4 cf[QK], sf[QK];
#pragma unroll
        for (int i = 0; i < QK; i++) {
            const int ai = a.rope == 0 ? 16 * (i >> 1) + 8 * hk + 4 * (i & 1) : 4 * (2 * i + hk);
            cf[i] = *(const float4*)(crow + ai);
            sf[i] = *(const float4*)(srow + ai);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();  // s_qw landed
        if (a.qn) {
            float ss = 0.0f;
#pragma unroll
            for (int ks = 0; ks < QK; ks++)
#pragma unroll
                for (int e = 0; e < 8; e++) ss = fmaf(x[ks][e], x[ks][e], ss);
            ss = sum_x32(ss);  // + the partner lane's 64 dims
            const float sc = 1.0f / sqrtf(ss / (float)HD + 1e-6f);
#pragma unroll
            for (int ks = 0; ks < QK; ks++) {
                const float4 w0 = *(const float4*)(s_qw + 16 * ks + 8 * hk);
                const float4 w1 = *(const float4*)(s_qw + 16 * ks + 8 * hk + 4);
                const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                for (int e = 0; e < 8; e++) x[ks][e] = rms_apply(x[ks][e], sc, wv[e]);
            }
        }
        if (a.rope == 0) {
            // NeoX: dim d < HD/2 pairs with d + HD/2, i.e. ks with ks + QK/2; angle d
#pragma unroll
            for (int ks = 0; ks < QK / 2; ks++) {
                const float cv[8] = {cf[2 * ks].x, cf[2 * ks].y, cf[2 * ks].z, cf[2 * ks].w,
                                     cf[2 * ks + 1].x, cf[2 * ks + 1].y, cf[2 * ks + 1].z, cf[2 * ks + 1].w};
                const float sv[8] = {sf[2 * ks].x, sf[2 * ks].y, sf[2 * ks].z, sf[2 * ks].w,
                                     sf[2 * ks + 1].x, sf[2 * ks + 1].y, sf[2 * ks + 1].z, sf[2 * ks + 1].w};
#pragma unroll
                for (int e = 0; e < 8; e++) rope_rotate(x[ks][e], x[ks + QK / 2][e], cv[e], sv[e]);
            }
        } else {
            // 8-dim chunk 2 ks + hk: block8 pairs (e, e+4), interleaved pairs (2i, 2i+1)
#pragma unroll
            for (int ks = 0; ks < QK; ks++) {
                const float cv[4] = {cf[ks].x, cf[ks].y, cf[ks].z, cf[ks].w};
                const float sv[4] = {sf[ks].x, sf[ks].y, sf[ks].z, sf[ks].w};
                if (a.rope == 1) {
#pragma unroll
                    for (int e = 0; e < 4; e++) rope_rotate(x[ks][e], x[ks][e + 4], cv[e], sv[e]);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) rope_rotate(x[ks][2 * e], x[ks][2 * e + 1], cv[e], sv[e]);
                }
            }
        }
        const float qs = rvalid ? a.qscale : 0.0f;
#pragma unroll
        for (int ks = 0; ks < QK; ks++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float xs = x[ks][e] * qs;
                const _Float16 hi = (_Float16)xs;
                qf[ks][e] = hi;
                if constexpr (SPLITQ) qfl[ks][e] = (_Float16)(xs - (float)hi);
            }
    }

    float m_run = NEG_INF, l_run = 0.0f;
    floatx16 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] = 0.0f;

    auto tile = [&](int kt, auto BUF) {
        constexpr int buf = decltype(BUF)::value;
        const int key0 = kt * kKeysPerTile;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's loads of tile kt
        __syncthreads();                                   // everyone's; the other buffer is free
        if (kt + 1 < ntiles) issue(kt + 1, buf ^ 1);
        if (key0 >= kend_w) return;  // wave-uniform: every row of this wave is done

        const char* kt_lds = lds[buf][0];
        const char* vt_lds = lds[buf][1];
        floatx16 sacc[2];
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++) {
            const char* kp = kt_lds + t2 * 32 * T::ROWB;
            half8 kf = *(const half8*)(kp + koff[0]);
            sacc[t2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[0], floatx16{}, 0, 0, 0);
            if constexpr (SPLITQ) sacc[t2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qfl[0], sacc[t2], 0, 0, 0);
#pragma unroll
            for (int ks = 1; ks < QK; ks++) {
                kf = *(const half8*)(kp + koff[ks]);
                sacc[t2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[ks], sacc[t2], 0, 0, 0);
                if constexpr (SPLITQ)
                    sacc[t2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qfl[ks], sacc[t2], 0, 0, 0);
            }
        }
        // lane holds keys key0 + 32*t2 + 8*(r/4) + 4*hk + r%4 of q row `col`
        if (key0 + kKeysPerTile - 1 > qpos_min_w) {
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = key0 + 32 * t2 + 8 * (r >> 2) + 4 * hk + (r & 3);
                    if (key > qpos) sacc[t2][r] = NEG_INF;
                }
        }
        float mx = NEG_INF;
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
            for (int r = 0; r < 16; r++) mx = fmaxf(mx, sacc[t2][r]);
        mx = max_x32(mx);
        if (__any(mx > m_run + kRescaleSlack)) {
            const float m_new = fmaxf(m_run, mx);
            const float corr = fast_exp2(m_run - m_new);
            m_run = m_new;
            l_run *= corr;
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[dt][r] *= corr;
        }
        half8 pf[4];
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
            for (int r = 0; r < 16; r++) pf[2 * t2 + (r >> 3)][r & 7] = (_Float16)fast_exp2(sacc[t2][r] - m_run);
        // row sum of the fp16 P the PV product consumes (v_dot2_f32_f16 with ones)
        const half2 one2 = {(_Float16)1.0f, (_Float16)1.0f};
        float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                ps[s] = __builtin_amdgcn_fdot2(half2{pf[s][2 * e], pf[s][2 * e + 1]}, one2, ps[s], false);
        l_run += (ps[0] + ps[1]) + (ps[2] + ps[3]);
#pragma unroll
        for (int s = 0; s < 4; s++) {
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                half4 part[2];
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const char* adr = vt_lds + voff[dt] + (16 * s + 8 * t) * T::ROWB;
                    const short4v raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) short4v*)adr);
                    part[t] = __builtin_bit_cast(half4, raw);
                }
                const half8 vf = {part[0][0], part[0][1], part[0][2], part[0][3],
                                  part[1][0], part[1][1], part[1][2], part[1][3]};
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[s], o[dt], 0, 0, 0);
            }
        }
    };

    for (int kt = 0; kt < ntiles; kt += 2) {
        tile(kt, std::integral_constant<int, 0>{});
        if (kt + 1 < ntiles) tile(kt + 1, std::integral_constant<int, 1>{});
    }

    const float l_tot = sum_x32(l_run);
    if (rvalid) {
        const float inv = 1.0f / l_tot;
        float* op = a.out + ((size_t)tok * a.nh + hq) * HD + 4 * hk;
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) {
                floatx4 vv = {o[dt][4 * r4] * inv, o[dt][4 * r4 + 1] * inv, o[dt][4 * r4 + 2] * inv,
                              o[dt][4 * r4 + 3] * inv};
                *(floatx4*)(op + 32 * dt + 8 * r4) = vv;
            }
    }
}

template <int HD>
static hipError_t launch_prefill_hd(pqa_ctx* ctx, int layer, int start, int n_tok, const float* q,
                                    const float* k, const float* v, float* out) {
    const bool norm = ctx->has_qk_norm[layer] != 0;
    const float* qn = norm ? ctx->qk_norm + (size_t)layer * 2 * HD : nullptr;
    const float* kn = norm ? ctx->qk_norm + (size_t)layer * 2 * HD + HD : nullptr;
    uint16_t* kc = ctx->key_cache + (size_t)layer * ctx->layer_elems;
    uint16_t* vc = ctx->val_cache + (size_t)layer * ctx->layer_elems;

    KvArgs p;
    p.k = k;
    p.v = v;
    p.kn = kn;
    p.wpad = ctx->qk_norm;
    p.cos_tab = ctx->rope_cos;
    p.sin_tab = ctx->rope_sin;
    p.kc = kc;
    p.vc = vc;
    p.start = start;
    p.n_tok = n_tok;
    p.nkv = ctx->n_kv_heads;
    p.rope = ctx->rope_style;
    constexpr int rows_per_wg = (kKvThreads / 64) * (64 / (HD / 4));
    const int n_items = n_tok * ctx->n_kv_heads;
    hipLaunchKernelGGL(prefill_kv_kernel<HD>, dim3((n_items + rows_per_wg - 1) / rows_per_wg), dim3(kKvThreads),
                       0, ctx->stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;

    AttnArgs a;
    a.q = q;
    a.qn = qn;
    a.wpad = ctx->qk_norm;
    a.cos_tab = ctx->rope_cos;
    a.sin_tab = ctx->rope_sin;
    a.kc = kc;
    a.vc = vc;
    a.out = out;
    a.start = start;
    a.n_tok = n_tok;
    a.nh = ctx->n_heads;
    a.g = ctx->kv_mul;
    a.n_kv = ctx->n_kv_heads;
    a.kv_dim = (int)ctx->kv_dim;
    a.rows = n_tok * ctx->kv_mul;
    a.nblk = (a.rows + kRowsPerBlock - 1) / kRowsPerBlock;
    a.rope = ctx->rope_style;
    a.qscale = 1.4426950408889634f / sqrtf((float)HD);
    dim3 grid(a.nblk * ctx->n_kv_heads);
    if (ctx->prefill_split_q)
        hipLaunchKernelGGL((prefill_attn_kernel<HD, true>), grid, dim3(kAttnThreads), 0, ctx->stream, a);
    else
        hipLaunchKernelGGL((prefill_attn_kernel<HD, false>), grid, dim3(kAttnThreads), 0, ctx->stream, a);
    return hipGetLastError();
}

hipError_t launch_prefill(pqa_ctx* ctx, int layer, int start, int n_tok, const float* q,
                          const float* k, const float* v, float* out) {
    if (ctx->head_dim == 64) return launch_prefill_hd<64>(ctx, layer, start, n_tok, q, k, v, out);
    if (ctx->head_dim == 128) return launch_prefill_hd<128>(ctx, layer, start, n_tok, q, k, v, out);
    return hipErrorInvalidValue;
}

}  // namespace pqa
