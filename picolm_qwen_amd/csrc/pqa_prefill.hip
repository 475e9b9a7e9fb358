// Causal prefill of one layer: the token loop of cpp/model.hpp:493-593 as two
// launches.
//
// 1. prefill_prep: one workgroup per token. QK-RMSNorm (reference reduction
//    order), RoPE at the token's position, K and V rounded to fp16 with the
//    reference's rounding into cache rows start..start+n-1, and q scaled by
//    log2(e)/sqrt(hd) and rounded to fp16 for the MFMA stage.
// 2. prefill_attn: flash attention over the fp16 cache on
//    v_mfma_f32_32x32x16_f16. The query heads of one KV head are packed as
//    rows R = token*g + h (g = query heads per KV head), so one K/V tile in
//    LDS serves the whole GQA group. A workgroup is 4 waves x 32 packed rows;
//    per 64-key tile each wave computes S^T = K Q^T (keys x rows), the online
//    softmax per row (a lane owns one row: its 32 scores plus the partner
//    lane 32 apart), and O^T += V^T P^T. With S^T in the MFMA result layout the
//    lane's scores are already the B operand of the PV product, so P never
//    leaves registers. V is stored transposed in LDS. Tiles past the causal
//    limit of every row in a wave are skipped. Workgroup blockIdx.x runs
//    query block nblk-1-x and then block x, so each workgroup does about the
//    same causal work.
#include "pqa_device.h"
#include "pqa_internal.h"

namespace pqa {

struct PrepArgs {
    const float* q;  // [n_tok][nh*HD]
    const float* k;  // [n_tok][kv_dim]
    const float* v;
    const float* qn;
    const float* kn;
    const float* wpad;     // 2*HD readable floats, loaded in place of absent norm weights
    const float* cos_tab;  // [S][HD/2]
    const float* sin_tab;
    uint16_t* kc;
    uint16_t* vc;
    _Float16* q16;     // [n_tok][nh][HD], fp16(q * qscale)
    _Float16* q16_lo;  // null, or the rounding residual fp16(q*qscale - q16)
    int start, nh, nkv, rope;
    float qscale;
};

constexpr int kPrepThreads = 256;

template <int HD>
__global__ __launch_bounds__(kPrepThreads) void prefill_prep_kernel(const PrepArgs a) {
    // [(nh + nkv) * HD] q and k heads, then [nh + nkv] scales, [HD] q/k norm
    // weights, [HD/2] cos and sin of the token's position
    extern __shared__ __attribute__((aligned(16))) float sx[];
    constexpr int H4 = HD / 4;
    constexpr int HALF = HD / 2;
    constexpr int MAXR = 8;  // float4 loads in flight per thread
    const int tid = threadIdx.x;
    const int tok = blockIdx.x;
    const int pos = a.start + tok;
    const int nheads = a.nh + a.nkv;
    const size_t q_dim = (size_t)a.nh * HD, kv_dim = (size_t)a.nkv * HD;
    float* scale = sx + (size_t)nheads * HD;
    float* s_qn = scale + ((nheads + 3) & ~3);
    float* s_kn = s_qn + HD;
    float* s_cs = s_kn + HD;  // cos then sin
    const float4* q4 = (const float4*)(a.q + tok * q_dim);
    const float4* k4 = (const float4*)(a.k + tok * kv_dim);
    const int nq4 = (int)(q_dim / 4), n4 = nheads * H4;

    // one round trip: every load of a chunk is issued before any store to LDS;
    // the loads are unconditional (index clamped) so none sits behind a branch
    for (int base = 0; base < n4; base += MAXR * kPrepThreads) {
        float4 r[MAXR];
#pragma unroll
        for (int u = 0; u < MAXR; u++) {
            const int i = min(base + tid + u * kPrepThreads, n4 - 1);
            const float4* src = i < nq4 ? q4 + i : k4 + (i - nq4);
            r[u] = *src;
        }
#pragma unroll
        for (int u = 0; u < MAXR; u++) pin(r[u]);
#pragma unroll
        for (int u = 0; u < MAXR; u++) {
            const int i = base + tid + u * kPrepThreads;
            if (i < n4) ((float4*)sx)[i] = r[u];
        }
    }
    {
        const int t = tid % H4;  // every thread loads (in bounds); the first H4 store
        const float4* cs = t < H4 / 2 ? (const float4*)(a.cos_tab + (size_t)pos * HALF) + t
                                      : (const float4*)(a.sin_tab + (size_t)pos * HALF) + (t - H4 / 2);
        const float4 c = *cs;
        const float* qn = a.qn ? a.qn : a.wpad;  // loads stay unconditional without a norm
        const float* kn = a.kn ? a.kn : a.wpad + HD;
        const float4 wq = ((const float4*)qn)[t];
        float4 wk = ((const float4*)kn)[t];
        float4 c2 = c, wq2 = wq;
        pin(c2);
        pin(wq2);
        pin(wk);
        if (tid < H4) {
            ((float4*)s_cs)[tid] = c2;
            ((float4*)s_qn)[tid] = wq2;
            ((float4*)s_kn)[tid] = wk;
        }
    }
    __syncthreads();
    if (a.qn) {
        for (int hb = 0; hb < nheads; hb += kPrepThreads / 4) {
            const int hh = hb + (tid >> 2);
            if (hh < nheads) scale[hh] = rms_scale_ref_quad(sx + (size_t)hh * HD, HD, tid & 3);
        }
        __syncthreads();
        for (int i = tid; i < nheads * HD; i += kPrepThreads) {
            const int hh = i / HD, d = i - (i / HD) * HD;
            sx[i] = rms_apply(sx[i], scale[hh], hh < a.nh ? s_qn[d] : s_kn[d]);
        }
        __syncthreads();
    }
    for (int i = tid; i < nheads * HALF; i += kPrepThreads) {
        const int hh = i / HALF, p = i - (i / HALF) * HALF;
        int e0, e1;
        rope_pair(a.rope, p, HD, e0, e1);
        float* x = sx + (size_t)hh * HD;
        rope_rotate(x[e0], x[e1], s_cs[p], s_cs[HALF + p]);
    }
    __syncthreads();
    // K and V rows in the reference fp16 rounding, four elements per thread-step
    const int nkv4 = (int)(kv_dim / 4);
    const float4* v4 = (const float4*)(a.v + tok * kv_dim);
    uint2* krow = (uint2*)(a.kc + (size_t)pos * kv_dim);
    uint2* vrow = (uint2*)(a.vc + (size_t)pos * kv_dim);
    for (int i = tid; i < nkv4; i += kPrepThreads) {
        const float4 vv = v4[i];
        const float4 kk = ((const float4*)(sx + q_dim))[i];
        krow[i] = uint2{(uint32_t)f32_to_f16_ref(kk.x) | ((uint32_t)f32_to_f16_ref(kk.y) << 16),
                        (uint32_t)f32_to_f16_ref(kk.z) | ((uint32_t)f32_to_f16_ref(kk.w) << 16)};
        vrow[i] = uint2{(uint32_t)f32_to_f16_ref(vv.x) | ((uint32_t)f32_to_f16_ref(vv.y) << 16),
                        (uint32_t)f32_to_f16_ref(vv.z) | ((uint32_t)f32_to_f16_ref(vv.w) << 16)};
    }
    _Float16* qrow = a.q16 + tok * q_dim;
    _Float16* qlo = a.q16_lo ? a.q16_lo + tok * q_dim : nullptr;
    for (int i = tid; i < nq4; i += kPrepThreads) {
        const float4 x4 = ((const float4*)sx)[i];
        const float xs[4] = {x4.x * a.qscale, x4.y * a.qscale, x4.z * a.qscale, x4.w * a.qscale};
        half4 hi, lo;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            hi[e] = (_Float16)xs[e];
            lo[e] = (_Float16)(xs[e] - (float)hi[e]);
        }
        ((half4*)qrow)[i] = hi;
        if (qlo) ((half4*)qlo)[i] = lo;
    }
}

struct AttnArgs {
    const _Float16* q16;
    const _Float16* q16_lo;  // used when SPLITQ
    const uint16_t* kc;
    const uint16_t* vc;
    float* out;
    int start, n_tok, nh, g, n_kv, kv_dim, rows, nblk;
};

constexpr int kAttnThreads = 256;
constexpr int kRowsPerBlock = 128;
constexpr int kKeysPerTile = 64;

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
    const int w = tid >> 6;
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

    const uint16_t* kbase = a.kc + (size_t)kvh * HD;
    const uint16_t* vbase = a.vc + (size_t)kvh * HD;

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

    // direct global -> LDS loads of tile kt into buffer buf (each wave its share)
    auto issue = [&](int kt, int buf) {
        const int key0 = kt * kKeysPerTile;
#pragma unroll
        for (int i = 0; i < T::NI; i++) {
            const int inst = w * T::NI + i;
            const int r = inst * T::RPI + lane / T::CH;
            const int p = lane % T::CH;
            const size_t row = (size_t)min(key0 + r, kend - 1) * a.kv_dim;
            const uint16_t* gk = kbase + row + 8 * (p ^ T::swz_k(r));
            const uint16_t* gv = vbase + row + 8 * (p ^ T::swz_v(r));
            __builtin_amdgcn_global_load_lds((const void*)gk, (__attribute__((address_space(3))) void*)&lds[buf][0][inst * 1024],
                                             16, 0, 0);
            __builtin_amdgcn_global_load_lds((const void*)gv, (__attribute__((address_space(3))) void*)&lds[buf][1][inst * 1024],
                                             16, 0, 0);
        }
    };

    issue(0, 0);

    half8 qf[QK], qfl[SPLITQ ? QK : 1];
    {
        const size_t qoff = ((size_t)tok * a.nh + hq) * HD + 8 * hk;
#pragma unroll
        for (int ks = 0; ks < QK; ks++) {
            const u32x4 raw = rvalid ? *(const u32x4*)(a.q16 + qoff + 16 * ks) : u32x4{0u, 0u, 0u, 0u};
            qf[ks] = __builtin_bit_cast(half8, raw);
            if constexpr (SPLITQ) {
                const u32x4 rl = rvalid ? *(const u32x4*)(a.q16_lo + qoff + 16 * ks) : u32x4{0u, 0u, 0u, 0u};
                qfl[ks] = __builtin_bit_cast(half8, rl);
            }
        }
    }

    float m_run = NEG_INF, l_run = 0.0f;
    floatx16 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] = 0.0f;

    // transposed-read geometry of this lane (see the V layout above)
    const int j16 = lane & 15, g16 = lane >> 4;
    const int tr_e = j16 >> 2, tr_q = j16 & 3;

    for (int kt = 0; kt < ntiles; kt++) {
        const int buf = kt & 1;
        const int key0 = kt * kKeysPerTile;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's loads of tile kt
        __syncthreads();                                   // everyone's; buffer buf^1 is free
        if (kt + 1 < ntiles) issue(kt + 1, buf ^ 1);
        if (key0 >= kend_w) continue;  // wave-uniform: every row of this wave is done

        const char* kt_lds = lds[buf][0];
        const char* vt_lds = lds[buf][1];
        floatx16 sacc[2];
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++) {
#pragma unroll
            for (int r = 0; r < 16; r++) sacc[t2][r] = 0.0f;
            const int row = 32 * t2 + col;
#pragma unroll
            for (int ks = 0; ks < QK; ks++) {
                const int c = 2 * ks + hk;
                const half8 kf = *(const half8*)(kt_lds + row * T::ROWB + 16 * (c ^ T::swz_k(row)));
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
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float corr = fast_exp2(m_run - m_new);
        m_run = m_new;
        float psum = 0.0f;
        half8 pf[4];
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float p = fast_exp2(sacc[t2][r] - m_new);
                psum += p;
                pf[2 * t2 + (r >> 3)][r & 7] = (_Float16)p;
            }
        l_run = l_run * corr + psum;
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[dt][r] *= corr;
#pragma unroll
        for (int s = 0; s < 4; s++) {
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                half4 part[2];
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const int row = 16 * s + 8 * t + 4 * hk + tr_e;
                    const int dim = 32 * dt + 16 * (g16 & 1) + 4 * tr_q;
                    const int c = dim >> 3;
                    const char* adr = vt_lds + row * T::ROWB + 16 * (c ^ T::swz_v(row)) + 2 * (dim & 7);
                    const short4v raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) short4v*)adr);
                    part[t] = __builtin_bit_cast(half4, raw);
                }
                const half8 vf = {part[0][0], part[0][1], part[0][2], part[0][3],
                                  part[1][0], part[1][1], part[1][2], part[1][3]};
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[s], o[dt], 0, 0, 0);
            }
        }
    }
    const float l_tot = l_run + __shfl_xor(l_run, 32);
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
    PrepArgs p;
    p.q = q;
    p.k = k;
    p.v = v;
    const bool norm = ctx->has_qk_norm[layer] != 0;
    p.qn = norm ? ctx->qk_norm + (size_t)layer * 2 * HD : nullptr;
    p.kn = norm ? ctx->qk_norm + (size_t)layer * 2 * HD + HD : nullptr;
    p.wpad = ctx->qk_norm;
    p.cos_tab = ctx->rope_cos;
    p.sin_tab = ctx->rope_sin;
    p.kc = ctx->key_cache + (size_t)layer * ctx->layer_elems;
    p.vc = ctx->val_cache + (size_t)layer * ctx->layer_elems;
    const bool splitq = ctx->prefill_split_q != 0;
    p.q16 = ctx->q16;
    p.q16_lo = splitq ? ctx->q16 + (size_t)n_tok * ctx->q_dim : nullptr;
    p.start = start;
    p.nh = ctx->n_heads;
    p.nkv = ctx->n_kv_heads;
    p.rope = ctx->rope_style;
    p.qscale = 1.4426950408889634f / sqrtf((float)HD);
    const int nheads = ctx->n_heads + ctx->n_kv_heads;
    const size_t shm = ((size_t)nheads * HD + ((nheads + 3) & ~3) + 2 * HD + HD) * sizeof(float);
    hipLaunchKernelGGL(prefill_prep_kernel<HD>, dim3(n_tok), dim3(kPrepThreads), shm, ctx->stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;

    AttnArgs a;
    a.q16 = ctx->q16;
    a.q16_lo = p.q16_lo;
    a.kc = p.kc;
    a.vc = p.vc;
    a.out = out;
    a.start = start;
    a.n_tok = n_tok;
    a.nh = ctx->n_heads;
    a.g = ctx->kv_mul;
    a.n_kv = ctx->n_kv_heads;
    a.kv_dim = (int)ctx->kv_dim;
    a.rows = n_tok * ctx->kv_mul;
    a.nblk = (a.rows + kRowsPerBlock - 1) / kRowsPerBlock;
    dim3 grid(a.nblk * ctx->n_kv_heads);
    if (splitq) hipLaunchKernelGGL((prefill_attn_kernel<HD, true>), grid, dim3(kAttnThreads), 0, ctx->stream, a);
    else hipLaunchKernelGGL((prefill_attn_kernel<HD, false>), grid, dim3(kAttnThreads), 0, ctx->stream, a);
    return hipGetLastError();
}

hipError_t launch_prefill(pqa_ctx* ctx, int layer, int start, int n_tok, const float* q,
                          const float* k, const float* v, float* out) {
    if (ctx->head_dim == 64) return launch_prefill_hd<64>(ctx, layer, start, n_tok, q, k, v, out);
    if (ctx->head_dim == 128) return launch_prefill_hd<128>(ctx, layer, start, n_tok, q, k, v, out);
    return hipErrorInvalidValue;
}

}  // namespace pqa
