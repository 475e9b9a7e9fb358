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
// The last split also owns the new row: one of its waves (see XW and LW
// below) applies the QK-norm and RoPE, rounds K and V to fp16 with the
// reference's rounding, stores them at row pos and adds that row's softmax
// term itself, so no workgroup reads a row written in the same launch.
//
// Inside a wave, per 16-row tile:
//   scores  S[16 rows][16 cols] = K_tile x Q^T on v_mfma_f32_16x16x32_f16;
//           q is split into fp16 hi + lo parts (two MFMAs into one fp32
//           accumulator) so scores keep fp32 precision; 1/sqrt(hd) and
//           log2(e) are folded into q.
//   softmax each 16-lane group keeps its own running max / sum per head over
//           the 4 rows of every tile that land in its registers; exp2; the
//           accumulator is rescaled only when a maximum moves.
//   PV      whole-row workgroups (HBM-bound): VALU FMA; the same lane group
//           loads those 4 V rows, each lane 8 head dims (HD/8 lanes per row),
//           and accumulates p[row][h] * v for the G heads; p comes from lane h
//           of the group by a DPP row broadcast.
//           per-column workgroups (short histories, latency-bound): MFMA, see
//           PVM below.
// Lane groups are merged once per wave, waves of a column once per workgroup
// (log-sum-exp weights); the workgroup writes the output (one split) or its
// partial (max, sum, acc) per head, and decode_combine_kernel merges splits.
#include <algorithm>
#include <mutex>
#include <string>
#include <type_traits>

#include "pqa_device.h"
#include "pqa_internal.h"

namespace pqa {

// Split partials of pqa_decode_noalloc: a file-scope device array, so that
// entry point allocates nothing. Every GPU the library runs on holds its own
// copy at its own address until the process ends. In host code `scratch` only
// names the symbol: its device address comes from hipGetSymbolAddress, once
// per device (scratch_init, called by pqa_create with that device current),
// and only that address is passed to kernels. Every pqa_decode_noalloc call on
// one GPU shares the array, so calls that overlap on one GPU (two streams,
// two threads) race. Nothing in it needs to start at zero: each split writes
// its whole partial before the combine launch reads it, and the combine reads
// only the splits of its own call.
constexpr size_t kScratchBytes = size_t(8) << 20;
constexpr int kScratchDevices = 64;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
static std::mutex g_scratch_mu;
static float* g_scratch_ptr[kScratchDevices] = {};

int scratch_init(int device) {
    if (device < 0 || device >= kScratchDevices)
        return set_err(nullptr, PQA_ERR_UNSUPPORTED, "pqa_create: device index above 63");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device]) return PQA_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return set_err(nullptr, PQA_ERR_HIP,
                       std::string("pqa_create: hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[device] = (float*)p;
    return PQA_OK;
}

// Phase stamps, compiled in only with -DPQA_PHASE_STAMPS (the build's
// stamps=True variant, libpqa_stamps.so; bench.py --phase-stamps reads them):
// s_memrealtime (a 100 MHz counter) at the phase boundaries of every wave,
// kStampSlots per workgroup, read back by pqa_decode_stamps_read.
constexpr int kStampSlots = 64;
constexpr int kStampWGs = 4096;
enum : int {
    kStStart = 0,      // workgroup start (thread 0)
    kStIssued = 1,     // + wave (up to 9 waves): prologue loads issued
    kStQReady = 10,    // + wave: q normalised, rotated and in LDS
    kStLoop0 = 19,     // + wave: history loop starts
    kStLoop1 = 28,     // + wave: history loop done
    kStMerge = 37,     // workgroup merge starts (after the barrier)
    kStEnd = 38,       // outputs stored
    kStNewRow0 = 39,   // the writer wave starts the new row
    kStNewRow1 = 40,   // the writer wave has its score and V
};
#ifdef PQA_PHASE_STAMPS
static __device__ unsigned long long g_decode_stamps[kStampWGs * kStampSlots];
#define PQA_STAMP(slot, cond)                                                                          \
    do {                                                                                               \
        const unsigned wg_ = blockIdx.y * gridDim.x + blockIdx.x;                                      \
        if ((cond) && wg_ < (unsigned)kStampWGs)                                                       \
            g_decode_stamps[(size_t)wg_ * kStampSlots + (slot)] = __builtin_amdgcn_s_memrealtime();    \
    } while (0)
#else
#define PQA_STAMP(slot, cond) \
    do {                      \
    } while (0)
#endif

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
    int cpw;    // columns per workgroup: 8 (whole cache rows) or 1 (short histories)
    float qscale;
};

constexpr int kDecodeWaves = 8;
constexpr int kDecodeTiles = 2;  // whole-row workgroups: 16-row K/V tiles in flight per wave
constexpr int kCombineThreads = 256;
constexpr int kCombineDims = 16;  // head dims per combine workgroup (HD / 16 workgroups per head)
constexpr int kMaxCombineSplits = 256;
constexpr int kSmallCombineSplits = 32;  // up to this many splits the merge runs one wave per workgroup
constexpr int kShortMaxTiles = 4;  // per-column workgroups: most tiles per wave (one split)
constexpr int kLateWriter = 3;     // per-column workgroups: the history wave that adds the new row last

// PVM: PV on MFMA (v_mfma_f32_16x16x16_f16). The score tile S[row][head] that
// the score MFMA leaves in lane (g, n), registers r = rows 4g + r of head n, is
// exactly the B operand P[rows 4g..4g+3][head n] of the 16x16x16 product
// O^T[dim][head] += V^T[dim][row] P[row][head]; V^T comes from a wave-private
// LDS copy of the tile by transposing reads (ds_read_b64_tr_b16). The softmax
// max then has to be common to the four lane groups (one max per head and
// tile), and each wave's O is complete: no lane-group merge after the loop.
// NT: 16-row tiles in flight per wave. PF: the loop requests the tiles of its
// next iteration (without it each wave runs one iteration of NT tiles).
// XW: a ninth wave that only appends the new row and scores it, so no history
// wave carries that chain (single-split per-column launches of 4 tiles per
// wave, where the history waves are long enough for it to pay: C1 7.31 ->
// 6.97 us; with shorter histories the new-row wave, third on its SIMD, ends
// later than a history wave doing it would). Raising its issue priority
// (1 or 2) measured slower: it then delays the two history waves beside it.
// LW: the writer appends the new row after its own history rows, at issue
// priority 2: in per-column launches of 1 or 2 tiles per wave (including the
// owner split of long histories) history wave kLateWriter (Qwen2.5-0.5B sweep
// 7.28 -> 7.11 us; with 4 tiles per wave it measured slower than XW, C1 6.20
// -> 6.46 us), in whole-row launches the first wave of each column of the
// owner split, whose loads then start with everyone else's (C3 26.03 ->
// 25.91 us, Qwen3-1.7B at ctx 8192 13.77 -> 13.47 us, C5 unchanged).
template <bool XW>
constexpr int decode_threads() {
    return 64 * (kDecodeWaves + (XW ? 1 : 0));
}

// The fields of the q, RoPE and K/V tile addresses come first, as scalar
// arguments (packed = g | rope << 16 | QK-norm << 18): built with
// -amdgpu-kernarg-preload-count, the dispatch puts these 14 words in SGPRs
// before the first instruction; only the struct (passed by reference into
// the argument segment, never preloaded) is loaded, in one round trip at the
// start. C1 5.91 -> 5.75 us, C3 25.77 -> 25.47 us with the combine launch,
// whose arguments are all preloaded. Holding the struct's first use (where
// the compiler waits for it) back behind the q and tile loads measured
// slower: C1 6.10-6.16 us.
template <int HD, int G, bool PVM, int NT, bool PF, bool XW, bool LW>
__global__ __launch_bounds__(decode_threads<XW>()) void decode_kernel(uint16_t* kc, uint16_t* vc, const float* q,
                                                                      const float* cosr, const float* sinr, int pos,
                                                                      int rows_per_split, int kv_dim, int packed,
                                                                      const DecodeArgs args) {
    DecodeArgs a = args;
    a.kc = kc, a.vc = vc, a.q = q, a.cosr = cosr, a.sinr = sinr;
    a.pos = pos, a.rows_per_split = rows_per_split, a.kv_dim = kv_dim;
    a.g = packed & 0xFFFF, a.nchunk = (a.g + 7) >> 3, a.rope = (packed >> 16) & 3;
    const bool norm = (packed >> 18) & 1;
    static_assert(!XW || PVM, "the new-row wave serves per-column workgroups");
    static_assert(!(LW && XW), "one new-row writer");
    constexpr int NW = kDecodeWaves;  // history waves
    constexpr int NT_THREADS = decode_threads<XW>();
    constexpr int KS = HD / 32;       // MFMA k-steps over the head dim
    constexpr int LPR = HD / 8;       // lanes per V row (8 fp16 each)
    constexpr int VL = 4 * LPR / 16;  // V loads per lane per 16-row tile
    constexpr int RPG = 16 / LPR;     // V rows per lane group per load (1 for HD 128, 2 for HD 64)
    constexpr int H4 = HD / 4;        // float4s per head
    constexpr int QL = (G * H4 + 63) / 64;  // q float4 loads per lane
    constexpr int QS = HD + 4;        // padded LDS row stride of a head
    constexpr float NEG_INF = -__builtin_huge_valf();

    // Per wave: its column's q heads ([G][QS], normalised, rotated and
    // scaled), later the wave's partial accumulator; the new K row for the
    // exact norm. Per column: the new row's V and scores. Every region but
    // the last three is private to one wave.
    __shared__ __attribute__((aligned(16))) float sq[NW][G * QS];
    __shared__ __attribute__((aligned(16))) float skr[NW][HD];
    __shared__ __attribute__((aligned(16))) float s_vnew[NW][HD];
    __shared__ float s_new[NW][G];
    __shared__ float wm[NW][G];
    __shared__ float wl[NW][G];
    // PVM: one V tile per wave, rows padded by 32 B so the four rows of a
    // transposing read fall in distinct banks
    constexpr int VSTR = 2 * HD + 32;
    __shared__ __attribute__((aligned(16))) char s_vt[PVM ? NW : 1][PVM ? 16 * VSTR : 16];

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int split = blockIdx.x;
    const int ybase = PVM ? (int)blockIdx.y : (int)blockIdx.y * a.cpw;
    PQA_STAMP(kStStart, threadIdx.x == 0);
    // Per-column workgroups (PVM) have one column, so the divisions below
    // fold away there (they sit on the path to the first loads: C1 6.06 ->
    // 5.87 us); a shift-based map for whole-row workgroups measured slower
    // (Qwen3-1.7B at ctx 8192 +0.1 us).
    const int cols = PVM ? 1 : min(a.ny - ybase, a.cpw);
    const int sub = NW / cols;
    const bool active = w < cols * sub;
    const int c = active ? w % cols : 0;
    const int sb = active ? w / cols : 0;
    // the last split (split == nsplit - 1 for nsplit = max(1, ceil(pos /
    // rows_per_split)), which the launch checks), from preloaded arguments only
    const bool owner = (split + 1) * a.rows_per_split >= a.pos;
    // the wave that adds column c's new row: the new-row wave (XW), history
    // wave kLateWriter (LW, per-column workgroups), else the column's first
    // history wave (after its rows with LW, before them without)
    const bool writer = owner && (XW ? w == NW : active && sb == (LW && PVM ? kLateWriter : 0));
    // column c = (KV head, chunk of at most G query heads)
    const int kvh = PVM && a.nchunk == 1 ? ybase + c : (ybase + c) / a.nchunk;
    const int hc = ybase + c - kvh * a.nchunk;
    const int Gc = min(G, a.g - hc * G);
    const int h0 = kvh * a.g + hc * G;

    // ---------------- this wave's history rows; first tiles in flight ----------------
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
    u32x4 kt[NT][KS], vt[NT][VL];

    // ---------------- prologue, one wave per column, no workgroup barrier ----------------
    // Lane layout: float4 i = lane + 64 r of the column's q heads is
    // (head i / H4, elements 4t..4t+3), t = lane mod H4; the K and V rows of
    // the KV head use the same t, so q[h][4t..] and k[4t..] share a lane.
    const int t = lane % H4;
    float4 vq[QL];
#pragma unroll
    for (int r = 0; r < QL; r++) {
        const int hh = min((lane + 64 * r) / H4, Gc - 1);
        vq[r] = ((const float4*)(a.q + (size_t)(h0 + hh) * HD))[t];
    }
    const int ci = rope_angle_f4<HD>(a.rope, t);
    float4 cs = ((const float4*)a.cosr)[ci];
    float4 sn = ((const float4*)a.sinr)[ci];
    float4 vk = ((const float4*)(a.k + (size_t)kvh * HD))[t];
    float4 vv = ((const float4*)(a.v + (size_t)kvh * HD))[t];
    const float* qn = norm ? a.qn : a.wpad;  // loads stay unconditional without a norm
    const float* kn = norm ? a.kn : a.wpad + HD;
    float4 wq = ((const float4*)qn)[t];
    float4 wk = ((const float4*)kn)[t];
    // Per-column workgroups with history: every wave's small loads enter the
    // memory pipe before any wave's tiles; otherwise the older wave of each
    // SIMD queues its tiles ahead of the younger one's q, and the younger wave
    // starts its loop a round trip late (an execution barrier only; nothing
    // waits for the loads). C1 7.03 -> 6.82 us, Qwen2.5-0.5B sweep 8.13 ->
    // 7.80 us. Whole-row workgroups keep the old order: with it C3 measured
    // +0.35 us (their older waves lose more by the later start of their tiles
    // than the younger ones gain) and C5 +0.3 us even with the barrier
    // skipped at run time.
    if constexpr (PVM) {
        if (r1 > r0) __builtin_amdgcn_s_barrier();  // the same for every wave of the workgroup
    }
#pragma unroll
    for (int b = 0; b < NT; b++) load_tile(w0 + 16 * b, kt[b], vt[b]);
#pragma unroll
    for (int r = 0; r < QL; r++) pin(vq[r]);
    pin(vk);
    pin(vv);
    pin(wq);
    pin(wk);
    pin(cs);
    pin(sn);
    PQA_STAMP(kStIssued + (threadIdx.x >> 6), (threadIdx.x & 63) == 0);

    // The new K/V row of column c: K normed in the reference's summation
    // order (cpp/tensor.hpp:146-176: quad j sums x[j], x[j+4], ...
    // sequentially), rotated and rounded to fp16 as the reference does,
    // stored once per KV head (chunk 0); the rounded V and the row's scores
    // against the column's (normed, rotated, scaled) q heads kept for the merge.
    auto new_row = [&]() {
        if (norm) {
            float* kr = skr[XW ? 0 : w];
            if (lane < H4) ((float4*)kr)[t] = vk;
            wave_sync();
            const float sc = rms_scale_ref_quad<HD>(kr, lane & 3);
            vk = float4{rms_apply(vk.x, sc, wk.x), rms_apply(vk.y, sc, wk.y), rms_apply(vk.z, sc, wk.z),
                        rms_apply(vk.w, sc, wk.w)};
        }
        vk = rope_lanes<HD>(vk, a.rope, t, cs, sn);
        const uint16_t kb0 = f32_to_f16_ref(vk.x), kb1 = f32_to_f16_ref(vk.y);
        const uint16_t kb2 = f32_to_f16_ref(vk.z), kb3 = f32_to_f16_ref(vk.w);
        const uint16_t vb0 = f32_to_f16_ref(vv.x), vb1 = f32_to_f16_ref(vv.y);
        const uint16_t vb2 = f32_to_f16_ref(vv.z), vb3 = f32_to_f16_ref(vv.w);
        if (hc == 0 && lane < H4) {
            const size_t off = (size_t)a.pos * a.kv_dim + (size_t)kvh * HD + 4 * t;
            *(u32x2*)(a.kc + off) = u32x2{kb0 | ((uint32_t)kb1 << 16), kb2 | ((uint32_t)kb3 << 16)};
            *(u32x2*)(a.vc + off) = u32x2{vb0 | ((uint32_t)vb1 << 16), vb2 | ((uint32_t)vb3 << 16)};
        }
        if (lane < H4)
            ((float4*)s_vnew[c])[t] = float4{f16_bits_to_f32(vb0), f16_bits_to_f32(vb1), f16_bits_to_f32(vb2),
                                             f16_bits_to_f32(vb3)};
        const float k0 = f16_bits_to_f32(kb0), k1 = f16_bits_to_f32(kb1);
        const float k2 = f16_bits_to_f32(kb2), k3 = f16_bits_to_f32(kb3);
#pragma unroll
        for (int r = 0; r < QL; r++) {
            float d = vq[r].x * k0 + vq[r].y * k1 + vq[r].z * k2 + vq[r].w * k3;
            d = group_sum<H4>(d);
            const int hh = (lane + 64 * r) / H4;
            if (t == 0 && hh < Gc) s_new[c][hh] = d;
        }
        wave_sync();
    };

    float* q_lds = sq[min(w, NW - 1)];
    if (active || writer) {
        // QK-RMSNorm of q: q only feeds scores, an fp32 tree sum over the
        // head's H4 lanes.
        if (norm) {
#pragma unroll
            for (int r = 0; r < QL; r++) {
                const float ss = group_sum<H4>(vq[r].x * vq[r].x + vq[r].y * vq[r].y + vq[r].z * vq[r].z +
                                               vq[r].w * vq[r].w);
                const float sc = 1.0f / sqrtf(ss / (float)HD + 1e-6f);
                vq[r] = float4{rms_apply(vq[r].x, sc, wq.x), rms_apply(vq[r].y, sc, wq.y),
                               rms_apply(vq[r].z, sc, wq.z), rms_apply(vq[r].w, sc, wq.w)};
            }
        }
#pragma unroll
        for (int r = 0; r < QL; r++) {
            vq[r] = rope_lanes<HD>(vq[r], a.rope, t, cs, sn);
            vq[r] = float4{vq[r].x * a.qscale, vq[r].y * a.qscale, vq[r].z * a.qscale, vq[r].w * a.qscale};
        }
        wave_sync();
#pragma unroll
        for (int r = 0; r < QL; r++) {
            const int i = lane + 64 * r;
            if (active && i < Gc * H4) ((float4*)(q_lds + (i / H4) * QS))[t] = vq[r];
        }
        if (!LW && writer) {
            PQA_STAMP(kStNewRow0, lane == 0);
            new_row();
            PQA_STAMP(kStNewRow1, lane == 0);
        }
    }
    wave_sync();
    PQA_STAMP(kStQReady + (threadIdx.x >> 6), (threadIdx.x & 63) == 0);

    // ---------------- wave loop over history rows ----------------
    // Lane (g, n), g = lane/16, n = lane%16. The score MFMA reads K row n of the
    // tile and puts S[row 4g+i][head n] in register i of lane (g, n). The same
    // lane group g also loads V rows 4g..4g+3, so each group runs its own
    // online softmax over its rows: no cross-group traffic per tile.
    half8 qh[KS], ql[KS];
    {
        const float* qrow = q_lds + min(n, Gc - 1) * QS + 8 * grp;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const float4 x0 = *(const float4*)(qrow + 32 * ks);
            const float4 x1 = *(const float4*)(qrow + 32 * ks + 4);
            const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float xv = n < Gc ? x[e] : 0.0f;
                const _Float16 hi = (_Float16)xv;
                qh[ks][e] = hi;
                ql[ks][e] = (_Float16)(xv - (float)hi);
            }
        }
    }
    wave_sync();  // q_lds is reused below for the wave partial
    PQA_STAMP(kStLoop0 + (threadIdx.x >> 6), (threadIdx.x & 63) == 0);

    float m_run = NEG_INF;
    float l_run = 0.0f;
    constexpr int AG = PVM ? 1 : G;
    float acc[AG][8];
#pragma unroll
    for (int h = 0; h < AG; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[h][e] = 0.0f;
    constexpr int NM = HD / 16;  // PVM: 16-dim blocks of O^T
    floatx4 o[PVM ? NM : 1];
#pragma unroll
    for (int m = 0; m < (PVM ? NM : 1); m++) o[m] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    // PVM: this lane's V row pieces in the staged tile, and its transposing-read
    // address (row 4 grp + n / 4, dims 4 (n % 4) .. +3 of each 16-dim block)
    char* vst = s_vt[PVM ? w : 0];
    const int tr_off = (4 * grp + (n >> 2)) * VSTR + 8 * (n & 3);

    if (w0 < w1) {
        auto scores = [&](int tb, const u32x4 (&kf)[KS], float (&s)[4]) {
            floatx4 S = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const half8 kh = __builtin_bit_cast(half8, kf[ks]);
                S = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[ks], S, 0, 0, 0);
                S = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[ks], S, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) s[i] = (tb + 4 * grp + i < w1 && n < Gc) ? S[i] : NEG_INF;
        };
        auto process = [&](int tb, const u32x4 (&kf)[KS], const u32x4 (&vf)[VL]) {
            float s[4];
            scores(tb, kf, s);
            if constexpr (PVM) {
                // stage the V tile (the previous tile's reads are done: one
                // wave's LDS accesses execute in order)
#pragma unroll
                for (int j = 0; j < VL; j++)
                    *(u32x4*)(vst + (4 * grp + vsub + RPG * j) * VSTR + 2 * vdim) = vf[j];
                // one max per head and tile: the four lane groups of head n
                const float mx = max_x32(max_x16(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]))));
                const float m_new = fmaxf(m_run, mx);
                const bool moved = m_new > m_run;
                if (__any(moved)) {
                    const float corr = moved ? fast_exp2(m_run - m_new) : 1.0f;
                    l_run *= corr;
                    m_run = m_new;
#pragma unroll
                    for (int m = 0; m < NM; m++) o[m] *= corr;
                }
                half4 pb;
                float ls = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const _Float16 ph = (_Float16)(s[i] == NEG_INF ? 0.0f : fast_exp2(s[i] - m_run));
                    pb[i] = ph;
                    ls += (float)ph;  // the weights the product uses
                }
                l_run += ls;
                wave_sync();
#pragma unroll
                for (int m = 0; m < NM; m++) {
                    const short4v raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) short4v*)(vst + tr_off + 32 * m));
                    o[m] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4, raw), pb, o[m], 0, 0, 0);
                }
                wave_sync();
            } else {
                const float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
                const float m_new = fmaxf(m_run, mx);
                const bool moved = m_new > m_run;
                if (__any(moved)) {
                    const float corr = moved ? fast_exp2(m_run - m_new) : 1.0f;
                    l_run *= corr;
                    m_run = m_new;
#pragma unroll
                    for (int h = 0; h < AG; h++) {
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
                    float pr[AG];
#pragma unroll
                    for (int h = 0; h < AG; h++) {
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
                        for (int h = 0; h < AG; h++) acc[h][e] = fmaf(pr[h], ve, acc[h][e]);
                    }
                }
            }
        };
        // Straight-line body: a tile past w1 (the second of the last pair) is
        // processed fully masked (its rows are clamped loads, its scores -inf,
        // so p = 0). A `break` here would give the compiler a path on which
        // tile b's loads are the newest, and its load waits would then drain
        // every tile in flight.
        // Per-column workgroups (short histories): the younger wave of each
        // SIMD (w >= 4) takes issue priority for its tiles, which the
        // older-first order would otherwise leave for last (C1 12.2 -> 11.7 us).
        // Whole-row workgroups measured slower with it and keep the default.
        if (a.cpw == 1 && w >= 4) __builtin_amdgcn_s_setprio(1);
        for (int tb = w0; tb < w1; tb += 16 * NT) {
#pragma unroll
            for (int b = 0; b < NT; b++) {
                process(tb + 16 * b, kt[b], vt[b]);
                if constexpr (PF) load_tile(tb + 16 * (b + NT), kt[b], vt[b]);
            }
        }
        __builtin_amdgcn_s_setprio(0);
    }

    PQA_STAMP(kStLoop1 + (threadIdx.x >> 6), (threadIdx.x & 63) == 0);
    if constexpr (LW) {
        // the late writer: the new row after its own history rows, at the
        // highest issue priority (the younger wave of its SIMD may still be
        // in its loop)
        if (writer) {
            PQA_STAMP(kStNewRow0, lane == 0);
            __builtin_amdgcn_s_setprio(2);
            new_row();
            __builtin_amdgcn_s_setprio(0);
            PQA_STAMP(kStNewRow1, lane == 0);
        }
    }
    // ---------------- merge the four lane groups, then write the wave partial ----------------
    // Cross-lane sums by DPP / permlane swaps: lane groups differ in lane bits
    // 4 and 5; with HD 64 the two V rows of a lane group differ in bit 3.
    if constexpr (PVM) {
        // m_run is already common to the lane groups and O^T complete: sum l,
        // store lane (g, n)'s O^T[16 m + 4 g + r][n] as head n's dims
        const float l = sum_x32(sum_x16(l_run));
        if (n < G && w < NW) {
#pragma unroll
            for (int m = 0; m < NM; m++) *(floatx4*)(q_lds + n * QS + 16 * m + 4 * grp) = o[m];
            if (grp == 0) {
                wm[w][n] = m_run;
                wl[w][n] = l;
            }
        }
    } else {
        const float M = max_x32(max_x16(m_run));
        const float e = (m_run == NEG_INF) ? 0.0f : fast_exp2(m_run - M);
        const float l = sum_x32(sum_x16(l_run * e));
        // The 8 dims of a lane are summed over the four lane groups by a
        // reduce-scatter: permlane32_swap(a, b) + its pair leaves a's sums over
        // lane ^ 32 in the lower half and b's in the upper; permlane16_swap
        // likewise over lane ^ 16 with odd and even rows. Lane group g ends
        // with dims 2 g and 2 g + 1 (6 swaps and 6 adds instead of 16 and 16).
        float2 part[AG];
#pragma unroll
        for (int h = 0; h < AG; h++) {
            const float eh = row_bcast(e, h);
            unsigned x[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                float xv = acc[h][k] * eh;
                if constexpr (RPG == 2) xv = xv + dpp_f<kDppXor8>(xv);
                x[k] = __builtin_bit_cast(unsigned, xv);
            }
            unsigned u[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const auto r = __builtin_amdgcn_permlane32_swap(x[k], x[k + 4], false, false);
                u[k] = __builtin_bit_cast(unsigned, __builtin_bit_cast(float, (unsigned)r[0]) +
                                                        __builtin_bit_cast(float, (unsigned)r[1]));
            }
            float y[2];
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const auto r = __builtin_amdgcn_permlane16_swap(u[k], u[k + 2], false, false);
                y[k] = __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
            }
            part[h] = float2{y[0], y[1]};
        }
        if (n < LPR) {
#pragma unroll
            for (int h = 0; h < AG; h++) *(float2*)(q_lds + h * QS + vdim + 2 * grp) = part[h];
        }
        if (lane < G) {
            wm[w][lane] = M;
            wl[w][lane] = l;
        }
    }
    __syncthreads();

    PQA_STAMP(kStMerge, threadIdx.x == 0);
    // ---------------- workgroup merge per column (+ the new row) ----------------
    // One float4 of head dims per thread and item: column cc (KV head yk,
    // chunk yc), head h; the column's nsub wave partials sit at waves
    // cc, cc + wstride, ...
    const int tid = threadIdx.x;
    constexpr int D4 = HD / 4;
    auto merge = [&](int cc, int h, int d4, int yk, int yc, int nsub, int wstride) {
        float M = owner ? s_new[cc][h] : NEG_INF;
        for (int s = 0; s < nsub; s++) M = fmaxf(M, wm[cc + s * wstride][h]);
        float L = 0.0f;
        floatx4 A = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int s = 0; s < nsub; s++) {
            const int wv = cc + s * wstride;
            const float e = fast_exp2(wm[wv][h] - M);
            L += e * wl[wv][h];
            A += e * *(const floatx4*)&sq[wv][h * QS + 4 * d4];
        }
        if (owner) {
            const float e = fast_exp2(s_new[cc][h] - M);
            L += e;
            A += e * *(const floatx4*)&s_vnew[cc][4 * d4];
        }
        if (a.nsplit == 1) {
            ((floatx4*)(a.out + (size_t)(yk * a.g + yc * G + h) * HD))[d4] = A * (1.0f / L);
        } else {
            const size_t pb = ((size_t)(ybase + cc) * a.nsplit + split) * G + h;
            ((floatx4*)(a.part_acc + pb * HD))[d4] = A;
            if (d4 == 0) *(float2*)(a.part_ml + pb * 2) = float2{M, L};
        }
    };
    if constexpr (PVM) {
        // Per-column workgroups: one column, its NW history waves in order,
        // counts known at compile time, so every LDS read of an item is
        // issued before the first is used; at most 256 items, one per thread.
        static_assert(G * D4 <= NT_THREADS, "one merge item per thread");
        if (tid < Gc * D4) merge(0, tid / D4, tid % D4, kvh, hc, NW, 1);
    } else {
        // Whole-row workgroups: the usual 8 or 4 columns (1 or 2 waves each)
        // get compile-time counts too; any other count takes the general loop.
        auto items = [&](auto ncol) {
            constexpr int NC = decltype(ncol)::value;
            const int nc = NC ? NC : cols;
            const int ns = NC ? NW / NC : sub;
            for (int i = tid; i < nc * G * D4; i += NT_THREADS) {
                const int cc = i / (G * D4), h = (i / D4) - cc * G, d4 = i - (i / D4) * D4;
                const int yk = a.nchunk == 1 ? ybase + cc : (ybase + cc) / a.nchunk;
                const int yc = ybase + cc - yk * a.nchunk;
                if (h >= min(G, a.g - yc * G)) continue;
                merge(cc, h, d4, yk, yc, ns, nc);
            }
        };
        if (cols == 8) items(std::integral_constant<int, 8>{});
        else if (cols == 4) items(std::integral_constant<int, 4>{});
        else items(std::integral_constant<int, 0>{});
    }
#ifdef PQA_PHASE_STAMPS
    __syncthreads();  // the stamped build only: every output stored before the end stamp
#endif
    PQA_STAMP(kStEnd, threadIdx.x == 0);
}

// Merge of the split partials of one column: workgroup (head h, column y,
// 16-dim slice). Thread (split group sg = tid / 4, float4 d4 = tid % 4) loads
// the slice of splits sg, sg + 64, ... (at most 256 splits: one batch), and
// thread tid the (max, sum) of split tid, all in one round trip. The launch is
// one memory round trip deep, so more, narrower workgroups finish sooner
// (16-dim slices: 0.25 us less per call than 32 at 256 splits).
// M = max_s m_s, w_s = exp2(m_s - M), out = sum_s w_s acc_s / sum_s w_s l_s.
// A separate launch: the kernel boundary makes every partial visible, so the
// split workgroups need no fences or atomics.
template <int HD>
__global__ __launch_bounds__(kCombineThreads) void decode_combine_kernel(const float* __restrict__ part_acc,
                                                                         const float* __restrict__ part_ml,
                                                                         float* __restrict__ out, int G, int g,
                                                                         int nchunk, int nsplit) {
    constexpr int D4 = kCombineDims / 4;         // float4s per slice
    constexpr int SG = kCombineThreads / D4;     // split groups
    constexpr int U = kMaxCombineSplits / SG;    // splits per thread
    constexpr int NWV = kCombineThreads / 64;
    constexpr float NEG_INF = -__builtin_huge_valf();
    __shared__ float s_w[kMaxCombineSplits];
    __shared__ float s_red[2][NWV];
    __shared__ __attribute__((aligned(16))) floatx4 s_acc[NWV][D4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int h = blockIdx.x, y = blockIdx.y, dslice = blockIdx.z;
    const int kvh = y / nchunk, hc = y - kvh * nchunk;
    const int Gc = min(G, g - hc * G);
    if (h >= Gc) return;
    const float* pml = part_ml + ((size_t)y * nsplit * G + h) * 2;
    const int d4 = tid % D4, sg = tid / D4;
    const floatx4* src = (const floatx4*)(part_acc + ((size_t)y * nsplit * G + h) * HD + kCombineDims * dslice) + d4;
    const size_t sstride = (size_t)G * HD / 4;

    const int ts = min(tid, nsplit - 1);
    const float2 ml = *(const float2*)(pml + (size_t)ts * G * 2);
    floatx4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = src[(size_t)min(sg + u * SG, nsplit - 1) * sstride];
    const float mloc = tid < nsplit ? ml.x : NEG_INF;
    float M = group_max<64>(mloc);
    if (lane == 0) s_red[0][w] = M;
    __syncthreads();
    M = s_red[0][0];
#pragma unroll
    for (int i = 1; i < NWV; i++) M = fmaxf(M, s_red[0][i]);
    float wl = 0.0f;
    if (tid < nsplit) {
        const float wt = fast_exp2(mloc - M);
        s_w[tid] = wt;
        wl = wt * ml.y;
    }
    wl = group_sum<64>(wl);
    if (lane == 0) s_red[1][w] = wl;
    __syncthreads();
    float L = 0.0f;
#pragma unroll
    for (int i = 0; i < NWV; i++) L += s_red[1][i];
    floatx4 A = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < U; u++)
        if (sg + u * SG < nsplit) A += s_w[sg + u * SG] * v[u];
    // sum over the split groups of the wave (lane bits 2..5), then over waves:
    // lanes i, i+4, i+8, i+12 of each 16-lane row, then the rows
    static_assert(D4 == 4, "the cross-lane sum below covers lane bits 2..5");
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float x = A[k];
        x = x + dpp_f<kDppRor4>(x);
        x = x + dpp_f<kDppXor8>(x);
        A[k] = sum_x32(sum_x16(x));
    }
    if (lane < D4) s_acc[w][lane] = A;
    __syncthreads();
    if (tid < D4) {
        floatx4 r = s_acc[0][tid];
#pragma unroll
        for (int q = 1; q < NWV; q++) r += s_acc[q][tid];
        const float inv = 1.0f / L;
        ((floatx4*)(out + (size_t)(kvh * g + hc * G + h) * HD + kCombineDims * dslice))[tid] = r * inv;
    }
}

// The same merge for at most kSmallCombineSplits splits (the per-column
// launches of short histories): one wave per (head, column, 16-dim slice),
// lane (split group sg = lane / 4, float4 d4 = lane % 4) on splits sg and
// sg + 16, lane s on the (max, sum) of split s; every reduction stays in the
// wave, with no LDS and no barrier.
template <int HD>
__global__ __launch_bounds__(64) void decode_combine_wave_kernel(const float* __restrict__ part_acc,
                                                                 const float* __restrict__ part_ml,
                                                                 float* __restrict__ out, int G, int g, int nchunk,
                                                                 int nsplit) {
    constexpr int D4 = kCombineDims / 4;           // float4s per slice
    constexpr int SG = 64 / D4;                    // split groups
    constexpr int U = kSmallCombineSplits / SG;    // splits per lane
    constexpr float NEG_INF = -__builtin_huge_valf();
    static_assert(kSmallCombineSplits <= 64, "one lane per split for the (max, sum) pairs");
    const int lane = threadIdx.x;
    const int h = blockIdx.x, y = blockIdx.y, dslice = blockIdx.z;
    const int kvh = y / nchunk, hc = y - kvh * nchunk;
    const int Gc = min(G, g - hc * G);
    if (h >= Gc) return;
    const float* pml = part_ml + ((size_t)y * nsplit * G + h) * 2;
    const int d4 = lane % D4, sg = lane / D4;
    const floatx4* src = (const floatx4*)(part_acc + ((size_t)y * nsplit * G + h) * HD + kCombineDims * dslice) + d4;
    const size_t sstride = (size_t)G * HD / 4;

    const float2 ml = *(const float2*)(pml + (size_t)min(lane, nsplit - 1) * G * 2);
    floatx4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = src[(size_t)min(sg + u * SG, nsplit - 1) * sstride];
    const float mloc = lane < nsplit ? ml.x : NEG_INF;
    const float M = group_max<64>(mloc);
    const float wt = lane < nsplit ? fast_exp2(mloc - M) : 0.0f;
    const float L = group_sum<64>(wt * ml.y);
    floatx4 A = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < U; u++) {
        const float ws = __shfl(wt, sg + u * SG);
        if (sg + u * SG < nsplit) A += ws * v[u];
    }
    // sum over the split groups (lane bits 2..5), as in decode_combine_kernel
    static_assert(D4 == 4, "the cross-lane sum below covers lane bits 2..5");
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float x = A[k];
        x = x + dpp_f<kDppRor4>(x);
        x = x + dpp_f<kDppXor8>(x);
        A[k] = sum_x32(sum_x16(x));
    }
    if (lane < D4)
        ((floatx4*)(out + (size_t)(kvh * g + hc * G + h) * HD + kCombineDims * dslice))[lane] = A * (1.0f / L);
}

void decode_split(const pqa_ctx* ctx, int hist, int max_splits, int* rows_per_split, int* nsplit, int* cols_per_wg,
                  int* tiles) {
    const int ny = ctx->n_kv_heads * ctx->n_chunk;
    if (ctx->split_override <= 0) {
        // Short histories: one workgroup per column and split. Up to 8 x 64
        // rows the column is one split with 1, 2 or 4 tiles per wave, and the
        // launch writes the output itself: no combine launch (C1 8.7 -> 7.3
        // us). Four tiles go two in flight, two iterations: all four requested
        // in the prologue measured 0.5 us slower at C1. Longer histories take
        // one tile per wave, requested in the prologue, and splits merged by
        // the combine launch (64 rows per wave there measured 10.5 against
        // 9.1 us per layer over Qwen2.5-0.5B at ctx 1024-4096); used while
        // these workgroups fill at most a quarter of the CUs.
        if (hist <= kDecodeWaves * 16 * kShortMaxTiles) {
            const int need = (hist + kDecodeWaves * 16 - 1) / (kDecodeWaves * 16);
            const int nt = need <= 1 ? 1 : need <= 2 ? 2 : 4;
            *rows_per_split = kDecodeWaves * 16 * nt;
            *nsplit = 1;
            *cols_per_wg = 1;
            *tiles = nt;
            return;
        }
        const int rps = kDecodeWaves * 16;
        const int ns = std::max(1, (hist + rps - 1) / rps);
        if (ns * ny <= ctx->cu_count / 4 && ns <= std::min(kMaxCombineSplits, max_splits)) {
            *rows_per_split = rps;
            *nsplit = ns;
            *cols_per_wg = 1;
            *tiles = 1;
            return;
        }
    }
    // Whole cache rows: a workgroup of 8 waves serves up to 8 columns, and
    // each wave should own at least one whole 16-row tile. Columns of at most
    // two query heads go 4 to a workgroup, two waves each: the same rows per
    // wave, half the splits, so half the partials for the combine launch
    // (C3 -0.35 us, Qwen3-1.7B at ctx 8192 -1.7 us; wider columns measured
    // slower this way).
    const int cols = std::min(ny, ctx->chunk_heads <= 2 ? kDecodeWaves / 2 : kDecodeWaves);
    const int quantum = 16 * (kDecodeWaves / cols);
    int rps;
    if (ctx->split_override > 0) {
        rps = ctx->split_override;
    } else {
        // About one workgroup (8 waves) per CU; a workgroup reads the cache
        // rows of all its columns.
        const int groups = (ny + cols - 1) / cols;
        const int target = std::max(1, ctx->cu_count / groups);
        rps = (hist + target - 1) / target;
        rps = std::max(quantum, (rps + quantum - 1) / quantum * quantum);
    }
    int ns = std::max(1, (hist + rps - 1) / rps);
    while (ns > max_splits) {
        rps += quantum;
        ns = std::max(1, (hist + rps - 1) / rps);
    }
    *rows_per_split = rps;
    *nsplit = ns;
    *cols_per_wg = cols;
    *tiles = kDecodeTiles;
}

int scratch_workspace(pqa_ctx* ctx, DecodeWorkspace* ws, const char* fn) {
    float* base = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (ctx->device >= 0 && ctx->device < kScratchDevices) base = g_scratch_ptr[ctx->device];
    }
    if (!base) return set_err(ctx, PQA_ERR_HIP, std::string(fn) + ": no scratch address for this device");
    // As many splits as fit: each takes ny * G * (hd + 2) floats. Fewer splits
    // than pqa_decode may use only lengthen each split's row range; when not
    // even two splits' partials fit, every call runs as one split, which
    // writes the output directly and needs no scratch (slow for long
    // histories, but never refused).
    const size_t ny = (size_t)ctx->n_kv_heads * ctx->n_chunk;
    const size_t per_split = ny * ctx->chunk_heads * (ctx->head_dim + 2);
    const size_t fit = kScratchBytes / sizeof(float) / per_split;
    ws->max_splits = fit < 2 ? 1 : (int)std::min<size_t>(fit, (size_t)ctx->max_splits);
    ws->part_acc = base;
    ws->part_ml = base + ny * ws->max_splits * ctx->chunk_heads * ctx->head_dim;
    return PQA_OK;
}

// PV on MFMA for the per-column workgroups of short histories (7-8 query
// heads per column made the VALU PV the bound there), with 1, 2 or 4 tiles per
// wave (4: two in flight, two iterations); whole-row workgroups stream HBM and
// keep the VALU PV.
template <int HD, bool PVM, int NT, bool PF, bool XW = false, bool LW = false>
static hipError_t launch_decode_pv(const DecodeArgs& a, int G, dim3 grid, hipStream_t st) {
    // the packed argument word, and the chunk count the kernel derives from g
    // and the owner split the kernel derives from pos and rows_per_split
    if (a.g < 1 || a.g > 0xFFFF || a.rope < 0 || a.rope > 3 || a.nchunk != (a.g + 7) / 8) return hipErrorInvalidValue;
    if (a.rows_per_split < 1 || a.nsplit != std::max(1, (a.pos + a.rows_per_split - 1) / a.rows_per_split))
        return hipErrorInvalidValue;
    switch (G) {
#define PQA_CASE(GG) \
    case GG:                                                                                                   \
        hipLaunchKernelGGL((decode_kernel<HD, GG, PVM, NT, PF, XW, LW>), grid, dim3(decode_threads<XW>()), 0, st, \
                           a.kc, a.vc, a.q, a.cosr, a.sinr, a.pos, a.rows_per_split, a.kv_dim,                  \
                           a.g | (a.rope << 16) | (a.qn ? 1 << 18 : 0), a);                                      \
        break;
        PQA_CASE(1) PQA_CASE(2) PQA_CASE(3) PQA_CASE(4) PQA_CASE(5) PQA_CASE(6) PQA_CASE(7) PQA_CASE(8)
#undef PQA_CASE
        default: return hipErrorInvalidValue;
    }
    return hipSuccess;
}

template <int HD>
static hipError_t launch_decode_hd(const DecodeArgs& a, int G, int tiles, dim3 grid, hipStream_t st) {
    hipError_t le = hipErrorInvalidValue;
    if (a.cpw != 1) le = launch_decode_pv<HD, false, kDecodeTiles, true, false, true>(a, G, grid, st);
    else if (tiles == 1) le = launch_decode_pv<HD, true, 1, false, false, true>(a, G, grid, st);
    else if (tiles == 2) le = launch_decode_pv<HD, true, 2, false, false, true>(a, G, grid, st);
    else if (tiles == 4) le = launch_decode_pv<HD, true, 2, true, true, false>(a, G, grid, st);  // one split
    if (le != hipSuccess) return le;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit == 1) return e;
    if (a.nsplit > kMaxCombineSplits) return hipErrorInvalidValue;
    if (a.nsplit <= kSmallCombineSplits)
        hipLaunchKernelGGL(decode_combine_wave_kernel<HD>, dim3(G, a.ny, HD / kCombineDims), dim3(64), 0, st,
                           a.part_acc, a.part_ml, a.out, G, a.g, a.nchunk, a.nsplit);
    else
        hipLaunchKernelGGL(decode_combine_kernel<HD>, dim3(G, a.ny, HD / kCombineDims), dim3(kCombineThreads), 0, st,
                       a.part_acc,
                       a.part_ml, a.out, G, a.g, a.nchunk, a.nsplit);
    return hipGetLastError();
}

#ifdef PQA_PHASE_STAMPS
// The stamped build's extra entry points (not in pqa.h): copy out / clear the
// stamps of the last decode launches; n = kStampWGs * kStampSlots values.
extern "C" int pqa_decode_stamps_read(unsigned long long* dst, int n) {
    if (!dst || n != kStampWGs * kStampSlots) return PQA_ERR_ARG;
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_decode_stamps), (size_t)n * 8, 0, hipMemcpyDeviceToHost) == hipSuccess
               ? PQA_OK
               : PQA_ERR_HIP;
}
extern "C" int pqa_decode_stamps_clear() {
    static unsigned long long zero[kStampWGs * kStampSlots];
    return hipMemcpyToSymbol(HIP_SYMBOL(g_decode_stamps), zero, sizeof(zero), 0, hipMemcpyHostToDevice) == hipSuccess
               ? PQA_OK
               : PQA_ERR_HIP;
}
#endif

hipError_t launch_decode(pqa_ctx* ctx, int layer, int pos, const float* q, const float* k,
                         const float* v, float* out, const DecodeWorkspace& ws) {
    if (!mfma_head_dim(ctx->head_dim)) return launch_decode_general(ctx, layer, pos, q, k, v, out, ws);
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
    a.part_acc = ws.part_acc;
    a.part_ml = ws.part_ml;
    a.pos = pos;
    a.g = ctx->kv_mul;
    a.nchunk = ctx->n_chunk;
    a.ny = ctx->n_kv_heads * ctx->n_chunk;
    a.rope = ctx->rope_style;
    a.kv_dim = (int)ctx->kv_dim;
    int tiles = kDecodeTiles;
    decode_split(ctx, pos, ws.max_splits, &a.rows_per_split, &a.nsplit, &a.cpw, &tiles);
    // One split writes the output itself; several write partials that
    // decode_combine_kernel merges in a second launch.
    a.qscale = 1.4426950408889634f / sqrtf((float)hd);
    dim3 grid(a.nsplit, (a.ny + a.cpw - 1) / a.cpw);
    if (hd == 64) return launch_decode_hd<64>(a, ctx->chunk_heads, tiles, grid, ctx->stream);
    if (hd == 128) return launch_decode_hd<128>(a, ctx->chunk_heads, tiles, grid, ctx->stream);
    return hipErrorInvalidValue;
}

}  // namespace pqa
