// Causal prefill of one layer: the token loop of cpp/model.hpp:493-593 as two
// launches.
//
// 1. prefill_kv: the new cache rows. One wave per 2 (token, KV head) rows:
//    K gets the QK-RMSNorm in the reference's summation order, RoPE at the
//    token's position and the reference's fp16 rounding; V the rounding
//    only. Rows start..start+n-1 of the layer slice are written.
// 2. prefill_attn: flash attention over the fp16 cache on
//    v_mfma_f32_16x16x32_f16 (on this GPU a stream of them moves 20 % more
//    MACs per second than v_mfma_f32_32x32x16_f16, with the same operand
//    traffic per tile). The query heads of one KV head are packed as
//    rows R = token*g + h (g = query heads per KV head), so one K/V tile in
//    LDS serves the whole GQA group. A workgroup of 8 waves takes a pair of
//    128-row blocks one after the other (a long and a short one, so every
//    workgroup has the same causal work). Waves w and w + 4 share a SIMD and
//    32 rows and take the even and the odd 64-key tiles; their partial
//    results are merged at the end of the block.
//    Per block: q rows are normed, rotated, scaled and rounded to fp16 into
//    LDS (each lane holds whole RoPE pairs of its row, so the rotation needs
//    no exchange). Per 64-key tile each wave computes S^T = K Q^T (keys x
//    rows) in 16x16 blocks, the online softmax per row (a lane holds 16
//    scores of each of two rows; a row's 64 scores sit in 4 lanes 16 apart),
//    and O^T += V^T P^T. With S^T in the
//    MFMA result layout the lane's scores are already the B operand of the
//    PV product, so P never leaves registers. The running maximum is raised
//    (and O, l rescaled) only when a score exceeds it by more than 2^8, so
//    most tiles skip the rescale. K/V tiles arrive by direct global->LDS
//    loads, double buffered, one barrier per tile pair; V fragments are read
//    with transposing LDS reads. Tiles past the causal limit of every row in
//    a wave are skipped. Outputs leave through LDS as whole 512-byte rows.
#include <type_traits>

#include "pqa_device.h"
#include "pqa_internal.h"

namespace pqa {

struct KvArgs {
    const float* k;  // row of token t at k + t * ld
    const float* v;
    const float* kn;       // [HD] or null
    const float* wpad;     // 2*HD readable floats, loaded in place of absent norm weights
    const float* cos_tab;  // [S][HD/2]
    const float* sin_tab;
    uint16_t* kc;  // layer slice [S][kv_dim]
    uint16_t* vc;
    int start, n_tok, nkv, rope;
    int ld;  // floats between the k (and v) rows of consecutive tokens
    // scaled inputs (YS): k = k * (kw[c] * x_inv[t]) + kb[c] for column c of
    // token t, v likewise; kb / vb may be null
    const float* kw;
    const float* vw;
    const float* x_inv;
    const uint8_t* kb;
    const uint8_t* vb;
    int kbt, vbt;
};

// y * (w * xi) + b[c .. c+3] (an exact power-of-two rescale, then vec_add,
// cpp/tensor.hpp:410-420), for 4 consecutive columns c of one token
__device__ __forceinline__ float bias_at(const uint8_t* b, int bt, int c) {
    return bt == GG_F32 ? ((const float*)b)[c] : f16_bits_to_f32(((const uint16_t*)b)[c]);
}
__device__ __forceinline__ float4 unscale4(float4 y, float4 w, float xi, const uint8_t* b, int bt, int c) {
    float4 r = float4{y.x * (w.x * xi), y.y * (w.y * xi), y.z * (w.z * xi), y.w * (w.w * xi)};
    if (b) r = float4{r.x + bias_at(b, bt, c), r.y + bias_at(b, bt, c + 1), r.z + bias_at(b, bt, c + 2),
                      r.w + bias_at(b, bt, c + 3)};
    return r;
}

constexpr int kKvThreads = 256;
// (token, KV head) rows per wave, at least one row per 16 lanes' float4s.
// Measured at Qwen3-4B shape (16384 rows): 2 -> 7.46 us, 4 -> 8.08, 8 -> 8.82,
// 16 -> 10.4 (fewer, fuller waves hide the load round trip worse).
#ifndef PQA_KV_ROWS_PER_WAVE
#define PQA_KV_ROWS_PER_WAVE 2
#endif
constexpr int kKvRowsPerWave = PQA_KV_ROWS_PER_WAVE;

// RPW rows per wave. Each lane holds NS float4s of K and of V: slot i, lane l
// -> row RPS i + l / H4 of the wave's RPW, elements 4 (l % H4) .. +3 (RPS =
// 64 / H4 rows per slot). All loads (K, V, the RoPE rows) are issued first.
// The K RMSNorm runs in the reference's order: the rows go to LDS, lane
// (r, j) = (l / 4, l % 4) sums SSE lane j of row r (rms_scale_ref_quad), and
// each lane reads back the scales of its slots' rows. RoPE partners come over
// lanes (rope_lanes), then the reference's fp16 rounding and 8-byte stores.
template <int HD>
constexpr int kv_rows_per_wave() { return kKvRowsPerWave < 256 / HD ? 256 / HD : kKvRowsPerWave; }

template <int HD, bool YS>
__global__ __launch_bounds__(kKvThreads) void prefill_kv_kernel(const KvArgs a) {
    constexpr int H4 = HD / 4;        // lanes per row
    constexpr int RPS = 64 / H4;      // rows per slot
    constexpr int RPW = kv_rows_per_wave<HD>();
    static_assert(RPW % RPS == 0 && RPW <= 16, "whole slots, at most 4 lanes per row for the norm chains");
    constexpr int NS = RPW / RPS;     // slots per lane
    constexpr int NW = kKvThreads / 64;
    constexpr int RS = HD + 4;        // LDS row stride in floats (rows r and r + 8 share banks: 2-way)
    __shared__ __attribute__((aligned(16))) float sk[NW][RPW * RS];
    __shared__ float s_scale[NW][RPW];
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int t = lane % H4, hh = lane / H4;
    const int n_items = a.n_tok * a.nkv;
    const int item0 = (blockIdx.x * NW + w) * RPW;
    const size_t kv_dim = (size_t)a.nkv * HD;
    const int ci = rope_angle_f4<HD>(a.rope, t);

    float4 kx[NS], vx[NS], cs[NS], sn[NS];
    int tok[NS], kvh[NS];
#pragma unroll
    for (int i = 0; i < NS; i++) {
        const int it = min(item0 + RPS * i + hh, n_items - 1);  // loads stay in bounds; stores are predicated
        tok[i] = it / a.nkv;
        kvh[i] = it - tok[i] * a.nkv;
        const size_t off = (size_t)tok[i] * a.ld + (size_t)kvh[i] * HD;
        kx[i] = ((const float4*)(a.k + off))[t];
        vx[i] = ((const float4*)(a.v + off))[t];
        const size_t pos = (size_t)(a.start + tok[i]);
        cs[i] = ((const float4*)(a.cos_tab + pos * (HD / 2)))[ci];
        sn[i] = ((const float4*)(a.sin_tab + pos * (HD / 2)))[ci];
    }
    const float4 wk = ((const float4*)(a.kn ? a.kn : a.wpad + HD))[t];
    if constexpr (YS) {
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const float xi = a.x_inv[tok[i]];
            const int c = kvh[i] * HD + 4 * t;
            kx[i] = unscale4(kx[i], ((const float4*)(a.kw + (size_t)kvh[i] * HD))[t], xi, a.kb, a.kbt, c);
            vx[i] = unscale4(vx[i], ((const float4*)(a.vw + (size_t)kvh[i] * HD))[t], xi, a.vb, a.vbt, c);
        }
    }
    if (a.kn) {
        float* rows = sk[w];
#pragma unroll
        for (int i = 0; i < NS; i++) ((float4*)(rows + (RPS * i + hh) * RS))[t] = kx[i];
        wave_sync();
        const int r = min(lane >> 2, RPW - 1);  // lane (r, j): SSE lane j of row r
        const float s = rms_scale_ref_quad<HD>(rows + r * RS, lane & 3);
        if ((lane & 3) == 0 && (lane >> 2) < RPW) s_scale[w][r] = s;
        wave_sync();
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const float sc = s_scale[w][RPS * i + hh];
            kx[i] = float4{rms_apply(kx[i].x, sc, wk.x), rms_apply(kx[i].y, sc, wk.y), rms_apply(kx[i].z, sc, wk.z),
                           rms_apply(kx[i].w, sc, wk.w)};
        }
    }
#pragma unroll
    for (int i = 0; i < NS; i++) {
        const float4 x = rope_lanes<HD>(kx[i], a.rope, t, cs[i], sn[i]);
        if (item0 + RPS * i + hh < n_items) {
            const size_t off = (size_t)(a.start + tok[i]) * kv_dim + (size_t)kvh[i] * HD + 4 * t;
            *(u32x2*)(a.kc + off) = u32x2{f32_to_f16_ref(x.x) | ((uint32_t)f32_to_f16_ref(x.y) << 16),
                                          f32_to_f16_ref(x.z) | ((uint32_t)f32_to_f16_ref(x.w) << 16)};
            *(u32x2*)(a.vc + off) = u32x2{f32_to_f16_ref(vx[i].x) | ((uint32_t)f32_to_f16_ref(vx[i].y) << 16),
                                          f32_to_f16_ref(vx[i].z) | ((uint32_t)f32_to_f16_ref(vx[i].w) << 16)};
        }
    }
}

// Phase stamps of prefill_attn_kernel, compiled in only with
// -DPQA_PHASE_STAMPS (bench.py --phase-stamps): s_memrealtime (100 MHz) per
// wave at the phase boundaries of each of the workgroup's two row blocks,
// kPStampSlots per workgroup (block j at 32 j), read back by
// pqa_prefill_stamps_read.
constexpr int kPStampSlots = 64;
constexpr int kPStampWGs = 4096;
enum : int {
    kPStStart = 0,   // block start (thread 0)
    kPStQReady = 1,  // + wave: q normed, rotated, fp16 in LDS
    kPStLoop = 9,    // + wave: tile loop done
    kPStMerged = 17, // odd-tile partials merged (thread 0)
    kPStStored = 18, // + wave (even-tile waves): output rows stored
    kPStQLanded = 22,  // wave 0: raw q rows (and the first tiles) landed in LDS
    kPStQMath = 23,    // wave 0: q normed, rotated and written as fp16
};
// Per-step stamps of the long block's tile loop, compiled in only with
// -DPQA_STEP_STAMPS as well (bench.py --phase-stamps reads them from the
// library built that way), so that the per-block stamps are taken without
// their cost: waves 0 (even tiles) and 4 (odd tiles) of the first
// kSStampWGs workgroups stamp kSStampEvents points of each of the first
// kSStampSteps steps.
constexpr int kSStampWGs = 256, kSStampSteps = 32, kSStampEvents = 8;
enum : int {
    kSStStart = 0,    // tile() entered
    kSStLanded = 1,   // after the wave's s_waitcnt for its tile loads
    kSStBarrier = 2,  // after the workgroup barrier
    kSStIssued = 3,   // the next tile's loads issued
    kSStScores = 4,   // score MFMAs done and the row maximum taken
    kSStSoftmax = 5,  // P in fp16 and the row sums done
    kSStPV = 6,       // PV MFMAs issued
};
#ifdef PQA_PHASE_STAMPS
static __device__ unsigned long long g_prefill_stamps[kPStampWGs * kPStampSlots];
static __device__ unsigned long long g_prefill_step_stamps[kSStampWGs * 2 * kSStampSteps * kSStampEvents];
#define PQA_PSTAMP(slot, cond)                                                                           \
    do {                                                                                                 \
        if ((cond) && blockIdx.x < (unsigned)kPStampWGs)                                                 \
            g_prefill_stamps[(size_t)blockIdx.x * kPStampSlots + (slot)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#endif
#if defined(PQA_PHASE_STAMPS) && defined(PQA_STEP_STAMPS)
#define PQA_SSTAMP(stepv, ev)                                                                                  \
    do {                                                                                                       \
        if (j == 0 && (tid & 63) == 0 && (w & 3) == 0 && (stepv) < kSStampSteps &&                             \
            blockIdx.x < (unsigned)kSStampWGs)                                                                 \
            g_prefill_step_stamps[(((size_t)blockIdx.x * 2 + (w >> 2)) * kSStampSteps + (stepv)) * kSStampEvents + \
                                  (ev)] = __builtin_amdgcn_s_memrealtime();                                    \
    } while (0)
#else
#define PQA_SSTAMP(stepv, ev) \
    do {                      \
    } while (0)
#endif
#ifndef PQA_PHASE_STAMPS
#define PQA_PSTAMP(slot, cond) \
    do {                       \
    } while (0)
#endif

struct AttnArgs {
    const float* q;   // fp32 projections: row of token t at q + t * q_ld, heads one after the other
    const float* qn;  // [HD] or null
    const float* wpad;
    const float* cos_tab;  // [S][HD/2]
    const float* sin_tab;
    const uint16_t* kc;
    const uint16_t* vc;
    float* out;
    int start, n_tok, nh, g, n_kv, kv_dim, rows, nblk, rope;
    float qscale;
    int q_ld;  // floats between the q rows of consecutive tokens
    // scaled q (YS): q = q * (qw[c] * x_inv[t]) + qb[c] for column c of token t
    const float* qw;
    const float* x_inv;
    const uint8_t* qb;
    int qbt;
};

// The prompt's q rows and output rows each cross the chip once: read and
// stored with the non-temporal hint, they stay out of the way of the K/V
// tiles that 32 workgroups share, and the output leaves no dirty lines behind
// for the next launch. Qwen3-4B prefill, per layer: 70.6 -> 68.9 us (attention
// 64.6-64.8 -> 62.9-63.3 us, the next layer's K/V prep 7.45 -> 7.24 us); the
// q hint alone changed nothing measurable.
#ifndef PQA_PF_NT
#define PQA_PF_NT 3
#endif
constexpr bool kNtQ = (PQA_PF_NT & 1) != 0;    // q rows read with the non-temporal hint
constexpr bool kNtOut = (PQA_PF_NT & 2) != 0;  // output rows stored with it
constexpr int kAttnThreads = 512;  // 2 groups of 4 waves: even and odd key tiles
constexpr int kGroupWaves = 4;
constexpr int kRowsPerBlock = 128;
constexpr int kKeysPerTile = 64;
constexpr float kRescaleSlack = 8.0f;  // log2 units: P stays <= 256 between rescales

// LDS tile layout: 64 rows of HD fp16 (row = one key), rows unpadded, the
// 16-byte chunks of row r stored at chunk index c ^ swz(r). The direct
// global->LDS loads pick, for each lane, the global chunk whose swizzled slot
// is the lane's LDS slot, so the tile is written already swizzled.
//   K: swz(r) = r mod chunks: the A-operand reads (16 rows x 4 chunk
//      columns per instruction) use every 16-byte bank slot 4 times, the
//      minimum for 1 KB.
//   V: swz(r) = 2 ((r / rows per 256 bytes) mod (chunks / 2)): the
//      transposing reads (16 rows x one 32-byte dim block per instruction)
//      use every 8-byte bank slot twice, the minimum for 512 bytes.
template <int HD>
struct PrefillTile {
    static_assert(HD == 64 || HD == 128, "head sizes of the MFMA prefill");
    static constexpr int CH = HD / 8;            // 16-byte chunks per row
    static constexpr int ROWB = HD * 2;          // bytes per row
    static constexpr int RPB = 256 / ROWB;       // rows per 256-byte bank window
    static constexpr int BYTES = kKeysPerTile * ROWB;
    static constexpr int RPI = 1024 / ROWB;      // rows per 1 KB wave-wide load
    static constexpr int NI = BYTES / 1024 / kGroupWaves;  // loads per wave per tile and operand
    __device__ static int swz_k(int r) { return r & (CH - 1); }
    __device__ static int swz_v(int r) { return 2 * ((r / RPB) & (CH / 2 - 1)); }
};

// SPLITQ: scores use q = hi + lo (two fp16 MFMAs into one fp32 accumulator),
// which keeps fp32-level score precision when keys carry large outliers.
template <int HD, bool SPLITQ, bool YS>
__global__ __launch_bounds__(kAttnThreads, 1) void prefill_attn_kernel(const AttnArgs a) {
    using T = PrefillTile<HD>;
    constexpr int KS = HD / 32;  // 32-dim k-steps of S^T = K Q^T
    constexpr int DB = HD / 16;  // 16-dim blocks of O^T
    constexpr float NEG_INF = -__builtin_huge_valf();
    __shared__ __attribute__((aligned(1024))) char lds[2][2][2][T::BYTES];  // [buffer][tile parity][K, V]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = w % kGroupWaves;   // row group: rows 32 wr .. 32 wr + 31 of the block
    const int par = w / kGroupWaves;  // key tiles 2 step + par
    // Work item: a pair of row blocks of one KV head, the longest remaining
    // (nblk - 1 - i) and then the shortest (i), so that every workgroup has
    // about the same work and the second block's prologue runs while the
    // first block's output stores drain. The pairs of one KV head run on the
    // same XCD (workgroups go round-robin over the 8 XCDs), keeping that
    // head's K/V in one L2. Inside the workgroup the two waves of a SIMD
    // (w and w + 4) own the same rows and alternate key tiles: equal work.
    const int kvh = (int)blockIdx.x % a.n_kv;
    const int pair = (int)blockIdx.x / a.n_kv;
    const int nb = a.nblk - 1 - pair == pair ? 1 : 2;

    const char* kbase = (const char*)(a.kc + (size_t)kvh * HD);
    const char* vbase = (const char*)(a.vc + (size_t)kvh * HD);
    const size_t rowb = (size_t)a.kv_dim * 2;  // bytes per cache row

    // q of the current block, normed, rotated, scaled, fp16 (see below)
    __shared__ __attribute__((aligned(16))) char sq[kGroupWaves][32 * HD * 2];

    for (int j = 0; j < nb; j++) {
        const int b = j == 0 ? a.nblk - 1 - pair : pair;
        if (j) __syncthreads();  // the previous block's epilogue is done with the LDS
        PQA_PSTAMP(32 * j + kPStStart, tid == 0);

        // Lane-derived offsets are rebuilt for each block (the empty asm hides
        // that the lane id is loop-invariant), so they are not held live, and
        // spilled, across the whole pair.
        int lane_j = tid & 63;
        asm volatile("" : "+v"(lane_j));
        const int lane = lane_j;
        const int col = lane & 31;  // the lane's row in the output staging
        // v_mfma_f32_16x16x32_f16 lane layout: A row / B column / D column
        // c16, k elements 8 g16 .. +7, D rows 4 g16 .. +3
        const int c16 = lane & 15, g16 = lane >> 4;

        // ---- per-lane offsets, fixed for the block's tile loop ----
        // global -> LDS: the waves of group par load tile 2 step + par; wave load i
        // of an operand fills LDS bytes [1024 (wr NI + i), +1024): tile row
        // r = (wr NI + i) RPI + lane / CH, source chunk (lane % CH) ^ swz(r)
        unsigned gk[T::NI], gv[T::NI];
#pragma unroll
        for (int i = 0; i < T::NI; i++) {
            const int r = (wr * T::NI + i) * T::RPI + lane / T::CH;
            const int p = lane % T::CH;
            gk[i] = (unsigned)(r * rowb) + 16u * (unsigned)(p ^ T::swz_k(r));
            gv[i] = (unsigned)(r * rowb) + 16u * (unsigned)(p ^ T::swz_v(r));
        }
        // K fragment of key block kb, k-step ks: row 16 kb + c16, chunk
        // (4 ks + g16) ^ swz_k(row), and swz_k(16 kb + c16) = swz_k(c16)
        int koff[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ks++) koff[ks] = c16 * T::ROWB + 16 * ((4 * ks + g16) ^ T::swz_k(c16));
        // V^T fragment of dim block db, keys 32 s + [0, 32): two transposing
        // reads (t = 0, 1). In each 16-lane group the lane gives key row
        // 32 s + 16 t + 4 g16 + c16 / 4, dims 16 db + 4 (c16 % 4) .. +3, and
        // receives dim 16 db + c16 of the group's 4 keys: k elements 8 g16 + 4 t
        // .. +3 are keys 32 s + 16 t + 4 g16 .. +3, the keys the lane's scores
        // hold (see the P layout below). swz_v of the row depends on 4 g16 +
        // c16 / 4 only.
        const int vr0 = 4 * g16 + (c16 >> 2);
        int voff[DB];
#pragma unroll
        for (int db = 0; db < DB; db++)
            voff[db] = vr0 * T::ROWB + 16 * ((2 * db + ((c16 & 3) >> 1)) ^ T::swz_v(vr0)) + 8 * (c16 & 1);

        const int R0 = b * kRowsPerBlock + wr * 32;
        const int R = R0 + col;
        const bool rvalid = R < a.rows;
        const int tok = rvalid ? R / a.g : 0;
        const int hq = kvh * a.g + (rvalid ? R - (R / a.g) * a.g : 0);
        // positions of the lane's two score rows R0 + 16 rb + c16 (padding
        // rows take the last row's: their q is zero and their output unused)
        int qpos[2];
#pragma unroll
        for (int rb = 0; rb < 2; rb++) qpos[rb] = a.start + min(R0 + 16 * rb + c16, a.rows - 1) / a.g;
        const int last_row_blk = min(a.rows, (b + 1) * kRowsPerBlock) - 1;
        const int kend = a.start + last_row_blk / a.g + 1;
        const int ntiles = (kend + kKeysPerTile - 1) / kKeysPerTile;
        const int kend_w = R0 < a.rows ? a.start + (min(a.rows, R0 + 32) - 1) / a.g + 1 : 0;
        const int qpos_min_w = R0 < a.rows ? a.start + R0 / a.g : 0;

        auto issue = [&](int step, int buf) {
            const int kt = 2 * step + par;
            if (kt >= ntiles) return;
            const int key0 = kt * kKeysPerTile;
            const char* kb = kbase + (size_t)key0 * rowb;
            const char* vb = vbase + (size_t)key0 * rowb;
            if (key0 + kKeysPerTile <= kend) {
#pragma unroll
                for (int i = 0; i < T::NI; i++) {
                    const int inst = wr * T::NI + i;
                    lds_dma_b128(kb, gk[i], lds_addr(&lds[buf][par][0][inst * 1024]));
                    lds_dma_b128(vb, gv[i], lds_addr(&lds[buf][par][1][inst * 1024]));
                }
            } else {  // last tile: rows past kend (never read unmasked) clamp to kend - 1
                const int rmax = kend - 1 - key0;
#pragma unroll
                for (int i = 0; i < T::NI; i++) {
                    const int inst = wr * T::NI + i;
                    const int r = inst * T::RPI + lane / T::CH;
                    const int p = lane % T::CH;
                    const unsigned row = (unsigned)(min(r, rmax) * rowb);
                    lds_dma_b128(kb, row + 16u * (p ^ T::swz_k(r)), lds_addr(&lds[buf][par][0][inst * 1024]));
                    lds_dma_b128(vb, row + 16u * (p ^ T::swz_v(r)), lds_addr(&lds[buf][par][1][inst * 1024]));
                }
            }
        };

        issue(0, 0);

        // ---- q: normed, rotated, scaled, fp16, into LDS (sq) ----
        // The q rows of the row group reach LDS (buffer 1, free until the loop)
        // by direct loads, whole rows per lane group: coalesced, unlike
        // fragment-shaped loads. Row r's 16-byte chunk c sits at slot c ^ (r mod
        // chunks per row), so both the reads below and the fragment reads of the
        // loop are conflict-free. The two waves of a row group prepare 16 rows
        // each: lane (rr, j) = (lane / 4, lane % 4) holds of row 16 par + rr the
        // dims j HD/8 .. +HD/8 of both halves, i.e. whole RoPE pairs of all three
        // pairings (NeoX d ~ d + HD/2; block8 and interleaved inside 8-dim
        // chunks), so the rotation stays in the lane and the norm is a quad sum.
        // Until sq is written the same space holds the norm weights.
        float* s_qw = (float*)&sq[0][0];
        if (w == 0 && lane < HD / 4)
            lds_dma_b128(a.qn ? a.qn : a.wpad, 16u * lane, lds_addr(s_qw));
        constexpr int CQ = HD / 4;            // 16-byte chunks per fp32 q row
        constexpr int RPQ = 1024 / (HD * 4);  // rows per 1 KB wave load
        constexpr int NQ = 32 / RPQ / 2;      // loads per wave (the two waves of a row group split them)
        char* qst = &lds[1][0][0][0] + wr * 32 * HD * 4;
        const int tq0 = min(R0, a.rows - 1) / a.g;  // first token of the row group
        const char* qbase = (const char*)(a.q + (size_t)tq0 * a.q_ld);
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            const int j = par * NQ + i;
            const int rr = j * RPQ + lane / CQ;
            const int Rq = min(R0 + rr, a.rows - 1);
            const int tq = Rq / a.g;
            const unsigned qoff = (unsigned)(((tq - tq0) * a.q_ld + (kvh * a.g + (Rq - tq * a.g)) * HD) * 4);
            const int c = (lane % CQ) ^ (rr & (CQ - 1));
            if constexpr (kNtQ) lds_dma_b128_nt(qbase, qoff + 16u * c, lds_addr(qst + j * 1024));
            else lds_dma_b128(qbase, qoff + 16u * c, lds_addr(qst + j * 1024));
        }
        constexpr int NF = HD / 16;       // float4s per lane: NF/2 in each half
        constexpr int NH4 = NF / 2;       // float4s per half
        const int prow = 16 * par + (lane >> 2), pj = lane & 3;
        const int pR = R0 + prow;
        const int pqpos = a.start + min(pR, a.rows - 1) / a.g;
        auto pchunk = [&](int i) { return (i / NH4) * (CQ / 2) + pj * NH4 + (i % NH4); };  // fp32 chunk of float4 i
        half8 qfl[SPLITQ ? 2 : 1][SPLITQ ? KS : 1];  // fp16 residual of q (split-q), B-operand layout [rb][ks]
        {
            // cos/sin float4 q: NeoX the angles of half-0 float4 q (4 * its chunk);
            // block8 / interleaved the four angles 2c .. 2c+3 of chunk pair (c, c+1)
            const float* crow = a.cos_tab + (size_t)pqpos * (HD / 2);
            const float* srow = a.sin_tab + (size_t)pqpos * (HD / 2);
            float4 cf[NH4], sf[NH4];
#pragma unroll
            for (int q = 0; q < NH4; q++) {
                const int ai = a.rope == 0 ? 4 * pchunk(q) : 2 * pchunk((q / (NH4 / 2)) * NH4 + 2 * (q % (NH4 / 2)));
                cf[q] = *(const float4*)(crow + ai);
                sf[q] = *(const float4*)(srow + ai);
            }
            // scaled q (YS): the column scales and biases of this lane's dims,
            // loaded with the RoPE rows so that one wait covers them
            float4 qwv[YS ? NF : 1], qbv[YS ? NF : 1];
            float qxi = 1.0f;
            if constexpr (YS) {
                const int pRc = min(pR, a.rows - 1);
                const int ptq = pRc / a.g;
                const int col0 = (kvh * a.g + (pRc - ptq * a.g)) * HD;
                qxi = a.x_inv[ptq];
#pragma unroll
                for (int i = 0; i < NF; i++) {
                    const int c = col0 + 4 * pchunk(i);
                    qwv[i] = *(const float4*)(a.qw + c);
                    qbv[i] = a.qb ? float4{bias_at(a.qb, a.qbt, c), bias_at(a.qb, a.qbt, c + 1),
                                           bias_at(a.qb, a.qbt, c + 2), bias_at(a.qb, a.qbt, c + 3)}
                                  : float4{0.0f, 0.0f, 0.0f, 0.0f};
                }
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();  // q rows and s_qw landed
            PQA_PSTAMP(32 * j + kPStQLanded, tid == 0);
            float x[NF][4];
            const char* rowp = qst + prow * HD * 4;
#pragma unroll
            for (int i = 0; i < NF; i++) {
                const float4 u = *(const float4*)(rowp + 16 * (pchunk(i) ^ (prow & (CQ - 1))));
                x[i][0] = u.x, x[i][1] = u.y, x[i][2] = u.z, x[i][3] = u.w;
            }
            if constexpr (YS) {  // q = y * (w * xi), then + b (vec_add) when the layer has a bias
#pragma unroll
                for (int i = 0; i < NF; i++) {
                    x[i][0] = x[i][0] * (qwv[i].x * qxi);
                    x[i][1] = x[i][1] * (qwv[i].y * qxi);
                    x[i][2] = x[i][2] * (qwv[i].z * qxi);
                    x[i][3] = x[i][3] * (qwv[i].w * qxi);
                    if (a.qb) {
                        x[i][0] = x[i][0] + qbv[i].x;
                        x[i][1] = x[i][1] + qbv[i].y;
                        x[i][2] = x[i][2] + qbv[i].z;
                        x[i][3] = x[i][3] + qbv[i].w;
                    }
                }
            }
            // the score scale (log2 e / sqrt(hd), 0 for padding rows) goes in
            // with the norm scale, or alone without a norm: q is not stored
            const float qs = pR < a.rows ? a.qscale : 0.0f;
            if (a.qn) {
                float ss = 0.0f;
#pragma unroll
                for (int i = 0; i < NF; i++)
#pragma unroll
                    for (int e = 0; e < 4; e++) ss = fmaf(x[i][e], x[i][e], ss);
                ss = group_sum<4>(ss);  // the row's four lanes
                const float sc = qs / sqrtf(ss / (float)HD + 1e-6f);
#pragma unroll
                for (int i = 0; i < NF; i++) {
                    const float4 wv = *(const float4*)(s_qw + 4 * pchunk(i));
                    x[i][0] = rms_apply(x[i][0], sc, wv.x);
                    x[i][1] = rms_apply(x[i][1], sc, wv.y);
                    x[i][2] = rms_apply(x[i][2], sc, wv.z);
                    x[i][3] = rms_apply(x[i][3], sc, wv.w);
                }
            } else {
#pragma unroll
                for (int i = 0; i < NF; i++)
#pragma unroll
                    for (int e = 0; e < 4; e++) x[i][e] *= qs;
            }
#pragma unroll
            for (int q = 0; q < NH4; q++) {
                const float cv[4] = {cf[q].x, cf[q].y, cf[q].z, cf[q].w};
                const float sv[4] = {sf[q].x, sf[q].y, sf[q].z, sf[q].w};
                if (a.rope == 0) {  // NeoX: float4 q of half 0 with float4 q of half 1
#pragma unroll
                    for (int e = 0; e < 4; e++) rope_rotate_fma(x[q][e], x[NH4 + q][e], cv[e], sv[e]);
                } else {
                    const int i0 = (q / (NH4 / 2)) * NH4 + 2 * (q % (NH4 / 2));  // chunk pair (i0, i0 + 1)
                    if (a.rope == 1) {  // block8: element e of the two halves of the 8-dim chunk
#pragma unroll
                        for (int e = 0; e < 4; e++) rope_rotate_fma(x[i0][e], x[i0 + 1][e], cv[e], sv[e]);
                    } else {  // interleaved: (2i, 2i+1), angles 2c .. 2c+3 over the chunk pair
                        rope_rotate_fma(x[i0][0], x[i0][1], cv[0], sv[0]);
                        rope_rotate_fma(x[i0][2], x[i0][3], cv[1], sv[1]);
                        rope_rotate_fma(x[i0 + 1][0], x[i0 + 1][1], cv[2], sv[2]);
                        rope_rotate_fma(x[i0 + 1][2], x[i0 + 1][3], cv[3], sv[3]);
                    }
                }
            }
            __syncthreads();  // every wave is done with the norm weights in sq
            // fp16 chunk (i0 / 2) = float4s (i0, i0 + 1); hi to sq, the residual
            // (split-q) over the row's own fp32 staging
#pragma unroll
            for (int i0 = 0; i0 < NF; i0 += 2) {
                half8 hi8, lo8;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float xs = x[i0 + e / 4][e % 4];
                    hi8[e] = (_Float16)xs;
                    lo8[e] = (_Float16)(xs - (float)hi8[e]);
                }
                const int slot = 16 * ((pchunk(i0) / 2) ^ (prow & (T::CH - 1)));
                *(half8*)(sq[wr] + prow * HD * 2 + slot) = hi8;
                if constexpr (SPLITQ) *(half8*)(qst + prow * HD * 4 + slot) = lo8;
            }
            PQA_PSTAMP(32 * j + kPStQMath, tid == 0);
            if constexpr (SPLITQ) {
                __syncthreads();  // both waves' residual rows landed
#pragma unroll
                for (int rb = 0; rb < 2; rb++)
#pragma unroll
                    for (int ks = 0; ks < KS; ks++)
                        qfl[rb][ks] = *(const half8*)(qst + (16 * rb + c16) * HD * 4 +
                                                      16 * ((4 * ks + g16) ^ (c16 & (T::CH - 1))));
            }
        }
        // q fragment of row block rb, k-step ks: row 16 rb + c16, chunk (4 ks + g16) ^ (row mod chunks)
        const char* sq_lane = sq[wr] + c16 * HD * 2;
        auto qread = [&](int ks, int rb) {
            return *(const half8*)(sq_lane + rb * 16 * HD * 2 + 16 * ((4 * ks + g16) ^ (c16 & (T::CH - 1))));
        };
        PQA_PSTAMP(32 * j + kPStQReady + w, (tid & 63) == 0);

        // The running max starts at -1e30 as in the reference (cpp/model.hpp:383):
        // a row whose keys in a tile are all masked (the odd group's first tile
        // can be) then gets p = exp2(-inf) = 0 and a rescale factor of 1, never
        // exp2(-inf - -inf).
        float m_run[2] = {-1e30f, -1e30f}, l_run[2] = {0.0f, 0.0f};  // rows 16 rb + c16
        floatx4 o[DB][2];  // O^T block (db, rb): dims 16 db + 4 g16 .. +3 of row 16 rb + c16
#pragma unroll
        for (int db = 0; db < DB; db++)
#pragma unroll
            for (int rb = 0; rb < 2; rb++) o[db][rb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

        auto tile = [&](int step, auto BUF) {
            constexpr int buf = decltype(BUF)::value;
            const int kt = 2 * step + par;
            const int key0 = kt * kKeysPerTile;
            PQA_SSTAMP(step, kSStStart);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's loads of step `step`
            PQA_SSTAMP(step, kSStLanded);
            __syncthreads();                                   // everyone's; the other buffer is free
            PQA_SSTAMP(step, kSStBarrier);
            issue(step + 1, buf ^ 1);
            PQA_SSTAMP(step, kSStIssued);
            if (kt >= ntiles || key0 >= kend_w) return;  // wave-uniform: nothing left for this wave

            const char* kt_lds = lds[buf][par][0];
            const char* vt_lds = lds[buf][par][1];
            // S^T = K Q^T in 16x16 blocks (key block kb, row block rb), KS
            // k-steps of 32 dims: 8 independent accumulators. Operands come from
            // LDS ahead of the MFMAs that use them: q one k-step ahead, K
            // fragments (sequence f = 4 ks + kb) through a ring RK deep.
            constexpr int RK = 4;
            floatx4 sacc[4][2];
            half8 rq[2][2], rk[RK];
            auto kread = [&](int f) {
                return *(const half8*)(kt_lds + (f & 3) * 16 * T::ROWB + koff[f >> 2]);
            };
            rq[0][0] = qread(0, 0);
            rq[0][1] = qread(0, 1);
#pragma unroll
            for (int f = 0; f < RK; f++) rk[f] = kread(f);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                if (ks + 1 < KS) {
                    rq[(ks + 1) & 1][0] = qread(ks + 1, 0);
                    rq[(ks + 1) & 1][1] = qread(ks + 1, 1);
                }
#pragma unroll
                for (int kp = 0; kp < 2; kp++) {
                    const int f0 = 4 * ks + 2 * kp;
                    half8 kf[2];
#pragma unroll
                    for (int q = 0; q < 2; q++) {
                        kf[q] = rk[(f0 + q) % RK];
                        if (f0 + q + RK < 4 * KS) rk[(f0 + q) % RK] = kread(f0 + q + RK);
                    }
                    // keep the reads ahead: the scheduler would otherwise sink them
                    // next to their MFMAs and expose the LDS latency again
                    __builtin_amdgcn_sched_barrier(0);
                    // two key blocks at a time: the hi and lo products of one
                    // accumulator sit 4 MFMAs apart (back to back they cost
                    // 0.45 us per Qwen3-4B layer)
#pragma unroll
                    for (int q = 0; q < 2; q++)
#pragma unroll
                        for (int rb = 0; rb < 2; rb++)
                            sacc[2 * kp + q][rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                kf[q], rq[ks & 1][rb], ks == 0 ? floatx4{0.0f, 0.0f, 0.0f, 0.0f} : sacc[2 * kp + q][rb], 0, 0, 0);
                    if constexpr (SPLITQ) {
#pragma unroll
                        for (int q = 0; q < 2; q++)
#pragma unroll
                            for (int rb = 0; rb < 2; rb++)
                                sacc[2 * kp + q][rb] =
                                    __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[q], qfl[rb][ks], sacc[2 * kp + q][rb], 0, 0, 0);
                    }
                }
            }
            // lane holds keys key0 + 16 kb + 4 g16 + e (e < 4) of rows 16 rb + c16
            if (key0 + kKeysPerTile - 1 > qpos_min_w) {
#pragma unroll
                for (int kb = 0; kb < 4; kb++)
#pragma unroll
                    for (int rb = 0; rb < 2; rb++)
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            if (key0 + 16 * kb + 4 * g16 + e > qpos[rb]) sacc[kb][rb][e] = NEG_INF;
            }
            // row maximum: the lane's 16 scores, then the row's 4 lanes (c16 + 16 g)
            float ml[2];
#pragma unroll
            for (int rb = 0; rb < 2; rb++) {
                float m = fmaxf(fmaxf(sacc[0][rb][0], sacc[0][rb][1]), fmaxf(sacc[0][rb][2], sacc[0][rb][3]));
#pragma unroll
                for (int kb = 1; kb < 4; kb++)
#pragma unroll
                    for (int e = 0; e < 4; e++) m = fmaxf(m, sacc[kb][rb][e]);
                ml[rb] = m;
            }
            // both rows at once: one swap leaves in the even 16-lane rows row 0's maximum of the
            // lane pair (l, l ^ 16) and in the odd ones row 1's; lanes l and l ^ 32 then agree
            // on the same row; a last swap hands each lane the other row's value (3 cross-lane
            // steps instead of 4; each sits on the tile's critical path: 0.8 us per Qwen3-4B
            // layer)
            float mx[2];
            {
                const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, ml[0]),
                                                                __builtin_bit_cast(unsigned, ml[1]), false, false);
                const float t = max_x32(fmaxf(__builtin_bit_cast(float, (unsigned)r[0]),
                                              __builtin_bit_cast(float, (unsigned)r[1])));
                pair16(t, mx[0], mx[1]);
            }
            PQA_SSTAMP(step, kSStScores);
            if (__any(mx[0] > m_run[0] + kRescaleSlack || mx[1] > m_run[1] + kRescaleSlack)) {
#pragma unroll
                for (int rb = 0; rb < 2; rb++) {
                    const float m_new = fmaxf(m_run[rb], mx[rb]);
                    const float corr = fast_exp2(m_run[rb] - m_new);
                    m_run[rb] = m_new;
                    l_run[rb] *= corr;
#pragma unroll
                    for (int db = 0; db < DB; db++)
#pragma unroll
                        for (int e = 0; e < 4; e++) o[db][rb][e] *= corr;
                }
            }
            // P^T as the B operand of the PV product, 32 keys per k-step s: k
            // elements 8 g16 .. +3 are keys 32 s + 4 g16 .. +3 (key block 2 s),
            // 8 g16 + 4 .. +7 are keys 32 s + 16 + 4 g16 .. +3 (block 2 s + 1),
            // exactly the lane's own scores, so P never leaves registers.
            half8 pf[2][2];  // [rb][s]
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
                for (int kb = 0; kb < 4; kb++)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        pf[rb][kb >> 1][4 * (kb & 1) + e] = (_Float16)fast_exp2(sacc[kb][rb][e] - m_run[rb]);
            // row sums of the fp16 P the PV product consumes (v_dot2_f32_f16 with ones)
            const half2 one2 = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
            for (int rb = 0; rb < 2; rb++) {
                float ps[2] = {0.0f, 0.0f};
#pragma unroll
                for (int s = 0; s < 2; s++)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        ps[s] = __builtin_amdgcn_fdot2(half2{pf[rb][s][2 * e], pf[rb][s][2 * e + 1]}, one2, ps[s], false);
                l_run[rb] += ps[0] + ps[1];
            }
            PQA_SSTAMP(step, kSStSoftmax);
            // O^T += V^T P^T: 2 key steps x DB dim blocks x 2 row blocks; V^T
            // fragments (two transposing reads each) through a ring RV deep.
            constexpr int NPV = 2 * DB, RV = 4;
            auto vread = [&](int idx) {
                const int s = idx / DB, db = idx % DB;
                half4 part[2];
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const char* adr = vt_lds + voff[db] + (32 * s + 16 * t) * T::ROWB;
                    const short4v raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)adr);
                    part[t] = __builtin_bit_cast(half4, raw);
                }
                return half8{part[0][0], part[0][1], part[0][2], part[0][3], part[1][0], part[1][1], part[1][2], part[1][3]};
            };
            half8 rv[RV];
#pragma unroll
            for (int i = 0; i < RV; i++) rv[i] = vread(i);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int idx = 0; idx < NPV; idx++) {
                const half8 vf = rv[idx % RV];
                if (idx + RV < NPV) rv[idx % RV] = vread(idx + RV);
                __builtin_amdgcn_sched_barrier(0);
                const int s = idx / DB, db = idx % DB;
#pragma unroll
                for (int rb = 0; rb < 2; rb++)
                    o[db][rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[rb][s], o[db][rb], 0, 0, 0);
            }
            PQA_SSTAMP(step, kSStPV);
        };

        const int nsteps = (ntiles + 1) / 2;
        for (int step = 0; step < nsteps; step += 2) {
            tile(step, std::integral_constant<int, 0>{});
            if (step + 1 < nsteps) tile(step + 1, std::integral_constant<int, 1>{});
        }

        PQA_PSTAMP(32 * j + kPStLoop + w, (tid & 63) == 0);
        // ---- merge the two parities' partials; each wave finishes one row block ----
        // The even-tile wave finishes rows 0..15 of the row group (row block 0)
        // and the odd-tile wave rows 16..31, so merging and storing are split
        // between the two waves of a SIMD (one wave storing all 32 rows took
        // 3 us more per Qwen3-4B layer: the stores are issue-bound per wave).
        // Each wave hands the other the half of its partial the other
        // finishes: LDS X[par][wr] holds, per lane, the DB float4s of O of
        // that row block and one float4 (m, l, 0, 0), as [slot][lane][4]
        // (16-byte accesses, conflict-free).
        constexpr int XS = DB + 1;  // float4 slots per lane
        constexpr int XB = XS * 64 * 16;  // bytes per wave
        constexpr int CPR = HD / 4;       // 16-byte chunks per output row
        constexpr int SB = 16 * HD * 4;   // staging bytes per wave: 16 rows of HD fp32
        static_assert(2 * kGroupWaves * XB + kGroupWaves * SB <= (int)sizeof(lds), "merge areas exceed the tile buffers");
        static_assert(SB <= (int)sizeof(sq[0]), "even-tile staging exceeds the q area");
        __syncthreads();  // tile buffers are free
        // RBO: the row block this wave finishes (a constant in each branch, so
        // o, m and l stay in registers)
        auto hand_over = [&](auto RBO) {
            constexpr int rbo = decltype(RBO)::value;
            floatx4* mine = (floatx4*)&lds[0][0][0][0] + (size_t)(par * kGroupWaves + wr) * XS * 64;
#pragma unroll
            for (int db = 0; db < DB; db++) mine[db * 64 + lane] = o[db][rbo ^ 1];
            mine[DB * 64 + lane] = floatx4{m_run[rbo ^ 1], l_run[rbo ^ 1], 0.0f, 0.0f};
        };
        auto finish = [&](auto RBO) {
            constexpr int rbo = decltype(RBO)::value;
            const floatx4* other = (const floatx4*)&lds[0][0][0][0] + (size_t)((par ^ 1) * kGroupWaves + wr) * XS * 64;
            floatx4 po[DB];
#pragma unroll
            for (int db = 0; db < DB; db++) po[db] = other[db * 64 + lane];
            const floatx4 ml = other[DB * 64 + lane];
            // the even-tile partial (e) and the odd-tile one (o) in the same
            // roles whichever wave merges, so both row blocks round alike: the
            // row's 1/l folded into both weights, one multiply and one fused
            // multiply-add per output value; l sums the row's 4 lanes
            const float me = rbo == 0 ? m_run[rbo] : ml[0], le = rbo == 0 ? l_run[rbo] : ml[1];
            const float mo = rbo == 0 ? ml[0] : m_run[rbo], lo = rbo == 0 ? ml[1] : l_run[rbo];
            const float M = fmaxf(me, mo);
            const float fe = fast_exp2(me - M);
            const float fo = fast_exp2(mo - M);
            const float inv = 1.0f / sum_x32(sum_x16(fmaf(le, fe, lo * fo)));
            const float we = fe * inv, wo = fo * inv;
#pragma unroll
            for (int db = 0; db < DB; db++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float xe = rbo == 0 ? o[db][rbo][e] : po[db][e];
                    const float xo = rbo == 0 ? po[db][e] : o[db][rbo][e];
                    o[db][rbo][e] = fmaf(xe, we, xo * wo);
                }

            // ---- normalise and store ----
            // The wave's 16 rows go through LDS (the even-tile waves' own q
            // area, the odd-tile waves' a slot past the exchange areas) as
            // [row][HD] fp32, 16-byte chunk c of row r at slot c ^ (r mod
            // chunks), so that each store instruction writes whole 512-byte
            // output rows.
            float* stg = par == 0 ? (float*)&sq[wr][0]
                                  : (float*)((char*)&lds[0][0][0][0] + 2 * kGroupWaves * XB + wr * SB);
#pragma unroll
            for (int db = 0; db < DB; db++) {
                const int c = 4 * db + g16;  // dims 16 db + 4 g16 .. +3
                *(floatx4*)(stg + c16 * HD + 4 * (c ^ (c16 & (CPR - 1)))) = o[db][rbo];
            }
            // output row of q row 16 rbo + (lane & 15)
            const int Rl = R0 + 16 * rbo + c16;
            const int orow = Rl < a.rows ? (Rl / a.g) * a.nh + kvh * a.g + (Rl - (Rl / a.g) * a.g) : -1;
            wave_sync();
            constexpr int RPS = 64 / CPR;          // rows per store instruction
            constexpr int NST = 16 * CPR / 64;     // store instructions per wave
            floatx4 vv[NST];
#pragma unroll
            for (int i = 0; i < NST; i++) {
                const int rr = RPS * i + lane / CPR, c = lane % CPR;
                vv[i] = *(const floatx4*)(stg + rr * HD + 4 * (c ^ (rr & (CPR - 1))));
            }
#pragma unroll
            for (int i = 0; i < NST; i++) {
                const int c = lane % CPR;
                int orr = -1;
#pragma unroll
                for (int u = 0; u < RPS; u++) {
                    const int v = __builtin_amdgcn_readlane(orow, RPS * i + u);
                    if (lane / CPR == u) orr = v;
                }
                if (orr >= 0) {
                    if constexpr (kNtOut) __builtin_nontemporal_store(vv[i], (floatx4*)(a.out + (size_t)orr * HD + 4 * c));
                    else *(floatx4*)(a.out + (size_t)orr * HD + 4 * c) = vv[i];
                }
            }
        };
        if (par == 0) hand_over(std::integral_constant<int, 0>{});
        else hand_over(std::integral_constant<int, 1>{});
        __syncthreads();
        PQA_PSTAMP(32 * j + kPStMerged, tid == 0);
        if (par == 0) finish(std::integral_constant<int, 0>{});
        else finish(std::integral_constant<int, 1>{});
        PQA_PSTAMP(32 * j + kPStStored + wr, lane == 0 && par == 0);
    }
}

#ifdef PQA_PHASE_STAMPS
// The stamped build's extra entry points (not in pqa.h), as for decode.
extern "C" int pqa_prefill_stamps_read(unsigned long long* dst, int n) {
    if (!dst || n != kPStampWGs * kPStampSlots) return PQA_ERR_ARG;
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_prefill_stamps), (size_t)n * 8, 0, hipMemcpyDeviceToHost) ==
                   hipSuccess
               ? PQA_OK
               : PQA_ERR_HIP;
}
extern "C" int pqa_prefill_step_stamps_read(unsigned long long* dst, int n) {
    if (!dst || n != kSStampWGs * 2 * kSStampSteps * kSStampEvents) return PQA_ERR_ARG;
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_prefill_step_stamps), (size_t)n * 8, 0, hipMemcpyDeviceToHost) ==
                   hipSuccess
               ? PQA_OK
               : PQA_ERR_HIP;
}
extern "C" int pqa_prefill_stamps_clear() {
    static unsigned long long zero[kPStampWGs * kPStampSlots];
    static_assert(sizeof(zero) >= sizeof(g_prefill_step_stamps), "one zero buffer clears both");
    return hipMemcpyToSymbol(HIP_SYMBOL(g_prefill_stamps), zero, sizeof(zero), 0, hipMemcpyHostToDevice) ==
                           hipSuccess &&
                   hipMemcpyToSymbol(HIP_SYMBOL(g_prefill_step_stamps), zero, sizeof(g_prefill_step_stamps), 0,
                                     hipMemcpyHostToDevice) == hipSuccess
               ? PQA_OK
               : PQA_ERR_HIP;
}
#endif

template <int HD, bool YS>
static hipError_t launch_prefill_hd(pqa_ctx* ctx, int layer, int start, int n_tok, const float* q,
                                    const float* k, const float* v, float* out, const PrefillScaled* ys) {
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
    p.ld = (int)ctx->kv_dim;
    p.kw = p.vw = p.x_inv = nullptr;
    p.kb = p.vb = nullptr;
    p.kbt = p.vbt = 0;
    const bool kv_scaled = YS && !ys->kv_plain;
    if (YS) {  // k and v are columns of the GEMM result; scaled unless the reference-order projection wrote them
        p.k = ys->y + ctx->q_dim;
        p.v = ys->y + ctx->q_dim + ctx->kv_dim;
        p.ld = ys->ld;
    }
    if (kv_scaled) {
        p.kw = ys->w_inv + ctx->q_dim;
        p.vw = ys->w_inv + ctx->q_dim + ctx->kv_dim;
        p.x_inv = ys->x_inv;
        p.kb = ys->b[1];
        p.kbt = ys->bt[1];
        p.vb = ys->b[2];
        p.vbt = ys->bt[2];
    }
    constexpr int rows_per_wg = (kKvThreads / 64) * kv_rows_per_wave<HD>();
    const int n_items = n_tok * ctx->n_kv_heads;
    const dim3 kv_grid((n_items + rows_per_wg - 1) / rows_per_wg);
    if (kv_scaled)
        hipLaunchKernelGGL((prefill_kv_kernel<HD, true>), kv_grid, dim3(kKvThreads), 0, ctx->stream, p);
    else
        hipLaunchKernelGGL((prefill_kv_kernel<HD, false>), kv_grid, dim3(kKvThreads), 0, ctx->stream, p);
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
    a.q_ld = (int)ctx->q_dim;
    a.qw = a.x_inv = nullptr;
    a.qb = nullptr;
    a.qbt = 0;
    if (YS) {
        a.q = ys->y;
        a.q_ld = ys->ld;
        a.qw = ys->w_inv;
        a.x_inv = ys->x_inv;
        a.qb = ys->b[0];
        a.qbt = ys->bt[0];
    }
    dim3 grid((a.nblk + 1) / 2 * ctx->n_kv_heads);  // pairs of row blocks
    if (ctx->prefill_split_q)
        hipLaunchKernelGGL((prefill_attn_kernel<HD, true, YS>), grid, dim3(kAttnThreads), 0, ctx->stream, a);
    else
        hipLaunchKernelGGL((prefill_attn_kernel<HD, false, YS>), grid, dim3(kAttnThreads), 0, ctx->stream, a);
    return hipGetLastError();
}

hipError_t launch_prefill(pqa_ctx* ctx, int layer, int start, int n_tok, const float* q,
                          const float* k, const float* v, float* out) {
    if (ctx->head_dim == 64) return launch_prefill_hd<64, false>(ctx, layer, start, n_tok, q, k, v, out, nullptr);
    if (ctx->head_dim == 128) return launch_prefill_hd<128, false>(ctx, layer, start, n_tok, q, k, v, out, nullptr);
    return launch_prefill_general(ctx, layer, start, n_tok, q, k, v, nullptr, out);
}

hipError_t launch_prefill_scaled(pqa_ctx* ctx, int layer, int start, int n_tok, const PrefillScaled& ys, float* out) {
    if (ctx->head_dim == 64)
        return launch_prefill_hd<64, true>(ctx, layer, start, n_tok, nullptr, nullptr, nullptr, out, &ys);
    if (ctx->head_dim == 128)
        return launch_prefill_hd<128, true>(ctx, layer, start, n_tok, nullptr, nullptr, nullptr, out, &ys);
    return launch_prefill_general(ctx, layer, start, n_tok, nullptr, nullptr, nullptr, &ys, out);
}

}  // namespace pqa
