// Q/K/V projections of one token on the GPU: TensorOps::matmul_bias
// (cpp/tensor.hpp:110-143) for ATTN_Q, ATTN_K and ATTN_V at
// cpp/model.hpp:320-366, in the reference's own summation order, so q, k and
// v equal the reference's bit for bit (as compiled without FMA contraction)
// and the K/V rows the decode appends stay bit-exact from xb on.
//
// Weights keep the GGUF block layout the reference reads (cpp/quant.hpp:33-63),
// one row per output element, uploaded once per layer with the row stride
// rounded up to 16 bytes. Orders reproduced (cpp/quant.hpp:297-356):
//   F32, F16, Q4_0, Q4_K, Q6_K  row dequantized element by element
//       (dequantize_row_*, same expressions), then vec_dot_f32_f32's SSE2
//       order: 8 sequential chains (element i goes to chain i mod 8), then
//       t = chain l + chain l+4, then (t0 + t2) + (t1 + t3);
//   Q8_0  per 32-block sequential sums of q*x, then sumf += d * sum in block
//       order.
// Then out = out + bias (vec_add), bias F32 or F16.
//
// Only the additions are ordered; dequantization and the products w * x are
// not. A workgroup of 16 waves owns 8 rows: the rows stream in chunks from
// HBM into a 4-slot LDS ring by direct global->LDS loads (chunk t + 3 in
// flight while t is used); waves 1-15 turn chunk t into fp32 products
// round(w * x) in LDS, chain-major (Q8_0: block-major with each block's d),
// while wave 0, lane 8 r + c, adds chunk t - 1 into chain c of row r. One
// barrier per chunk. Each producer item issues all its LDS reads (quant
// bytes, scales, x) before its first product store, since the compiler
// cannot move a read of x past a store into the same LDS block. The work is
// VALU- and latency-bound by the fixed order (no MFMA or packed math can
// keep it).
#include <algorithm>
#include <cstring>
#include <string>

#include "pqa_device.h"
#include "pqa_internal.h"

namespace pqa {

constexpr int kProjWaves = 16;        // wave 0 sums the chains, waves 1-15 produce
constexpr int kProjProducers = 64 * (kProjWaves - 1);
constexpr int kProjRows = 8;          // rows per workgroup
constexpr int kProjChunkMax = 512;    // largest chunk bytes per row
constexpr int kProjKC = 64;           // largest chain elements per chunk
constexpr int kPS = kProjKC + 4;      // product row stride (floats): chains off the bank period
constexpr int kProjSlots = 4;         // raw chunk ring: chunk t + 3 loads while t is used
constexpr int kProjSlotBytes = kProjRows * kProjChunkMax;  // 16 DMA loads of 256 bytes
constexpr int kProjDmaPerWave = kProjSlotBytes / 256 / kProjWaves;

struct ProjMat {
    const uint8_t* w;  // [rows][stride] GGUF rows
    const uint8_t* b;  // bias row or null
    float* out;        // with add_out: out[row] += result (vec_add into the residual stream)
    int add_out;
    int rows, wtype, btype, stride, wg0;  // wg0: first workgroup of this matrix
    int fast;  // rows summed in any order (gemv_wg), one row per wave; else the reference's order (proj_wg)
};

struct ProjArgs {
    ProjMat m[3];
    const float* x;
    int n, nmat;
};

__device__ __forceinline__ float h2f(unsigned h) { return (float)__builtin_bit_cast(_Float16, (unsigned short)h); }
__device__ __forceinline__ unsigned ld16(const uint8_t* p) { return *(const unsigned short*)p; }

// chunk geometry per type: elements and bytes per row, both whole blocks with
// 4-byte aligned offsets
template <int T> struct QT;
template <> struct QT<GG_F32> { static constexpr int CE = 128, CB = 512; };
template <> struct QT<GG_F16> { static constexpr int CE = 256, CB = 512; };
template <> struct QT<GG_Q4_0> { static constexpr int CE = 512, CB = 288; };
template <> struct QT<GG_Q8_0> { static constexpr int CE = 256, CB = 272; };
template <> struct QT<GG_Q4_K> { static constexpr int CE = 512, CB = 288; };
template <> struct QT<GG_Q6_K> { static constexpr int CE = 512, CB = 420; };

// get_scale_min_k4 (cpp/quant.hpp:210-218) on the 12 scale bytes held as
// three little-endian words
__device__ __forceinline__ unsigned scale_byte(unsigned s0, unsigned s1, unsigned s2, int i) {
    const unsigned wd = i < 4 ? s0 : (i < 8 ? s1 : s2);
    return (wd >> (8 * (i & 3))) & 0xFF;
}
__device__ __forceinline__ void scale_min_k4_regs(int j, unsigned s0, unsigned s1, unsigned s2, unsigned& sc,
                                                  unsigned& mn) {
    if (j < 4) {
        sc = scale_byte(s0, s1, s2, j) & 63;
        mn = scale_byte(s0, s1, s2, j + 4) & 63;
    } else {
        sc = (scale_byte(s0, s1, s2, j + 4) & 0xF) | ((scale_byte(s0, s1, s2, j - 4) >> 6) << 4);
        mn = (scale_byte(s0, s1, s2, j + 4) >> 4) | ((scale_byte(s0, s1, s2, j) >> 6) << 4);
    }
}

// Products of one chunk, round(w * x) in fp32 with w dequantized by the
// expressions of dequantize_row_* (cpp/quant.hpp:176-281). Chain types:
// element e of row r at prod[(8 r + e % 8) * kPS + e / 8] (a chain lane reads
// its products as consecutive floats). Q8_0: q * x of element j of block bi at
// prod[(8 r + bi) * kPS + j], the block's d at slot 32. Every element of the
// chunk is written, past the row end too (never summed).
template <int T>
__device__ __forceinline__ void produce(const uint8_t* raw, const float* xs, float* prod, int pt) {
    constexpr int CB = QT<T>::CB, RB = (CB + 3) / 4 * 4;  // LDS bytes per raw row
    auto put = [&](int r, int e, float v) __attribute__((always_inline)) { prod[(8 * r + (e & 7)) * kPS + (e >> 3)] = v; };
    if constexpr (T == GG_F32) {  // 8 rows x 32 float4
        for (int it = pt; it < 8 * 32; it += kProjProducers) {
            const int r = it >> 5, f = it & 31;
            const floatx4 v = *(const floatx4*)(raw + r * RB + 16 * f);
            const floatx4 x = *(const floatx4*)(xs + 4 * f);
#pragma unroll
            for (int b = 0; b < 4; b++) put(r, 4 * f + b, v[b] * x[b]);
        }
    } else if constexpr (T == GG_F16) {  // 8 rows x 64 groups of 4 halfs
        for (int it = pt; it < 8 * 64; it += kProjProducers) {
            const int r = it >> 6, g = it & 63;
            const u32x2 v = *(const u32x2*)(raw + r * RB + 8 * g);
            const floatx4 x = *(const floatx4*)(xs + 4 * g);
            put(r, 4 * g + 0, h2f(v.x & 0xFFFF) * x[0]);
            put(r, 4 * g + 1, h2f(v.x >> 16) * x[1]);
            put(r, 4 * g + 2, h2f(v.y & 0xFFFF) * x[2]);
            put(r, 4 * g + 3, h2f(v.y >> 16) * x[3]);
        }
    } else if constexpr (T == GG_Q4_0) {  // 8 rows x 16 blocks x 8 byte pairs: d * ((float)nibble - 8)
        for (int it = pt; it < 8 * 128; it += kProjProducers) {
            const int r = it >> 7, bi = (it >> 3) & 15, j2 = 2 * (it & 7);
            const uint8_t* blk = raw + r * RB + 18 * bi;
            const int e = 32 * bi + j2;
            const unsigned dh = ld16(blk), two = ld16(blk + 2 + j2);
            const float2 xl = *(const float2*)(xs + e), xh = *(const float2*)(xs + e + 16);
            const float d = h2f(dh);
            const float xlo[2] = {xl.x, xl.y}, xhi[2] = {xh.x, xh.y};
#pragma unroll
            for (int b = 0; b < 2; b++) {
                const unsigned byte = (two >> (8 * b)) & 0xFF;
                put(r, e + b, d * ((float)(byte & 0xF) - 8.0f) * xlo[b]);
                put(r, e + b + 16, d * ((float)(byte >> 4) - 8.0f) * xhi[b]);
            }
        }
    } else if constexpr (T == GG_Q8_0) {  // 8 rows x 8 blocks x 8 groups of 4: (float)q * x
        for (int it = pt; it < 8 * 64; it += kProjProducers) {
            const int r = it >> 6, bi = (it >> 3) & 7, g = it & 7;
            const uint8_t* blk = raw + r * RB + 34 * bi;
            const unsigned lo = ld16(blk + 2 + 4 * g), hi = ld16(blk + 4 + 4 * g), dh = ld16(blk);
            const floatx4 x = *(const floatx4*)(xs + 32 * bi + 4 * g);
            const unsigned q4 = lo | (hi << 16);
            float* pr = prod + (8 * r + bi) * kPS;
            floatx4 v;
#pragma unroll
            for (int b = 0; b < 4; b++) v[b] = (float)(int)(int8_t)((q4 >> (8 * b)) & 0xFF) * x[b];
            *(floatx4*)(pr + 4 * g) = v;
            if (g == 0) pr[32] = h2f(dh);
        }
    } else if constexpr (T == GG_Q4_K) {  // 8 rows x 2 blocks x 32 qs dwords: (d * sc) * q - dmin * mn
        for (int it = pt; it < 8 * 64; it += kProjProducers) {
            const int r = it >> 6, bk = (it >> 5) & 1, w = it & 31, jj = w >> 3, l0 = 4 * (w & 7);
            const uint8_t* blk = raw + r * RB + 144 * bk;
            const int e0 = 256 * bk + 64 * jj + l0;
            // every LDS read of the item first (d and dmin, the 12 scale bytes,
            // the 4 quant bytes, x), so they share one round trip
            const unsigned dd = *(const unsigned*)blk;
            const unsigned s0 = *(const unsigned*)(blk + 4), s1 = *(const unsigned*)(blk + 8),
                           s2 = *(const unsigned*)(blk + 12);
            const unsigned q4 = *(const unsigned*)(blk + 16 + 4 * w);
            const floatx4 xa = *(const floatx4*)(xs + e0), xb = *(const floatx4*)(xs + e0 + 32);
            const float d = h2f(dd & 0xFFFF), dmin = h2f(dd >> 16);
            unsigned sc, mn;
            scale_min_k4_regs(2 * jj, s0, s1, s2, sc, mn);
            const float d1 = d * (float)sc, m1 = dmin * (float)mn;
            scale_min_k4_regs(2 * jj + 1, s0, s1, s2, sc, mn);
            const float d2 = d * (float)sc, m2 = dmin * (float)mn;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const unsigned byte = (q4 >> (8 * b)) & 0xFF;
                put(r, e0 + b, (d1 * (float)(byte & 0xF) - m1) * xa[b]);
                put(r, e0 + 32 + b, (d2 * (float)(byte >> 4) - m2) * xb[b]);
            }
        }
    } else if constexpr (T == GG_Q6_K) {  // 8 rows x 2 blocks x 2 halves x 16 l-pairs: (d * sc) * q
        for (int it = pt; it < 8 * 64; it += kProjProducers) {
            const int r = it >> 6, bk = (it >> 5) & 1, h = (it >> 4) & 1, l = 2 * (it & 15);
            const uint8_t* blk = raw + r * RB + 210 * bk;
            const int e0 = 256 * bk + 128 * h + l;
            // every LDS read of the item first: d, the quant bytes, the four
            // scale pairs (scale of quad q is byte l / 16 of pair q) and x
            const unsigned dh = ld16(blk + 208);
            const unsigned la = ld16(blk + 64 * h + l), lb = ld16(blk + 64 * h + 32 + l);
            const unsigned hb = ld16(blk + 128 + 32 * h + l);
            unsigned sp[4];
            float2 xv[4];
#pragma unroll
            for (int quad = 0; quad < 4; quad++) {
                sp[quad] = ld16(blk + 192 + 8 * h + 2 * quad);
                xv[quad] = *(const float2*)(xs + e0 + 32 * quad);
            }
            const float d = h2f(dh);
#pragma unroll
            for (int quad = 0; quad < 4; quad++) {
                const float ds = d * (float)(int)(int8_t)((sp[quad] >> (8 * (l >> 4))) & 0xFF);
                const unsigned lq = (quad & 1) ? lb : la;
                const float xq[2] = {xv[quad].x, xv[quad].y};
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    const unsigned lo = ((lq >> (8 * b)) >> (quad < 2 ? 0 : 4)) & 0xF;
                    const unsigned hi = ((hb >> (8 * b)) >> (2 * quad)) & 3;
                    const int q = (int)(lo | (hi << 4)) - 32;
                    put(r, e0 + 32 * quad + b, ds * (float)q * xq[b]);
                }
            }
        }
    }
}

// s_waitcnt vmcnt(n) for a run-time n in [0, 15] (the count is an immediate)
__device__ __forceinline__ void wait_loads_but(int n) {
    switch (n) {
#define PQA_VMCNT(N) case N: asm volatile("s_waitcnt vmcnt(" #N ")" ::: "memory"); break;
        PQA_VMCNT(1) PQA_VMCNT(2) PQA_VMCNT(3) PQA_VMCNT(4) PQA_VMCNT(5) PQA_VMCNT(6) PQA_VMCNT(7)
        PQA_VMCNT(8) PQA_VMCNT(9) PQA_VMCNT(10) PQA_VMCNT(11) PQA_VMCNT(12) PQA_VMCNT(13) PQA_VMCNT(14)
        PQA_VMCNT(15)
#undef PQA_VMCNT
        default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    }
}
static_assert(kProjDmaPerWave * (kProjSlots - 1) <= 15, "loads in flight exceed the waits written out");

template <int T>
__device__ void proj_wg(const ProjMat& m, const float* __restrict__ x, float* xs, uint8_t* ring, float* prod, int n,
                        int lwg) {
    constexpr int CE = QT<T>::CE, CB = QT<T>::CB;
    constexpr int CDW = (CB + 3) / 4;  // dwords per row and chunk
    constexpr int KC = CE / 8;         // chain elements per chunk
    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int pt = tid - 64;  // producer thread index (waves 1-3)
    const int row0 = lwg * kProjRows;
    const int nch = (n + CE - 1) / CE;
    const unsigned ring_lds = lds_addr(ring);
    // Chunk t's rows go to slot t % kProjSlots as [row][CDW dwords]: 16 loads of
    // 64 dwords, 4 per wave. Dword d: row d / CDW (rows past the matrix and the
    // slot tail read clamped, unused data), word d % CDW (words past the row
    // end stay inside its stride).
    unsigned voff[kProjDmaPerWave];
#pragma unroll
    for (int i = 0; i < kProjDmaPerWave; i++) {
        const int d = 64 * (kProjDmaPerWave * w + i) + lane;
        const int rr = min(d / CDW, kProjRows - 1), wd = d - (d / CDW) * CDW;
        voff[i] = (unsigned)(min(row0 + rr, m.rows - 1) * m.stride) + 4u * (unsigned)min(wd, CDW - 1);
    }
    auto issue = [&](int t) __attribute__((always_inline)) {
        const unsigned slot = ring_lds + (unsigned)((t % kProjSlots) * kProjSlotBytes);
#pragma unroll
        for (int i = 0; i < kProjDmaPerWave; i++) {
            // the last chunk of a row may end inside the row's 16-byte padding
            const unsigned off = min(voff[i] + (unsigned)(t * CB),
                                     voff[i] - voff[i] % (unsigned)m.stride + (unsigned)m.stride - 4u);
            lds_dma_b32(m.w, off, slot + 256u * (unsigned)(kProjDmaPerWave * w + i));
        }
    };
    // chain wave: lane (r, c)
    const int r = lane >> 3, c = lane & 7;
    float acc = 0.0f;
    auto chains = [&](int t) __attribute__((always_inline)) {  // products of chunk t
        const float* pr = prod + (t & 1) * 64 * kPS + (8 * r + c) * kPS;
        const int ne = min(CE, n - t * CE);
        if constexpr (T == GG_Q8_0) {  // lane c: block c; then d * sum into sumf in block order
            const int nb = ne >> 5;
            float sum = 0.0f;
            if (c < nb) {
#pragma unroll
                for (int j = 0; j < 32; j += 4) {
                    const floatx4 p4 = *(const floatx4*)(pr + j);
#pragma unroll
                    for (int b = 0; b < 4; b++) sum = sum + p4[b];
                }
            }
            const float tb = pr[32] * sum;
            for (int bi = 0; bi < nb; bi++) acc = acc + __shfl(tb, (lane & ~7) + bi);
        } else if (ne == CE) {
#pragma unroll
            for (int k = 0; k < KC; k += 4) {
                const floatx4 p4 = *(const floatx4*)(pr + k);
#pragma unroll
                for (int b = 0; b < 4; b++) acc = acc + p4[b];
            }
        } else {
            for (int k = 0; k < (ne >> 3); k++) acc = acc + pr[k];
        }
    };
    for (int t = 0; t < kProjSlots - 1 && t < nch; t++) issue(t);
    // x goes to LDS while the first chunks load (loads complete in issue
    // order, so its wait covers them too: one round trip for both)
    for (int i = tid; i < n; i += 64 * kProjWaves) xs[i] = x[i];
    // this wave's loads of chunk t are done once only those of later chunks
    // (kProjDmaPerWave each) are outstanding
    wait_loads_but(kProjDmaPerWave * min(kProjSlots - 2, nch - 1));
    __syncthreads();  // x and chunk 0 in LDS
    // step t: chunk t + 3 starts loading into the slot chunk t - 1 left;
    // producers turn chunk t into products while the chain wave sums chunk
    // t - 1; every wave then waits for its loads of chunk t + 1, and one
    // barrier publishes the products, ends the reads of chunk t - 1's products
    // and makes chunk t + 1 visible
    for (int t = 0; t <= nch; t++) {
        if (t + kProjSlots - 1 < nch) issue(t + kProjSlots - 1);
        if (w > 0) {
            if (t < nch) produce<T>(ring + (t % kProjSlots) * kProjSlotBytes, xs + t * CE, prod + (t & 1) * 64 * kPS, pt);
        } else if (t > 0) {
            chains(t - 1);
        }
        if (t + 1 < nch) wait_loads_but(kProjDmaPerWave * min(kProjSlots - 2, nch - 2 - t));
        __syncthreads();
    }
    if (w == 0) {
        float total;
        if constexpr (T == GG_Q8_0) {
            total = acc;
        } else {
            const float t4 = acc + __shfl(acc, lane + 4);  // lanes c < 4: acc0[c] + acc1[c]
            const float t2 = t4 + __shfl(t4, lane + 2);    // c = 0: t0 + t2, c = 1: t1 + t3
            total = t2 + __shfl(t2, lane + 1);             // c = 0: (t0 + t2) + (t1 + t3)
        }
        const int row = row0 + r;
        if (c == 0 && row < m.rows) {
            if (m.b) {
                const float bv = m.btype == GG_F32 ? ((const float*)m.b)[row] : h2f(ld16(m.b + 2 * row));
                total = total + bv;
            }
            m.out[row] = m.add_out ? m.out[row] + total : total;
        }
    }
}

// The q rows of one token without the fixed order. q feeds only the
// attention scores (its bits reach no cache row), so its sums may take any
// order: one row per wave, the lanes over interleaved units of the row (a
// float4 of F32, 8 halfs of F16, a quarter block of Q4_K: its 16-byte header
// and 32 quant bytes, 64 elements), one fp32 fused sum per lane, then a
// butterfly sum over the wave and the bias. Every weight byte is read once,
// x comes from LDS. F32 and F16 weights multiply x as they are; a Q4_K
// group of 32 elements w = d q - m (cpp/quant.hpp:220-236) contributes
// d sum q x - m sum x, with sum x per group computed once per workgroup.
// Error against the reference's order: at most (n + 12) 2^-24 sum_i |w_i x_i|
// for F32 and F16, and (n + 12) 2^-24 sum_i (|d q_i| + |m|) |x_i| for Q4_K.
__host__ __device__ constexpr bool gemv_type(int t) { return t == GG_F32 || t == GG_F16 || t == GG_Q4_K; }

template <int T>
__device__ void gemv_wg(const ProjMat& m, const float* __restrict__ x, float* xs, int n, int lwg) {
    static_assert(gemv_type(T), "types with 16-byte aligned units");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row = lwg * kProjWaves + w;
    // waves past the last row load the last row again and store nothing: every
    // wave reaches the barrier below
    const uint8_t* wr = m.w + (size_t)min(row, m.rows - 1) * m.stride;
    // F32 / F16: lane l takes unit l + 64 k of EU elements (n is a multiple of
    // 8, so a unit is whole or past the row), 8 units per batch. Q4_K: unit
    // u = 4 sb + jj is the quarter block of elements 256 sb + 64 jj + [0, 64)
    // (cpp/quant.hpp:220-236), its 16-byte header and 32 quant bytes; n <= 8192
    // gives at most 2 units per lane.
    constexpr int EU = T == GG_F32 ? 4 : 8;
    constexpr int NB = T == GG_Q4_K ? 6 : 8;  // 16-byte loads held per lane
    u32x4 wv[NB];
    auto load_batch = [&](int e0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int e = e0 + EU * (64 * u + lane);
            wv[u] = e < n ? *(const u32x4*)(wr + (T == GG_F32 ? 4 : 2) * e) : u32x4{0u, 0u, 0u, 0u};
        }
    };
    const int nu = n / 64;
    if constexpr (T == GG_Q4_K) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int u = min(64 * k + lane, nu - 1);  // loads stay in the row; the sum skips it
            const uint8_t* blk = wr + 144 * (u >> 2);
            wv[3 * k] = *(const u32x4*)blk;
            wv[3 * k + 1] = *(const u32x4*)(blk + 16 + 32 * (u & 3));
            wv[3 * k + 2] = *(const u32x4*)(blk + 32 + 32 * (u & 3));
        }
    } else {
        load_batch(0);
    }
    // Q4_K: lane u reads x[64 u, 64 u + 64); in LDS every 64 floats are
    // followed by 4 of padding, so the lanes' 16-byte reads fall on different
    // banks (unpadded, all 64 lanes hit the same four banks)
    auto xp = [&](int e) __attribute__((always_inline)) { return T == GG_Q4_K ? e + 4 * (e >> 6) : e; };
    {  // x to LDS while the weights load: every load of the thread issued before its stores
        constexpr int XPT = PQA_MAX_EMBD / (64 * kProjWaves);
        float xv[XPT];
#pragma unroll
        for (int k = 0; k < XPT; k++) {
            const int i = tid + 64 * kProjWaves * k;
            xv[k] = i < n ? x[i] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < XPT; k++) {
            const int i = tid + 64 * kProjWaves * k;
            if (i < n) xs[xp(i)] = xv[k];
        }
    }
    __syncthreads();
    float* xg = xs + xp(n);  // Q4_K: the sum of each 32-element group of x, shared by every row
    if constexpr (T == GG_Q4_K) {
        if (tid < n / 32) {
            float sg = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const floatx4 v4 = *(const floatx4*)(xs + xp(32 * tid) + 4 * i);
                sg = sg + ((v4[0] + v4[1]) + (v4[2] + v4[3]));
            }
            xg[tid] = sg;
        }
        __syncthreads();
    }
    if (row >= m.rows) return;
    float acc = 0.0f;
    if constexpr (T == GG_F32 || T == GG_F16) {
        for (int e0 = 0; e0 < n; e0 += 64 * EU * 8) {
            if (e0) load_batch(e0);
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int e = e0 + EU * (64 * u + lane);
                if (e < n) {
                    if constexpr (T == GG_F32) {
                        const floatx4 xq = *(const floatx4*)(xs + e);
#pragma unroll
                        for (int b = 0; b < 4; b++) acc = fmaf(__uint_as_float(wv[u][b]), xq[b], acc);
                    } else {
                        const floatx4 xa = *(const floatx4*)(xs + e), xb = *(const floatx4*)(xs + e + 4);
#pragma unroll
                        for (int b = 0; b < 4; b++) {
                            const float xl = b < 2 ? xa[2 * b] : xb[2 * b - 4];
                            const float xh = b < 2 ? xa[2 * b + 1] : xb[2 * b - 3];
                            acc = fmaf(h2f(wv[u][b] & 0xFFFF), xl, acc);
                            acc = fmaf(h2f(wv[u][b] >> 16), xh, acc);
                        }
                    }
                }
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int u = 64 * k + lane;
            if (u < nu) {
                const u32x4 hdr = wv[3 * k], qa = wv[3 * k + 1], qb = wv[3 * k + 2];
                const int jj = u & 3;
                const float* xu = xs + xp(64 * u);
                const float d = h2f(hdr.x & 0xFFFF), dmin = h2f(hdr.x >> 16);
                unsigned sc, mn;
                scale_min_k4_regs(2 * jj, hdr.y, hdr.z, hdr.w, sc, mn);
                const float d1 = d * (float)sc, m1 = dmin * (float)mn;
                scale_min_k4_regs(2 * jj + 1, hdr.y, hdr.z, hdr.w, sc, mn);
                const float d2 = d * (float)sc, m2 = dmin * (float)mn;
                // sum over a group of (d q - m) x = d sum q x - m sum x: per
                // element one nibble, one conversion and one fused product
                const unsigned q8[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
                float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const floatx4 xl = *(const floatx4*)(xu + 4 * i), xh = *(const floatx4*)(xu + 32 + 4 * i);
#pragma unroll
                    for (int b = 0; b < 4; b++) {
                        const unsigned byte = (q8[i] >> (8 * b)) & 0xFF;
                        s1 = fmaf((float)(byte & 0xF), xl[b], s1);
                        s2 = fmaf((float)(byte >> 4), xh[b], s2);
                    }
                }
                acc = fmaf(d1, s1, acc);
                acc = fmaf(-m1, xg[2 * u], acc);
                acc = fmaf(d2, s2, acc);
                acc = fmaf(-m2, xg[2 * u + 1], acc);
            }
        }
    }
    acc = group_sum<64>(acc);
    if (lane == 0) {
        if (m.b) acc = acc + (m.btype == GG_F32 ? ((const float*)m.b)[row] : h2f(ld16(m.b + 2 * row)));
        m.out[row] = m.add_out ? m.out[row] + acc : acc;
    }
}

// LDS: x [n] floats, the raw chunk ring (kProjSlots x 8 x kProjChunkMax
// bytes) and two product buffers (64 x kPS floats each).
__host__ __device__ inline size_t proj_x_bytes(int n) { return ((size_t)n * 4 + 15) / 16 * 16; }
constexpr int kProjFixedLds = kProjSlots * kProjSlotBytes + 2 * 64 * kPS * 4;

__global__ __launch_bounds__(64 * kProjWaves) void proj_kernel(const ProjArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    float* xs = (float*)smem;
    uint8_t* ring = smem + proj_x_bytes(a.n);
    float* prod = (float*)(ring + kProjSlots * kProjSlotBytes);
    int mi = 0;
    while (mi + 1 < a.nmat && (int)blockIdx.x >= a.m[mi + 1].wg0) mi++;
    const ProjMat& m = a.m[mi];
    const int lwg = (int)blockIdx.x - m.wg0;
    if (m.fast) {
        switch (m.wtype) {
            case GG_F32: gemv_wg<GG_F32>(m, a.x, xs, a.n, lwg); break;
            case GG_F16: gemv_wg<GG_F16>(m, a.x, xs, a.n, lwg); break;
            case GG_Q4_K: gemv_wg<GG_Q4_K>(m, a.x, xs, a.n, lwg); break;
            default: break;
        }
        return;
    }
    switch (m.wtype) {
        case GG_F32: proj_wg<GG_F32>(m, a.x, xs, ring, prod, a.n, lwg); break;
        case GG_F16: proj_wg<GG_F16>(m, a.x, xs, ring, prod, a.n, lwg); break;
        case GG_Q4_0: proj_wg<GG_Q4_0>(m, a.x, xs, ring, prod, a.n, lwg); break;
        case GG_Q8_0: proj_wg<GG_Q8_0>(m, a.x, xs, ring, prod, a.n, lwg); break;
        case GG_Q4_K: proj_wg<GG_Q4_K>(m, a.x, xs, ring, prod, a.n, lwg); break;
        case GG_Q6_K: proj_wg<GG_Q6_K>(m, a.x, xs, ring, prod, a.n, lwg); break;
        default: break;
    }
}

size_t proj_lds_bytes(int n) { return proj_x_bytes(n) + kProjFixedLds; }
// the any-order q rows use the front of the same allocation: x with 4 floats
// of padding per 64 and one sum per 32-element group
static_assert((PQA_MAX_EMBD + PQA_MAX_EMBD / 16 + PQA_MAX_EMBD / 32) * 4 <= PQA_MAX_EMBD * 4 + kProjFixedLds,
              "padded x and group sums exceed the projection LDS");

}  // namespace pqa

using pqa::hip_check;
using pqa::set_err;

namespace {

int block_elems(int t) {
    switch (t) {
        case pqa::GG_F32: case pqa::GG_F16: return 1;
        case pqa::GG_Q4_0: case pqa::GG_Q8_0: return 32;
        case pqa::GG_Q4_K: case pqa::GG_Q6_K: return 256;
        default: return 0;
    }
}

int block_bytes(int t) {
    switch (t) {
        case pqa::GG_F32: return 4;
        case pqa::GG_F16: return 2;
        case pqa::GG_Q4_0: return 18;
        case pqa::GG_Q8_0: return 34;
        case pqa::GG_Q4_K: return 144;
        case pqa::GG_Q6_K: return 210;
        default: return 0;
    }
}

// Rows are whole blocks; the chunk loop also needs whole 8-element groups
// (F32/F16, no scalar tail) and 4-byte aligned chunk offsets (Q6_K rows of an
// even number of blocks).
const char* shape_problem(int t, int n) {
    const int be = block_elems(t);
    if (!be) return "unsupported weight type (F32, F16, Q4_0, Q8_0, Q4_K, Q6_K)";
    if (n % be) return "n_embd is not a whole number of blocks";
    if ((t == pqa::GG_F32 || t == pqa::GG_F16) && n % 8) return "F32/F16 rows need a multiple of 8 elements";
    if (t == pqa::GG_Q6_K && n % 512) return "Q6_K rows need a multiple of 512 elements";
    if ((t == pqa::GG_Q4_0 || t == pqa::GG_Q8_0) && n % 64) return "Q4_0/Q8_0 rows need a multiple of 64 elements";
    return nullptr;
}

void free_proj(pqa_ctx* c, int layer) {
    auto& p = c->proj[layer];
    for (int i = 0; i < 4; i++) {
        if (p.w[i]) (void)hipFree(p.w[i]);
        if (p.b[i]) (void)hipFree(p.b[i]);
        p.w[i] = p.b[i] = nullptr;
    }
    p.n_embd = 0;
    p.out_rows = 0;
    if (p.split) (void)hipFree(p.split);
    p.split = nullptr;
    if (p.out_split) (void)hipFree(p.out_split);
    p.out_split = nullptr;
    if (p.exact) (void)hipFree(p.exact);
    p.exact = nullptr;
}

}  // namespace

void pqa_free_projections(pqa_ctx* c) {
    for (int l = 0; l < (int)c->proj.size(); l++) free_proj(c, l);
}

// Uploads matrix i of a layer: rows x GGUF rows of n elements, bias or null.
static int upload_matrix(pqa_ctx* ctx, pqa_proj_weights& p, int i, const char* fn, int n, int rows, const void* w,
                         int wt, const void* b, int bt) {
    const size_t rb = (size_t)(n / block_elems(wt)) * block_bytes(wt);
    const size_t stride = (rb + 15) & ~(size_t)15;
    // rows repacked at a 16-byte stride, plus a tail a chunk load may touch
    if (int rc = hip_check(ctx, hipMalloc(&p.w[i], stride * rows + 64), fn)) return rc;
    if (int rc = hip_check(ctx, hipMemset(p.w[i], 0, stride * rows + 64), fn)) return rc;
    if (int rc = hip_check(ctx, hipMemcpy2D(p.w[i], stride, w, rb, rb, rows, hipMemcpyHostToDevice), fn)) return rc;
    p.wtype[i] = wt;
    p.stride[i] = (int)stride;
    p.btype[i] = pqa::GG_NONE;
    if (b && bt != pqa::GG_NONE) {
        const size_t bb = (size_t)rows * (bt == pqa::GG_F32 ? 4 : 2);
        if (int rc = hip_check(ctx, hipMalloc(&p.b[i], bb), fn)) return rc;
        if (int rc = hip_check(ctx, hipMemcpy(p.b[i], b, bb, hipMemcpyHostToDevice), fn)) return rc;
        p.btype[i] = bt;
    }
    return PQA_OK;
}

static void free_matrix(pqa_proj_weights& p, int i) {
    if (p.w[i]) (void)hipFree(p.w[i]);
    if (p.b[i]) (void)hipFree(p.b[i]);
    p.w[i] = p.b[i] = nullptr;
}

static int allow_lds(pqa_ctx* ctx, const char* fn) {
    // x and the chunk rings can exceed the default 64 KB of dynamic LDS. The
    // attribute belongs to the kernel, process-wide, not to a context or a
    // layer: it is always set to what the widest allowed input needs, so a
    // later call for a narrower matrix never lowers it below what another
    // matrix's launches request.
    return hip_check(ctx, hipFuncSetAttribute((const void*)pqa::proj_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                              (int)pqa::proj_lds_bytes(PQA_MAX_EMBD)), fn);
}

extern "C" int pqa_set_qkv_weights(pqa_ctx* ctx, int layer, int n_embd, const void* wq, int wq_type, const void* bq,
                                   int bq_type, const void* wk, int wk_type, const void* bk, int bk_type,
                                   const void* wv, int wv_type, const void* bv, int bv_type) {
    static const char* fn = "pqa_set_qkv_weights";
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_set_qkv_weights: ctx is NULL");
    if (layer < 0 || layer >= ctx->n_layers) return set_err(ctx, PQA_ERR_ARG, "pqa_set_qkv_weights: bad layer");
    if (n_embd <= 0 || n_embd > PQA_MAX_EMBD)
        return set_err(ctx, PQA_ERR_UNSUPPORTED, "pqa_set_qkv_weights: n_embd outside [1, 8192]");
    const void* w[3] = {wq, wk, wv};
    const void* b[3] = {bq, bk, bv};
    const int wt[3] = {wq_type, wk_type, wv_type};
    const int bt[3] = {bq_type, bk_type, bv_type};
    const int rows[3] = {(int)ctx->q_dim, (int)ctx->kv_dim, (int)ctx->kv_dim};
    for (int i = 0; i < 3; i++) {
        if (!w[i]) return set_err(ctx, PQA_ERR_ARG, "pqa_set_qkv_weights: weight pointer is NULL");
        if (const char* why = shape_problem(wt[i], n_embd))
            return set_err(ctx, PQA_ERR_UNSUPPORTED, std::string(fn) + ": " + why);
        if (b[i] && bt[i] != pqa::GG_NONE && bt[i] != pqa::GG_F32 && bt[i] != pqa::GG_F16)
            return set_err(ctx, PQA_ERR_UNSUPPORTED, "pqa_set_qkv_weights: bias type must be F32 or F16");
    }
    if (ctx->proj.empty()) ctx->proj.resize(ctx->n_layers);
    auto& p = ctx->proj[layer];
    for (int i = 0; i < 3; i++) free_matrix(p, i);
    if (p.split) (void)hipFree(p.split);  // the batched path's copies of the old rows
    p.split = nullptr;
    if (p.exact) (void)hipFree(p.exact);
    p.exact = nullptr;
    p.n_embd = 0;
    for (int i = 0; i < 3; i++)
        if (int rc = upload_matrix(ctx, p, i, fn, n_embd, rows[i], w[i], wt[i], b[i], bt[i])) {
            for (int j = 0; j < 3; j++) free_matrix(p, j);
            return rc;
        }
    p.n_embd = n_embd;
    return allow_lds(ctx, fn);
}

extern "C" int pqa_set_out_weights(pqa_ctx* ctx, int layer, int n_embd, const void* wo, int wo_type, const void* bo,
                                   int bo_type) {
    static const char* fn = "pqa_set_out_weights";
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_set_out_weights: ctx is NULL");
    if (layer < 0 || layer >= ctx->n_layers) return set_err(ctx, PQA_ERR_ARG, "pqa_set_out_weights: bad layer");
    if (n_embd <= 0 || !wo) return set_err(ctx, PQA_ERR_ARG, "pqa_set_out_weights: bad n_embd or NULL weights");
    const int width = (int)ctx->q_dim;  // attn_output rows are q_dim wide
    if (width > PQA_MAX_EMBD)
        return set_err(ctx, PQA_ERR_UNSUPPORTED, "pqa_set_out_weights: n_heads * head_dim above 8192");
    if (const char* why = shape_problem(wo_type, width))
        return set_err(ctx, PQA_ERR_UNSUPPORTED, std::string(fn) + ": " + why);
    if (bo && bo_type != pqa::GG_NONE && bo_type != pqa::GG_F32 && bo_type != pqa::GG_F16)
        return set_err(ctx, PQA_ERR_UNSUPPORTED, "pqa_set_out_weights: bias type must be F32 or F16");
    if (ctx->proj.empty()) ctx->proj.resize(ctx->n_layers);
    auto& p = ctx->proj[layer];
    free_matrix(p, 3);
    if (p.out_split) (void)hipFree(p.out_split);  // the batched path's copy of the old rows
    p.out_split = nullptr;
    p.out_rows = 0;
    if (int rc = upload_matrix(ctx, p, 3, fn, width, n_embd, wo, wo_type, bo, bo_type)) {
        free_matrix(p, 3);
        return rc;
    }
    p.out_rows = n_embd;
    return allow_lds(ctx, fn);
}

namespace pqa {

hipError_t launch_qkv_project(pqa_ctx* ctx, int layer, const float* xb, float* q, float* k, float* v) {
    const auto& p = ctx->proj[layer];
    ProjArgs a;
    float* outs[3] = {q, k, v};
    const int rows[3] = {(int)ctx->q_dim, (int)ctx->kv_dim, (int)ctx->kv_dim};
    // q on the any-order rows when its type has them: its workgroups (one row
    // per wave) come after K's and V's, which keep the reference's order and
    // take longer, so both kinds share the CUs in one round
    const bool fast_q = !ctx->token_exact_q && gemv_type(p.wtype[0]);
    const int order[3] = {fast_q ? 1 : 0, fast_q ? 2 : 1, fast_q ? 0 : 2};
    int wgs = 0;
    for (int j = 0; j < 3; j++) {
        const int i = order[j];
        a.m[j].w = (const uint8_t*)p.w[i];
        a.m[j].b = (const uint8_t*)p.b[i];
        a.m[j].out = outs[i];
        a.m[j].add_out = 0;
        a.m[j].rows = rows[i];
        a.m[j].wtype = p.wtype[i];
        a.m[j].btype = p.btype[i];
        a.m[j].stride = p.stride[i];
        a.m[j].wg0 = wgs;
        a.m[j].fast = i == 0 && fast_q;
        wgs += a.m[j].fast ? (rows[i] + kProjWaves - 1) / kProjWaves : (rows[i] + kProjRows - 1) / kProjRows;
    }
    a.x = xb;
    a.n = p.n_embd;
    a.nmat = 3;
    hipLaunchKernelGGL(proj_kernel, dim3(wgs), dim3(64 * kProjWaves), proj_lds_bytes(a.n), ctx->stream, a);
    return hipGetLastError();
}

hipError_t launch_out_project(pqa_ctx* ctx, int layer, const float* attn, float* x) {
    const auto& p = ctx->proj[layer];
    ProjArgs a;
    a.m[0].w = (const uint8_t*)p.w[3];
    a.m[0].b = (const uint8_t*)p.b[3];
    a.m[0].out = x;
    a.m[0].add_out = 1;
    a.m[0].rows = p.out_rows;
    a.m[0].wtype = p.wtype[3];
    a.m[0].btype = p.btype[3];
    a.m[0].stride = p.stride[3];
    a.m[0].wg0 = 0;
    a.m[0].fast = !ctx->out_exact && gemv_type(p.wtype[3]);
    a.x = attn;
    a.n = (int)ctx->q_dim;
    a.nmat = 1;
    const int rpw = a.m[0].fast ? kProjWaves : kProjRows;  // rows per workgroup
    hipLaunchKernelGGL(proj_kernel, dim3((p.out_rows + rpw - 1) / rpw), dim3(64 * kProjWaves),
                       proj_lds_bytes(a.n), ctx->stream, a);
    return hipGetLastError();
}

}  // namespace pqa

static int check_proj(pqa_ctx* ctx, int layer, const char* fn) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, std::string(fn) + ": ctx is NULL");
    if (layer < 0 || layer >= ctx->n_layers) return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": bad layer");
    if (ctx->proj.empty() || !ctx->proj[layer].n_embd)
        return set_err(ctx, PQA_ERR_ARG, std::string(fn) + ": no projection weights for this layer");
    return PQA_OK;
}

extern "C" int pqa_set_token_projection(pqa_ctx* ctx, int exact_q) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_set_token_projection: ctx is NULL");
    if (exact_q != 0 && exact_q != 1) return set_err(ctx, PQA_ERR_ARG, "pqa_set_token_projection: exact_q must be 0 or 1");
    ctx->token_exact_q = exact_q;
    return PQA_OK;
}

extern "C" int pqa_set_out_projection(pqa_ctx* ctx, int exact) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_set_out_projection: ctx is NULL");
    if (exact != 0 && exact != 1) return set_err(ctx, PQA_ERR_ARG, "pqa_set_out_projection: exact must be 0 or 1");
    ctx->out_exact = exact;
    return PQA_OK;
}

extern "C" int pqa_qkv_project(pqa_ctx* ctx, int layer, const float* xb, float* q, float* k, float* v) {
    if (int rc = check_proj(ctx, layer, "pqa_qkv_project")) return rc;
    if (!xb || !q || !k || !v) return set_err(ctx, PQA_ERR_ARG, "pqa_qkv_project: NULL pointer");
    return hip_check(ctx, pqa::launch_qkv_project(ctx, layer, xb, q, k, v), "pqa_qkv_project");
}

extern "C" int pqa_decode_x(pqa_ctx* ctx, int layer, int pos, const float* xb, float* out) {
    if (int rc = check_proj(ctx, layer, "pqa_decode_x")) return rc;
    if (!xb || !out) return set_err(ctx, PQA_ERR_ARG, "pqa_decode_x: NULL pointer");
    float* q = ctx->qkv;
    float* k = q + ctx->q_dim;
    float* v = k + ctx->kv_dim;
    if (int rc = hip_check(ctx, pqa::launch_qkv_project(ctx, layer, xb, q, k, v), "pqa_decode_x")) return rc;
    return pqa_decode(ctx, layer, pos, q, k, v, out);
}

extern "C" int pqa_out_project(pqa_ctx* ctx, int layer, const float* attn, float* x) {
    if (!ctx) return set_err(nullptr, PQA_ERR_ARG, "pqa_out_project: ctx is NULL");
    if (layer < 0 || layer >= ctx->n_layers) return set_err(ctx, PQA_ERR_ARG, "pqa_out_project: bad layer");
    if (ctx->proj.empty() || !ctx->proj[layer].out_rows)
        return set_err(ctx, PQA_ERR_ARG, "pqa_out_project: no attn_output weights for this layer");
    if (!attn || !x) return set_err(ctx, PQA_ERR_ARG, "pqa_out_project: NULL pointer");
    return hip_check(ctx, pqa::launch_out_project(ctx, layer, attn, x), "pqa_out_project");
}

extern "C" int pqa_attention_block(pqa_ctx* ctx, int layer, int pos, const float* xb, float* x) {
    if (int rc = check_proj(ctx, layer, "pqa_attention_block")) return rc;
    if (!ctx->proj[layer].out_rows)
        return set_err(ctx, PQA_ERR_ARG, "pqa_attention_block: no attn_output weights for this layer");
    if (!xb || !x) return set_err(ctx, PQA_ERR_ARG, "pqa_attention_block: NULL pointer");
    float* attn = ctx->qkv + ctx->q_dim + 2 * ctx->kv_dim;
    if (int rc = pqa_decode_x(ctx, layer, pos, xb, attn)) return rc;
    return hip_check(ctx, pqa::launch_out_project(ctx, layer, attn, x), "pqa_attention_block");
}
