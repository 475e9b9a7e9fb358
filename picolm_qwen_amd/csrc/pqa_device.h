// Device-side building blocks shared by the decode and prefill kernels:
// the reference's fp16 rounding, its per-head RMSNorm reduction order and the
// three RoPE pairings. Everything that feeds a K row written to the cache is
// evaluated without FMA contraction so the fp16 bits match the reference.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pqa {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short short4v __attribute__((ext_vector_type(4)));

// fp32 -> fp16 exactly as cpp/quant.hpp:102-135 rounds: the magnitude gets
// half an fp16 ulp added and is truncated (nearest, ties away from zero;
// |x| >= 2^16 -> infinity, |x| < 2^-25 -> signed zero, NaN -> sign|0x7E00).
// Computed branch-free with the hardware conversion, which rounds to nearest
// even with fp16 subnormals kept: when the first bit the fp16 value drops
// (bit sh1 of the significand with its hidden bit: 12 for normal results,
// 13..23 for subnormal ones, clamped to 24 below them, where it is 0) is
// set, fp32 bit 0 is set too, which turns an exact tie into "above half"
// and changes no other rounding; NaN gets the reference's bits. Equal to
// the reference's bit procedure on all 2^32 inputs.
__device__ __forceinline__ uint16_t f32_to_f16_ref(float f) {
    const uint32_t bits = __float_as_uint(f);
    const uint32_t be = (bits >> 23) & 0xFFu;
    const int sh1 = min(max(125 - (int)be, 12), 24);
    const uint32_t m1 = (bits & 0x7FFFFFu) | 0x800000u;  // significand with the hidden bit
    const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)__uint_as_float(bits | ((m1 >> sh1) & 1u)));
    return (be == 255u && (bits & 0x7FFFFFu)) ? (uint16_t)(((bits >> 16) & 0x8000u) | 0x7E00u) : h;
}

// fp16 bits -> fp32: exact widening (the hardware conversion equals
// cpp/quant.hpp:73-100 for every input, subnormals included).
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// Inverse RMS of one head the way cpp/tensor.hpp:146-176 computes it on x86:
// four SSE lane sums (lane j takes x[i] for i = j mod 4 while i+3 < n, in
// increasing i), horizontal sum (l0+l2)+(l1+l3) (cpp/quant.hpp:296-302),
// scalar tail, then 1/sqrt(ss/n + 1e-6). Called by one thread per head.
__device__ __forceinline__ float rms_scale_ref(const float* x, int n) {
#pragma clang fp contract(off)
    float l0 = 0.0f, l1 = 0.0f, l2 = 0.0f, l3 = 0.0f;
    int i = 0;
    for (; i + 3 < n; i += 4) {
        l0 = l0 + x[i] * x[i];
        l1 = l1 + x[i + 1] * x[i + 1];
        l2 = l2 + x[i + 2] * x[i + 2];
        l3 = l3 + x[i + 3] * x[i + 3];
    }
    float ss = (l0 + l2) + (l1 + l3);
    for (; i < n; i++) ss = ss + x[i] * x[i];
    return 1.0f / sqrtf(ss / (float)n + 1e-6f);
}

// Same reduction split over the 4 lanes of a quad (lane j owns SSE lane j);
// every lane of the quad returns the scale. The lane sums are sequential in
// i exactly as above; the quad exchange only moves finished values.
// Must be called by all 4 lanes of the quad together.
__device__ __forceinline__ float rms_scale_ref_quad(const float* x, int n, int j) {
#pragma clang fp contract(off)
    float l = 0.0f;
    const int nfull = n & ~3;
    // the reads do not depend on the sums: unrolled, they are all in flight
    // before the (sequential) adds need them
#pragma unroll 8
    for (int i = j; i < nfull; i += 4) l = l + x[i] * x[i];
    const float L0 = __shfl(l, 0, 4), L1 = __shfl(l, 1, 4);
    const float L2 = __shfl(l, 2, 4), L3 = __shfl(l, 3, 4);
    float ss = (L0 + L2) + (L1 + L3);
    for (int i = nfull; i < n; i++) ss = ss + x[i] * x[i];
    return 1.0f / sqrtf(ss / (float)n + 1e-6f);
}

// The same for a head size known at compile time (N a multiple of 4): a fixed
// trip count, so all N / 4 reads of lane j are issued before the adds, which
// keep their order (a loop with the lane-dependent bound above read one value
// per LDS round trip: 1.8 us at N = 128).
template <int N>
__device__ __forceinline__ float rms_scale_ref_quad(const float* x, int j) {
#pragma clang fp contract(off)
    static_assert(N % 4 == 0, "whole SSE groups");
    float v[N / 4];
#pragma unroll
    for (int k = 0; k < N / 4; k++) v[k] = x[4 * k + j];
    float l = 0.0f;
#pragma unroll
    for (int k = 0; k < N / 4; k++) l = l + v[k] * v[k];
    const float L0 = __shfl(l, 0, 4), L1 = __shfl(l, 1, 4);
    const float L2 = __shfl(l, 2, 4), L3 = __shfl(l, 3, 4);
    const float ss = (L0 + L2) + (L1 + L3);
    return 1.0f / sqrtf(ss / (float)N + 1e-6f);
}

// Element indices of RoPE pair p (0 <= p < hd/2) for each pairing; the angle
// is always p. Block8: full blocks of 4 pairs (4b+3 < half) pair 8b+j with
// 8b+4+j (j = p mod 4); pairs past the last full block use the interleaved
// tail (cpp/tensor.hpp:316-323).
__device__ __forceinline__ void rope_pair(int style, int p, int hd, int& e0, int& e1) {
    const int half = hd >> 1;
    if (style == 0) {
        e0 = p;
        e1 = p + half;
    } else if (style == 1 && (p | 3) < half) {
        e0 = ((p >> 2) << 3) + (p & 3);
        e1 = e0 + 4;
    } else {
        e0 = 2 * p;
        e1 = 2 * p + 1;
    }
}

// x' = x0*c - x1*s, y' = x0*s + x1*c with separate roundings (no FMA), as the
// SSE and scalar code of cpp/tensor.hpp does.
__device__ __forceinline__ void rope_rotate(float& x0, float& x1, float c, float s) {
#pragma clang fp contract(off)
    const float a = x0, b = x1;
    x0 = a * c - b * s;
    x1 = a * s + b * c;
}

// The same rotation with fused multiply-adds, for values that are not stored
// (q): two instructions per element instead of three.
__device__ __forceinline__ void rope_rotate_fma(float& x0, float& x1, float c, float s) {
    const float a = x0, b = x1;
    x0 = fmaf(a, c, -(b * s));
    x1 = fmaf(a, s, b * c);
}

// (x * s) * w, rounded twice (cpp/tensor.hpp:168-171).
__device__ __forceinline__ float rms_apply(float x, float s, float w) {
#pragma clang fp contract(off)
    return (x * s) * w;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Materialises a loaded value in registers at this point. Placed after a batch
// of loads whose results are only stored under a predicate, it stops the
// compiler from sinking each load into its predicated block (which would turn
// one memory round trip per batch into one per load).
__device__ __forceinline__ void pin(floatx4& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(float4& x) {
    floatx4 v = {x.x, x.y, x.z, x.w};
    asm volatile("" : "+v"(v));
    x = float4{v[0], v[1], v[2], v[3]};
}

// Orders the calling wave's LDS accesses before this point against those
// after it, for data exchanged between lanes of the same wave (the LDS
// executes one wave's requests in order; this stops the compiler moving
// accesses across the point).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A pointer the caller knows to be wave-uniform, moved to scalar registers.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
    const unsigned long long v = (unsigned long long)p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    return (const void*)(((unsigned long long)hi << 32) | lo);
}

// Byte address in LDS of a pointer into a __shared__ object (take it once,
// outside loops: the generic -> LDS conversion carries a null check).
__device__ __forceinline__ unsigned lds_addr(const void* p) {
    return (unsigned)(size_t)(const __attribute__((address_space(3))) void*)p;
}

// 16 bytes per lane from global memory straight into LDS
// (global_load_lds_dwordx4): lane l's bytes land at LDS byte address
// lds + 16 l. base and lds must be wave-uniform; voff is the lane's byte
// offset from base. Issued from inline asm on purpose: the compiler then does
// not track the LDS write, so it does not make every later LDS read wait for
// this load (the callers order these loads against reads of the same bytes
// with an explicit s_waitcnt vmcnt(0) and a barrier, and never read a buffer
// that has a load in flight).
__device__ __forceinline__ void lds_dma_b128(const void* base, unsigned voff, unsigned lds) {
    base = uniform_ptr(base);
    lds = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}

// The same with the non-temporal hint: data read once (streaming), kept from
// displacing reused lines in the caches.
__device__ __forceinline__ void lds_dma_b128_nt(const void* base, unsigned voff, unsigned lds) {
    base = uniform_ptr(base);
    lds = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt"
                 :
                 : "v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}

// 4 bytes per lane (global_load_lds_dword): lane l's dword lands at LDS byte
// address lds + 4 l. Same contract as lds_dma_b128.
__device__ __forceinline__ void lds_dma_b32(const void* base, unsigned voff, unsigned lds) {
    base = uniform_ptr(base);
    lds = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1"
                 :
                 : "v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}

// ---- cross-lane exchanges without LDS round trips ----
// DPP controls: quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1] (lane ^ 2),
// row_half_mirror (lane ^ 7 within 8), row_mirror (lane ^ 15 within 16),
// row_ror:8 (lane ^ 8 within 16), row_ror:4 (not an involution).
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppXor7 = 0x141;
constexpr int kDppXor15 = 0x140;
constexpr int kDppXor8 = 0x128;
constexpr int kDppRor4 = 0x124;  // row_ror:4: lane i of a 16-lane row reads lane (i + 4) mod 16

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// gfx950 v_permlane16_swap / v_permlane32_swap with both operands = x: both
// lanes of a pair (lane, lane ^ 16) resp. (lane, lane ^ 32) receive lo = the
// value of the pair's lower lane and hi = that of its upper lane.
__device__ __forceinline__ void pair16(float x, float& lo, float& hi) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    lo = __builtin_bit_cast(float, (unsigned)r[0]);
    hi = __builtin_bit_cast(float, (unsigned)r[1]);
}
__device__ __forceinline__ void pair32(float x, float& lo, float& hi) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    lo = __builtin_bit_cast(float, (unsigned)r[0]);
    hi = __builtin_bit_cast(float, (unsigned)r[1]);
}
__device__ __forceinline__ float sum_x16(float x) {
    float lo, hi;
    pair16(x, lo, hi);
    return lo + hi;
}
__device__ __forceinline__ float sum_x32(float x) {
    float lo, hi;
    pair32(x, lo, hi);
    return lo + hi;
}
__device__ __forceinline__ float max_x16(float x) {
    float lo, hi;
    pair16(x, lo, hi);
    return fmaxf(lo, hi);
}
__device__ __forceinline__ float max_x32(float x) {
    float lo, hi;
    pair32(x, lo, hi);
    return fmaxf(lo, hi);
}

// Sum / max over aligned groups of N lanes (N = 2..64) by butterflies whose
// partner relation is symmetric, so every lane of a group ends with the same
// bits (a + b == b + a exactly).
template <int N>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (N > 1) x = x + dpp_f<kDppXor1>(x);
    if constexpr (N > 2) x = x + dpp_f<kDppXor2>(x);
    if constexpr (N > 4) x = x + dpp_f<kDppXor7>(x);
    if constexpr (N > 8) x = x + dpp_f<kDppXor15>(x);
    if constexpr (N > 16) x = sum_x16(x);
    if constexpr (N > 32) x = sum_x32(x);
    return x;
}
template <int N>
__device__ __forceinline__ float group_max(float x) {
    if constexpr (N > 1) x = fmaxf(x, dpp_f<kDppXor1>(x));
    if constexpr (N > 2) x = fmaxf(x, dpp_f<kDppXor2>(x));
    if constexpr (N > 4) x = fmaxf(x, dpp_f<kDppXor7>(x));
    if constexpr (N > 8) x = fmaxf(x, dpp_f<kDppXor15>(x));
    if constexpr (N > 16) x = max_x16(x);
    if constexpr (N > 32) x = max_x32(x);
    return x;
}

// Value of lane `src` of the caller's 16-lane row (DPP row_newbcast). `src`
// must fold to a constant after unrolling; the switch then disappears.
template <int L>
__device__ __forceinline__ float row_bcast_c(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x150 + L, 0xF, 0xF, false));
}

__device__ __forceinline__ float row_bcast(float x, int src) {
    switch (src & 15) {
        case 0: return row_bcast_c<0>(x);
        case 1: return row_bcast_c<1>(x);
        case 2: return row_bcast_c<2>(x);
        case 3: return row_bcast_c<3>(x);
        case 4: return row_bcast_c<4>(x);
        case 5: return row_bcast_c<5>(x);
        case 6: return row_bcast_c<6>(x);
        case 7: return row_bcast_c<7>(x);
        case 8: return row_bcast_c<8>(x);
        case 9: return row_bcast_c<9>(x);
        case 10: return row_bcast_c<10>(x);
        case 11: return row_bcast_c<11>(x);
        case 12: return row_bcast_c<12>(x);
        case 13: return row_bcast_c<13>(x);
        case 14: return row_bcast_c<14>(x);
        default: return row_bcast_c<15>(x);
    }
}

// RoPE of a head spread over lanes as float4s: the caller's lane holds
// elements 4t..4t+3, t = lane mod HD/4, and every lane of the wave calls this
// together (style is uniform). The partner of each element comes from the
// lane that holds it: NeoX pairs (p, p + HD/2) sit HD/8 lanes apart (lane ^ 16
// for HD 128, lane ^ 8 for HD 64), block8 pairs (8b+j, 8b+4+j) in adjacent
// lanes (lane ^ 1), interleaved pairs inside the lane. cs/sn are the cos/sin
// float4 at index rope_angle_f4(style, t): NeoX and block8 element e uses
// component e, interleaved component 2(t&1) + e/2. Same roundings as
// rope_rotate, so K rows stay bit-exact.
template <int HD>
__device__ __forceinline__ int rope_angle_f4(int style, int t) {
    return style == 0 ? t % (HD / 8) : t >> 1;
}

template <int HD>
__device__ __forceinline__ float4 rope_lanes(float4 x, int style, int t, float4 cs, float4 sn) {
    static_assert(HD == 64 || HD == 128, "head_dim");
    float o[4] = {x.x, x.y, x.z, x.w};
    const float cc[4] = {cs.x, cs.y, cs.z, cs.w};
    const float ss[4] = {sn.x, sn.y, sn.z, sn.w};
    if (style == 2) {
        const int b = 2 * (t & 1);
        rope_rotate(o[0], o[1], cc[b], ss[b]);
        rope_rotate(o[2], o[3], cc[b + 1], ss[b + 1]);
        return float4{o[0], o[1], o[2], o[3]};
    }
    float x0[4], x1[4];
    bool first;
    if (style == 0 && HD == 128) {
        first = (t & 16) == 0;
#pragma unroll
        for (int e = 0; e < 4; e++) pair16(o[e], x0[e], x1[e]);
    } else {
        first = style == 0 ? (t & 8) == 0 : (t & 1) == 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float p = style == 0 ? dpp_f<kDppXor8>(o[e]) : dpp_f<kDppXor1>(o[e]);
            x0[e] = first ? o[e] : p;
            x1[e] = first ? p : o[e];
        }
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
        rope_rotate(x0[e], x1[e], cc[e], ss[e]);
        o[e] = first ? x0[e] : x1[e];
    }
    return float4{o[0], o[1], o[2], o[3]};
}

}  // namespace pqa
