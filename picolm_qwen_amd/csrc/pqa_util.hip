// Element-wise device helpers: the reference fp16 rounding as a standalone
// op, and the seeded synthetic cache history used by benchmarks and tests.
#include "pqa_device.h"
#include "pqa_internal.h"

namespace pqa {

__global__ void f32_to_f16_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = f32_to_f16_ref(src[i]);
}

hipError_t launch_f32_to_f16(pqa_ctx* ctx, const float* src, uint16_t* dst, size_t n) {
    if (n == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((n + 255) / 256, (size_t)ctx->cu_count * 16);
    hipLaunchKernelGGL(f32_to_f16_kernel, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, src, dst, n);
    return hipGetLastError();
}

// SplitMix64 output number i of a generator seeded with `key` (the state
// after i+1 increments of the golden-ratio gamma, then the finaliser).
__host__ __device__ inline uint64_t splitmix64_at(uint64_t key, uint64_t i) {
    uint64_t z = key + (i + 1u) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ inline double unit_open(uint64_t r) { return ((double)(r >> 11) + 0.5) * 0x1.0p-53; }

// Standard normal number i of stream `key`: Box-Muller on uniforms 2i, 2i+1.
__device__ inline float normal_at(uint64_t key, uint64_t i) {
    const double u1 = unit_open(splitmix64_at(key, 2 * i));
    const double u2 = unit_open(splitmix64_at(key, 2 * i + 1));
    return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

__global__ void synth_kv_kernel(uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int kv_dim, int pos0,
                                int n, uint64_t kkey, uint64_t vkey, uint64_t okey, float prob) {
    const size_t total = (size_t)n * kv_dim;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const size_t r = i / (size_t)kv_dim;
        const uint64_t pos = (uint64_t)pos0 + r;
        const float scale = (prob > 0.0f && unit_open(splitmix64_at(okey, pos)) < (double)prob) ? 8.0f : 1.0f;
        const uint64_t gi = pos * (uint64_t)kv_dim + (i - r * (size_t)kv_dim);
        const size_t off = (size_t)pos * kv_dim + (i - r * (size_t)kv_dim);
        kc[off] = f32_to_f16_ref(normal_at(kkey, gi) * scale);
        vc[off] = f32_to_f16_ref(normal_at(vkey, gi) * scale);
    }
}

static uint64_t stream_key(uint64_t seed, uint32_t kind, uint32_t layer) {
    return splitmix64_at(seed, ((uint64_t)kind << 32) | layer);
}

hipError_t launch_synth_kv(pqa_ctx* ctx, int layer, int pos0, int n, uint64_t seed, float prob) {
    if (n <= 0) return hipSuccess;
    uint16_t* kc = ctx->key_cache + (size_t)layer * ctx->layer_elems;
    uint16_t* vc = ctx->val_cache + (size_t)layer * ctx->layer_elems;
    const size_t total = (size_t)n * ctx->kv_dim;
    const size_t blocks = std::min<size_t>((total + 255) / 256, (size_t)ctx->cu_count * 32);
    // stream kinds 4 (K history), 5 (V history), 8 (outlier flags)
    hipLaunchKernelGGL(synth_kv_kernel, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, kc, vc,
                       (int)ctx->kv_dim, pos0, n, stream_key(seed, 4, (uint32_t)layer),
                       stream_key(seed, 5, (uint32_t)layer), stream_key(seed, 8, (uint32_t)layer), prob);
    return hipGetLastError();
}

}  // namespace pqa
