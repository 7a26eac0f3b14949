// synth.hip -- on-device synthetic weights and states for the benchmark model.
//
// Counter-based generator: value i of stream `seed` is a function of (seed, i)
// only (splitmix64 finaliser), so results do not depend on launch geometry.
// Normals by Box-Muller.  Distributions follow the benchmark configs: e4m3 bytes
// uniform with the NaN codes redrawn, block scales log-uniform, N(mean, std).
#include "internal.h"

using namespace rl;

namespace {

__device__ inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ inline float unit01(uint64_t r) { return (static_cast<float>(r >> 40) + 0.5f) * (1.f / 16777216.f); }

__device__ inline float normal(uint64_t seed, size_t i) {
    const uint64_t r = mix64(seed ^ mix64(i));
    const float u1 = unit01(r), u2 = unit01(mix64(r));
    return sqrtf(-2.f * logf(u1)) * cospif(2.f * u2);
}

__global__ void fill_fp8_kernel(uint8_t* p, size_t n, uint64_t seed) {
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        uint64_t r = mix64(seed ^ mix64(i));
        uint8_t b = static_cast<uint8_t>(r);
        while ((b & 0x7f) == 0x7f) {  // 0x7F / 0xFF are NaN in e4m3fn: redraw
            r = mix64(r);
            b = static_cast<uint8_t>(r);
        }
        p[i] = b;
    }
}

__global__ void fill_loguniform_kernel(float* p, size_t n, float lo, float hi, uint64_t seed) {
    const float a = logf(lo), b = logf(hi);
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        p[i] = expf(a + (b - a) * unit01(mix64(seed ^ mix64(i))));
}

__global__ void fill_normal_f32_kernel(float* p, size_t n, float mean, float stdv, uint64_t seed) {
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        p[i] = mean + stdv * normal(seed, i);
}

__global__ void fill_normal_16_kernel(uint16_t* p, size_t n, float stdv, uint64_t seed, int bf16) {
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const float v = stdv * normal(seed, i);
        p[i] = bf16 ? static_cast<uint16_t>(__float_as_uint(v) >> 16)
                    : __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
    }
}

// GGML K-quant super-blocks: random quant / scale bytes, fp16 d (and dmin)
// log-uniform in [1e-4, 1e-2]
__global__ void fill_kquant_kernel(uint8_t* p, size_t n_bytes, int bsz, int d_off, int n_d, uint64_t seed) {
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n_bytes;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const size_t b = i / bsz;
        const int off = static_cast<int>(i % bsz);
        uint8_t v;
        if (off >= d_off && off < d_off + 2 * n_d) {
            const int f = (off - d_off) >> 1;
            const float u = unit01(mix64(seed ^ mix64(2 * b + f + 0x5bd1e995ull)));
            const float d = expf(logf(1e-4f) + (logf(1e-2f) - logf(1e-4f)) * u);
            const uint16_t h = __builtin_bit_cast(uint16_t, static_cast<_Float16>(d));
            v = static_cast<uint8_t>(((off - d_off) & 1) ? h >> 8 : h & 0xff);
        } else {
            v = static_cast<uint8_t>(mix64(seed ^ mix64(i)));
        }
        p[i] = v;
    }
}

constexpr int kGrid = 4096;

}  // namespace

namespace rl {

void fill_kquant(uint8_t* p, int type, size_t n_blocks, uint64_t seed, hipStream_t s) {
    const int bsz = type == RL_Q_Q4_K ? 144 : 210;
    const int d_off = type == RL_Q_Q4_K ? 0 : 208, n_d = type == RL_Q_Q4_K ? 2 : 1;
    hipLaunchKernelGGL(fill_kquant_kernel, dim3(kGrid), dim3(256), 0, s, p, n_blocks * bsz, bsz, d_off, n_d, seed);
    check_launch("fill_kquant_kernel");
}

void fill_fp8(uint8_t* p, size_t n, uint64_t seed, hipStream_t s) {
    hipLaunchKernelGGL(fill_fp8_kernel, dim3(kGrid), dim3(256), 0, s, p, n, seed);
    check_launch("fill_fp8_kernel");
}
void fill_loguniform(float* p, size_t n, float lo, float hi, uint64_t seed, hipStream_t s) {
    hipLaunchKernelGGL(fill_loguniform_kernel, dim3(kGrid), dim3(256), 0, s, p, n, lo, hi, seed);
    check_launch("fill_loguniform_kernel");
}
void fill_normal_f32(float* p, size_t n, float mean, float stdv, uint64_t seed, hipStream_t s) {
    hipLaunchKernelGGL(fill_normal_f32_kernel, dim3(kGrid), dim3(256), 0, s, p, n, mean, stdv, seed);
    check_launch("fill_normal_f32_kernel");
}
void fill_normal_bf16(uint16_t* p, size_t n, float stdv, uint64_t seed, hipStream_t s) {
    hipLaunchKernelGGL(fill_normal_16_kernel, dim3(kGrid), dim3(256), 0, s, p, n, stdv, seed, 1);
    check_launch("fill_normal_16_kernel");
}
void fill_normal_f16(uint16_t* p, size_t n, float stdv, uint64_t seed, hipStream_t s) {
    hipLaunchKernelGGL(fill_normal_16_kernel, dim3(kGrid), dim3(256), 0, s, p, n, stdv, seed, 0);
    check_launch("fill_normal_16_kernel");
}

}  // namespace rl
