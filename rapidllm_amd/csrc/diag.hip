// diag.hip -- calibration and comparison kernels (no counterpart in the reference).
//
// A plain streaming copy and a streaming read of a known number of bytes.  They
// give the achievable HBM rate on the box and the scale factor between rocprof's
// FETCH_SIZE / WRITE_SIZE counters and bytes actually moved.  A VALU T=1 FP8 GEMV
// over the product's weight layout, timed against the matrix-core kernel.
#include <cstdlib>

#include "common.h"
#include "internal.h"

using namespace rl;

namespace {

__global__ void copy_probe_kernel(const i32x4* __restrict__ src, i32x4* __restrict__ dst, size_t n16) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride)
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// Each thread keeps UNROLL independent 16-byte loads in flight.  NT: non-temporal.
template <int UNROLL, bool NT>
__global__ void read_probe_kernel(const i32x4* __restrict__ src, size_t n16, unsigned* __restrict__ out) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    i32x4 acc = {0, 0, 0, 0};
    for (; i + (UNROLL - 1) * stride < n16; i += UNROLL * stride) {
        i32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) v[u] = NT ? __builtin_nontemporal_load(src + i + u * stride) : src[i + u * stride];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc ^= v[u];
    }
    for (; i < n16; i += stride) acc ^= src[i];
    const unsigned x = static_cast<unsigned>(acc[0] ^ acc[1] ^ acc[2] ^ acc[3]);
    if (x == 0x9e3779b9u) out[0] = x;  // practically never taken; keeps the loads live
}

// T=1 block-FP8 GEMV on the VALU, for the comparison with the matrix-core kernel:
// the same tiled weights (tile = 16 rows x 128 columns; lane (g, row) holds row `row`
// at columns 32 g .. 32 g + 31 of each block), 16 waves per row tile as the store
// launches, x staged in LDS as fp32.  Per block: 32 e4m3 -> fp32 conversions and 32
// FMAs per lane, scaled by the block's tile scale; lane groups summed by shuffles,
// waves through LDS.
constexpr int kValuWaves = 16;
__global__ __launch_bounds__(64 * kValuWaves) void valu_gemv_t1_kernel(const uint8_t* __restrict__ W,
                                                                        const float* __restrict__ ts,
                                                                        const float* __restrict__ x,
                                                                        float* __restrict__ y, int m, int n_kb) {
    extern __shared__ float xs[];  // n_kb * 128 floats
    __shared__ float red[kValuWaves][16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, row = lane & 15;
    const int rt = blockIdx.x;
    const uint8_t* wb = W + static_cast<size_t>(rt) * n_kb * 2048;
    const float* sb = ts + static_cast<size_t>(rt) * n_kb;
    for (int i = tid; i < n_kb * 32; i += 64 * kValuWaves)
        reinterpret_cast<float4*>(xs)[i] = reinterpret_cast<const float4*>(x)[i];
    __syncthreads();
    float acc = 0.f;
    for (int kb = wave; kb < n_kb; kb += kValuWaves) {
        const i32x4* tile = reinterpret_cast<const i32x4*>(wb + static_cast<size_t>(kb) * 2048);
        const i32x4 w0 = __builtin_nontemporal_load(tile + lane);
        const i32x4 w1 = __builtin_nontemporal_load(tile + 64 + lane);
        const float s = sb[kb];
        const float4* xp = reinterpret_cast<const float4*>(xs + kb * 128 + 32 * g);
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            const int word = d < 4 ? w0[d] : w1[d - 4];
            const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(word, false);
            const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(word, true);
            const float4 xv = xp[d];
            a0 = fmaf(lo[0], xv.x, a0);
            a1 = fmaf(lo[1], xv.y, a1);
            a0 = fmaf(hi[0], xv.z, a0);
            a1 = fmaf(hi[1], xv.w, a1);
        }
        acc = fmaf(a0 + a1, s, acc);
    }
    acc += __shfl_xor(acc, 16, 64);
    acc += __shfl_xor(acc, 32, 64);
    if (g == 0) red[wave][row] = acc;
    __syncthreads();
    if (tid < 16) {
        float t = 0.f;
        for (int w = 0; w < kValuWaves; ++w) t += red[w][tid];
        const int r = rt * 16 + tid;
        if (r < m) y[r] = t;
    }
}

}  // namespace

extern "C" {

int rl_hip_copy_probe(const void* src, void* dst, size_t bytes, void* stream) {
    return guard([&] {
        RL_REQUIRE(bytes % 16 == 0 && src && dst, RL_ERR_RANGE, "copy_probe: bytes must be a multiple of 16");
        hipLaunchKernelGGL(copy_probe_kernel, dim3(256 * 8), dim3(256), 0, S(stream),
                           static_cast<const i32x4*>(src), static_cast<i32x4*>(dst), bytes / 16);
        check_launch("copy_probe_kernel");
    });
}

int rl_hip_read_probe(const void* src, size_t bytes, void* out4, void* stream) {
    return guard([&] {
        RL_REQUIRE(bytes % 16 == 0 && src && out4, RL_ERR_RANGE, "read_probe: bytes must be a multiple of 16");
        // env RL_PROBE_TEMPORAL=1: ordinary loads (allocate in caches) instead of non-temporal
        static const bool temporal = [] {
            const char* v = std::getenv("RL_PROBE_TEMPORAL");
            return v && v[0] == '1';
        }();
        if (temporal)
            hipLaunchKernelGGL((read_probe_kernel<8, false>), dim3(256 * 8), dim3(256), 0, S(stream),
                               static_cast<const i32x4*>(src), bytes / 16, static_cast<unsigned*>(out4));
        else
            hipLaunchKernelGGL((read_probe_kernel<8, true>), dim3(256 * 8), dim3(256), 0, S(stream),
                               static_cast<const i32x4*>(src), bytes / 16, static_cast<unsigned*>(out4));
        check_launch("read_probe_kernel");
    });
}

int rl_hip_norm_group_rows(void) { return norm_group_rows(); }

int rl_hip_time_gemm_fp8(const void* const* w_copies, int n_copies, const float* tile_scales, const void* frag,
                         float* Y, void* frag_out, const float* gamma, float* sumsq, const float* block_sumsq,
                         const float* sumsq_in, int m, int n, int T, int epilogue, int split, int iters,
                         void* stream, float* avg_ms) {
    return guard([&] {
        RL_REQUIRE(w_copies && n_copies >= 1 && iters >= 1 && avg_ms, RL_ERR_RANGE, "time_gemm: bad arguments");
        RL_REQUIRE(epilogue == kEpiStore || epilogue == kEpiPartial || epilogue == kEpiSwiGLU ||
                       epilogue == kEpiSwiGLUH || epilogue == kEpiAddNorm,
                   RL_ERR_RANGE, "time_gemm: epilogue must be store, partial, swiglu or add-norm");
        const hipStream_t s = S(stream);
        const bool sw = epilogue == kEpiSwiGLU || epilogue == kEpiSwiGLUH;
        const int ldy = sw ? m / 2 : m;
        const int m_valid = ldy;
        const int S_ = epilogue == kEpiPartial ? split : 1;
        void* fo = sw || epilogue == kEpiAddNorm ? frag_out : nullptr;
        NormIO io;
        io.gamma_out = gamma;
        io.ss_out = sumsq;
        RL_REQUIRE(!block_sumsq || epilogue == kEpiAddNorm, RL_ERR_RANGE, "time_gemm: block scale with add-norm only");
        io.kss = block_sumsq;
        io.kss_n = 128;
        io.kss_eps = 1e-6f;
        RL_REQUIRE(!sumsq_in || epilogue == kEpiStore || sw, RL_ERR_RANGE,
                   "time_gemm: input sums of squares with store or swiglu only");
        if (sumsq_in) {
            io.ss_in = sumsq_in;
            io.groups_in = add_norm_groups(n);
            io.n_norm = n;
            io.eps = 1e-6f;
        }
        const NormIO* iop = epilogue == kEpiAddNorm || sumsq_in ? &io : nullptr;
        hipEvent_t a, b;
        RL_HIP(hipEventCreate(&a));
        RL_HIP(hipEventCreate(&b));
        RL_HIP(hipEventRecord(a, s));
        for (int i = 0; i < iters; ++i)
            rl::gemm_fp8_frag(static_cast<const uint8_t*>(w_copies[i % n_copies]), tile_scales, frag,
                              fo && sw ? nullptr : Y, m, n, T, epilogue, ldy, m_valid, s, S_, fo,
                              iop);
        RL_HIP(hipEventRecord(b, s));
        RL_HIP(hipEventSynchronize(b));
        float ms = 0.f;
        RL_HIP(hipEventElapsedTime(&ms, a, b));
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        *avg_ms = ms / iters;
    });
}

// The VALU T=1 GEMV above: `iters` launches cycling over n_copies weight copies,
// one event pair around the loop.  No counterpart in the reference.
int rl_hip_time_gemv_fp8_valu(const void* const* w_copies, int n_copies, const float* tile_scales, const float* X,
                              float* Y, int m, int n, int iters, void* stream, float* avg_ms) {
    return guard([&] {
        RL_REQUIRE(w_copies && n_copies >= 1 && iters >= 1 && avg_ms && tile_scales && X && Y, RL_ERR_RANGE,
                   "time_gemv_valu: bad arguments");
        RL_REQUIRE(m > 0 && n > 0 && n % 128 == 0 && n <= 16384, RL_ERR_RANGE,
                   "time_gemv_valu: n a multiple of 128, at most 16384 (x in LDS)");
        const hipStream_t s = S(stream);
        const int n_kb = n / 128, mt = (m + 15) / 16;
        hipEvent_t a, b;
        RL_HIP(hipEventCreate(&a));
        RL_HIP(hipEventCreate(&b));
        RL_HIP(hipEventRecord(a, s));
        for (int i = 0; i < iters; ++i)
            hipLaunchKernelGGL(valu_gemv_t1_kernel, dim3(mt), dim3(64 * kValuWaves), static_cast<size_t>(n) * 4, s,
                               static_cast<const uint8_t*>(w_copies[i % n_copies]), tile_scales, X, Y, m, n_kb);
        check_launch("valu_gemv_t1_kernel");
        RL_HIP(hipEventRecord(b, s));
        RL_HIP(hipEventSynchronize(b));
        float ms = 0.f;
        RL_HIP(hipEventElapsedTime(&ms, a, b));
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        *avg_ms = ms / iters;
    });
}

// Average duration of `iters` back-to-back K-quant GEMVs (HIP events on the launch
// stream), cycling over n_copies weight copies so every launch reads from HBM.
int rl_hip_time_gemm_kquant(int type, const void* const* w_copies, int n_copies, const float* X, float* Y,
                            void* workspace, size_t workspace_bytes, int m, int n, int T, int iters, void* stream,
                            float* avg_ms) {
    return guard([&] {
        RL_REQUIRE(w_copies && n_copies >= 1 && iters >= 1 && avg_ms, RL_ERR_RANGE, "time_kquant: bad arguments");
        RL_REQUIRE(type == RL_Q_Q4_K || type == RL_Q_Q6_K, RL_ERR_UNSUPPORTED, "time_kquant: Q4_K or Q6_K only");
        const hipStream_t s = S(stream);
        hipEvent_t a, b;
        RL_HIP(hipEventCreate(&a));
        RL_HIP(hipEventCreate(&b));
        RL_HIP(hipEventRecord(a, s));
        for (int i = 0; i < iters; ++i)
            rl::kq_gemm(type == RL_Q_Q4_K ? 4 : 6, static_cast<const uint8_t*>(w_copies[i % n_copies]), X, Y,
                        workspace, workspace_bytes, m, n, T, 0, m, s);
        RL_HIP(hipEventRecord(b, s));
        RL_HIP(hipEventSynchronize(b));
        float ms = 0.f;
        RL_HIP(hipEventElapsedTime(&ms, a, b));
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        *avg_ms = ms / iters;
    });
}

// Average duration of one DeltaNet decode launch (rl_hip_gdn_decode semantics, S
// updated in place) over `iters` passes across n_layers separate layer states.
int rl_hip_time_gdn(float* const* S_layers, int n_layers, const float* qkv, const float* a, const float* b, int ld_in,
                    const float* A_log, const float* dt_bias, const float* conv_w, const float* conv_in,
                    float* conv_out, float* o, int T, int nk, int nv, int dk, int dv, int conv_k, int v_tiled,
                    int iters, void* stream, float* avg_ms) {
    return guard([&] {
        RL_REQUIRE(S_layers && n_layers >= 1 && iters >= 1 && avg_ms, RL_ERR_RANGE, "time_gdn: bad arguments");
        RL_REQUIRE(rl::gdn_fused_supported(dk, dv, conv_k), RL_ERR_UNSUPPORTED, "time_gdn: fused kernel shapes only");
        const hipStream_t s = S(stream);
        hipEvent_t ea, eb;
        RL_HIP(hipEventCreate(&ea));
        RL_HIP(hipEventCreate(&eb));
        RL_HIP(hipEventRecord(ea, s));
        for (int i = 0; i < iters; ++i)
            for (int l = 0; l < n_layers; ++l)
                rl::gdn_decode_fused(qkv, a, b, ld_in, A_log, dt_bias, conv_w, conv_in, conv_out, S_layers[l],
                                     S_layers[l], nullptr, 0, 0, nullptr, o, nullptr, nullptr, nullptr, nullptr, T, nk,
                                     nv, dk, dv, conv_k, v_tiled, s);
        RL_HIP(hipEventRecord(eb, s));
        RL_HIP(hipEventSynchronize(eb));
        float ms = 0.f;
        RL_HIP(hipEventElapsedTime(&ms, ea, eb));
        (void)hipEventDestroy(ea);
        (void)hipEventDestroy(eb);
        *avg_ms = ms / (static_cast<float>(iters) * n_layers);
    });
}

}  // extern "C"
