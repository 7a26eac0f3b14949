// seam.hip -- single-op kernels behind the reference's kernel-name device seam.
//
// rapidllm::Device::launch(name, args, params) (include/rapidllm/backend/device.h:
// 49-60, params.h:5-22) dispatches single ops by name.  The decode engine never
// uses these: its step runs the fused kernels (gdn.hip, attn.hip).  These three
// cover the seam names whose data layout is the reference CPU path's own, so a
// HipDevice can serve them with the reference's buffers unchanged:
//   conv1d_update   ops::conv1d_update   (src/kernels/ops.cpp:458-468)
//   delta_recurrent ops::delta_recurrent_step (ops.cpp:495-540), S row-major
//                   [n_v][dk][dv] as the CPU Session keeps it (not the engine's
//                   transposed state)
//   attn_decode     ops::attn_decode     (ops.cpp:575-605) over fp32 caches
//                   [seq][n_kv][head_dim] (DualCache's CPU layout)
// One workgroup per head (channel block for the conv); these are small launches,
// not the bandwidth-bound hot path.
#include "internal.h"

using namespace rl;
namespace {

__device__ inline float silu_ref(float x) { return x / (1.f + expf(-x)); }

// state [dim][k] (tap 0 oldest): shift left, append x_t, y = silu(sum w * st) with
// a double accumulator (ops.cpp:458-468).
__global__ void conv1d_update_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                     float* __restrict__ state, float* __restrict__ y, int dim, int k) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= dim) return;
    float* st = state + static_cast<size_t>(c) * k;
    for (int p = 0; p + 1 < k; ++p) st[p] = st[p + 1];
    st[k - 1] = x[c];
    double acc = 0.0;
    for (int p = 0; p < k; ++p) acc += static_cast<double>(w[static_cast<size_t>(c) * k + p]) * st[p];
    y[c] = silu_ref(static_cast<float>(acc));
}

// Block-wide double sum over 256 threads (4 waves): wave sums, then the four wave
// results added in wave order.
__device__ inline double block_sum_d(double v, double* red) {
    v = wave_sum_d(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    const double s = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return s;
}

constexpr int kSeamThreads = 256;
constexpr int kSeamMaxDk = 256;

// One head per workgroup; thread j owns value columns j, j + 256, ...
// q, k <- l2norm (x / sqrt(sum x^2 + eps), double sum); q *= 1/sqrt(dk);
// S *= exp(g); kv = S^T k; delta = (v - kv) * beta; S += k delta^T; o = S^T q.
__global__ __launch_bounds__(kSeamThreads) void delta_recurrent_kernel(
    float* __restrict__ S, const float* __restrict__ q_in, const float* __restrict__ k_in,
    const float* __restrict__ v, const float* __restrict__ beta, const float* __restrict__ g_log,
    float* __restrict__ o, int dk, int dv, float eps) {
    __shared__ float qs[kSeamMaxDk], ks[kSeamMaxDk];
    __shared__ double red[4];
    const int h = blockIdx.x;
    const int tid = threadIdx.x;
    const float* qh = q_in + static_cast<size_t>(h) * dk;
    const float* kh = k_in + static_cast<size_t>(h) * dk;
    const float qv = tid < dk ? qh[tid] : 0.f;
    const float kvv = tid < dk ? kh[tid] : 0.f;
    const double sq = block_sum_d(static_cast<double>(qv) * qv, red);
    const double sk = block_sum_d(static_cast<double>(kvv) * kvv, red);
    const float qinv = 1.f / sqrtf(static_cast<float>(sq) + eps);
    const float kinv = 1.f / sqrtf(static_cast<float>(sk) + eps);
    const float scale = 1.f / sqrtf(static_cast<float>(dk));
    if (tid < dk) {
        qs[tid] = (qv * qinv) * scale;
        ks[tid] = kvv * kinv;
    }
    __syncthreads();
    const float g = expf(g_log[h]);
    const float b = beta[h];
    float* Sh = S + static_cast<size_t>(h) * dk * dv;
    for (int j = tid; j < dv; j += kSeamThreads) {
        float kv = 0.f;
        for (int i = 0; i < dk; ++i) {
            const float s = Sh[static_cast<size_t>(i) * dv + j] * g;
            Sh[static_cast<size_t>(i) * dv + j] = s;
            kv += s * ks[i];
        }
        const float delta = (v[static_cast<size_t>(h) * dv + j] - kv) * b;
        float acc = 0.f;
        for (int i = 0; i < dk; ++i) {
            const float s = Sh[static_cast<size_t>(i) * dv + j] + ks[i] * delta;
            Sh[static_cast<size_t>(i) * dv + j] = s;
            acc += s * qs[i];
        }
        o[static_cast<size_t>(h) * dv + j] = acc;
    }
}

// One query head per workgroup, 4 waves.  Wave w takes positions w, w + 4, ...
// with a running max / sum / output (online softmax); lane l holds dims
// l, l + 64, ... (head_dim <= 256).  The four waves' states are merged at the end.
__global__ __launch_bounds__(kSeamThreads) void attn_decode_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ kc, const float* __restrict__ vc, float* __restrict__ o,
    int pos, int n_q, int n_kv, int hd) {
    constexpr int kMaxPer = 4;
    __shared__ float wm[4], wl[4];
    __shared__ float wo[4][256];
    const int hq = blockIdx.x;
    const int hkv = hq / (n_q / n_kv);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const float scale = 1.f / sqrtf(static_cast<float>(hd));
    float qv[kMaxPer], acc[kMaxPer];
#pragma unroll
    for (int e = 0; e < kMaxPer; ++e) {
        const int d = lane + 64 * e;
        qv[e] = d < hd ? q[static_cast<size_t>(hq) * hd + d] : 0.f;
        acc[e] = 0.f;
    }
    float m = -INFINITY, l = 0.f;
    for (int s = w; s <= pos; s += 4) {
        const float* ks = kc + (static_cast<size_t>(s) * n_kv + hkv) * hd;
        const float* vs = vc + (static_cast<size_t>(s) * n_kv + hkv) * hd;
        float part = 0.f;
#pragma unroll
        for (int e = 0; e < kMaxPer; ++e) {
            const int d = lane + 64 * e;
            if (d < hd) part += qv[e] * ks[d];
        }
        const float sc = wave_sum(part) * scale;
        const float mn = fmaxf(m, sc);
        const float corr = expf(m - mn);
        const float p = expf(sc - mn);
        l = l * corr + p;
#pragma unroll
        for (int e = 0; e < kMaxPer; ++e) {
            const int d = lane + 64 * e;
            acc[e] = acc[e] * corr + (d < hd ? p * vs[d] : 0.f);
        }
        m = mn;
    }
    if (lane == 0) {
        wm[w] = m;
        wl[w] = l;
    }
#pragma unroll
    for (int e = 0; e < kMaxPer; ++e) {
        const int d = lane + 64 * e;
        if (d < hd) wo[w][d] = acc[e];
    }
    __syncthreads();
    const float M = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    float f[4], L = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[i] = wl[i] > 0.f ? expf(wm[i] - M) : 0.f;  // a wave with no position has l = 0
        L += wl[i] * f[i];
    }
    for (int d = threadIdx.x; d < hd; d += kSeamThreads) {
        float v = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) v += wo[i][d] * f[i];
        o[static_cast<size_t>(hq) * hd + d] = v / L;
    }
}

}  // namespace

extern "C" {

int rl_hip_conv1d_update(const float* x_t, const float* w, float* state, float* y, int dim, int k, void* stream) {
    return guard([&] {
        RL_REQUIRE(dim > 0 && k >= 1 && x_t && w && state && y, RL_ERR_RANGE, "conv1d_update: bad arguments");
        hipLaunchKernelGGL(conv1d_update_kernel, dim3((dim + 255) / 256), dim3(256), 0, S(stream), x_t, w, state, y,
                           dim, k);
        check_launch("conv1d_update_kernel");
    });
}

int rl_hip_delta_recurrent(float* S_, const float* q, const float* k, const float* v, const float* beta,
                           const float* g_log, float* o, int n_v, int dk, int dv, float eps_l2, void* stream) {
    return guard([&] {
        RL_REQUIRE(n_v > 0 && dk >= 1 && dk <= kSeamMaxDk && dv >= 1, RL_ERR_RANGE,
                   "delta_recurrent: n_v > 0, dk in 1..256, dv > 0");
        RL_REQUIRE(S_ && q && k && v && beta && g_log && o, RL_ERR_RANGE, "delta_recurrent: null pointer");
        hipLaunchKernelGGL(delta_recurrent_kernel, dim3(n_v), dim3(kSeamThreads), 0, S(stream), S_, q, k, v, beta,
                           g_log, o, dk, dv, eps_l2);
        check_launch("delta_recurrent_kernel");
    });
}

int rl_hip_attn_decode_f32(const float* q, const float* k_cache, const float* v_cache, float* o, int pos, int n_q,
                           int n_kv, int head_dim, void* stream) {
    return guard([&] {
        RL_REQUIRE(pos >= 0 && n_kv > 0 && n_q > 0 && n_q % n_kv == 0 && head_dim >= 1 && head_dim <= 256,
                   RL_ERR_RANGE, "attn_decode_f32: pos >= 0, n_q a multiple of n_kv, head_dim in 1..256");
        RL_REQUIRE(q && k_cache && v_cache && o, RL_ERR_RANGE, "attn_decode_f32: null pointer");
        hipLaunchKernelGGL(attn_decode_f32_kernel, dim3(n_q), dim3(kSeamThreads), 0, S(stream), q, k_cache, v_cache,
                           o, pos, n_q, n_kv, head_dim);
        check_launch("attn_decode_f32_kernel");
    });
}

}  // extern "C"
