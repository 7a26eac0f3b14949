// norms.hip -- normalisations fused with the activation packing of the next linear,
// and the embedding lookup.
//
//   rmsnorm_pack : Qwen3 RMSNorm y = x / sqrt(mean(x^2) + eps) * (1 + gamma)
//                  (reference src/kernels/ops.cpp:107-127), written as fp32 and/or as
//                  the bf16 hi/mid fragments the GEMM consumes (gemm.hip).
//   gnorm_pack   : gated RMSNorm y = gamma * (o / rms(o)) * silu(z), per head when
//                  gamma_n < n, n % gamma_n == 0, n >= 256, else over the vector
//                  (ops.cpp:129-156); output to fragments for out_proj.
//   embed_rows   : token ids -> fp32 rows of an F32 / F16 / BF16 table
//                  (src/runtime/session.cpp:122-140).
// Sums of squares are accumulated in double as in the reference scalar path.
#include "internal.h"

using namespace rl;

namespace {

constexpr int kBlockCols = 128;

__device__ inline float silu_f(float x) { return x / (1.f + expf(-x)); }

// Residual update + Qwen RMSNorm + packing.  One workgroup of 1024 threads per
// token; thread u owns the 8 columns [8u, 8u+8) (a second pass for n > 8192).  Each
// thread loads its x and partial-sum slices at once (no serial chain), forms
// v = x_in + P[0] + ... + P[S-1] in slice order, and the block sums v^2 in double.
// Columns past n up to the next multiple of 128 are written as zero fragments.
constexpr int kNormThreads = 1024;
constexpr int kNormMaxUnits = 2 * kNormThreads;  // n <= 16384
constexpr int kNormMaxSplit = 4;                 // split-K partial slices

__global__ __launch_bounds__(kNormThreads) void residual_rmsnorm_kernel(const float* __restrict__ x_in, int ld_x,
                                                                        const float* __restrict__ P, int S,
                                                                        float* __restrict__ x_out,
                                                                        const float* __restrict__ gamma,
                                                                        float* __restrict__ y,
                                                                        i32x4* __restrict__ frag, int n, int T,
                                                                        float eps) {
    __shared__ double red[kNormThreads / 64];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float* xt = x_in + static_cast<size_t>(t) * ld_x;
    const size_t pstride = static_cast<size_t>(T) * n;
    const int nu = n / 8;
    const int units = ((n + kBlockCols - 1) / kBlockCols) * 16;
    float v[2][8];
    double ss = 0.0;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        const int u = tid + pass * kNormThreads;
        if (u < nu) {
            float4 a = reinterpret_cast<const float4*>(xt)[2 * u];
            float4 b = reinterpret_cast<const float4*>(xt)[2 * u + 1];
            // all partial slices are loaded before the first add: one memory round
            // trip instead of S dependent ones; the sum keeps slice order
            float4 pa[kNormMaxSplit], pb[kNormMaxSplit];
#pragma unroll
            for (int q = 0; q < kNormMaxSplit; ++q) {
                if (q < S) {
                    const float4* pp =
                        reinterpret_cast<const float4*>(P + q * pstride + static_cast<size_t>(t) * n);
                    pa[q] = pp[2 * u];
                    pb[q] = pp[2 * u + 1];
                }
            }
#pragma unroll
            for (int q = 0; q < kNormMaxSplit; ++q) {
                if (q < S) {
                    a.x += pa[q].x, a.y += pa[q].y, a.z += pa[q].z, a.w += pa[q].w;
                    b.x += pb[q].x, b.y += pb[q].y, b.z += pb[q].z, b.w += pb[q].w;
                }
            }
            const float r[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[pass][e] = r[e];
                ss += static_cast<double>(r[e]) * r[e];
            }
            if (x_out) {
                float4* xo = reinterpret_cast<float4*>(x_out + static_cast<size_t>(t) * n);
                xo[2 * u] = a;
                xo[2 * u + 1] = b;
            }
        }
    }
    ss = wave_sum_d(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int w = 0; w < kNormThreads / 64; ++w) tot += red[w];
    const float inv = 1.f / sqrtf(static_cast<float>(tot / n) + eps);
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        const int u = tid + pass * kNormThreads;
        if (u >= units) continue;
        float o[8];
        if (u < nu) {
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = v[pass][e] * inv * (gamma ? 1.f + gamma[8 * u + e] : 1.f);
            if (y) {
                float4* yo = reinterpret_cast<float4*>(y + static_cast<size_t>(t) * n);
                yo[2 * u] = make_float4(o[0], o[1], o[2], o[3]);
                yo[2 * u + 1] = make_float4(o[4], o[5], o[6], o[7]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = 0.f;
        }
        if (frag) write_frag8(frag, u, t, T, o);
    }
}

// RMSNorm + packing for many tokens (prefill): one wave per token, 4 tokens per
// workgroup; lane l owns the 8-column units l, l + 64, ... (NU of them at most), all
// loaded before the wave's double sum of squares (no LDS, no barrier).  Same
// arithmetic per element as residual_rmsnorm_kernel without partials.
template <int NU>
__global__ __launch_bounds__(256) void rmsnorm_wave_kernel(const float* __restrict__ x, int ld_x,
                                                           const float* __restrict__ gamma, float* __restrict__ y,
                                                           i32x4* __restrict__ frag, int n, int T, float eps) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= T) return;  // whole waves
    const float* xt = x + static_cast<size_t>(t) * ld_x;
    const int nu = n / 8;
    const int units = ((n + kBlockCols - 1) / kBlockCols) * 16;
    float v[NU][8];
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const int u = lane + 64 * k;
        if (u < nu) {
            const float4 a = reinterpret_cast<const float4*>(xt)[2 * u];
            const float4 b = reinterpret_cast<const float4*>(xt)[2 * u + 1];
            v[k][0] = a.x, v[k][1] = a.y, v[k][2] = a.z, v[k][3] = a.w;
            v[k][4] = b.x, v[k][5] = b.y, v[k][6] = b.z, v[k][7] = b.w;
        }
    }
#pragma unroll
    for (int k = 0; k < NU; ++k)
        if (lane + 64 * k < nu)
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += static_cast<double>(v[k][e]) * v[k][e];
    ss = wave_sum_d(ss);
    const float inv = 1.f / sqrtf(static_cast<float>(ss / n) + eps);
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const int u = lane + 64 * k;
        if (u >= units) break;
        float o[8];
        if (u < nu) {
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = v[k][e] * inv * (gamma ? 1.f + gamma[8 * u + e] : 1.f);
            if (y) {
                float4* yo = reinterpret_cast<float4*>(y + static_cast<size_t>(t) * n);
                yo[2 * u] = make_float4(o[0], o[1], o[2], o[3]);
                yo[2 * u + 1] = make_float4(o[4], o[5], o[6], o[7]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = 0.f;
        }
        if (frag) write_frag8(frag, u, t, T, o);
    }
}

// Gated RMSNorm + packing.  grid (segments, T), one wave per segment (a head when
// per_head, else the whole vector).  seg % 8 == 0.
__global__ __launch_bounds__(64) void gnorm_pack_kernel(const float* __restrict__ o, const float* __restrict__ z,
                                                        int ld_z, const float* __restrict__ gamma, int gamma_n,
                                                        int per_head, float* __restrict__ y,
                                                        i32x4* __restrict__ frag, int n, int T, float eps) {
    const int t = blockIdx.y, lane = threadIdx.x;
    const int seg = per_head ? gamma_n : n;
    const int h0 = blockIdx.x * seg;
    const float* ot = o + static_cast<size_t>(t) * n;
    const float* zt = z + static_cast<size_t>(t) * ld_z;
    // segments up to 512 (the common case: 128-wide heads): the lane's z and gamma
    // are loaded together with o, before the reduction
    float zp[8], gp[8];
    const bool pre = seg <= 512 && lane < seg / 8;
    if (pre) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int i = h0 + 8 * lane + e;
            zp[e] = zt[i];
            gp[e] = gamma ? gamma[per_head ? (i - h0) : (i % gamma_n)] : 1.f;
        }
    }
    double ss = 0.0;
    for (int i = lane; i < seg; i += 64) ss += static_cast<double>(ot[h0 + i]) * ot[h0 + i];
    ss = wave_sum_d(ss);
    const float inv = 1.f / sqrtf(static_cast<float>(ss / seg) + eps);
    for (int u = lane; u < seg / 8; u += 64) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int i = h0 + 8 * u + e;
            const bool p = pre && u == lane;
            const float g = p ? gp[e] : (gamma ? gamma[per_head ? (i - h0) : (i % gamma_n)] : 1.f);
            const float zz = p ? zp[e] : zt[i];
            v[e] = g * (ot[i] * inv) * silu_f(zz);
            if (y) y[static_cast<size_t>(t) * n + i] = v[e];
        }
        if (frag) write_frag8(frag, (h0 >> 3) + u, t, T, v);
    }
    // zero the padding columns of the last 128-block (last segment only)
    if (frag && blockIdx.x == gridDim.x - 1) {
        const int units = ((n + kBlockCols - 1) / kBlockCols) * 16;
        for (int u = n / 8 + lane; u < units; u += 64) {
            const float zero8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            write_frag8(frag, u, t, T, zero8);
        }
    }
}

// The same for 128-wide heads with one gamma per head position: 16 lanes per head
// (8 columns each, vector loads), 16 heads per 256-thread workgroup, grid
// (heads / 16, T); the head's sum of squares in double over its 16 lanes.
__global__ __launch_bounds__(256) void gnorm_pack128_kernel(const float* __restrict__ o, const float* __restrict__ z,
                                                            int ld_z, const float* __restrict__ gamma,
                                                            float* __restrict__ y, i32x4* __restrict__ frag, int n,
                                                            int T, float eps) {
    const int t = blockIdx.y, tid = threadIdx.x;
    const int hh = blockIdx.x * 16 + (tid >> 4), u = tid & 15;
    const bool ok = hh * 128 < n;  // whole 16-lane groups, so the shuffles below stay within valid groups
    const int c0 = hh * 128 + 8 * u;
    float ov[8], zv[8], gv[8];
    double ss = 0.0;
    if (ok) {
        const float4* op = reinterpret_cast<const float4*>(o + static_cast<size_t>(t) * n + c0);
        const float4* zp = reinterpret_cast<const float4*>(z + static_cast<size_t>(t) * ld_z + c0);
        const float4 o0 = op[0], o1 = op[1], z0 = zp[0], z1 = zp[1];
        ov[0] = o0.x, ov[1] = o0.y, ov[2] = o0.z, ov[3] = o0.w, ov[4] = o1.x, ov[5] = o1.y, ov[6] = o1.z, ov[7] = o1.w;
        zv[0] = z0.x, zv[1] = z0.y, zv[2] = z0.z, zv[3] = z0.w, zv[4] = z1.x, zv[5] = z1.y, zv[6] = z1.z, zv[7] = z1.w;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            gv[e] = gamma ? gamma[8 * u + e] : 1.f;
            ss += static_cast<double>(ov[e]) * ov[e];
        }
    }
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) ss += __shfl_xor(ss, m, 64);
    if (!ok) return;
    const float inv = 1.f / sqrtf(static_cast<float>(ss / 128) + eps);
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = gv[e] * (ov[e] * inv) * silu_f(zv[e]);
    if (y) {
        float4* yp = reinterpret_cast<float4*>(y + static_cast<size_t>(t) * n + c0);
        yp[0] = make_float4(v[0], v[1], v[2], v[3]);
        yp[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    if (frag) write_frag8(frag, c0 >> 3, t, T, v);
}

// tokens[t] -> out[t][H]; kind: RL_Q_F32 / RL_Q_F16 / RL_Q_BF16 table [vocab][H].
__global__ void embed_rows_kernel(const void* __restrict__ table, int kind, const int* __restrict__ tokens,
                                  float* __restrict__ out, int H, int vocab) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= H) return;
    int id = tokens[t];
    id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);  // ids are validated on the host
    const size_t k = static_cast<size_t>(id) * H + i;
    float v;
    if (kind == RL_Q_F32)
        v = static_cast<const float*>(table)[k];
    else if (kind == RL_Q_BF16)
        v = __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(table)[k]) << 16);
    else
        v = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(table)[k]));
    out[static_cast<size_t>(t) * H + i] = v;
}

__global__ void swiglu_kernel(const float* __restrict__ g, int ldg, const float* __restrict__ u, int ldu,
                              float* __restrict__ h, int n) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    h[static_cast<size_t>(t) * n + i] = silu_f(g[static_cast<size_t>(t) * ldg + i]) * u[static_cast<size_t>(t) * ldu + i];
}

__global__ void copy_int_kernel(const int* __restrict__ src, int* __restrict__ dst) { *dst = *src; }

}  // namespace

namespace rl {

// silu(g) * u (reference ops.cpp:607-609), rows at strides ldg / ldu, h dense [T][n].
void swiglu(const float* g, int ldg, const float* u, int ldu, float* h, int n, int T, hipStream_t s) {
    hipLaunchKernelGGL(swiglu_kernel, dim3((n + 255) / 256, T), dim3(256), 0, s, g, ldg, u, ldu, h, n);
    check_launch("swiglu_kernel");
}

// one int device-to-device as a kernel (graph-safe, no memcpy node)
void copy_int(const int* src, int* dst, hipStream_t s) {
    hipLaunchKernelGGL(copy_int_kernel, dim3(1), dim3(1), 0, s, src, dst);
    check_launch("copy_int_kernel");
}

void residual_rmsnorm_pack(const float* x_in, const float* P, int S, float* x_out, const float* gamma, float* y,
                           void* frag, int n, int T, float eps, hipStream_t s) {
    RL_REQUIRE(n > 0 && n % 8 == 0 && T >= 1 && T <= 65535, RL_ERR_RANGE, "rmsnorm: n % 8 == 0, T in 1..65535");
    RL_REQUIRE(x_in && (y || frag || x_out), RL_ERR_RANGE, "rmsnorm: null pointer");
    RL_REQUIRE(x_out != x_in, RL_ERR_RANGE, "rmsnorm: residual output must not alias the input");
    RL_REQUIRE(!P || (S >= 1 && S <= kNormMaxSplit), RL_ERR_RANGE, "rmsnorm: 1..4 partial slices");
    RL_REQUIRE(((n + kBlockCols - 1) / kBlockCols) * 16 <= kNormMaxUnits, RL_ERR_RANGE, "rmsnorm: n > 16384");
    hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3(T), dim3(kNormThreads), 0, s, x_in, n, P, P ? S : 0, x_out,
                       gamma, y, static_cast<i32x4*>(frag), n, T, eps);
    check_launch("residual_rmsnorm_kernel");
}

void rmsnorm_pack(const float* x, int ld_x, const float* gamma, float* y, void* frag, int n, int T, float eps,
                  hipStream_t s) {
    RL_REQUIRE(n > 0 && n % 8 == 0 && T >= 1 && T <= 65535, RL_ERR_RANGE, "rmsnorm_pack: n % 8 == 0, T in 1..65535");
    RL_REQUIRE(x && (y || frag), RL_ERR_RANGE, "rmsnorm_pack: null pointer");
    RL_REQUIRE(ld_x % 4 == 0, RL_ERR_RANGE, "rmsnorm_pack: row stride must be a multiple of 4");
    RL_REQUIRE(((n + kBlockCols - 1) / kBlockCols) * 16 <= kNormMaxUnits, RL_ERR_RANGE, "rmsnorm: n > 16384");
    // prefill-sized T: one wave per token (the decode sizes keep the kernel below,
    // so every decode step width uses the same summation order)
    const int units = ((n + kBlockCols - 1) / kBlockCols) * 16;
    const bool aligned = reinterpret_cast<uintptr_t>(x) % 16 == 0 && (!y || reinterpret_cast<uintptr_t>(y) % 16 == 0);
    if (T >= 64 && aligned && units <= 64 * 12) {
        const dim3 grid((T + 3) / 4);
        if (units <= 64 * 4)
            hipLaunchKernelGGL(rmsnorm_wave_kernel<4>, grid, dim3(256), 0, s, x, ld_x, gamma, y,
                               static_cast<i32x4*>(frag), n, T, eps);
        else if (units <= 64 * 8)
            hipLaunchKernelGGL(rmsnorm_wave_kernel<8>, grid, dim3(256), 0, s, x, ld_x, gamma, y,
                               static_cast<i32x4*>(frag), n, T, eps);
        else
            hipLaunchKernelGGL(rmsnorm_wave_kernel<12>, grid, dim3(256), 0, s, x, ld_x, gamma, y,
                               static_cast<i32x4*>(frag), n, T, eps);
        check_launch("rmsnorm_wave_kernel");
        return;
    }
    hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3(T), dim3(kNormThreads), 0, s, x, ld_x, nullptr, 0, nullptr,
                       gamma, y, static_cast<i32x4*>(frag), n, T, eps);
    check_launch("residual_rmsnorm_kernel");
}

void gnorm_pack(const float* o, const float* z, int ld_z, const float* gamma, int gamma_n, float* y, void* frag,
                int n, int T, float eps, hipStream_t s) {
    if (gamma_n <= 0) gamma_n = n;
    const bool per_head = gamma_n < n && n % gamma_n == 0 && n >= 256;
    const int seg = per_head ? gamma_n : n;
    RL_REQUIRE(seg % 8 == 0 && T >= 1 && T <= 65535, RL_ERR_RANGE, "gnorm_pack: segment % 8 == 0, T in 1..65535");
    RL_REQUIRE(o && z && (y || frag), RL_ERR_RANGE, "gnorm_pack: null pointer");
    const bool vec = reinterpret_cast<uintptr_t>(o) % 16 == 0 && reinterpret_cast<uintptr_t>(z) % 16 == 0 &&
                     (!y || reinterpret_cast<uintptr_t>(y) % 16 == 0) && ld_z % 4 == 0;
    if (per_head && seg == 128 && vec) {
        hipLaunchKernelGGL(gnorm_pack128_kernel, dim3((n / 128 + 15) / 16, T), dim3(256), 0, s, o, z, ld_z, gamma, y,
                           static_cast<i32x4*>(frag), n, T, eps);
        check_launch("gnorm_pack128_kernel");
        return;
    }
    hipLaunchKernelGGL(gnorm_pack_kernel, dim3(n / seg, T), dim3(64), 0, s, o, z, ld_z, gamma, gamma_n,
                       per_head ? 1 : 0, y, static_cast<i32x4*>(frag), n, T, eps);
    check_launch("gnorm_pack_kernel");
}

void embed_rows(const void* table, int kind, const int* tokens, float* out, int H, int vocab, int T, hipStream_t s) {
    RL_REQUIRE(kind == RL_Q_F32 || kind == RL_Q_F16 || kind == RL_Q_BF16, RL_ERR_UNSUPPORTED,
               "embed: table must be F32, F16 or BF16");
    hipLaunchKernelGGL(embed_rows_kernel, dim3((H + 255) / 256, T), dim3(256), 0, s, table, kind, tokens, out, H,
                       vocab);
    check_launch("embed_rows_kernel");
}

}  // namespace rl

extern "C" {

int rl_hip_rmsnorm_pack(const float* x, int ld_x, const float* gamma, float* y, void* frag, int n, int T, float eps,
                        void* stream) {
    return guard([&] { rl::rmsnorm_pack(x, ld_x, gamma, y, frag, n, T, eps, S(stream)); });
}

int rl_hip_gated_rmsnorm_pack(const float* o, const float* z, int ld_z, const float* gamma, int gamma_n, float* y,
                              void* frag, int n, int T, float eps, void* stream) {
    return guard([&] { rl::gnorm_pack(o, z, ld_z, gamma, gamma_n, y, frag, n, T, eps, S(stream)); });
}

int rl_hip_embed_rows(const void* table, int kind, const int* tokens, float* out, int H, int vocab, int T,
                      void* stream) {
    return guard([&] { rl::embed_rows(table, kind, tokens, out, H, vocab, T, S(stream)); });
}

}  // extern "C"
