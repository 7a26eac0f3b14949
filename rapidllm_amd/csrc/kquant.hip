// kquant.hip -- GGUF Q4_K / Q6_K dequantisation and dequant-dot GEMV (T = 1..4).
//
// Dequant follows the reference CPU exactly (bit-exact, no FMA contraction):
//   Q4_K (ops.cpp:245-284): w = (d * sc_j) * q - (dmin * m_j), each product rounded
//   Q6_K (ops.cpp:357-387): w = (d * sc) * (q - 32)
// The GEMV (ops.cpp:292-305, 389-402; threaded by cpu_caps.cpp:200-222) is computed
// in the factorised form sum_j [ (d sc_j) * sum_l q_l x_l - (dmin m_j) * sum_l x_l ]
// with an fp32 accumulator: the same real number, within the 1e-3 relative-L2
// budget of the north star.
//
// Device layout ("K-tiled"): a tile = 64 rows x 1 super-block.  Lane l of a wave
// owns row 64*rg + l; the 144-byte (Q4_K) / 208+2-byte (Q6_K) block of that row is
// cut into 16-byte chunks stored chunk-major, lane-minor, so each of the wave's
// 16-byte loads is one contiguous 1 KiB stream.  The Q6_K fp16 d of the 64 rows
// follows the 13 chunks.  Bytes are only moved, never re-rounded.
//
// All 64 lanes of a wave work on the same super-block at the same time, so the
// activation element multiplying every lane's weight is the same: x is read with
// scalar loads into SGPRs and used directly as the FMA operand (no LDS, no VGPRs).
#include <algorithm>
#include <cstdlib>

#include "internal.h"

using namespace rl;

namespace {

constexpr int kRows = 64;  // rows per tile (one per lane)

template <int QT>
struct KFmt;
template <>
struct KFmt<4> {
    static constexpr int kBlockBytes = 144;
    static constexpr int kChunks = 9;
    static constexpr int kTileBytes = kRows * 144;
};
template <>
struct KFmt<6> {
    static constexpr int kBlockBytes = 210;
    static constexpr int kChunks = 13;
    static constexpr int kTileBytes = kRows * 210;
};

__device__ inline float half_bits_to_f32(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// byte e of a dword as float (the compiler selects v_cvt_f32_ubyte{0..3})
__device__ inline float ubyte(uint32_t w, int e) { return static_cast<float>((w >> (8 * e)) & 0xffu); }

__device__ inline uint32_t lane_dword(const i32x4 (&c)[16], int byte_off) {
    return static_cast<uint32_t>(c[byte_off >> 4][(byte_off >> 2) & 3]);
}

// 6-bit scale and min of sub-block j from the 12 scale bytes (block bytes 4..15).
__device__ inline void q4k_scale_min(const uint8_t* s12, int j, int& sc, int& mn) {
    if (j < 4) {
        sc = s12[j] & 63;
        mn = s12[j + 4] & 63;
    } else {
        sc = (s12[j + 4] & 15) | ((s12[j - 4] >> 6) << 4);
        mn = (s12[j + 4] >> 4) | ((s12[j] >> 6) << 4);
    }
}

// One super-block of one row (this lane), accumulated into y[t].
// xs32: sums of x over the 32-element sub-blocks of this workgroup's K-slice
// (sub-block sbl*8 + j of token t at xs32[t * xs_ld + sbl*8 + j]).
template <int T>
__device__ inline void q4k_block(const i32x4 (&c)[16], const float* __restrict__ x, const float* xs32, int xs_ld,
                                 int n, int sb, int sbl, float (&y)[4]) {
    union {
        i32x4 v;
        uint8_t b[16];
    } hdr;
    hdr.v = c[0];
    const float d = half_bits_to_f32(hdr.b[0] | (hdr.b[1] << 8));
    const float dmin = half_bits_to_f32(hdr.b[2] | (hdr.b[3] << 8));
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
        int s0, m0, s1, m1;
        q4k_scale_min(hdr.b + 4, 2 * grp, s0, m0);
        q4k_scale_min(hdr.b + 4, 2 * grp + 1, s1, m1);
        float acc_lo[T], acc_hi[T];
#pragma unroll
        for (int t = 0; t < T; ++t) acc_lo[t] = acc_hi[t] = 0.f;
        const int k0 = sb * 256 + 64 * grp;
#pragma unroll
        for (int dw = 0; dw < 8; ++dw) {
            const uint32_t w = lane_dword(c, 16 + 32 * grp + 4 * dw);
            const uint32_t lo = w & 0x0f0f0f0fu;
            const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const float4 xl = *reinterpret_cast<const float4*>(x + static_cast<size_t>(t) * n + k0 + 4 * dw);
                const float4 xh = *reinterpret_cast<const float4*>(x + static_cast<size_t>(t) * n + k0 + 32 + 4 * dw);
                acc_lo[t] += ubyte(lo, 0) * xl.x + ubyte(lo, 1) * xl.y + ubyte(lo, 2) * xl.z + ubyte(lo, 3) * xl.w;
                acc_hi[t] += ubyte(hi, 0) * xh.x + ubyte(hi, 1) * xh.y + ubyte(hi, 2) * xh.z + ubyte(hi, 3) * xh.w;
            }
        }
        const float a0 = d * static_cast<float>(s0), b0 = dmin * static_cast<float>(m0);
        const float a1 = d * static_cast<float>(s1), b1 = dmin * static_cast<float>(m1);
        const int j0 = sbl * 8 + 2 * grp;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float* st = xs32 + t * xs_ld + j0;
            y[t] += a0 * acc_lo[t] - b0 * st[0] + a1 * acc_hi[t] - b1 * st[1];
        }
    }
}

// xs16: sums of x over the 16-element sub-blocks of the K-slice (as q4k_block).
template <int T>
__device__ inline void q6k_block(const i32x4 (&c)[16], float d, const float* __restrict__ x, const float* xs16,
                                 int xs_ld, int n, int sb, int sbl, float (&y)[4]) {
    union {
        i32x4 v;
        int8_t b[16];
    } scb;
    scb.v = c[12];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
#pragma unroll
        for (int l16 = 0; l16 < 2; ++l16) {
            float acc[4][T];
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int t = 0; t < T; ++t) acc[k][t] = 0.f;
#pragma unroll
            for (int dw = 0; dw < 4; ++dw) {
                const uint32_t qa = lane_dword(c, 64 * half + 16 * l16 + 4 * dw);
                const uint32_t qb = lane_dword(c, 64 * half + 32 + 16 * l16 + 4 * dw);
                const uint32_t qh = lane_dword(c, 128 + 32 * half + 16 * l16 + 4 * dw);
                uint32_t q[4];
                q[0] = (qa & 0x0f0f0f0fu) | ((qh & 0x03030303u) << 4);
                q[1] = (qb & 0x0f0f0f0fu) | (((qh >> 2) & 0x03030303u) << 4);
                q[2] = ((qa >> 4) & 0x0f0f0f0fu) | (((qh >> 4) & 0x03030303u) << 4);
                q[3] = ((qb >> 4) & 0x0f0f0f0fu) | (((qh >> 6) & 0x03030303u) << 4);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int kk = sb * 256 + 128 * half + 32 * k + 16 * l16 + 4 * dw;
#pragma unroll
                    for (int t = 0; t < T; ++t) {
                        const float4 xv = *reinterpret_cast<const float4*>(x + static_cast<size_t>(t) * n + kk);
                        acc[k][t] += ubyte(q[k], 0) * xv.x + ubyte(q[k], 1) * xv.y + ubyte(q[k], 2) * xv.z +
                                     ubyte(q[k], 3) * xv.w;
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float a = d * static_cast<float>(scb.b[8 * half + l16 + 2 * k]);
                const int j = sbl * 16 + 8 * half + 2 * k + l16;
#pragma unroll
                for (int t = 0; t < T; ++t) y[t] += a * (acc[k][t] - 32.f * xs16[t * xs_ld + j]);
            }
        }
    }
}

// Split-K tickets: one counter per row group, 64 bytes apart (atomics on one cache
// line serialise).  Zero at load; the workgroup that takes a group's last ticket
// resets it, so every launch finds them zero.  Launches on one device must not
// overlap in time (they share the counters).
constexpr int kKqMaxGroups = 4096;
__device__ unsigned g_kq_ticket[kKqMaxGroups * 16];

// Grid: blockIdx.x = row-group * S + k-slice; KS waves per workgroup split the
// slice's super-blocks.  The sub-block sums of x that the min / offset terms need
// are computed per workgroup for its slice, into LDS (summed in double, as
// written by ops.cpp's dot of the dequantised block).  S == 1: the workgroup writes
// Y (store or add).  S > 1: it writes partial[slice][t][row] and takes a ticket;
// the last workgroup of the row group adds the S partials in slice order (a fixed
// order) and writes Y.  Partials and tickets use agent-scope atomic accesses,
// which are coherent across the XCDs' L2 caches without cache maintenance.
template <int QT, int T, int KS>
__global__ __launch_bounds__(64 * KS) void kq_gemm_kernel(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                          float* __restrict__ Y, float* __restrict__ partial, int m,
                                                          int n, int S, int accumulate, int ldy) {
    using F = KFmt<QT>;
    constexpr int kSubPerSb = QT == 4 ? 8 : 16;
    constexpr int kSubLen = 256 / kSubPerSb;
    extern __shared__ float xs_l[];  // [T][per_slice * kSubPerSb]
    const int lane = threadIdx.x & 63;
    // wave index is uniform: make that visible so the super-block loop (and the x
    // addresses derived from it) stay scalar
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rg = blockIdx.x / S;
    const int slice = blockIdx.x % S;
    const int nsb = n / 256;
    const int per_slice = (nsb + S - 1) / S;
    const int s0 = min(nsb, slice * per_slice), s1 = min(nsb, s0 + per_slice);
    const int per = (s1 - s0 + KS - 1) / KS;
    const int b0 = min(s1, s0 + wave * per), b1 = min(s1, b0 + per);
    const int xs_ld = per_slice * kSubPerSb;

    float y[4] = {0.f, 0.f, 0.f, 0.f};
    const uint8_t* rowtiles = W + static_cast<size_t>(rg) * nsb * F::kTileBytes;
    i32x4 cur[16], nxt[16];
    auto load = [&](int sb, i32x4 (&c)[16]) {
        const uint8_t* tile = rowtiles + static_cast<size_t>(sb) * F::kTileBytes;
#pragma unroll
        for (int k = 0; k < F::kChunks; ++k)
            c[k] = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(tile + k * 1024 + 16 * lane));
        if constexpr (QT == 6) {
            const uint16_t dh = reinterpret_cast<const uint16_t*>(tile + F::kChunks * 1024)[lane];
            c[15] = i32x4{static_cast<int>(dh), 0, 0, 0};
        }
    };
    // the first weights are requested before the slice's x sums are formed
    if (b0 < b1) load(b0, cur);
    {
        const int nsub = (s1 - s0) * kSubPerSb;
        for (int i = threadIdx.x; i < T * nsub; i += 64 * KS) {
            const int t = i / nsub, j = i % nsub;
            const float* p = x + static_cast<size_t>(t) * n + static_cast<size_t>(s0) * 256 + j * kSubLen;
            double acc = 0.0;
#pragma unroll
            for (int e = 0; e < kSubLen; e += 4) {
                const float4 v = *reinterpret_cast<const float4*>(p + e);
                acc += v.x;
                acc += v.y;
                acc += v.z;
                acc += v.w;
            }
            xs_l[t * xs_ld + j] = static_cast<float>(acc);
        }
    }
    __syncthreads();
    for (int sb = b0; sb < b1; ++sb) {
        if (sb + 1 < b1) load(sb + 1, nxt);
        if constexpr (QT == 4)
            q4k_block<T>(cur, x, xs_l, xs_ld, n, sb, sb - s0, y);
        else
            q6k_block<T>(cur, half_bits_to_f32(static_cast<uint32_t>(cur[15][0])), x, xs_l, xs_ld, n, sb, sb - s0, y);
        if (sb + 1 < b1) {
#pragma unroll
            for (int k = 0; k < F::kChunks; ++k) cur[k] = nxt[k];
            if constexpr (QT == 6) cur[15] = nxt[15];
        }
    }

    __shared__ float red[KS][4][64];
    __shared__ int s_last;
#pragma unroll
    for (int t = 0; t < 4; ++t) red[wave][t][lane] = y[t];
    __syncthreads();
    if (S > 1) {
        for (int it = threadIdx.x; it < T * kRows; it += 64 * KS) {
            const int t = it / kRows, l = it % kRows;
            const int row = rg * kRows + l;
            if (row >= m) continue;
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < KS; ++w) s += red[w][t][l];
            __hip_atomic_store(partial + (static_cast<size_t>(slice) * T + t) * m + row, s, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // partial stores complete before the ticket
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned* tk = g_kq_ticket + static_cast<size_t>(rg) * 16;
            const unsigned old = __hip_atomic_fetch_add(tk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int last = old == static_cast<unsigned>(S - 1);
            if (last) __hip_atomic_store(tk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = last;
        }
        __syncthreads();
        if (!s_last) return;
        for (int it = threadIdx.x; it < T * kRows; it += 64 * KS) {
            const int t = it / kRows, l = it % kRows;
            const int row = rg * kRows + l;
            if (row >= m) continue;
            float s = 0.f;
            for (int q = 0; q < S; ++q)
                s += __hip_atomic_load(partial + (static_cast<size_t>(q) * T + t) * m + row, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            float* dst = Y + static_cast<size_t>(t) * ldy + row;
            if (accumulate)
                *dst += s;
            else
                *dst = s;
        }
        return;
    }
    for (int it = threadIdx.x; it < T * kRows; it += 64 * KS) {
        const int t = it / kRows, l = it % kRows;
        const int row = rg * kRows + l;
        if (row >= m) continue;
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < KS; ++w) s += red[w][t][l];
        if (accumulate)
            Y[static_cast<size_t>(t) * ldy + row] += s;
        else
            Y[static_cast<size_t>(t) * ldy + row] = s;
    }
}

// Row-major GGUF blocks [m][n/256 * bb] -> K-tiled.
template <int QT>
__global__ void kq_pack_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int m, int nsb) {
    // rows past m are written as zero blocks (d = 0: every weight is 0)
    using F = KFmt<QT>;
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // (rg, sb, lane)
    const int m_groups = (m + kRows - 1) / kRows;
    if (idx >= static_cast<size_t>(m_groups) * nsb * kRows) return;
    const int lane = idx % kRows;
    const int sb = (idx / kRows) % nsb;
    const int rg = static_cast<int>(idx / (static_cast<size_t>(kRows) * nsb));
    const int row = rg * kRows + lane;
    uint8_t* tile = dst + (static_cast<size_t>(rg) * nsb + sb) * F::kTileBytes;
    const uint8_t* blk = src + (static_cast<size_t>(row) * nsb + sb) * F::kBlockBytes;
    const bool ok = row < m;
    for (int k = 0; k < F::kChunks; ++k)
        for (int e = 0; e < 16; ++e) tile[k * 1024 + 16 * lane + e] = ok ? blk[16 * k + e] : 0;
    if constexpr (QT == 6) {
        tile[F::kChunks * 1024 + 2 * lane] = ok ? blk[208] : 0;
        tile[F::kChunks * 1024 + 2 * lane + 1] = ok ? blk[209] : 0;
    }
}

// Exact dequantisation of row-major blocks (one thread per block).
__global__ void q4k_dequant_kernel(const uint8_t* __restrict__ src, float* __restrict__ out, size_t nblocks) {
#pragma clang fp contract(off)
    const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* blk = src + b * 144;
    const float d = half_bits_to_f32(blk[0] | (blk[1] << 8));
    const float dmin = half_bits_to_f32(blk[2] | (blk[3] << 8));
    float* o = out + b * 256;
    for (int g = 0; g < 4; ++g) {
        int s0, m0, s1, m1;
        q4k_scale_min(blk + 4, 2 * g, s0, m0);
        q4k_scale_min(blk + 4, 2 * g + 1, s1, m1);
        const float d0 = __fmul_rn(d, static_cast<float>(s0)), mm0 = __fmul_rn(dmin, static_cast<float>(m0));
        const float d1 = __fmul_rn(d, static_cast<float>(s1)), mm1 = __fmul_rn(dmin, static_cast<float>(m1));
        for (int l = 0; l < 32; ++l) {
            const uint8_t q = blk[16 + 32 * g + l];
            o[64 * g + l] = __fsub_rn(__fmul_rn(d0, static_cast<float>(q & 15)), mm0);
            o[64 * g + 32 + l] = __fsub_rn(__fmul_rn(d1, static_cast<float>(q >> 4)), mm1);
        }
    }
}

__global__ void q6k_dequant_kernel(const uint8_t* __restrict__ src, float* __restrict__ out, size_t nblocks) {
#pragma clang fp contract(off)
    const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* blk = src + b * 210;
    const float d = half_bits_to_f32(blk[208] | (blk[209] << 8));
    for (int half = 0; half < 2; ++half) {
        const uint8_t* ql = blk + 64 * half;
        const uint8_t* qh = blk + 128 + 32 * half;
        const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192 + 8 * half);
        float* o = out + b * 256 + 128 * half;
        for (int l = 0; l < 32; ++l) {
            const int v0 = ((ql[l] & 15) | ((qh[l] & 3) << 4)) - 32;
            const int v1 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int v2 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int v3 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            const int s = l / 16;
            o[l] = __fmul_rn(__fmul_rn(d, static_cast<float>(sc[s])), static_cast<float>(v0));
            o[l + 32] = __fmul_rn(__fmul_rn(d, static_cast<float>(sc[s + 2])), static_cast<float>(v1));
            o[l + 64] = __fmul_rn(__fmul_rn(d, static_cast<float>(sc[s + 4])), static_cast<float>(v2));
            o[l + 96] = __fmul_rn(__fmul_rn(d, static_cast<float>(sc[s + 6])), static_cast<float>(v3));
        }
    }
}

size_t kq_tiled_bytes(int qt, int m, int n) {
    const size_t tile = qt == 4 ? KFmt<4>::kTileBytes : KFmt<6>::kTileBytes;
    return static_cast<size_t>((m + kRows - 1) / kRows) * (n / 256) * tile;
}

// Work split: keep >= ~512 workgroups where the row groups alone are too few, and
// the slice's x sums within 32 KiB of LDS.
constexpr size_t kKqXsLds = 32768;
size_t kq_xs_bytes(int qt, int nsb, int S, int T) {
    return static_cast<size_t>(T) * ((nsb + S - 1) / S) * (qt == 4 ? 8 : 16) * sizeof(float);
}
void kq_split(int qt, int m, int nsb, int T, int& S, int& KS) {
    const int groups = (m + kRows - 1) / kRows;
    KS = 4;
    S = 1;
    while (groups * S < 512 && nsb / (S * 2) >= 4) S *= 2;
    while (kq_xs_bytes(qt, nsb, S, T) > kKqXsLds) S *= 2;
    static const char* env = std::getenv("RL_KQ_SPLIT");  // measurement override "S"
    if (env && std::atoi(env) > 0) S = std::atoi(env);
    S = std::min(S, nsb);
}

template <int QT, int T>
void launch_kq_t(const uint8_t* W, const float* x, float* Y, float* partial, int m, int n, int S, int accumulate,
                 int ldy, hipStream_t s) {
    const int groups = (m + kRows - 1) / kRows;
    const size_t lds = kq_xs_bytes(QT, n / 256, S, T);
    hipLaunchKernelGGL((kq_gemm_kernel<QT, T, 4>), dim3(groups * S), dim3(256), lds, s, W, x, Y, partial, m, n, S,
                       accumulate, ldy);
}

template <int QT>
void launch_kq(const uint8_t* W, const float* x, float* Y, float* partial, int m, int n, int T, int S, int accumulate,
               int ldy, hipStream_t s) {
    switch (T) {
    case 1: launch_kq_t<QT, 1>(W, x, Y, partial, m, n, S, accumulate, ldy, s); break;
    case 2: launch_kq_t<QT, 2>(W, x, Y, partial, m, n, S, accumulate, ldy, s); break;
    case 3: launch_kq_t<QT, 3>(W, x, Y, partial, m, n, S, accumulate, ldy, s); break;
    default: launch_kq_t<QT, 4>(W, x, Y, partial, m, n, S, accumulate, ldy, s); break;
    }
}

}  // namespace

namespace rl {

size_t kq_workspace_bytes(int m, int n, int T) {
    // partials for the largest split either type uses: S*T*m floats
    int S4, S6, KS;
    kq_split(4, m, n / 256, T, S4, KS);
    kq_split(6, m, n / 256, T, S6, KS);
    const int S = std::max(S4, S6);
    return (S > 1 ? static_cast<size_t>(S) * T * m : 0) * 4 + 256;
}

// Y[T][m] (=, +=) W . x for Q4_K (qt=4) / Q6_K (qt=6) K-tiled weights.
void kq_gemm(int qt, const uint8_t* W, const float* x, float* Y, void* ws, size_t ws_bytes, int m, int n, int T,
             int accumulate, int ldy, hipStream_t s) {
    RL_REQUIRE(qt == 4 || qt == 6, RL_ERR_UNSUPPORTED, "kquant: type must be Q4_K or Q6_K");
    RL_REQUIRE(m > 0 && n > 0 && n % 256 == 0, RL_ERR_RANGE, "kquant: n must be a positive multiple of 256");
    RL_REQUIRE(T >= 1 && T <= 4, RL_ERR_RANGE, "kquant: T must be in 1..4");
    RL_REQUIRE(W && x && Y && ws, RL_ERR_RANGE, "kquant: null pointer");
    RL_REQUIRE(ws_bytes >= kq_workspace_bytes(m, n, T), RL_ERR_RANGE, "kquant: workspace too small");
    int S, KS;
    kq_split(qt, m, n / 256, T, S, KS);
    RL_REQUIRE(S == 1 || (m + kRows - 1) / kRows <= kKqMaxGroups, RL_ERR_UNSUPPORTED, "kquant: too many rows");
    RL_REQUIRE(kq_xs_bytes(qt, n / 256, S, T) <= kKqXsLds, RL_ERR_UNSUPPORTED, "kquant: K-slice too long");
    float* partial = static_cast<float*>(ws);
    if (qt == 4)
        launch_kq<4>(W, x, Y, partial, m, n, T, S, accumulate, ldy, s);
    else
        launch_kq<6>(W, x, Y, partial, m, n, T, S, accumulate, ldy, s);
    check_launch("kq_gemm_kernel");
}

}  // namespace rl

extern "C" {

size_t rl_hip_kquant_tiled_bytes(int type, int m, int n) {
    if ((type != RL_Q_Q4_K && type != RL_Q_Q6_K) || n % 256 != 0 || m <= 0) return 0;
    return kq_tiled_bytes(type == RL_Q_Q4_K ? 4 : 6, m, n);
}

size_t rl_hip_kquant_workspace_bytes(int m, int n, int T) { return rl::kq_workspace_bytes(m, n, T); }

int rl_hip_pack_kquant(int type, const uint8_t* blocks, uint8_t* tiled, int m, int n, void* stream) {
    return guard([&] {
        RL_REQUIRE(type == RL_Q_Q4_K || type == RL_Q_Q6_K, RL_ERR_UNSUPPORTED, "pack_kquant: Q4_K or Q6_K only");
        RL_REQUIRE(m > 0 && n > 0 && n % 256 == 0 && blocks && tiled, RL_ERR_RANGE, "pack_kquant: bad shape");
        const int nsb = n / 256;
        const size_t total = static_cast<size_t>((m + kRows - 1) / kRows) * nsb * kRows;
        if (type == RL_Q_Q4_K)
            hipLaunchKernelGGL(kq_pack_kernel<4>, dim3((total + 255) / 256), dim3(256), 0, S(stream), blocks, tiled, m,
                               nsb);
        else
            hipLaunchKernelGGL(kq_pack_kernel<6>, dim3((total + 255) / 256), dim3(256), 0, S(stream), blocks, tiled, m,
                               nsb);
        check_launch("kq_pack_kernel");
    });
}

int rl_hip_gemm_kquant(int type, const uint8_t* tiled, const float* X, float* Y, void* workspace,
                       size_t workspace_bytes, int m, int n, int T, int accumulate, void* stream) {
    return guard([&] {
        RL_REQUIRE(type == RL_Q_Q4_K || type == RL_Q_Q6_K, RL_ERR_UNSUPPORTED, "gemm_kquant: Q4_K or Q6_K only");
        rl::kq_gemm(type == RL_Q_Q4_K ? 4 : 6, tiled, X, Y, workspace, workspace_bytes, m, n, T, accumulate, m,
                    S(stream));
    });
}

int rl_hip_dequant_kquant(int type, const uint8_t* blocks, float* out, size_t n_blocks, void* stream) {
    return guard([&] {
        RL_REQUIRE(type == RL_Q_Q4_K || type == RL_Q_Q6_K, RL_ERR_UNSUPPORTED, "dequant: Q4_K or Q6_K only");
        if (n_blocks == 0) return;
        RL_REQUIRE(blocks && out, RL_ERR_RANGE, "dequant: null pointer");
        const dim3 grid((n_blocks + 127) / 128);
        if (type == RL_Q_Q4_K)
            hipLaunchKernelGGL(q4k_dequant_kernel, grid, dim3(128), 0, S(stream), blocks, out, n_blocks);
        else
            hipLaunchKernelGGL(q6k_dequant_kernel, grid, dim3(128), 0, S(stream), blocks, out, n_blocks);
        check_launch("dequant_kernel");
    });
}

}  // extern "C"
