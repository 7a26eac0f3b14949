// kquant.hip -- GGUF Q4_K / Q6_K dequantisation and dequant-dot GEMV (T = 1..16).
//
// Dequant follows the reference CPU exactly (bit-exact, no FMA contraction):
//   Q4_K (ops.cpp:245-284): w = (d * sc_j) * q - (dmin * m_j), each product rounded
//   Q6_K (ops.cpp:357-387): w = (d * sc) * (q - 32)
// The GEMV (ops.cpp:292-305, 389-402; threaded by cpu_caps.cpp:200-222) is computed
// per sub-block j in the factorised form a_j * sum_l q_l x_l - b_j * sum_l x_l with
// fp32 accumulation: the same real number, within the 1e-3 relative-L2 budget of
// the north star.
//
// The quant dot products run on the matrix cores (v_mfma_i32_16x16x64_i8):
//   * quants are the B operand as they are stored: a Q4_K nibble or a Q6_K 6-bit
//     value is an int8 in 0..63 after a mask (and, for Q6_K, an or of the two high
//     bits), no conversion;
//   * x is quantised per 32-value block and token to int8 hi + lo with one scale:
//     x ~ s * (hi + lo / 254), s = max|x| / 127 (15 significant bits of the block
//     maximum; about 1e-5 relative error on the outputs), in LDS;
//   * A-operand row 4g + p carries token column p only in the k-range of lane group
//     g (block-diagonal), so the MFMA returns, in every lane, the exact int32 dot
//     product of that lane's own 16 quants with x hi / lo for up to 4 token
//     columns (hi, lo of two tokens) -- no cross-lane sums;
//   * a lane's 16-quant runs never cross a sub-block, so the MFMAs of a sub-block
//     accumulate exactly in place and the per-(row, sub-block) scale is applied
//     once: y += a_j * s * (C_hi + C_lo / 254) - b_j * X_j (Q4_K, b_j = dmin * m_j;
//     Q6_K: b_j = 32 a_j), with X_j the sub-block sum of the quantised x.
//
// Device layout: a tile = 16 rows x 1 super-block (256 quants).  Lane l of a wave
// owns row 16rt + l % 16 and a quarter of the super-block (g = l / 16):
//   Q4_K: bytes 16+32g .. 16+32g+31 of the block (sub-blocks 2g low nibbles and
//         2g+1 high nibbles) as two 16-byte chunks, chunk-major and lane-minor (each
//         wave load is one contiguous 1 KiB run), then the 16 rows' 16-byte headers
//         (d, dmin, 12 scale bytes): 2304 B = 16 x 144;
//   Q6_K: ql[64h + 16e .. +16], ql[64h + 32 + 16e .. +16], qh[32h + 16e .. +16]
//         with h = g / 2, e = g % 2 (three chunks), then the rows' 16 int8 scales
//         (16 B each) and fp16 d (2 B each): 3360 B = 16 x 210.
// Bytes are only moved, never re-rounded.
#include <algorithm>
#include <cstdlib>

#include "internal.h"

#include <mutex>

using namespace rl;

namespace {

constexpr int kTR = 16;       // rows per tile
// Work split: keep >= ~512 workgroups where the row groups alone are too few, and a
// K-slice short enough for the LDS fragments of four tokens (so the split, and
// with it every token's summation order, does not depend on T).
constexpr int kKqMaxSlice = 12;
constexpr int kKqMaxSsPerLane = 8;  // folded input norm: up to 512 partial groups

template <int QT>
struct KFmt;
template <>
struct KFmt<4> {
    static constexpr int kBlockBytes = 144;
    static constexpr int kChunks = 2;       // 16-byte quant chunks per lane
    static constexpr int kHdr = 2048;       // offset of the row headers
    static constexpr int kTileBytes = 2304;
    static constexpr int kNSub = 8;         // sub-blocks per super-block
    static constexpr int kSubLen = 32;
};
template <>
struct KFmt<6> {
    static constexpr int kBlockBytes = 210;
    static constexpr int kChunks = 3;
    static constexpr int kHdr = 3072;       // row scales (16 B each), then d (2 B each)
    static constexpr int kTileBytes = 3360;
    static constexpr int kNSub = 16;
    static constexpr int kSubLen = 16;
};

__device__ inline float half_bits_to_f32(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
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

// q4k_scale_min on the 16 header bytes held in registers (h[1..3] = scale bytes
// s12[0..11]); j may differ per lane, so bytes are taken by shifts, not by index
// (an indexed local array would live in scratch memory).
__device__ inline void q4k_scale_min_reg(const i32x4& h, int j, int& sc, int& mn) {
    const int sh = 8 * (j & 3);
    const int b1 = (static_cast<uint32_t>(h[1]) >> sh) & 255;  // s12[j & 3]
    const int b2 = (static_cast<uint32_t>(h[2]) >> sh) & 255;  // s12[4 + (j & 3)]
    const int b3 = (static_cast<uint32_t>(h[3]) >> sh) & 255;  // s12[8 + (j & 3)]
    const bool lo = j < 4;
    sc = lo ? (b1 & 63) : ((b3 & 15) | ((b1 >> 6) << 4));
    mn = lo ? (b2 & 63) : ((b3 >> 4) | ((b2 >> 6) << 4));
}

// Offset (within the super-block) of the 16 x values multiplying the quants of MFMA
// mi of lane group g.  Q4_K: mi = 2 * (high nibble) + chunk; Q6_K: mi = kk.
template <int QT>
__device__ inline int x_off16(int g, int mi) {
    if constexpr (QT == 4)
        return 64 * g + 32 * (mi >> 1) + 16 * (mi & 1);
    else
        return 128 * (g >> 1) + 32 * mi + 16 * (g & 1);
}

// Weight sub-block (scale index) of MFMA mi of lane group g.
template <int QT>
__device__ inline int sub_of(int g, int mi) {
    if constexpr (QT == 4)
        return 2 * g + (mi >> 1);
    else
        return 8 * (g >> 1) + 2 * mi + (g & 1);
}

// 16 ints in [-127, 127] -> 16 int8 bytes.
__device__ inline i32x4 pack_i8x16(const int (&v)[16]) {
    i32x4 r;
#pragma unroll
    for (int d = 0; d < 4; ++d)
        r[d] = (v[4 * d] & 255) | ((v[4 * d + 1] & 255) << 8) | ((v[4 * d + 2] & 255) << 16) |
               (static_cast<int>(static_cast<uint32_t>(v[4 * d + 3]) << 24));
    return r;
}

// Split-K tickets live at the start of the caller's workspace: one counter per row
// group, 64 bytes apart (atomics on one cache line serialise), then the partials.
// The workspace is zero-filled once when allocated; the workgroup that takes a
// group's last ticket resets it, so every launch finds them zero.  Launches that
// share one workspace must not overlap in time.
inline size_t kq_ticket_bytes(int groups) { return (static_cast<size_t>(groups) * 64 + 255) / 256 * 256; }
// Token groups of a launch: T <= 4 tokens in one, T = 5..16 in groups of four
// (each with its own tickets).
inline int kq_token_groups(int T) { return (T + 3) / 4; }

// Target of the pipeline's idle load slots (never written).
constexpr int kKqDummyWindows = 64;
__device__ __align__(4096) uint8_t g_kq_dummy[kKqDummyWindows * 4096];

// LDS of a workgroup (K-slice of P super-blocks, NSET token sets of 2 tokens):
//   afrag[set][sbl][mi][p][g]: 16 B (16 int8) -- x hi (p even) / lo (p odd) of
//                              token 2*set + p/2 at x_off16(g, mi)
//   zero16: 16 zero bytes (A operand of the off-diagonal lanes)
//   xinf[t][sbl][j]:           float2 per weight sub-block j: s / 254 (s the scale of
//                              its 32-value x block) and the sub-block's sum of the
//                              quantised x, s * (sum hi + sum lo / 254)
template <int QT>
__host__ __device__ constexpr int kq_afrag_bytes(int P, int nset) { return nset * P * 4 * 4 * 4 * 16; }
template <int QT>
__host__ __device__ constexpr int kq_lds_bytes(int P, int nset, int T) {
    return kq_afrag_bytes<QT>(P, nset) + 16 + T * P * KFmt<QT>::kNSub * 8;
}

// Extra workgroup u of a launch with BF16 rows beside the K-quant ones (KqNorm::ab_w):
// row tile u / ab_slices, K-slice u % ab_slices of the BF16 matrix, over the same
// fp32 x (slices past the last column block write zeros).  Lane (g, r) of wave w
// holds row r at columns 32 g .. 32 g + 31 of each 128-column block (four 16-byte
// chunks); waves take blocks w, w + 4, ...; lane groups summed by shuffles, waves
// in order through LDS.
// Tokens t0 .. t0 + tn - 1 of Tg (the launch's token group; T = 4 per group when Tg > 4).
template <int T, int NRM>
__device__ void kq_ab_rows(const KqNorm& nrm, const float* __restrict__ x, int n, int u, int t0, int tn, int Tg) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int rt = u / nrm.ab_slices, sl = u % nrm.ab_slices;
    const int n_kb = n / 128;
    const int per = (n_kb + nrm.ab_slices - 1) / nrm.ab_slices;
    const int b0 = min(n_kb, sl * per), b1 = min(n_kb, b0 + per);
    __shared__ float red[4][4][16];  // [wave][token][row]
    __shared__ float inv_s[4];
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.f;
    for (int kb = b0 + wave; kb < b1; kb += 4) {
        const uint8_t* tile = reinterpret_cast<const uint8_t*>(nrm.ab_w) + (static_cast<size_t>(rt) * n_kb + kb) * 4096;
        i32x4 w[4];
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) w[c4] = *reinterpret_cast<const i32x4*>(tile + c4 * 1024 + 16 * lane);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            if (t >= tn) break;
            const float4* xp = reinterpret_cast<const float4*>(x + static_cast<size_t>(t0 + t) * n + kb * 128 + 32 * g);
            float s0 = 0.f, s1 = 0.f;
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) {
                const float4 xa = xp[2 * c4], xb = xp[2 * c4 + 1];
                const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t d = static_cast<uint32_t>(w[c4][q]);
                    s0 = fmaf(__uint_as_float(d << 16), xv[2 * q], s0);
                    s1 = fmaf(__uint_as_float(d & 0xffff0000u), xv[2 * q + 1], s1);
                }
            }
            acc[t] += s0 + s1;
        }
    }
    float inv = 1.f;
    if constexpr (NRM == 1) {
        // token w's 1/rms from the input's partial sums (groups in order, then a
        // fixed butterfly), as the K-quant rows
        if (wave < tn) {
            double ss = 0.0;
            for (int gi = lane; gi < nrm.groups_in; gi += 64) ss += static_cast<double>(nrm.ss_in[gi * Tg + t0 + wave]);
            ss = wave_sum_d(ss);
            if (lane == 0) inv_s[wave] = 1.f / sqrtf(static_cast<float>(ss / nrm.n_norm) + nrm.eps);
        }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
        acc[t] += __shfl_xor(acc[t], 16, 64);
        acc[t] += __shfl_xor(acc[t], 32, 64);
        if (g == 0) red[wave][t][r16] = acc[t];
    }
    __syncthreads();
    if (static_cast<int>(threadIdx.x) < tn * 16) {
        const int t = threadIdx.x / 16, r = threadIdx.x % 16;
        const int row = rt * 16 + r;
        float v = ((red[0][t][r] + red[1][t][r]) + red[2][t][r]) + red[3][t][r];
        if constexpr (NRM == 1) v *= inv_s[t];
        (void)inv;
        if (row < nrm.ab_rows) nrm.ab_out[(static_cast<size_t>(sl) * Tg + t0 + t) * nrm.ab_ld + row] = v;
    }
}

// Grid: blockIdx.x = row-group * S + k-slice.  Wave w of the workgroup takes tile
// row RW * row-group + w over the slice's super-blocks.  S == 1: the workgroup writes
// Y (store or add).  S > 1: it writes partial[slice][t][row] and takes a ticket; the
// last workgroup of the row group adds the S partials in slice order (a fixed
// order) and writes Y.  Partials and tickets use agent-scope atomic accesses,
// which are coherent across the XCDs' L2 caches without cache maintenance.
// NRM: 0 plain; 1 consumer of a folded RMSNorm (outputs scaled by 1/rms from
// nrm.ss_in); 2 producer (accumulates into the residual rows and writes nrm.ss_out,
// and the next linear's inputs x * (1 + gamma) as fp32 rows / bf16 fragments);
// 3 producer whose input's 128-column blocks are scaled per token by their
// gated RMSNorm's 1/rms (nrm.bss) as the x fragments are built.
template <int QT, int T, int D, int RW, int NRM = 0>
__global__ __launch_bounds__(64 * RW) void kq_gemm_kernel(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                      float* __restrict__ Y, float* __restrict__ partial,
                                                      unsigned* __restrict__ tickets, int m, int n, int S,
                                                      int accumulate, int ldy, KqNorm nrm, int Tg, int nb) {
    using F = KFmt<QT>;
    constexpr int NSET = (T + 1) / 2;  // token sets of two (hi, mid, hi, mid columns)
    // Token groups: Tg tokens (rows of x) in groups of T; the workgroups of one
    // (row group, slice) for each group are blockIdx 8 apart, so they run on one XCD
    // (workgroups go to the XCDs round-robin) and read the same weight tiles at about
    // the same time: the second read hits that XCD's L2.  Each group runs the
    // T-token kernel on its own rows: every token's sums are those of a launch with
    // that token alone.  nb workgroups per group (launch_kq_rw); the padding exits.
    const int ngrp = (Tg + T - 1) / T;
    const int tgi = (blockIdx.x / 8) % ngrp, bix = (blockIdx.x / (8 * ngrp)) * 8 + blockIdx.x % 8;
    const int t0 = tgi * T, tn = min(T, Tg - t0);  // this workgroup's tokens t0 .. t0 + tn - 1
    if (ngrp > 1 && bix >= nb) return;
    if constexpr (NRM < 2) {
        // extra workgroups past the K-quant ones: the BF16 rows (KqNorm::ab_w)
        const int ab_wgs = nrm.ab_w ? ((nrm.ab_rows + 15) / 16) * nrm.ab_slices : 0;
        if (bix >= nb - ab_wgs) {
            kq_ab_rows<T, NRM>(nrm, x, n, bix - (nb - ab_wgs), t0, tn, Tg);
            return;
        }
    }
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int rgp = bix / S;
    const int slice = bix % S;
    const int nsb = n / 256;
    const int per_slice = (nsb + S - 1) / S;
    const int s0 = min(nsb, slice * per_slice), s1 = min(nsb, s0 + per_slice);
    const int P = per_slice;
    const int m_tiles = (m + kTR - 1) / kTR;
    const int rt = min(rgp * RW + wave, m_tiles - 1);
    const bool wave_live = rgp * RW + wave < m_tiles;

    i32x4* afrag = reinterpret_cast<i32x4*>(lds);
    i32x4* zero16 = reinterpret_cast<i32x4*>(lds + kq_afrag_bytes<QT>(P, NSET));
    float2* xinf = reinterpret_cast<float2*>(lds + kq_afrag_bytes<QT>(P, NSET) + 16);

    const uint8_t* tiles = W + static_cast<size_t>(rt) * nsb * F::kTileBytes;
    // loads per lane per tile: quant chunks, the row's header (Q4_K d, dmin and scale
    // bytes; Q6_K the 16 int8 scales) and, for Q6_K, the row's fp16 d
    constexpr int NL = F::kChunks + 1;
    // D tiles in flight per wave.  Pipeline slots past the slice still issue their
    // loads (so every wait has a static count), from a zero block that stays in the
    // caches; each wave reads its own 4 KiB window of it (one shared address would
    // queue every wave on one L2 channel).
    i32x4 buf[D][NL];
    uint32_t dbits[D];
    const uint8_t* dummy = g_kq_dummy + ((bix * RW + wave) % kKqDummyWindows) * 4096;
    auto load = [&](int d, int sb, bool live) {
        const uint8_t* tile = live ? tiles + static_cast<size_t>(sb) * F::kTileBytes : dummy;
#pragma unroll
        for (int k = 0; k < F::kChunks; ++k) {
            const i32x4* p = reinterpret_cast<const i32x4*>(tile + k * 1024 + 16 * lane);
            buf[d][k] = live ? __builtin_nontemporal_load(p) : *p;
        }
        buf[d][NL - 1] = *reinterpret_cast<const i32x4*>(tile + F::kHdr + 16 * r16);
        if constexpr (QT == 6) dbits[d] = reinterpret_cast<const uint16_t*>(tile + F::kHdr + 256)[r16];
    };
    // folded input RMSNorm: wave w < T holds token w's partial sums of squares
    // (group l + 64k in lane l), reduced in the epilogue
    float ssr[NRM == 1 ? kKqMaxSsPerLane : 1];
    const bool ss_wave = NRM == 1 && wave < tn;
    if constexpr (NRM == 1) {
#pragma unroll
        for (int k = 0; k < kKqMaxSsPerLane; ++k) {
            const int gi = lane + 64 * k;
            ssr[k] = ss_wave && gi < nrm.groups_in ? nrm.ss_in[static_cast<size_t>(gi) * Tg + t0 + wave] : 0.f;
        }
    }

    // ---- x fragments of this slice: each 32-value block of a token is quantised
    // to int8 hi + lo with one scale s = max|x| / 127:  x ~ s * (hi + lo / 254),
    // |hi|, |lo| <= 127 (15 significant bits of the block maximum)
    {
        const int nsl = s1 - s0;
        if (threadIdx.x == 0) *zero16 = i32x4{0, 0, 0, 0};
        // items (token, sbl, r): the 16-value run r of the super-block; the two runs
        // of a 32-value block sit in adjacent lanes
        const int items = tn * P * 16;
        // at most kPer items per thread: every item's x loads are issued before the
        // first item is processed (one memory round trip for the whole build)
        constexpr int kPer = (T * kKqMaxSlice * 16 + 64 * RW - 1) / (64 * RW);
        float4 xv[kPer][4];
        float4 bs4[NRM == 3 ? kPer : 1];  // the run's 128-column block's partial sums
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int it = threadIdx.x + k * 64 * RW;
            const int r = it & 15, sbl = (it >> 4) % P, t = (it >> 4) / P;
#pragma unroll
            for (int q = 0; q < 4; ++q) xv[k][q] = make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (NRM == 3) bs4[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (it < items && sbl < nsl) {
                const int col = (s0 + sbl) * 256 + 16 * r;
                const float4* px = reinterpret_cast<const float4*>(x + static_cast<size_t>(t0 + t) * n + col);
#pragma unroll
                for (int q = 0; q < 4; ++q) xv[k][q] = px[q];
                if constexpr (NRM == 3)
                    bs4[k] = *reinterpret_cast<const float4*>(nrm.bss + (static_cast<size_t>(col >> 7) * Tg + t0 + t) * 4);
            }
        }
        // the first weights are requested after the x loads and before the build:
        // vector loads return in issue order, so the build waits only for x (L2),
        // not for the weights (HBM)
#pragma unroll
        for (int d = 0; d < D; ++d) load(d, s0 + d, s0 + d < s1);
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int it = threadIdx.x + k * 64 * RW;
            if (k * 64 * RW >= items) break;  // uniform: whole waves past the items
            const int r = it & 15, sbl = (it >> 4) % P, t = (it >> 4) / P;
            float v[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                v[4 * q] = xv[k][q].x;
                v[4 * q + 1] = xv[k][q].y;
                v[4 * q + 2] = xv[k][q].z;
                v[4 * q + 3] = xv[k][q].w;
            }
            if constexpr (NRM == 3) {
                // the run's gated RMSNorm block (sums in a fixed order)
                const float sum = (bs4[k].x + bs4[k].y) + (bs4[k].z + bs4[k].w);
                const float inv = 1.f / sqrtf(sum / 128.f + 1e-6f);
#pragma unroll
                for (int e = 0; e < 16; ++e) v[e] *= inv;
            }
            float mx = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) mx = fmaxf(mx, fabsf(v[e]));
            mx = fmaxf(mx, __shfl_xor(mx, 1, 64));  // the 32-value block's maximum
            // hardware reciprocal (about 1 ulp): the quantised values stay in
            // [-127, 127] (|v * inv| <= 127 (1 + 2^-22) rounds to 127) and x ~ sc * (hi +
            // lo / 254) to the same 15 bits; the correctly rounded divisions were two
            // long sequences per item on every workgroup's path to its first tile
            const float sc = mx * (1.f / 127.f);
            const float inv = mx > 0.f ? 127.f * __builtin_amdgcn_rcpf(mx) : 0.f;
            int hi[16], lo[16], shi = 0, slo = 0;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float u = v[e] * inv;
                const float h = rintf(u);
                hi[e] = static_cast<int>(h);
                lo[e] = static_cast<int>(rintf((u - h) * 254.f));
                shi += hi[e];
                slo += lo[e];
            }
            // the weight sub-block's sum of the quantised x: Q4_K sub-blocks are the
            // 32-value blocks (both runs), Q6_K sub-blocks the 16-value runs
            if constexpr (QT == 4) {
                shi += __shfl_xor(shi, 1, 64);
                slo += __shfl_xor(slo, 1, 64);
            }
            if (it < items && sbl < nsl) {
                int g, mi;
                if constexpr (QT == 4) {
                    g = r >> 2;
                    mi = r & 3;
                } else {
                    g = 2 * (r >> 3) + (r & 1);
                    mi = (r >> 1) & 3;
                }
                const int set = t >> 1, tt = t & 1;
                const int base = (((set * P + sbl) * 4 + mi) * 4) * 4;  // [set][sbl][mi][p][g]
                afrag[base + (2 * tt) * 4 + g] = pack_i8x16(hi);
                afrag[base + (2 * tt + 1) * 4 + g] = pack_i8x16(lo);
                const float X = sc * (static_cast<float>(shi) + static_cast<float>(slo) * (1.f / 254.f));
                if (QT == 6 || (r & 1) == 0)
                    xinf[(t * P + sbl) * F::kNSub + (QT == 4 ? (r >> 1) : sub_of<6>(g, mi))] =
                        make_float2(sc * (1.f / 254.f), X);
            }
        }
        // (entries past the slice and the second column of an odd T's last set are
        // never used: the loop stops at the slice end, and an unused token column
        // only reaches its own output rows)
    }
    __syncthreads();

    // A operand source of this lane: token column p = r16 % 4 of lane group g when
    // r16 / 4 == g, else the zero block
    const bool diag = (r16 >> 2) == g;
    const int p_lane = r16 & 3;

    float tot[4] = {0.f, 0.f, 0.f, 0.f};  // per token
    for (int sb0 = s0; sb0 < s1; sb0 += D) {
#pragma unroll
        for (int ps = 0; ps < D; ++ps) {
            const int sb = sb0 + ps;
            if (sb < s1) {
                const int sbl = sb - s0;
                const i32x4* cb = buf[ps];
                const float dq6d = QT == 6 ? half_bits_to_f32(dbits[ps]) : 0.f;
                // this super-block's x fragments (A operands), scales and sub-block
                // sums, read from LDS together before the MFMAs need them
                i32x4 af[NSET][4];
                {
                    const i32x4* fa = diag ? afrag + (((sbl * 4) * 4 + p_lane) * 4 + g) : zero16;
                    const int fstep = diag ? 16 : 0;  // i32x4 per mi
#pragma unroll
                    for (int st = 0; st < NSET; ++st)
#pragma unroll
                        for (int mi = 0; mi < 4; ++mi) af[st][mi] = fa[(st * P * 4 + mi) * fstep];
                }
                constexpr int kLaneSubs = QT == 4 ? 2 : 4;
                float2 xi[T][kLaneSubs];
#pragma unroll
                for (int t = 0; t < T; ++t)
#pragma unroll
                    for (int k = 0; k < kLaneSubs; ++k)
                        xi[t][k] = xinf[(t * P + sbl) * F::kNSub + sub_of<QT>(g, QT == 4 ? 2 * k : k)];
                // quants as int8 B operands (16 per MFMA, one sub-block), exact int32
                // dot products with x hi / lo per sub-block
                i32x4 acc[NSET][kLaneSubs];
#pragma unroll
                for (int st = 0; st < NSET; ++st)
#pragma unroll
                    for (int k = 0; k < kLaneSubs; ++k) acc[st][k] = i32x4{0, 0, 0, 0};
#pragma unroll
                for (int mi = 0; mi < 4; ++mi) {
                    i32x4 bq;
                    if constexpr (QT == 4) {
                        // chunk mi & 1, nibble mi >> 1: the 16 quants of sub-block 2g + (mi >> 1)
                        const i32x4 ch = cb[mi & 1];
#pragma unroll
                        for (int d = 0; d < 4; ++d)
                            bq[d] = static_cast<int>((static_cast<uint32_t>(ch[d]) >> (4 * (mi >> 1))) & 0x0f0f0f0fu);
                    } else {
                        // kk = mi: low 4 bits from ql chunk kk & 1 (nibble kk >> 1), high 2 bits
                        // from qh bits 2kk, 2kk+1
                        const i32x4 ql = cb[mi & 1];
                        const i32x4 qh = cb[2];
#pragma unroll
                        for (int d = 0; d < 4; ++d) {
                            const uint32_t low = (static_cast<uint32_t>(ql[d]) >> (4 * (mi >> 1))) & 0x0f0f0f0fu;
                            const uint32_t h2 = (static_cast<uint32_t>(qh[d]) >> (2 * mi)) & 0x03030303u;
                            bq[d] = static_cast<int>(low | (h2 << 4));
                        }
                    }
                    const int k = QT == 4 ? (mi >> 1) : mi;
#pragma unroll
                    for (int st = 0; st < NSET; ++st)
                        acc[st][k] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[st][mi], bq, acc[st][k], 0, 0, 0);
                }
                // per (row, sub-block) scales of this lane's sub-blocks:
                // y += a_j * (s / 254) * (254 C_hi + C_lo) - b_j * X_j (the integer
                // 254 C_hi + C_lo is exact; below 2^24 for Q4_K)
                if constexpr (QT == 4) {
                    // header dwords: d | dmin, then scale bytes s12[0..3], [4..7], [8..11]
                    const uint32_t h0 = static_cast<uint32_t>(cb[NL - 1][0]);
                    const float d = half_bits_to_f32(h0 & 0xffffu);
                    const float dmin = half_bits_to_f32(h0 >> 16);
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        int sc, mn;
                        q4k_scale_min_reg(cb[NL - 1], 2 * g + k, sc, mn);
                        const float a = d * static_cast<float>(sc);
                        const float c = dmin * static_cast<float>(mn);
#pragma unroll
                        for (int t = 0; t < T; ++t) {
                            const int ci = __mul24(acc[t >> 1][k][2 * (t & 1)], 254) + acc[t >> 1][k][2 * (t & 1) + 1];
                            tot[t] = fmaf(a * xi[t][k].x, static_cast<float>(ci), fmaf(-c, xi[t][k].y, tot[t]));
                        }
                    }
                } else {
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) {
                        // scale j = 8h + 2kk + e (h = g / 2, e = g % 2): dword 2h + kk / 2,
                        // byte 2 (kk % 2) + e of the row's 16 int8 scales
                        const i32x4 sv = cb[NL - 1];
                        const int dw = (g >> 1) ? ((kk >> 1) ? sv[3] : sv[2]) : ((kk >> 1) ? sv[1] : sv[0]);
                        const int scv = __builtin_amdgcn_sbfe(dw, 8 * (2 * (kk & 1) + (g & 1)), 8);
                        const float a = dq6d * static_cast<float>(scv);
                        const float c = 32.f * a;
#pragma unroll
                        for (int t = 0; t < T; ++t) {
                            const int ci = __mul24(acc[t >> 1][kk][2 * (t & 1)], 254) + acc[t >> 1][kk][2 * (t & 1) + 1];
                            tot[t] = fmaf(a * xi[t][kk].x, static_cast<float>(ci), fmaf(-c, xi[t][kk].y, tot[t]));
                        }
                    }
                }
            }
            load(ps, sb + D, sb + D < s1);
        }
    }

    // the four lane groups of a row hold quarters of it: fixed-order sum (every lane
    // ends with its row's totals); from here lane group g finishes token g
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        tot[t] += __shfl_xor(tot[t], 16, 64);
        tot[t] += __shfl_xor(tot[t], 32, 64);
    }
    const int te = g;  // this lane's token
    const int row = rt * kTR + r16;
    const bool own = wave_live && te < tn && row < m;
    const int tw = t0 + te;  // the token's row of x / Y
    __shared__ int s_last;
    float v = tot[0];
#pragma unroll
    for (int t = 1; t < T; ++t) v = te == t ? tot[t] : v;
    // the row's old value (accumulate) is requested now, so its round trip overlaps
    // the ticket and the partial loads
    const float y_old = own && accumulate ? Y[static_cast<size_t>(tw) * ldy + row] : 0.f;
    if (S > 1) {
        if (own)
            __hip_atomic_store(partial + (static_cast<size_t>(slice) * Tg + tw) * m + row, v, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // partial stores complete before the ticket
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned* tk = tickets + (static_cast<size_t>(rgp) * ngrp + tgi) * 16;
            const unsigned old = __hip_atomic_fetch_add(tk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int last = old == static_cast<unsigned>(S - 1);
            if (last) __hip_atomic_store(tk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = last;
        }
        __syncthreads();
        if (!s_last) return;
        if (own) {
            // the partials of 8 slices requested together (one memory round trip per
            // 8 slices), then added in slice order
            v = 0.f;
            for (int q0 = 0; q0 < S; q0 += 8) {
                float pv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    pv[j] = q0 + j < S ? __hip_atomic_load(partial + (static_cast<size_t>(q0 + j) * Tg + tw) * m + row,
                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                       : 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (q0 + j < S) v += pv[j];
            }
        }
    }

    // ---- final write of the row group (one writer per row and token)
    __shared__ float s_inv[4];
    __shared__ double s_sq[4][4];  // [wave][token]
    if constexpr (NRM == 1) {
        // folded input norm: token w's 1/rms from its partial sums (groups in order,
        // then a fixed butterfly)
        if (ss_wave) {
            double ss = 0.0;
#pragma unroll
            for (int k = 0; k < kKqMaxSsPerLane; ++k) ss += static_cast<double>(ssr[k]);
            ss = wave_sum_d(ss);
            if (lane == 0) s_inv[wave] = 1.f / sqrtf(static_cast<float>(ss / nrm.n_norm) + nrm.eps);
        }
        __syncthreads();
    }
    float y = NRM == 1 ? v * s_inv[te < tn ? te : 0] : v;
    if (NRM < 2 && nrm.swiglu) {
        // gate / up half tiles: tile rows 8..15 are the up rows of rows 0..7, so
        // lane r16 < 8 pairs its gate value with lane r16 + 8's up value
        // (silu(g) * u, reference ops.cpp:607-609)
        const float u = __shfl_down(y, 8, 64);
        if (own && r16 < 8) Y[static_cast<size_t>(tw) * ldy + rt * 8 + r16] = y / (1.f + expf(-y)) * u;
        return;
    }
    if (own) {
        y = accumulate ? y_old + y : y;
        Y[static_cast<size_t>(tw) * ldy + row] = y;
    }
    if constexpr (NRM >= 2) {
        // residual add fused with the next RMSNorm's data: the row group's sum of
        // x^2 per token (16 rows per wave by a fixed butterfly within the token's lane
        // group, the waves in order, double) and the next linear's inputs
        // x * (1 + gamma): fp32 rows (xg_out) and, if asked, bf16 fragments
        double sq = own ? static_cast<double>(y) * y : 0.0;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) sq += __shfl_xor(sq, o, 64);
        if (r16 == 0 && te < tn) s_sq[wave][te] = sq;
        if (own) {
            const float xg = y * (1.f + nrm.gamma_out[row]);
            nrm.xg_out[static_cast<size_t>(tw) * m + row] = xg;
            if (nrm.frag_out) {
                uint16_t* f16 = static_cast<uint16_t*>(nrm.frag_out);
                uint16_t hi, mid;
                split_bf16(xg, hi, mid);
                const size_t u = frag_unit(row >> 3, tw, Tg);
                f16[u * 8 + (row & 7)] = hi;
                f16[(u + Tg) * 8 + (row & 7)] = mid;
            }
        }
        __syncthreads();
        if (static_cast<int>(threadIdx.x) < tn) {
            double sq = 0.0;
            for (int w = 0; w < RW; ++w) sq += s_sq[w][threadIdx.x];
            nrm.ss_out[static_cast<size_t>(rgp) * Tg + t0 + threadIdx.x] = static_cast<float>(sq);
        }
    }
}

// Row-major GGUF blocks [m][n/256 * bb] -> tiles.  One thread per (tile, lane).
// With src_up, the tiles are gate / up half tiles: tile rt holds rows 8 rt .. 8 rt + 7
// of src (gate) as its rows 0..7 and the same rows of src_up as its rows 8..15.
template <int QT>
__global__ void kq_pack_kernel(const uint8_t* __restrict__ src, const uint8_t* __restrict__ src_up,
                               uint8_t* __restrict__ dst, int m, int nsb) {
    // rows past m are written as zero blocks (d = 0: every weight is 0)
    using F = KFmt<QT>;
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // (rt, sb, lane)
    const int m_tiles = src_up ? (m + 7) / 8 : (m + kTR - 1) / kTR;
    if (idx >= static_cast<size_t>(m_tiles) * nsb * 64) return;
    const int lane = idx % 64;
    const int sb = (idx / 64) % nsb;
    const int rt = static_cast<int>(idx / (static_cast<size_t>(64) * nsb));
    const int r16 = lane & 15, g = lane >> 4;
    const int row = src_up ? rt * 8 + (r16 & 7) : rt * kTR + r16;
    uint8_t* tile = dst + (static_cast<size_t>(rt) * nsb + sb) * F::kTileBytes;
    const uint8_t* blk = (src_up && r16 >= 8 ? src_up : src) + (static_cast<size_t>(row) * nsb + sb) * F::kBlockBytes;
    const bool ok = row < m;
    auto put = [&](int chunk, int off) {
        for (int e = 0; e < 16; ++e) tile[chunk * 1024 + 16 * lane + e] = ok ? blk[off + e] : 0;
    };
    if constexpr (QT == 4) {
        put(0, 16 + 32 * g);
        put(1, 16 + 32 * g + 16);
        if (g == 0)
            for (int e = 0; e < 16; ++e) tile[F::kHdr + 16 * r16 + e] = ok ? blk[e] : 0;
    } else {
        const int h = g >> 1, e16 = g & 1;
        put(0, 64 * h + 16 * e16);
        put(1, 64 * h + 32 + 16 * e16);
        put(2, 128 + 32 * h + 16 * e16);
        if (g == 0) {
            for (int e = 0; e < 16; ++e) tile[F::kHdr + 16 * r16 + e] = ok ? blk[192 + e] : 0;
            tile[F::kHdr + 256 + 2 * r16] = ok ? blk[208] : 0;
            tile[F::kHdr + 256 + 2 * r16 + 1] = ok ? blk[209] : 0;
        }
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

// Eight consecutive weights of row r16 of a K-quant tile row, columns c0 .. c0 + 7
// of super-block tile `tile` (c0 a multiple of 8), dequantised with the reference's
// operation order (q4k_dequant_kernel / q6k_dequant_kernel: separate products and
// difference, no contraction).
template <int QT>
__device__ inline void kq_dequant8(const uint8_t* __restrict__ tile, int r16, int c0, float (&w)[8]) {
#pragma clang fp contract(off)
    using F = KFmt<QT>;
    const uint8_t* hdr = tile + F::kHdr + 16 * r16;
    if constexpr (QT == 4) {
        const int g64 = c0 / 64, high = (c0 % 64) >= 32, l0 = c0 % 32;
        const uint8_t* qs = tile + (l0 / 16) * 1024 + 16 * (r16 + 16 * g64) + (l0 % 16);
        const float d = half_bits_to_f32(hdr[0] | (hdr[1] << 8));
        const float dmin = half_bits_to_f32(hdr[2] | (hdr[3] << 8));
        int sc, mn;
        q4k_scale_min(hdr + 4, 2 * g64 + high, sc, mn);
        const float a = __fmul_rn(d, static_cast<float>(sc)), b = __fmul_rn(dmin, static_cast<float>(mn));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int q = high ? (qs[e] >> 4) : (qs[e] & 15);
            w[e] = __fsub_rn(__fmul_rn(a, static_cast<float>(q)), b);
        }
    } else {
        const int half = c0 / 128, rem = c0 % 128, sel = rem / 32, l0 = rem % 32;
        const int g = 2 * half + l0 / 16, off = l0 % 16;
        const uint8_t* ql = tile + (sel & 1) * 1024 + 16 * (r16 + 16 * g) + off;  // ql[l] or ql[l + 32]
        const uint8_t* qh = tile + 2 * 1024 + 16 * (r16 + 16 * g) + off;
        const float d = half_bits_to_f32(tile[F::kHdr + 256 + 2 * r16] | (tile[F::kHdr + 256 + 2 * r16 + 1] << 8));
        const int8_t scv = static_cast<int8_t>(hdr[8 * half + l0 / 16 + 2 * sel]);
        const float a = __fmul_rn(d, static_cast<float>(scv));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int lq = sel < 2 ? (ql[e] & 15) : (ql[e] >> 4);
            const int v = (lq | (((qh[e] >> (2 * sel)) & 3) << 4)) - 32;
            w[e] = __fmul_rn(a, static_cast<float>(v));
        }
    }
}

// Tiled K-quant -> BF16 tiles hi + lo (the gemm.hip BF16 tile: 16 rows x 128
// columns, unit (chunk q, lane (row, g)) = columns 32 g + 8 q .. + 8).  One thread
// per (row tile, super-block, row, 8 columns): the eight weights dequantised
// (kq_dequant8), each split into its top 16 bits and the top 16 bits of the
// remainder.
template <int QT>
__global__ void kq_to_bf16x2_kernel(const uint8_t* __restrict__ tiled, uint16_t* __restrict__ hi,
                                    uint16_t* __restrict__ lo, int m_tiles, int nsb) {
    using F = KFmt<QT>;
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // (rt, sb, u, r16)
    if (idx >= static_cast<size_t>(m_tiles) * nsb * 32 * 16) return;
    const int r16 = idx & 15;
    const int u = (idx >> 4) & 31;  // 8-column group of the super-block
    const int sb = static_cast<int>((idx >> 9) % nsb);
    const int rt = static_cast<int>((idx >> 9) / nsb);
    const uint8_t* tile = tiled + (static_cast<size_t>(rt) * nsb + sb) * F::kTileBytes;
    const int c0 = 8 * u;  // first column within the super-block
    float w[8];
    kq_dequant8<QT>(tile, r16, c0, w);
    // BF16 tile (rt, kb) and its unit for columns j .. j + 7 of the 128-column block
    const int kb = 2 * sb + c0 / 128, j = c0 % 128;
    const int g = j / 32, q = (j % 32) / 8;
    const size_t unit = (static_cast<size_t>(rt) * (2 * nsb) + kb) * 2048 + q * 512 + 8 * (r16 + 16 * g);
    union {
        uint16_t h[8];
        i32x4 v;
    } H, L;
#pragma unroll
    for (int e = 0; e < 8; ++e) split_bf16(w[e], H.h[e], L.h[e]);
    *reinterpret_cast<i32x4*>(hi + unit) = H.v;
    *reinterpret_cast<i32x4*>(lo + unit) = L.v;
}

// Power of two s with max / s in [2^14, 2^15) (1 for max = 0): values scaled by 1/s
// keep fp16's full precision and range.
__device__ inline float f16_block_scale(float mx) {
    if (!(mx > 0.f)) return 1.f;
    int e;
    frexpf(mx, &e);  // mx = f * 2^e, f in [0.5, 1)
    return ldexpf(1.f, e - 15);
}

// Tiled K-quant -> fp16 tiles in the BF16 tile layout, one power-of-two scale per
// (16-row tile, 128-column block): workgroup = one (row tile, block), thread =
// (row, 8 columns).  Each weight is dequantised exactly (kq_dequant8), divided by
// the block's scale (exact) and rounded to fp16 (nearest even): 11 significant bits.
template <int QT>
__global__ __launch_bounds__(256) void kq_to_f16_kernel(const uint8_t* __restrict__ tiled, _Float16* __restrict__ w16,
                                                        float* __restrict__ tscale, int nsb) {
    using F = KFmt<QT>;
    const int rt = blockIdx.x, kb = blockIdx.y, n_kb = 2 * nsb;
    const int tid = threadIdx.x, r16 = tid & 15, u = tid >> 4;  // 8-column group u of the block
    const int sb = kb >> 1, c0 = (kb & 1) * 128 + 8 * u;
    const uint8_t* tile = tiled + (static_cast<size_t>(rt) * nsb + sb) * F::kTileBytes;
    float w[8];
    kq_dequant8<QT>(tile, r16, c0, w);
    float mx = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(w[e]));
    mx = wave_max(mx);
    __shared__ float wmax[4];
    if ((tid & 63) == 0) wmax[tid >> 6] = mx;
    __syncthreads();
    const float s = f16_block_scale(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])));
    const float inv = 1.f / s;  // a power of two: exact
    const int j = 8 * u, g = j / 32, q = (j % 32) / 8;
    const size_t unit = (static_cast<size_t>(rt) * n_kb + kb) * 2048 + q * 512 + 8 * (r16 + 16 * g);
    union {
        _Float16 h[8];
        i32x4 v;
    } H;
#pragma unroll
    for (int e = 0; e < 8; ++e) H.h[e] = static_cast<_Float16>(w[e] * inv);
    *reinterpret_cast<i32x4*>(w16 + unit) = H.v;
    if (tid == 0) tscale[static_cast<size_t>(rt) * n_kb + kb] = s;
}

size_t kq_tiled_bytes(int qt, int m, int n) {
    const size_t tile = qt == 4 ? KFmt<4>::kTileBytes : KFmt<6>::kTileBytes;
    return static_cast<size_t>((m + kTR - 1) / kTR) * (n / 256) * tile;
}

constexpr int kKqDepth = 4;  // tiles in flight per wave
// Row tiles (waves) per workgroup.  RL_KQ_RW overrides it for measurement.
int kq_rw() {
    static const int rw = [] {
        const char* v = std::getenv("RL_KQ_RW");
        const int r = v ? std::atoi(v) : 0;
        return r == 1 || r == 2 || r == 4 ? r : 4;
    }();
    return rw;
}
void kq_split(int m, int nsb, int& S) {
    // about two workgroups per CU in total (5120 x 17408: 80 row groups x 6 slices
    // measured best, 15.5 us against 17.1 us with 8 slices and 21.6 us with 16),
    // slices of at least 4 super-blocks
    const int groups = (m + kTR * kq_rw() - 1) / (kTR * kq_rw());
    S = std::max(1, std::min(512 / groups, nsb / 4));
    while ((nsb + S - 1) / S > kKqMaxSlice) ++S;
    // one round instead: when slices of at most 8 super-blocks give every row group
    // its slices on one CU each (5120 x 6144 Q4_K: 80 x 3 workgroups, 8.1 -> 7.1 us
    // at T = 1 and 9.4 -> 9.1 us at T = 4 against 80 x 6)
    const int s1 = (nsb + 7) / 8;
    if (s1 < S && groups * s1 <= device_cus()) S = s1;
    static const char* env = std::getenv("RL_KQ_SPLIT");  // measurement override
    if (env && std::atoi(env) > 0) S = std::max(std::atoi(env), (nsb + kKqMaxSlice - 1) / kKqMaxSlice);
    S = std::min(S, nsb);
}

// T tokens per workgroup; Tg (> T only for T = 4) tokens in groups of T, one
// workgroup per group for each (row group, slice).
template <int QT, int T, int RW, int NRM>
void launch_kq_rw(const uint8_t* W, const float* x, float* Y, float* partial, unsigned* tickets, int m, int n, int S,
                  int accumulate, int ldy, hipStream_t s, const KqNorm& nrm, int Tg) {
    const int groups = (m + kTR * RW - 1) / (kTR * RW);
    const int P = (n / 256 + S - 1) / S;
    const size_t lds = kq_lds_bytes<QT>(P, (T + 1) / 2, T);
    const int ab_wgs = nrm.ab_w ? ((nrm.ab_rows + 15) / 16) * nrm.ab_slices : 0;
    const int ngrp = (Tg + T - 1) / T;
    const int nb = groups * S + ab_wgs;  // workgroups per token group
    const int grid = ngrp == 1 ? nb : (nb + 7) / 8 * 8 * ngrp;
    hipLaunchKernelGGL((kq_gemm_kernel<QT, T, kKqDepth, RW, NRM>), dim3(grid), dim3(64 * RW), lds, s, W, x, Y, partial,
                       tickets, m, n, S, accumulate, ldy, nrm, Tg, nb);
}

template <int QT, int T>
void launch_kq_t(const uint8_t* W, const float* x, float* Y, float* partial, unsigned* tickets, int m, int n, int S,
                 int accumulate, int ldy, hipStream_t s, const KqNorm& nrm, int Tg) {
    // the folded-norm variants use the default work split only
    if (nrm.ss_in) {
        RL_REQUIRE(kq_rw() == 4, RL_ERR_UNSUPPORTED, "kquant: folded RMSNorm needs four row tiles per workgroup");
        launch_kq_rw<QT, T, 4, 1>(W, x, Y, partial, tickets, m, n, S, accumulate, ldy, s, nrm, Tg);
        return;
    }
    if (nrm.ss_out) {
        RL_REQUIRE(kq_rw() == 4, RL_ERR_UNSUPPORTED, "kquant: folded RMSNorm needs four row tiles per workgroup");
        if (nrm.bss)
            launch_kq_rw<QT, T, 4, 3>(W, x, Y, partial, tickets, m, n, S, accumulate, ldy, s, nrm, Tg);
        else
            launch_kq_rw<QT, T, 4, 2>(W, x, Y, partial, tickets, m, n, S, accumulate, ldy, s, nrm, Tg);
        return;
    }
    switch (kq_rw()) {
    case 1: launch_kq_rw<QT, T, 1, 0>(W, x, Y, partial, tickets, m, n, S, accumulate, ldy, s, nrm, Tg); break;
    case 2: launch_kq_rw<QT, T, 2, 0>(W, x, Y, partial, tickets, m, n, S, accumulate, ldy, s, nrm, Tg); break;
    default: launch_kq_rw<QT, T, 4, 0>(W, x, Y, partial, tickets, m, n, S, accumulate, ldy, s, nrm, Tg); break;
    }
}

template <int QT>
void launch_kq(const uint8_t* W, const float* x, float* Y, float* partial, unsigned* tickets, int m, int n, int T, int S,
               int accumulate, int ldy, hipStream_t s, const KqNorm& nrm) {
    const int Tg = T;
    switch (T) {
    case 1: launch_kq_t<QT, 1>(W, x, Y, partial, tickets, m, n, S, accumulate, ldy, s, nrm, Tg); break;
    case 2: launch_kq_t<QT, 2>(W, x, Y, partial, tickets, m, n, S, accumulate, ldy, s, nrm, Tg); break;
    case 3: launch_kq_t<QT, 3>(W, x, Y, partial, tickets, m, n, S, accumulate, ldy, s, nrm, Tg); break;
    default: launch_kq_t<QT, 4>(W, x, Y, partial, tickets, m, n, S, accumulate, ldy, s, nrm, Tg); break;
    }
}

}  // namespace

namespace rl {

void kq_to_bf16x2(int qt, const uint8_t* tiled, uint16_t* hi, uint16_t* lo, int m, int n, hipStream_t s) {
    RL_REQUIRE((qt == 4 || qt == 6) && m > 0 && n > 0 && n % 256 == 0 && tiled && hi && lo, RL_ERR_RANGE,
               "kquant_to_bf16x2: Q4_K / Q6_K, n a multiple of 256");
    const int m_tiles = (m + kTR - 1) / kTR, nsb = n / 256;
    const size_t threads = static_cast<size_t>(m_tiles) * nsb * 512;
    const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
    if (qt == 4)
        hipLaunchKernelGGL(kq_to_bf16x2_kernel<4>, grid, dim3(256), 0, s, tiled, hi, lo, m_tiles, nsb);
    else
        hipLaunchKernelGGL(kq_to_bf16x2_kernel<6>, grid, dim3(256), 0, s, tiled, hi, lo, m_tiles, nsb);
    check_launch("kq_to_bf16x2_kernel");
}


void kq_to_f16(int qt, const uint8_t* tiled, void* w16, float* tscale, int m, int n, hipStream_t s) {
    RL_REQUIRE((qt == 4 || qt == 6) && m > 0 && n > 0 && n % 256 == 0 && tiled && w16 && tscale, RL_ERR_RANGE,
               "kquant_to_f16: Q4_K / Q6_K, n a multiple of 256");
    const int m_tiles = (m + kTR - 1) / kTR, nsb = n / 256;
    const dim3 grid(m_tiles, 2 * nsb);
    _Float16* w = static_cast<_Float16*>(w16);
    if (qt == 4)
        hipLaunchKernelGGL(kq_to_f16_kernel<4>, grid, dim3(256), 0, s, tiled, w, tscale, nsb);
    else
        hipLaunchKernelGGL(kq_to_f16_kernel<6>, grid, dim3(256), 0, s, tiled, w, tscale, nsb);
    check_launch("kq_to_f16_kernel");
}

size_t kq_workspace_bytes(int m, int n, int T) {
    // split-K tickets, then the partials of the split: S*T*m floats
    int S;
    kq_split(m, n / 256, S);
    if (S == 1) return 256;
    const int groups = (m + kTR * kq_rw() - 1) / (kTR * kq_rw());
    return kq_ticket_bytes(groups * kq_token_groups(T)) + static_cast<size_t>(S) * T * m * 4;
}

// Y[T][m] (=, +=) W . x for Q4_K (qt=4) / Q6_K (qt=6) K-tiled weights.
int kq_norm_groups(int m) { return (m + kTR * kq_rw() - 1) / (kTR * kq_rw()); }
bool kq_fold_supported() { return kq_rw() == 4; }

void kq_gemm(int qt, const uint8_t* W, const float* x, float* Y, void* ws, size_t ws_bytes, int m, int n, int T,
             int accumulate, int ldy, hipStream_t s, const KqNorm* norm) {
    const KqNorm nrm = norm ? *norm : KqNorm{};
    RL_REQUIRE(qt == 4 || qt == 6, RL_ERR_UNSUPPORTED, "kquant: type must be Q4_K or Q6_K");
    RL_REQUIRE(!nrm.ss_in || (nrm.groups_in >= 1 && nrm.groups_in <= 64 * kKqMaxSsPerLane && nrm.n_norm > 0),
               RL_ERR_RANGE, "kquant: folded RMSNorm needs 1..512 partial groups");
    RL_REQUIRE(!nrm.ss_out || (accumulate && ldy == m && nrm.gamma_out && nrm.xg_out && !nrm.ss_in), RL_ERR_RANGE,
               "kquant: the add-norm output accumulates into the [T][m] residual rows and needs gamma and the "
               "x * (1 + gamma) rows");
    RL_REQUIRE(!nrm.frag_out || nrm.ss_out, RL_ERR_RANGE, "kquant: fragment output needs the add-norm output");
    RL_REQUIRE(!nrm.bss || nrm.ss_out, RL_ERR_RANGE, "kquant: block-scaled input with the add-norm output only");
    RL_REQUIRE(!nrm.ab_w || (!nrm.ss_out && !nrm.swiglu && nrm.ab_rows > 0 && nrm.ab_slices >= 1 &&
                             nrm.ab_out && nrm.ab_ld >= nrm.ab_rows && kq_rw() == 4),
               RL_ERR_RANGE, "kquant: BF16 rows need a plain or folded-norm input launch and an output");
    RL_REQUIRE(!nrm.swiglu || (!nrm.ss_out && !accumulate && m % kTR == 0 && ldy >= m / 2), RL_ERR_RANGE,
               "kquant: the SwiGLU output needs whole gate / up half tiles, no accumulate and no add-norm output");
    RL_REQUIRE(m > 0 && n > 0 && n % 256 == 0, RL_ERR_RANGE, "kquant: n must be a positive multiple of 256");
    RL_REQUIRE(T >= 1 && T <= 16, RL_ERR_RANGE, "kquant: T must be in 1..16 (groups of 4 above 4)");
    RL_REQUIRE(W && x && Y && ws, RL_ERR_RANGE, "kquant: null pointer");
    RL_REQUIRE(ws_bytes >= kq_workspace_bytes(m, n, T), RL_ERR_RANGE, "kquant: workspace too small");
    int S;
    kq_split(m, n / 256, S);
    const int groups = (m + kTR * kq_rw() - 1) / (kTR * kq_rw());
    unsigned* tickets = static_cast<unsigned*>(ws);
    float* partial = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kq_ticket_bytes(groups * kq_token_groups(T)));
    if (qt == 4)
        launch_kq<4>(W, x, Y, partial, tickets, m, n, T, S, accumulate, ldy, s, nrm);
    else
        launch_kq<6>(W, x, Y, partial, tickets, m, n, T, S, accumulate, ldy, s, nrm);
    check_launch("kq_gemm_kernel");
}

// ---- the allocation-free entry point's scratch ------------------------------
// Split-K tickets and partials of rl_hip_gemm_kquant_noalloc live in this array
// (each device holds its own copy until the process ends).  Host code never passes
// the array's name to a kernel: it resolves the device address once per device
// with hipGetSymbolAddress and uses that pointer.
constexpr size_t kKqScratchBytes = size_t(4) << 20;
static __device__ __align__(256) uint8_t scratch[kKqScratchBytes];

namespace {

__global__ void kq_zero_kernel(uint32_t* p, size_t n_words) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_words;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        p[i] = 0u;
}

constexpr int kKqMaxDevices = 64;
std::mutex g_scratch_mu;
struct KqScratch {
    void* ptr = nullptr;          // device address of `scratch`
    hipEvent_t cleared = nullptr; // recorded after the clear on `clear_stream`
    hipStream_t clear_stream = nullptr;
    bool clear_done = false;      // the event has been seen complete
};
KqScratch g_scratch[kKqMaxDevices];

// Device address of `scratch` on the current device.  The first call for a device
// resolves it and clears the array with a fill kernel on that call's stream `s`,
// then records an event.  Until the host has seen that event complete, a call on
// any other stream makes its stream wait for the event first, so a first use on
// two streams (or threads) at once cannot run a GEMM on uncleared tickets.
void* kq_scratch(hipStream_t s) {
    int dev = 0;
    RL_HIP(hipGetDevice(&dev));
    RL_REQUIRE(dev >= 0 && dev < kKqMaxDevices, RL_ERR_DEVICE, "gemm_kquant_noalloc: device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    KqScratch& g = g_scratch[dev];
    if (!g.ptr) {
        void* p = nullptr;
        RL_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        RL_REQUIRE(p != nullptr, RL_ERR_DEVICE, "gemm_kquant_noalloc: scratch symbol has no device address");
        if (!g.cleared) RL_HIP(hipEventCreateWithFlags(&g.cleared, hipEventDisableTiming));
        hipLaunchKernelGGL(kq_zero_kernel, dim3(256), dim3(256), 0, s, static_cast<uint32_t*>(p), kKqScratchBytes / 4);
        check_launch("kq_zero_kernel");
        RL_HIP(hipEventRecord(g.cleared, s));
        g.clear_stream = s;
        g.ptr = p;
    } else if (!g.clear_done) {
        const hipError_t q = hipEventQuery(g.cleared);
        if (q == hipSuccess) {
            g.clear_done = true;
        } else {
            RL_REQUIRE(q == hipErrorNotReady, RL_ERR_DEVICE, "gemm_kquant_noalloc: scratch clear failed");
            if (s != g.clear_stream) RL_HIP(hipStreamWaitEvent(s, g.cleared, 0));
        }
    }
    return g.ptr;
}

}  // namespace

size_t kq_noalloc_max_bytes() { return kKqScratchBytes; }

}  // namespace rl

extern "C" {

int rl_hip_gemm_kquant_noalloc(int type, const uint8_t* tiled, const float* X, float* Y, int m, int n, int T,
                               int accumulate, void* stream) {
    return guard([&] {
        RL_REQUIRE(type == RL_Q_Q4_K || type == RL_Q_Q6_K, RL_ERR_UNSUPPORTED, "gemm_kquant_noalloc: Q4_K or Q6_K only");
        RL_REQUIRE(m > 0 && n > 0 && n % 256 == 0 && T >= 1 && T <= 4, RL_ERR_RANGE,
                   "gemm_kquant_noalloc: m > 0, n a positive multiple of 256, T in 1..4");
        const size_t need = rl::kq_workspace_bytes(m, n, T);
        if (need > rl::kKqScratchBytes)
            throw Error(RL_ERR_RANGE, "gemm_kquant_noalloc: shape needs " + std::to_string(need) +
                                          " scratch bytes, more than the fixed " +
                                          std::to_string(rl::kKqScratchBytes) + " (use rl_hip_gemm_kquant)");
        void* ws = rl::kq_scratch(S(stream));
        rl::kq_gemm(type == RL_Q_Q4_K ? 4 : 6, tiled, X, Y, ws, rl::kKqScratchBytes, m, n, T, accumulate, m,
                    S(stream));
    });
}

size_t rl_hip_gemm_kquant_noalloc_max_scratch(void) { return rl::kq_noalloc_max_bytes(); }


size_t rl_hip_kquant_tiled_bytes(int type, int m, int n) {
    if ((type != RL_Q_Q4_K && type != RL_Q_Q6_K) || n % 256 != 0 || m <= 0) return 0;
    return kq_tiled_bytes(type == RL_Q_Q4_K ? 4 : 6, m, n);
}

size_t rl_hip_kquant_workspace_bytes(int m, int n, int T) { return rl::kq_workspace_bytes(m, n, T); }

namespace {
void kq_pack(int type, const uint8_t* blocks, const uint8_t* up, uint8_t* tiled, int m, int n, hipStream_t s) {
    const int nsb = n / 256;
    const size_t total = static_cast<size_t>(up ? (m + 7) / 8 : (m + kTR - 1) / kTR) * nsb * 64;
    if (type == RL_Q_Q4_K)
        hipLaunchKernelGGL(kq_pack_kernel<4>, dim3((total + 255) / 256), dim3(256), 0, s, blocks, up, tiled, m, nsb);
    else
        hipLaunchKernelGGL(kq_pack_kernel<6>, dim3((total + 255) / 256), dim3(256), 0, s, blocks, up, tiled, m, nsb);
    check_launch("kq_pack_kernel");
}
}  // namespace

int rl_hip_pack_kquant(int type, const uint8_t* blocks, uint8_t* tiled, int m, int n, void* stream) {
    return guard([&] {
        RL_REQUIRE(type == RL_Q_Q4_K || type == RL_Q_Q6_K, RL_ERR_UNSUPPORTED, "pack_kquant: Q4_K or Q6_K only");
        RL_REQUIRE(m > 0 && n > 0 && n % 256 == 0 && blocks && tiled, RL_ERR_RANGE, "pack_kquant: bad shape");
        kq_pack(type, blocks, nullptr, tiled, m, n, S(stream));
    });
}

int rl_hip_pack_kquant_gate_up(int type, const uint8_t* gate_blocks, const uint8_t* up_blocks, uint8_t* tiled,
                               int I, int n, void* stream) {
    return guard([&] {
        RL_REQUIRE(type == RL_Q_Q4_K || type == RL_Q_Q6_K, RL_ERR_UNSUPPORTED, "pack_kquant_gate_up: Q4_K or Q6_K only");
        RL_REQUIRE(I > 0 && I % 8 == 0 && n > 0 && n % 256 == 0 && gate_blocks && up_blocks && tiled, RL_ERR_RANGE,
                   "pack_kquant_gate_up: I a positive multiple of 8, n of 256");
        kq_pack(type, gate_blocks, up_blocks, tiled, I, n, S(stream));
    });
}

int rl_hip_gemm_kquant_swiglu(int type, const uint8_t* tiled, const float* X, float* H, void* workspace,
                              size_t workspace_bytes, int I, int n, int T, void* stream) {
    return guard([&] {
        RL_REQUIRE(type == RL_Q_Q4_K || type == RL_Q_Q6_K, RL_ERR_UNSUPPORTED, "gemm_kquant_swiglu: Q4_K or Q6_K only");
        RL_REQUIRE(I > 0 && I % 8 == 0, RL_ERR_RANGE, "gemm_kquant_swiglu: I a positive multiple of 8");
        rl::KqNorm kn;
        kn.swiglu = 1;
        rl::kq_gemm(type == RL_Q_Q4_K ? 4 : 6, tiled, X, H, workspace, workspace_bytes, 2 * I, n, T, 0, I, S(stream),
                    &kn);
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

int rl_hip_kquant_to_bf16x2(int type, const uint8_t* tiled, uint16_t* w_hi, uint16_t* w_lo, int m, int n,
                            void* stream) {
    return guard([&] {
        RL_REQUIRE(type == RL_Q_Q4_K || type == RL_Q_Q6_K, RL_ERR_UNSUPPORTED, "kquant_to_bf16x2: Q4_K or Q6_K");
        rl::kq_to_bf16x2(type == RL_Q_Q4_K ? 4 : 6, tiled, w_hi, w_lo, m, n, S(stream));
    });
}

int rl_hip_kquant_to_f16(int type, const uint8_t* tiled, void* w16, float* tile_scale, int m, int n, void* stream) {
    return guard([&] {
        RL_REQUIRE(type == RL_Q_Q4_K || type == RL_Q_Q6_K, RL_ERR_UNSUPPORTED, "kquant_to_f16: Q4_K or Q6_K");
        rl::kq_to_f16(type == RL_Q_Q4_K ? 4 : 6, tiled, w16, tile_scale, m, n, S(stream));
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
