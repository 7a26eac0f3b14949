// prefill.hip -- block-FP8 linears over many tokens (prompt prefill), on MFMA.
//
// Same arithmetic as ops::gemv_fp8 (reference src/kernels/ops.cpp:182-194) applied
// to every prompt token, i.e. the reference's prefill linears
// (src/kernels/cuda/cuda_engine.cu:18338-18590 launch_prefill_chunk -> launch_linear
// for T > 8, cuda_engine.cu:12008-12016).  At prefill sizes the work is
// matrix-core bound, not HBM bound: one 128-row x 128-token output block per
// workgroup reads each weight tile once for 128 tokens.
//
// Operands as in gemm.hip: A = 16 weight rows x 32 k, e4m3 decoded to bf16 by the
// hardware converter (exact); B = 32 k x 16 tokens of the activation fragments
// (bf16 hi and mid parts, two MFMAs into the same accumulator, so products carry
// 16 significant bits of x); the 128x128 block scale multiplies each 128-column
// block's fp32 partial.  Weights use the decode GEMM's tiled layout (16 rows x 128
// columns per 2 KiB tile), activations its fragment layout for T tokens.
//
// Workgroup: 4 waves, 8 row tiles (128 rows) x 128 tokens; wave w owns tokens
// 32w .. 32w+31 of the block (two 16-token column tiles, so each weight fragment
// read from LDS feeds four MFMAs) for all 8 row tiles.  The 8 weight tiles of a column
// block (16 KiB) are staged once in LDS (double buffered, the next block's loads in
// flight during the MFMAs) and read by all four waves.
#include "internal.h"

using namespace rl;

namespace {

constexpr int kPfNT = 2;     // 16-token column tiles per wave
constexpr int kPfTok = 64 * kPfNT;  // tokens per workgroup
constexpr int kTileRows = 16;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

union Frag8 {
    bf16x8 v;
    f16x8 h;
    uint32_t u[4];
    i32x4 i;
};

__device__ inline void e4m3x4_to_bf16(uint32_t w, uint32_t& lo, uint32_t& hi) {
    const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(w), 1.0f, false);
    const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(w), 1.0f, true);
    lo = __builtin_bit_cast(uint32_t, a);
    hi = __builtin_bit_cast(uint32_t, b);
}

__device__ inline float silu_f(float x) { return x / (1.f + __expf(-x)); }

// EPI: 0 store, 1 add (Y += W.x), 2 SwiGLU over interleaved gate/up row tiles
// (even tile = gate rows, odd = up rows of the same 16 outputs; Y row = output row),
// 5 SwiGLU over half tiles (tile k: gate rows 8k..8k+7, up rows 8k..8k+7; scales
// [tile][kb][2]).
// WK: the weight tiles.  0: block-FP8 (2 KiB tiles, tile scales).  1: BF16 (4 KiB
// tiles of the decode GEMM's BF16 layout, no scales).  2: two BF16 matrices W_hi +
// W_lo (a weight split into 16 significant bits): three MFMAs per step,
// hi.x_hi + hi.x_mid + lo.x_hi.  3: fp16 tiles in the BF16 layout with one
// power-of-two scale per (tile, column block) (the K-quant linears as dequantised
// for prefill), activations as fp16 hi + lo fragments with one power-of-two scale
// per (column block, token): two fp16 MFMAs per step.
// RT row tiles per workgroup: 8 for FP8, 4 for BF16 and fp16 (the same 16 KiB of
// weights staged per column block; 32 KiB for hi + lo).
template <int EPI, int WK = 0>
__global__ __launch_bounds__(256) void gemm_prefill_kernel(const uint8_t* __restrict__ W,
                                                           const float* __restrict__ tscale,
                                                           const i32x4* __restrict__ frag, float* __restrict__ Y,
                                                           int m, int n_kb, int T, int ldy, int m_valid,
                                                           const uint8_t* __restrict__ W_lo = nullptr,
                                                           const float* __restrict__ xscale = nullptr) {
    constexpr int kPfRT = WK == 0 ? 8 : 4;  // row tiles per workgroup (fp16 at 8: one wave per SIMD, slower)
    constexpr int kCh = WK == 0 ? 2 : 4;            // 16-B chunks per lane per tile
    constexpr int kTileB = WK == 0 ? 2048 : 4096;   // bytes per tile
    constexpr int kMat = WK == 2 ? 2 : 1;           // weight matrices staged
    constexpr int kUnits = kPfRT * kCh * 64 * kMat / 256;  // 16-B staging units per thread
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, col = lane & 15;
    const int m_tiles = (m + kTileRows - 1) / kTileRows;
    const int rt0 = blockIdx.x * kPfRT;
    int tokv[kPfNT], tokcv[kPfNT];
#pragma unroll
    for (int nt = 0; nt < kPfNT; ++nt) {
        tokv[nt] = blockIdx.y * kPfTok + (wave * kPfNT + nt) * 16 + col;  // B column of this lane
        tokcv[nt] = min(tokv[nt], T - 1);
    }
    const int NC = 2 * T;
    // the input fragments as a buffer resource (gfx9 raw dword buffer; the host keeps
    // them under 4 GiB) and the byte offset of the unit of (k-step i, lane group g,
    // token) within a column block
    const __amdgpu_buffer_rsrc_t frsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<i32x4*>(frag), 0, static_cast<int>(static_cast<uint32_t>(n_kb) * 16u * 2u * T * 16u), 0x00020000);
    uint32_t boff[kPfNT][4];
#pragma unroll
    for (int nt = 0; nt < kPfNT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) boff[nt][i] = static_cast<uint32_t>((i * 4 + g) * NC + tokcv[nt]) * 16u;

    __shared__ i32x4 wl[2][kMat][kPfRT][kCh][64];  // [buffer][matrix][row tile][16-B chunk][lane]

    // staging: unit u = (matrix, row tile, chunk, lane), kUnits per thread.  Every
    // address is a uniform base for the column block plus a loop-invariant 32-bit
    // lane offset (the host keeps weights and fragments under 4 GiB), so the loads
    // take the scalar-base form with no 64-bit address arithmetic per iteration.
    uint32_t woff[kUnits];
#pragma unroll
    for (int q = 0; q < kUnits; ++q) {
        const int u = tid + 256 * q;
        const int l = u & 63, c = (u >> 6) % kCh, r = (u / (64 * kCh)) % kPfRT;
        const int rt = min(rt0 + r, m_tiles - 1);
        woff[q] = static_cast<uint32_t>(rt) * static_cast<uint32_t>(n_kb * kTileB) + c * 1024 + 16 * l;
    }
    // weights as buffer resources too (non-temporal loads: aux bit 1)
    const int wbytes = static_cast<int>(static_cast<uint32_t>(m_tiles) * static_cast<uint32_t>(n_kb * kTileB));
    const __amdgpu_buffer_rsrc_t wrsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(W), 0, wbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t wlrsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(kMat > 1 ? W_lo : W), 0, wbytes, 0x00020000);
    i32x4 stg[kUnits];
    auto stage_load = [&](int kb) {
#pragma unroll
        for (int q = 0; q < kUnits; ++q) {
            const int mat = (tid + 256 * q) / (64 * kCh * kPfRT);
            stg[q] = __builtin_amdgcn_raw_buffer_load_b128(mat ? wlrsrc : wrsrc, static_cast<int>(woff[q]),
                                                           kb * kTileB, 2);
        }
    };
    auto stage_store = [&](int buf) {
#pragma unroll
        for (int q = 0; q < kUnits; ++q) {
            const int u = tid + 256 * q;
            wl[buf][u / (64 * kCh * kPfRT)][(u / (64 * kCh)) % kPfRT][(u >> 6) % kCh][u & 63] = stg[q];
        }
    };

    f32x4 tot[kPfNT][kPfRT];
#pragma unroll
    for (int nt = 0; nt < kPfNT; ++nt)
#pragma unroll
        for (int r = 0; r < kPfRT; ++r) tot[nt][r] = f32x4{0.f, 0.f, 0.f, 0.f};

    stage_load(0);
    stage_store(0);
    __syncthreads();
    for (int kb = 0; kb < n_kb; ++kb) {
        const int buf = kb & 1;
        if (kb + 1 < n_kb) stage_load(kb + 1);
        // activation fragments of this lane's token: 4 k-steps x (hi, mid); WK 3: the
        // fp16 hi / lo fragments and the token's block scale
        i32x4 bh[kPfNT][4], bm[kPfNT][4];
        float xs[kPfNT];
        if constexpr (WK == 3) {
#pragma unroll
            for (int nt = 0; nt < kPfNT; ++nt) xs[nt] = xscale[static_cast<size_t>(kb) * T + tokcv[nt]];
        }
        // buffer loads: the column block's offset as the scalar offset, the lane's
        // as the vector offset (no per-load address arithmetic)
        const int kbo = kb * 16 * NC * 16;
#pragma unroll
        for (int nt = 0; nt < kPfNT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                bh[nt][i] = __builtin_amdgcn_raw_buffer_load_b128(frsrc, static_cast<int>(boff[nt][i]), kbo, 0);
                bm[nt][i] = __builtin_amdgcn_raw_buffer_load_b128(frsrc, static_cast<int>(boff[nt][i]), kbo + 16 * T, 0);
            }
#pragma unroll
        for (int r = 0; r < kPfRT; ++r) {
            const int rt = min(rt0 + r, m_tiles - 1);
            f32x4 acc[kPfNT];
#pragma unroll
            for (int nt = 0; nt < kPfNT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                Frag8 a, b;
                if constexpr (WK == 0) {
                    const i32x4 wv = wl[buf][0][r][i >> 1][lane];
                    e4m3x4_to_bf16(static_cast<uint32_t>((i & 1) ? wv[2] : wv[0]), a.u[0], a.u[1]);
                    e4m3x4_to_bf16(static_cast<uint32_t>((i & 1) ? wv[3] : wv[1]), a.u[2], a.u[3]);
                } else {
                    a.i = wl[buf][0][r][i][lane];
                }
#pragma unroll
                for (int nt = 0; nt < kPfNT; ++nt) {
                    if constexpr (WK == 3) {
                        b.i = bh[nt][i];
                        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, b.h, acc[nt], 0, 0, 0);
                        b.i = bm[nt][i];
                        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, b.h, acc[nt], 0, 0, 0);
                    } else {
                        b.i = bh[nt][i];
                        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, acc[nt], 0, 0, 0);
                        b.i = bm[nt][i];
                        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, acc[nt], 0, 0, 0);
                    }
                }
                if constexpr (WK == 2) {
                    a.i = wl[buf][1][r][i][lane];
#pragma unroll
                    for (int nt = 0; nt < kPfNT; ++nt) {
                        b.i = bh[nt][i];
                        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, acc[nt], 0, 0, 0);
                    }
                }
            }
            if constexpr (WK == 0) {
                // C rows 4g..4g+3 of a half-tile matrix: gate (g < 2) or up scale
                // (rt, kb) is uniform: the scales are scalar loads; the lane picks its half's
                float sc;
                if constexpr (EPI == 5 || EPI == 6) {
                    const float2 s2 = *reinterpret_cast<const float2*>(tscale + (static_cast<size_t>(rt) * n_kb + kb) * 2);
                    sc = g >= 2 ? s2.y : s2.x;
                } else {
                    sc = tscale[static_cast<size_t>(rt) * n_kb + kb];
                }
#pragma unroll
                for (int nt = 0; nt < kPfNT; ++nt) tot[nt][r] += sc * acc[nt];
            } else if constexpr (WK == 3) {
                const float sc = tscale[static_cast<size_t>(rt) * n_kb + kb];
#pragma unroll
                for (int nt = 0; nt < kPfNT; ++nt) tot[nt][r] += (sc * xs[nt]) * acc[nt];
            } else {
#pragma unroll
                for (int nt = 0; nt < kPfNT; ++nt) tot[nt][r] += acc[nt];
            }
        }
        if (kb + 1 < n_kb) stage_store(buf ^ 1);
        __syncthreads();
    }

    // lane (g, col) holds rows 4g .. 4g+3 of each row tile for token tokv[nt]
#pragma unroll
    for (int nt = 0; nt < kPfNT; ++nt) {
        const int tok = tokv[nt];
        if (tok >= T) break;
        float* yrow = Y + static_cast<size_t>(tok) * ldy;
        if constexpr (EPI == 5) {
            // lane (g < 2, col) holds gate rows 4g..4g+3; lane + 32 the matching up rows
#pragma unroll
            for (int r = 0; r < kPfRT; ++r) {
                if (rt0 + r >= m_tiles) break;
                const int orow = (rt0 + r) * 8 + 4 * g;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float up = __shfl_xor(tot[nt][r][v], 32, 64);
                    if (g < 2 && orow + v < m_valid) yrow[orow + v] = silu_f(tot[nt][r][v]) * up;
                }
            }
        } else if constexpr (EPI == 6) {
            // as 5; lanes g = 0 and 1 hold output rows 0..3 and 4..7 of the half tile,
            // one 8-column fragment unit of the next GEMM's input, which lane g = 0
            // writes (the same bf16 hi + mid split as pack_act)
            i32x4* fo = reinterpret_cast<i32x4*>(Y);
#pragma unroll
            for (int r = 0; r < kPfRT; ++r) {
                if (rt0 + r >= m_tiles) break;
                float h8[8];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float up = __shfl_xor(tot[nt][r][v], 32, 64);
                    h8[v] = silu_f(tot[nt][r][v]) * up;
                }
#pragma unroll
                for (int v = 0; v < 4; ++v) h8[4 + v] = __shfl_xor(h8[v], 16, 64);
                if (g == 0) write_frag8(fo, rt0 + r, tok, T, h8);
            }
        } else if constexpr (EPI == 2) {
#pragma unroll
            for (int r = 0; r < kPfRT; r += 2) {
                if (rt0 + r + 1 >= m_tiles) break;
                const int orow = ((rt0 + r) / 2) * kTileRows + 4 * g;
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (orow + v < m_valid) yrow[orow + v] = silu_f(tot[nt][r][v]) * tot[nt][r + 1][v];
            }
        } else {
#pragma unroll
            for (int r = 0; r < kPfRT; ++r) {
                if (rt0 + r >= m_tiles) break;
                const int row = (rt0 + r) * kTileRows + 4 * g;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if (row + v >= m_valid) break;
                    if constexpr (EPI == 1)
                        yrow[row + v] += tot[nt][r][v];
                    else
                        yrow[row + v] = tot[nt][r][v];
                }
            }
        }
    }
}


// bf16 hi + mid activation fragments -> fp16 hi + lo fragments, one thread per
// (128-column block kb, token t): x = hi + mid (exact, 16 significant bits), scaled
// by a power of two xscale[kb][t] that puts the block's largest |x| in
// [2^14, 2^15), then split into fp16 hi = rn(x / s) and lo = rn(x / s - hi), which
// together hold every bit of x.  Same layout as the input (units (kb, i, g): hi in
// column t, lo in column T + t).
__global__ void act_frag_to_f16_kernel(const i32x4* __restrict__ frag, i32x4* __restrict__ out,
                                       float* __restrict__ xscale, int n_kb, int T) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_kb * T) return;
    const int t = idx % T, kb = idx / T;
    const size_t NC = 2 * static_cast<size_t>(T);
    auto unit = [&](int gi) { return (static_cast<size_t>(kb) * 16 + gi) * NC + t; };
    auto value = [&](const Frag8& h, const Frag8& md, int e) {
        const uint32_t hb = (h.u[e >> 1] >> (16 * (e & 1))) & 0xffffu;
        const uint32_t mb = (md.u[e >> 1] >> (16 * (e & 1))) & 0xffffu;
        return __uint_as_float(hb << 16) + __uint_as_float(mb << 16);
    };
    float mx = 0.f;
    for (int gi = 0; gi < 16; ++gi) {
        Frag8 h, md;
        h.i = frag[unit(gi)];
        md.i = frag[unit(gi) + T];
#pragma unroll
        for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(value(h, md, e)));
    }
    float sc = 1.f;
    if (mx > 0.f) {
        int ex;
        frexpf(mx, &ex);
        sc = ldexpf(1.f, ex - 15);
    }
    const float inv = 1.f / sc;
    for (int gi = 0; gi < 16; ++gi) {
        Frag8 h, md, oh, ol;
        h.i = frag[unit(gi)];
        md.i = frag[unit(gi) + T];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float v = value(h, md, e) * inv;
            const _Float16 vh = static_cast<_Float16>(v);
            oh.h[e] = vh;
            ol.h[e] = static_cast<_Float16>(v - static_cast<float>(vh));
        }
        out[unit(gi)] = oh.i;
        out[unit(gi) + T] = ol.i;
    }
    xscale[static_cast<size_t>(kb) * T + t] = sc;
}

}  // namespace

namespace rl {

void gemm_prefill_any(int wk, const uint8_t* W, const uint8_t* W_lo, const float* ts, const void* frag, float* Y,
                      int m, int n, int T, int epi, int ldy, int m_valid, hipStream_t s, const float* xscale) {
    RL_REQUIRE(m > 0 && n > 0 && T >= 1, RL_ERR_RANGE, "gemm_prefill: empty shape");
    RL_REQUIRE(W && frag && Y && ((wk != 0 && wk != 3) || ts) && (wk != 2 || W_lo) && (wk != 3 || xscale),
               RL_ERR_RANGE, "gemm_prefill: null pointer");
    RL_REQUIRE(wk >= 0 && wk <= 3, RL_ERR_RANGE, "gemm_prefill: weight kind");
    RL_REQUIRE(epi == kEpiStore || epi == kEpiAdd || epi == kEpiSwiGLU || epi == kEpiSwiGLUH ||
                   epi == kEpiSwiGLUHFrag,
               RL_ERR_RANGE, "gemm_prefill: epilogue must be store, add or swiglu");
    if (epi == kEpiSwiGLUH) RL_REQUIRE(m % 16 == 0, RL_ERR_RANGE, "gemm_prefill swiglu: rows a multiple of 16");
    if (epi == kEpiSwiGLUHFrag)
        RL_REQUIRE(m % 256 == 0 && m_valid == m / 2, RL_ERR_RANGE,
                   "gemm_prefill swiglu to fragments: outputs a multiple of 128");
    const int m_tiles = (m + kTileRows - 1) / kTileRows;
    if (epi == kEpiSwiGLU) RL_REQUIRE(m % 32 == 0, RL_ERR_RANGE, "gemm_prefill swiglu: rows must be a multiple of 32");
    const int n_kb = (n + 127) / 128;
    // the kernel addresses weights and fragments with 32-bit offsets
    RL_REQUIRE(static_cast<size_t>(m_tiles) * n_kb * (wk == 0 ? 2048 : 4096) < (size_t{1} << 32) &&
                   static_cast<size_t>(n_kb) * 16 * 2 * T * 16 < (size_t{1} << 32),
               RL_ERR_RANGE, "gemm_prefill: weights and input fragments must each stay under 4 GiB");
    const int rt = wk == 0 ? 8 : 4;
    const dim3 grid((m_tiles + rt - 1) / rt, (T + kPfTok - 1) / kPfTok);
    RL_REQUIRE(grid.y <= 65535, RL_ERR_RANGE, "gemm_prefill: too many tokens");
    const i32x4* fr = static_cast<const i32x4*>(frag);
#define RL_PF(E, K)                                                                                                 \
    if (epi == E && wk == K) {                                                                                      \
        hipLaunchKernelGGL((gemm_prefill_kernel<E == kEpiSwiGLUH ? 5 : E, K>), grid, dim3(256), 0, s, W, ts, fr, Y, m, \
                           n_kb, T, ldy, m_valid, W_lo, xscale);                                                    \
        check_launch("gemm_prefill_kernel");                                                                        \
        return;                                                                                                     \
    }
    RL_PF(kEpiStore, 0) RL_PF(kEpiAdd, 0) RL_PF(kEpiSwiGLU, 0) RL_PF(kEpiSwiGLUH, 0)
    RL_PF(kEpiStore, 1) RL_PF(kEpiAdd, 1) RL_PF(kEpiSwiGLU, 1) RL_PF(kEpiSwiGLUH, 1)
    RL_PF(kEpiStore, 2) RL_PF(kEpiAdd, 2) RL_PF(kEpiSwiGLU, 2) RL_PF(kEpiSwiGLUH, 2)
    RL_PF(kEpiStore, 3) RL_PF(kEpiAdd, 3) RL_PF(kEpiSwiGLU, 3) RL_PF(kEpiSwiGLUH, 3)
    RL_PF(kEpiSwiGLUHFrag, 0) RL_PF(kEpiSwiGLUHFrag, 1) RL_PF(kEpiSwiGLUHFrag, 2) RL_PF(kEpiSwiGLUHFrag, 3)
#undef RL_PF
}

void act_frag_to_f16(const void* frag, void* frag16, float* xscale, int n, int T, hipStream_t s) {
    RL_REQUIRE(frag && frag16 && xscale && n > 0 && T >= 1 && frag != frag16, RL_ERR_RANGE,
               "act_frag_to_f16: bad arguments");
    const int n_kb = (n + 127) / 128;
    const int total = n_kb * T;
    hipLaunchKernelGGL(act_frag_to_f16_kernel, dim3((total + 255) / 256), dim3(256), 0, s,
                       static_cast<const i32x4*>(frag), static_cast<i32x4*>(frag16), xscale, n_kb, T);
    check_launch("act_frag_to_f16_kernel");
}

void gemm_fp8_prefill(const uint8_t* W, const float* ts, const void* frag, float* Y, int m, int n, int T, int epi,
                      int ldy, int m_valid, hipStream_t s) {
    gemm_prefill_any(0, W, nullptr, ts, frag, Y, m, n, T, epi, ldy, m_valid, s);
}

}  // namespace rl

extern "C" {

int rl_hip_gemm_fp8_prefill(const uint8_t* w_tiled, const float* tile_scale, const void* frag, float* Y, int m, int n,
                            int T, int epilogue, int ldy, void* stream) {
    return guard([&] {
        const int mv = epilogue == kEpiSwiGLU || epilogue == kEpiSwiGLUH || epilogue == kEpiSwiGLUHFrag ? m / 2 : m;
        rl::gemm_fp8_prefill(w_tiled, tile_scale, frag, Y, m, n, T, epilogue, ldy > 0 ? ldy : mv, mv, S(stream));
    });
}

int rl_hip_gemm_bf16_prefill(const uint16_t* w_tiled, const uint16_t* w_lo_tiled, const void* frag, float* Y, int m,
                             int n, int T, int epilogue, int ldy, void* stream) {
    return guard([&] {
        const int mv = epilogue == kEpiSwiGLU || epilogue == kEpiSwiGLUH || epilogue == kEpiSwiGLUHFrag ? m / 2 : m;
        rl::gemm_prefill_any(w_lo_tiled ? 2 : 1, reinterpret_cast<const uint8_t*>(w_tiled),
                             reinterpret_cast<const uint8_t*>(w_lo_tiled), nullptr, frag, Y, m, n, T, epilogue,
                             ldy > 0 ? ldy : mv, mv, S(stream));
    });
}

int rl_hip_act_frag_to_f16(const void* frag, void* frag16, float* xscale, int n, int T, void* stream) {
    return guard([&] { rl::act_frag_to_f16(frag, frag16, xscale, n, T, S(stream)); });
}

int rl_hip_gemm_f16_prefill(const void* w16, const float* tile_scale, const void* frag16, const float* xscale,
                            float* Y, int m, int n, int T, int epilogue, int ldy, void* stream) {
    return guard([&] {
        const int mv = epilogue == kEpiSwiGLU || epilogue == kEpiSwiGLUH || epilogue == kEpiSwiGLUHFrag ? m / 2 : m;
        rl::gemm_prefill_any(3, static_cast<const uint8_t*>(w16), nullptr, tile_scale, frag16, Y, m, n, T, epilogue,
                             ldy > 0 ? ldy : mv, mv, S(stream), xscale);
    });
}

}  // extern "C"
