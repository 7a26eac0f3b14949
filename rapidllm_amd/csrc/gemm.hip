// gemm.hip -- skinny block-FP8 / BF16 linears for T = 1..8 tokens on gfx950 MFMA.
//
// Computes Y[t][i] = sum_j W[i][j] * scale(i/128, j/128) * X[t][j], the arithmetic
// of ops::gemv_fp8 (reference src/kernels/ops.cpp:182-194), for all T tokens in one
// pass over the weights (the reference's CUDA T=4 verify runs four T=1 GEMVs,
// src/kernels/cuda/cuda_engine.cu:11997-12005; reading W once is the point here).
//
// Mapping onto v_mfma_f32_16x16x32_bf16:
//   A (16 rows x 32 k)  = 16 weight rows, e4m3 decoded to bf16 by the hardware
//                         converter (exact: every finite e4m3 value is a bf16);
//   B (32 k x 16 cols)  = activations: column t = bf16 "hi" part of token t,
//                         column T+t = bf16 "mid" part (x - hi), so hi+mid carries
//                         16 significant bits and fp32's exponent range;
//   C (16 x 16, fp32)   = per 128-column block; scaled by the block's fp32 scale and
//                         added to the running fp32 total (the scale is uniform over
//                         a 16-row x 128-column tile).
// Products of a <=4-bit e4m3 mantissa and an 8-bit bf16 mantissa are exact in fp32.
//
// Weight layout in HBM ("tiled"): for row-tile rt (16 rows) and column block kb
// (128 columns), one contiguous tile of 2048 B (FP8) / 4096 B (BF16).  Lane l of a
// wave owns row r = l%16, columns [32g, 32g+32) with g = l/16; its FP8 bytes sit
// at tile offsets 16l and 1024+16l, so every 16-byte wave load is one contiguous
// 1 KiB stream.  Tiles of one row-tile are contiguous along kb.
//
// Work split: a workgroup = KSPLIT waves over RT row-tiles; wave w walks a
// contiguous 1/KSPLIT of the column blocks, partial C tiles are summed through LDS
// in a fixed order (deterministic), then the epilogue stores or accumulates Y.
#include "common.h"

using namespace rl;
namespace {

constexpr int kTileRows = 16;
constexpr int kBlockCols = 128;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

union Frag8 {
    bf16x8 v;
    uint32_t u[4];
    i32x4 i;
};

// Four e4m3 bytes packed in a dword -> four bf16 (two dwords), exact.
__device__ inline void e4m3x4_to_bf16(uint32_t w, uint32_t& lo, uint32_t& hi) {
    bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(w), 1.0f, false);
    bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(w), 1.0f, true);
    lo = __builtin_bit_cast(uint32_t, a);
    hi = __builtin_bit_cast(uint32_t, b);
}

enum Epilogue { kStore = 0, kAdd = 1, kSwiGLU = 2 };

template <int RT, int KSPLIT, bool kFp8>
__global__ __launch_bounds__(64 * KSPLIT) void gemm_frag_kernel(const uint8_t* __restrict__ W,
                                                                const float* __restrict__ tscale,
                                                                const i32x4* __restrict__ frag,
                                                                float* __restrict__ Y, int m, int n_kb, int T,
                                                                int epilogue) {
    constexpr int kTileBytes = kFp8 ? 2048 : 4096;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4;
    const int col = lane & 15;
    const int NC = 2 * T;
    const int rt0 = blockIdx.x * RT;
    const int m_tiles = (m + kTileRows - 1) / kTileRows;

    const int per = (n_kb + KSPLIT - 1) / KSPLIT;
    const int kb_begin = min(n_kb, wave * per);
    const int kb_end = min(n_kb, kb_begin + per);

    f32x4 tot[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) tot[r] = f32x4{0.f, 0.f, 0.f, 0.f};

    const bool has_col = col < NC;
    const i32x4 zero4 = {0, 0, 0, 0};

    auto load_w = [&](int kb, i32x4 (&wv)[RT][kFp8 ? 2 : 4]) {
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const int rt = min(rt0 + r, m_tiles - 1);
            const uint8_t* tile = W + (static_cast<size_t>(rt) * n_kb + kb) * kTileBytes;
#pragma unroll
            for (int c = 0; c < (kFp8 ? 2 : 4); ++c)
                wv[r][c] = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(tile + c * 1024 + 16 * lane));
        }
    };
    auto load_b = [&](int kb, i32x4 (&bv)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            bv[i] = has_col ? frag[((static_cast<size_t>(kb) * 4 + i) * 4 + g) * NC + col] : zero4;
    };

    i32x4 wcur[RT][kFp8 ? 2 : 4], wnext[RT][kFp8 ? 2 : 4];
    i32x4 bcur[4], bnext[4];
    if (kb_begin < kb_end) {
        load_w(kb_begin, wcur);
        load_b(kb_begin, bcur);
    }
    for (int kb = kb_begin; kb < kb_end; ++kb) {
        if (kb + 1 < kb_end) {
            load_w(kb + 1, wnext);
            load_b(kb + 1, bnext);
        }
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                Frag8 a, b;
                b.i = bcur[i];
                if constexpr (kFp8) {
                    const i32x4 wv = wcur[r][i >> 1];
                    const uint32_t d0 = static_cast<uint32_t>((i & 1) ? wv[2] : wv[0]);
                    const uint32_t d1 = static_cast<uint32_t>((i & 1) ? wv[3] : wv[1]);
                    e4m3x4_to_bf16(d0, a.u[0], a.u[1]);
                    e4m3x4_to_bf16(d1, a.u[2], a.u[3]);
                } else {
                    a.i = wcur[r][i];
                }
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, acc, 0, 0, 0);
            }
            if constexpr (kFp8) {
                const int rt = min(rt0 + r, m_tiles - 1);
                const float s = tscale[static_cast<size_t>(rt) * n_kb + kb];
                tot[r] += s * acc;
            } else {
                tot[r] += acc;
            }
        }
        if (kb + 1 < kb_end) {
#pragma unroll
            for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int c = 0; c < (kFp8 ? 2 : 4); ++c) wcur[r][c] = wnext[r][c];
#pragma unroll
            for (int i = 0; i < 4; ++i) bcur[i] = bnext[i];
        }
    }

    // Cross-wave reduction in a fixed order.  red[w][r][lane] holds C rows
    // 4*(lane/16)+v, column lane%16.
    __shared__ f32x4 red[KSPLIT][RT][64];
#pragma unroll
    for (int r = 0; r < RT; ++r) red[wave][r][lane] = tot[r];
    __syncthreads();

    const int items = (epilogue == kSwiGLU ? RT / 2 : RT) * T * kTileRows;
    for (int it = threadIdx.x; it < items; it += 64 * KSPLIT) {
        const int row = it % kTileRows;
        const int t = (it / kTileRows) % T;
        const int r = it / (kTileRows * T);
        const int src_lane = (row >> 2) * 16;
        const int v = row & 3;
        auto cval = [&](int rr, int c) {
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < KSPLIT; ++w) s += red[w][rr][src_lane + c][v];
            return s;
        };
        if (epilogue == kSwiGLU) {
            // interleaved tiles: even = gate rows, odd = up rows of the same 16 outputs
            const int rt_g = rt0 + 2 * r;
            const int orow = (rt_g / 2) * kTileRows + row;
            if (rt_g + 1 < m_tiles + 1 && orow < m / 2) {
                const float gv = cval(2 * r, t) + cval(2 * r, T + t);
                const float uv = cval(2 * r + 1, t) + cval(2 * r + 1, T + t);
                Y[static_cast<size_t>(t) * (m / 2) + orow] = gv / (1.f + __expf(-gv)) * uv;
            }
        } else {
            const int orow = (rt0 + r) * kTileRows + row;
            if (orow < m) {
                const float val = cval(r, t) + cval(r, T + t);
                float* dst = Y + static_cast<size_t>(t) * m + orow;
                if (epilogue == kAdd)
                    *dst += val;
                else
                    *dst = val;
            }
        }
    }
}

// X fp32 [T][n] -> fragments [kb][i][g][c][8 bf16]; c < T: hi of token c, else mid of
// token c - T.  Column j of block kb for (i, g, e) is 32g + 8i + e.
__global__ void pack_act_kernel(const float* __restrict__ X, i32x4* __restrict__ frag, int n, int n_kb, int T) {
    const int total = n_kb * 16 * T;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int t = idx % T;
    const int gi = (idx / T) % 16;  // i*4 + g
    const int kb = idx / (T * 16);
    const int i = gi >> 2, g = gi & 3;
    const int j0 = kb * kBlockCols + 32 * g + 8 * i;
    union {
        uint16_t h[8];
        i32x4 v;
    } hi, mid;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int j = j0 + e;
        const float x = j < n ? X[static_cast<size_t>(t) * n + j] : 0.f;
        split_bf16(x, hi.h[e], mid.h[e]);
    }
    const int NC = 2 * T;
    const size_t base = ((static_cast<size_t>(kb) * 4 + i) * 4 + g) * NC;
    frag[base + t] = hi.v;
    frag[base + T + t] = mid.v;
}

// Row-major e4m3 [m][n] + block scales -> tiled bytes + per-tile scales.
// One thread per (row-tile, column block, lane): 32 bytes.
__global__ void pack_fp8_kernel(const uint8_t* __restrict__ w, const float* __restrict__ scale,
                                uint8_t* __restrict__ out, float* __restrict__ tscale, int m, int n, int n_kb) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int m_tiles = (m + kTileRows - 1) / kTileRows;
    if (idx >= static_cast<size_t>(m_tiles) * n_kb * 64) return;
    const int lane = idx & 63;
    const int kb = (idx >> 6) % n_kb;
    const int rt = static_cast<int>((idx >> 6) / n_kb);
    const int row = rt * kTileRows + (lane & 15);
    const int c0 = kb * kBlockCols + 32 * (lane >> 4);
    uint8_t b[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) b[e] = (row < m && c0 + e < n) ? w[static_cast<size_t>(row) * n + c0 + e] : 0;
    uint8_t* tile = out + (static_cast<size_t>(rt) * n_kb + kb) * 2048;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        tile[16 * lane + e] = b[e];
        tile[1024 + 16 * lane + e] = b[16 + e];
    }
    if (lane == 0) {
        const int sb_cols = (n + 127) / 128;
        tscale[static_cast<size_t>(rt) * n_kb + kb] = scale[static_cast<size_t>((rt * kTileRows) / 128) * sb_cols + kb];
    }
}

__global__ void pack_bf16_kernel(const uint16_t* __restrict__ w, uint16_t* __restrict__ out, int m, int n,
                                 int n_kb) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int m_tiles = (m + kTileRows - 1) / kTileRows;
    if (idx >= static_cast<size_t>(m_tiles) * n_kb * 64) return;
    const int lane = idx & 63;
    const int kb = (idx >> 6) % n_kb;
    const int rt = static_cast<int>((idx >> 6) / n_kb);
    const int row = rt * kTileRows + (lane & 15);
    const int c0 = kb * kBlockCols + 32 * (lane >> 4);
    uint16_t* tile = out + (static_cast<size_t>(rt) * n_kb + kb) * 2048;  // 4096 B = 2048 halves
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int c = c0 + 8 * q + e;
            tile[q * 512 + 8 * lane + e] = (row < m && c < n) ? w[static_cast<size_t>(row) * n + c] : 0;
        }
}

__global__ void e4m3_decode_kernel(const uint8_t* __restrict__ in, float* __restrict__ out, size_t n) {
    const size_t i4 = (static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
    if (i4 >= n) return;
    uint32_t w = 0;
    for (int e = 0; e < 4; ++e)
        if (i4 + e < n) w |= static_cast<uint32_t>(in[i4 + e]) << (8 * e);
    uint32_t lo, hi;
    e4m3x4_to_bf16(w, lo, hi);
    const uint32_t h[4] = {lo & 0xffffu, lo >> 16, hi & 0xffffu, hi >> 16};
    for (int e = 0; e < 4; ++e)
        if (i4 + e < n) out[i4 + e] = __uint_as_float(h[e] << 16);
}

inline int n_kb_of(int n) { return (n + kBlockCols - 1) / kBlockCols; }
inline int m_tiles_of(int m) { return (m + kTileRows - 1) / kTileRows; }

template <bool kFp8>
void launch_gemm(const void* W, const float* tscale, const void* frag, float* Y, int m, int n, int T, int epilogue,
                 hipStream_t s) {
    RL_REQUIRE(m > 0 && n > 0, RL_ERR_RANGE, "gemm: empty shape");
    RL_REQUIRE(T >= 1 && T <= 8, RL_ERR_RANGE, "gemm: T must be in 1..8");
    RL_REQUIRE(W && frag && Y, RL_ERR_RANGE, "gemm: null pointer");
    RL_REQUIRE(!kFp8 || tscale, RL_ERR_RANGE, "gemm: FP8 weights need tile scales");
    const int n_kb = n_kb_of(n);
    const int m_tiles = m_tiles_of(m);
    constexpr int RT = 2, KS = 4;
    if (epilogue == kSwiGLU)
        RL_REQUIRE(m % 32 == 0, RL_ERR_RANGE, "gemm swiglu: interleaved rows must be a multiple of 32");
    const int grid = (m_tiles + RT - 1) / RT;
    hipLaunchKernelGGL((gemm_frag_kernel<RT, KS, kFp8>), dim3(grid), dim3(64 * KS), 0, s,
                       static_cast<const uint8_t*>(W), tscale, static_cast<const i32x4*>(frag), Y, m, n_kb, T,
                       epilogue);
    check_launch("gemm_frag_kernel");
}

void launch_pack_act(const float* X, void* frag, int n, int T, hipStream_t s) {
    RL_REQUIRE(n > 0 && T >= 1 && T <= 8, RL_ERR_RANGE, "pack_act: bad shape");
    const int n_kb = n_kb_of(n);
    const int total = n_kb * 16 * T;
    hipLaunchKernelGGL(pack_act_kernel, dim3((total + 255) / 256), dim3(256), 0, s, X, static_cast<i32x4*>(frag), n,
                       n_kb, T);
    check_launch("pack_act_kernel");
}

}  // namespace

namespace rl {
// Internal entry points shared with the engine.
void gemm_fp8_frag(const uint8_t* W, const float* ts, const void* frag, float* Y, int m, int n, int T, int epi,
                   hipStream_t s) {
    launch_gemm<true>(W, ts, frag, Y, m, n, T, epi, s);
}
void gemm_bf16_frag(const uint16_t* W, const void* frag, float* Y, int m, int n, int T, int epi, hipStream_t s) {
    launch_gemm<false>(W, nullptr, frag, Y, m, n, T, epi, s);
}
void pack_act(const float* X, void* frag, int n, int T, hipStream_t s) { launch_pack_act(X, frag, n, T, s); }
}  // namespace rl

using namespace rl;

extern "C" {

size_t rl_hip_fp8_packed_bytes(int m, int n) { return static_cast<size_t>(m_tiles_of(m)) * n_kb_of(n) * 2048; }
size_t rl_hip_fp8_tile_scales(int m, int n) { return static_cast<size_t>(m_tiles_of(m)) * n_kb_of(n); }
size_t rl_hip_bf16_packed_bytes(int m, int n) { return static_cast<size_t>(m_tiles_of(m)) * n_kb_of(n) * 4096; }
size_t rl_hip_act_frag_bytes(int n, int T) { return static_cast<size_t>(n_kb_of(n)) * 16 * 2 * T * 16; }

int rl_hip_pack_fp8(const uint8_t* w, const float* scale, uint8_t* w_tiled, float* tile_scale, int m, int n,
                    void* stream) {
    return guard([&] {
        RL_REQUIRE(m > 0 && n > 0 && w && scale && w_tiled && tile_scale, RL_ERR_RANGE, "pack_fp8: bad args");
        const size_t total = static_cast<size_t>(m_tiles_of(m)) * n_kb_of(n) * 64;
        hipLaunchKernelGGL(pack_fp8_kernel, dim3((total + 255) / 256), dim3(256), 0, S(stream), w, scale, w_tiled,
                           tile_scale, m, n, n_kb_of(n));
        check_launch("pack_fp8_kernel");
    });
}

int rl_hip_pack_bf16(const uint16_t* w, uint16_t* w_tiled, int m, int n, void* stream) {
    return guard([&] {
        RL_REQUIRE(m > 0 && n > 0 && w && w_tiled, RL_ERR_RANGE, "pack_bf16: bad args");
        const size_t total = static_cast<size_t>(m_tiles_of(m)) * n_kb_of(n) * 64;
        hipLaunchKernelGGL(pack_bf16_kernel, dim3((total + 255) / 256), dim3(256), 0, S(stream), w, w_tiled, m, n,
                           n_kb_of(n));
        check_launch("pack_bf16_kernel");
    });
}

int rl_hip_pack_act(const float* X, void* frag, int n, int T, void* stream) {
    return guard([&] { launch_pack_act(X, frag, n, T, S(stream)); });
}

int rl_hip_gemm_fp8_frag(const uint8_t* w_tiled, const float* tile_scale, const void* frag, float* Y, int m, int n,
                         int T, int accumulate, void* stream) {
    return guard([&] { launch_gemm<true>(w_tiled, tile_scale, frag, Y, m, n, T, accumulate ? kAdd : kStore, S(stream)); });
}

int rl_hip_gemm_bf16_frag(const uint16_t* w_tiled, const void* frag, float* Y, int m, int n, int T, int accumulate,
                          void* stream) {
    return guard([&] { launch_gemm<false>(w_tiled, nullptr, frag, Y, m, n, T, accumulate ? kAdd : kStore, S(stream)); });
}

int rl_hip_gemm_fp8(const uint8_t* w_tiled, const float* tile_scale, const float* X, float* Y, void* frag_scratch,
                    int m, int n, int T, void* stream) {
    return guard([&] {
        launch_pack_act(X, frag_scratch, n, T, S(stream));
        launch_gemm<true>(w_tiled, tile_scale, frag_scratch, Y, m, n, T, kStore, S(stream));
    });
}

int rl_hip_e4m3_to_f32(const uint8_t* in, float* out, size_t n, void* stream) {
    return guard([&] {
        if (n == 0) return;
        RL_REQUIRE(in && out, RL_ERR_RANGE, "e4m3_to_f32: null pointer");
        const size_t threads = (n + 3) / 4;
        hipLaunchKernelGGL(e4m3_decode_kernel, dim3((threads + 255) / 256), dim3(256), 0, S(stream), in, out, n);
        check_launch("e4m3_decode_kernel");
    });
}

}  // extern "C"
