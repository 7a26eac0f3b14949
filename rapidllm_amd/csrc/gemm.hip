// gemm.hip -- skinny block-FP8 / BF16 linears for T = 1..16 tokens on gfx950 MFMA.
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
// Work split: a workgroup = KSPLIT waves over RT row-tiles; wave w walks every
// KSPLIT-th column block (depth 1) or a contiguous 1/KSPLIT of them (deeper
// pipelines), partial C tiles are summed through LDS
// in a fixed order (deterministic), then the epilogue stores or accumulates Y.
#include "internal.h"

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

// kPartial: split-K over S workgroups per row group; slice s writes its partial sum
// to Y + (s*T + t)*ldy (the consumer adds the S slices in order).
// Weight loads are non-temporal: every weight byte is streamed once per launch.

enum Epilogue { kStore = 0, kAdd = 1, kSwiGLU = 2, kPartial = 3, kAddNorm = 4, kSwiGLUH = 5 };

// Grid: one workgroup per RT row-tiles.  Each workgroup: KSPLIT waves, each wave a
// contiguous run of column blocks.  D = load pipeline depth (D-1 column blocks of
// weights in flight while one is computed).
// kKs: per-column-block input scale (NormIO::kss, the folded gated RMSNorm); depth 1.
// TT > 0: T is the compile-time token count TT.  For TT <= 4 each column block's
// activation fragments (16 * 2T units of 16 B) are fetched by 1 or 2 coalesced loads
// (every lane one distinct unit) and handed to the lanes that need them by
// ds_bpermute; for TT = 5..8 the four per-lane loads are all but distinct units
// already (NC = 2T of the 16 B columns), so each lane loads its own.
// Loading each lane's B operand directly takes four 64-lane loads per block for
// 128 * T distinct bytes; those load instructions, not the bytes, measured 2-4 us
// per launch (34816 x 5120 at T=1: 31.5 -> 27.5 us cold).
// EPI >= 0 / SSIN >= 0: the epilogue and whether the input RMSNorm is folded in
// (io.ss_in) are compile-time, so an instantiation keeps no registers for the
// others' state across the main loop (eight waves per SIMD need <= 64 VGPRs).
// kGuh: gate/up in half tiles (SwiGLU epilogue): 16-row tile k holds gate rows
// 8k .. 8k+7 (tile rows 0-7) and up rows 8k .. 8k+7 (rows 8-15), with one block scale
// per half (tscale [tile][kb][2]); one tile gives 8 outputs, so a workgroup needs
// only one row tile (the whole-tile interleave needs two).
template <int RT, int KSPLIT, int D, bool kFp8, bool kKs = false, int TT = 0, int EPI = -1, int SSIN = -1,
          bool kGuh = false>
__global__ __launch_bounds__(64 * KSPLIT) void gemm_frag_kernel(const uint8_t* __restrict__ W,
                                                                const float* __restrict__ tscale,
                                                                const i32x4* __restrict__ frag,
                                                                float* __restrict__ Y, int m, int n_kb, int T_,
                                                                int epilogue_, int ldy, int m_valid, int S,
                                                                i32x4* __restrict__ frag_out, NormIO io) {
    const int T = TT > 0 ? TT : T_;
    const int epilogue = EPI >= 0 ? EPI : epilogue_;
    // Partial sums per workgroup: column block kb goes to partial kb % KP, which
    // wave kb % KSPLIT accumulates (KP / KSPLIT of them per wave), and the partials
    // are added in index order.  The residual add-norm kernels use 16 partials
    // with 8 or 16 waves, so every work split gives identical sums (a row of a
    // T = 1 step equals the same row of a T = 2..4 verify or batch step).
    constexpr int KP = (EPI == kAddNorm && RT == 2 && KSPLIT <= 16) ? 16 : KSPLIT;
    constexpr int NP = KP / KSPLIT;
    static_assert(KP % KSPLIT == 0 && (NP == 1 || D == 1), "partials: a multiple of the waves, depth 1");
    if constexpr (SSIN == 0) io.ss_in = nullptr;
    const bool has_ss = SSIN == 1 || (SSIN < 0 && io.ss_in != nullptr);
    constexpr int kTileBytes = kFp8 ? 2048 : 4096;
    constexpr int NW = kFp8 ? 2 : 4;  // 16-byte loads per lane per tile
    const int lane = threadIdx.x & 63;
    // wave-uniform: keeps the column-block bounds, the tile-scale loads and the loop
    // control in scalar registers (scale loads then wait on their own counter and
    // never on the weight loads queued behind them)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4;
    const int col = lane & 15;
    const int NC = 2 * T;
    const int slice = blockIdx.x % S;
    const int rt0 = (blockIdx.x / S) * RT;
    const int m_tiles = (m + kTileRows - 1) / kTileRows;

    // column blocks of this workgroup's slice; for depth > 1 a contiguous run per wave
    const int per_s = (n_kb + S - 1) / S;
    const int s_begin = min(n_kb, slice * per_s), s_end = min(n_kb, s_begin + per_s);
    const int per = (s_end - s_begin + KSPLIT - 1) / KSPLIT;
    const int kb_begin = min(s_end, s_begin + wave * per);
    const int kb_end = min(s_end, kb_begin + per);

    // TT = 9..16: the 2T B columns (hi of each token, then mid) span two 16-column
    // MFMA tiles; every weight fragment feeds one MFMA per tile
    constexpr int NCT = TT > 8 ? 2 : 1;
    constexpr int kMaxTok = TT > 8 ? 16 : 8;
    f32x4 tots[NP][RT][NCT];
#pragma unroll
    for (int q = 0; q < NP; ++q)
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int c = 0; c < NCT; ++c) tots[q][r][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto* tot = tots[0];

    // RMSNorm folded into this GEMM (io.ss_in): the input fragments hold x * (1+gamma)
    // unnormalised, and the outputs are scaled by 1/rms(x_t).  Wave w < T sums the
    // producer's per-group sums of squares of token w (issued here, consumed in the
    // epilogue, so the loads overlap the weight stream).
    // add-norm epilogue: thread `it` owns item it = (r, t, row) of the epilogue; its
    // residual value is loaded now, not after the main loop
    // (token-major: item it = t * RT*16 + r*16 + row, so each token's rows are one
    // run of RT*16 lanes), together with its gamma
    float xpre = 0.f, gpre = 0.f;
    // (indices recomputed where used, so only the two values stay live)
    auto an_orow_of = [&]() { return (rt0 + (threadIdx.x / kTileRows) % RT) * kTileRows + threadIdx.x % kTileRows; };
    auto an_valid_of = [&]() {
        return epilogue == kAddNorm && static_cast<int>(threadIdx.x) < RT * T * kTileRows &&
               rt0 + static_cast<int>((threadIdx.x / kTileRows) % RT) < m_tiles && an_orow_of() < m_valid;
    };
    if (an_valid_of()) {
        xpre = Y[static_cast<size_t>(threadIdx.x / (RT * kTileRows)) * ldy + an_orow_of()];
        gpre = 1.f + io.gamma_out[an_orow_of()];
    }

    // The sums are copied straight into LDS (global_load_lds: no registers held
    // through the main loop) and reduced in the epilogue.
    constexpr int kMaxSsPerLane = 4;  // groups <= 256
    __shared__ float ss_lds[kMaxTok][64 * kMaxSsPerLane];
    // wave w takes tokens w, w + KSPLIT, ...
    const bool ss_wave = has_ss && wave < T;
    if (ss_wave) {
        for (int t = wave; t < T; t += KSPLIT) {
#pragma unroll
            for (int k = 0; k < kMaxSsPerLane; ++k) {
                const int gi = lane + 64 * k;
                const float* src = io.ss_in + static_cast<size_t>(gi < io.groups_in ? gi : 0) * T + t;
                __builtin_amdgcn_global_load_lds(src, &ss_lds[t][64 * k], 4, 0, 0);
            }
        }
    }
    __shared__ f32x4 red[KP][RT][NCT][64];
    __shared__ float s_inv[kMaxTok];
    // Token `wave`'s 1/rms from the sums of squares in LDS (every load of this wave,
    // the copies included, has completed: the wait is explicit for waves that had no
    // column block to wait on).
    auto reduce_ss = [&]() {
        if (ss_wave) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            for (int t = wave; t < T; t += KSPLIT) {
                double ss = 0.0;
#pragma unroll
                for (int k = 0; k < kMaxSsPerLane; ++k) {
                    const int gi = lane + 64 * k;
                    ss += gi < io.groups_in ? static_cast<double>(ss_lds[t][gi]) : 0.0;  // group order
                }
                ss = wave_sum_d(ss);                                  // fixed butterfly order
                if (lane == 0) s_inv[t] = 1.f / sqrtf(static_cast<float>(ss / io.n_norm) + io.eps);
            }
        }
    };

    // Lanes of B columns >= 2T read a valid column: those MFMA output columns are
    // never used, and unconditional loads keep the load count identical on every
    // path, so the compiler's waits stay exact.
    int bcolv[NCT];
#pragma unroll
    for (int c = 0; c < NCT; ++c) bcolv[c] = min(16 * c + col, NC - 1);
    const int bcol = bcolv[0];
    const uint8_t* wbase[RT];
    const float* sbase[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int rt = min(rt0 + r, m_tiles - 1);
        wbase[r] = W + static_cast<size_t>(rt) * n_kb * kTileBytes;  // uniform tile-row base
        sbase[r] = kFp8 ? tscale + static_cast<size_t>(rt) * n_kb * (kGuh ? 2 : 1) : nullptr;
    }
    const i32x4* fbase = frag + static_cast<size_t>(g) * NC;
    const size_t fstride = static_cast<size_t>(16) * NC;  // per column block

    i32x4 wbuf[D][RT][NW];
    i32x4 bbuf[D][NCT][4];
    float sbuf[D][RT];
    float sbuf2[D][RT];  // kGuh: the up half's scale
    // kKs: this lane's token (B column hi / mid of token ktok) and the block scale
    // 1 / rms of the block's four partial sums of squares
    int ktokv[NCT];
#pragma unroll
    for (int c = 0; c < NCT; ++c) ktokv[c] = bcolv[c] < T ? bcolv[c] : bcolv[c] - T;
    const float kss_inv_n = kKs ? 1.f / static_cast<float>(io.kss_n) : 0.f;
    auto block_sums = [&](int kb, int c = 0) {
        // this lane's token's four sums of the block, requested just before the
        // block's weights (loads return in issue order, so they are there first)
        return reinterpret_cast<const float4*>(io.kss)[static_cast<size_t>(kb) * T + ktokv[c]];
    };
    auto block_scale = [&](const float4 q) {
        return __builtin_amdgcn_rsqf(((q.x + q.y) + (q.z + q.w)) * kss_inv_n + io.kss_eps);
    };
    // kb >= kb_end: a pipeline slot past the wave's range.  Its loads still issue (so
    // the load count is the same on every path) but read the small, cache-resident
    // activation fragments instead of weights; the values are never used.
    // (the fragments hold n_kb * 512 * T bytes; narrower inputs use this group's
    // first weight tile instead)
    const uint8_t* dummy = n_kb * 512 * T >= kTileBytes ? reinterpret_cast<const uint8_t*>(frag) : wbase[0];
    auto load = [&](int d, int kb, bool live) {
        if constexpr (kFp8 && kGuh) {
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                sbuf[d][r] = sbase[r][2 * (live ? kb : 0)];
                sbuf2[d][r] = sbase[r][2 * (live ? kb : 0) + 1];
            }
        } else if constexpr (kFp8) {
#pragma unroll
            for (int r = 0; r < RT; ++r) sbuf[d][r] = sbase[r][live ? kb : 0];
        }
        // TT > 0: the block's fragment loads go first, so the permutes that consume
        // them wait only for them (the load counter retires in issue order), with
        // the block's weight loads still in flight
        const int kbw = kb;
        kb = live ? kb : 0;
        auto load_weights = [&]() {
#pragma unroll
            for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int c = 0; c < NW; ++c) {
                    const uint8_t* base = live ? wbase[r] + static_cast<size_t>(kbw) * kTileBytes : dummy;
                    const i32x4* p = reinterpret_cast<const i32x4*>(base + c * 1024) + lane;
                    wbuf[d][r][c] = __builtin_nontemporal_load(p);
                }
        };
        if constexpr (TT == 0 || TT > 4) load_weights();
        if constexpr (TT > 0 && TT <= 4) {
            // L loads of P units: load j, lane l holds unit j*P + l; MFMA i of lane
            // (g, col) needs unit (i*4 + g)*NC + bcol, which is in load j = i*L/4
            constexpr int NCc = 2 * TT;
            constexpr int L = NCc <= 4 ? 1 : (NCc <= 8 ? 2 : 4);
            constexpr int P = 16 * NCc / L;
            const i32x4* fb = frag + kb * fstride;
            const int li = lane < P ? lane : 0;
            i32x4 src[L];
#pragma unroll
            for (int j = 0; j < L; ++j) src[j] = fb[j * P + li];
            load_weights();
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = i * L / 4;
                const int addr = ((i * 4 + g) * NCc + bcol - j * P) * 4;  // source lane, in bytes
#pragma unroll
                for (int c = 0; c < 4; ++c) bbuf[d][0][i][c] = __builtin_amdgcn_ds_bpermute(addr, src[j][c]);
            }
        } else {
#pragma unroll
            for (int c = 0; c < NCT; ++c)
#pragma unroll
                for (int i = 0; i < 4; ++i) bbuf[d][c][i] = fbase[kb * fstride + i * 4 * NC + bcolv[c]];
        }
    };
    // ks0 / ks1: the kKs block scale of the lane's token in column tile 0 / 1
    auto compute = [&](int d, int kb, float ks0 = 1.f, int q = 0, float ks1 = 1.f) {
        auto* tot = tots[q];
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            f32x4 acc[NCT];
#pragma unroll
            for (int c = 0; c < NCT; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                Frag8 a;
                if constexpr (kFp8) {
                    const i32x4 wv = wbuf[d][r][i >> 1];
                    const uint32_t d0 = static_cast<uint32_t>((i & 1) ? wv[2] : wv[0]);
                    const uint32_t d1 = static_cast<uint32_t>((i & 1) ? wv[3] : wv[1]);
                    e4m3x4_to_bf16(d0, a.u[0], a.u[1]);
                    e4m3x4_to_bf16(d1, a.u[2], a.u[3]);
                } else {
                    a.i = wbuf[d][r][i];
                }
#pragma unroll
                for (int c = 0; c < NCT; ++c) {
                    Frag8 b;
                    b.i = bbuf[d][c][i];
                    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, acc[c], 0, 0, 0);
                }
            }
#pragma unroll
            for (int c = 0; c < NCT; ++c) {
                const float ks = c == 0 ? ks0 : ks1;
                if constexpr (kFp8 && kGuh)
                    tot[r][c] += (g < 2 ? sbuf[d][r] : sbuf2[d][r]) * acc[c];  // C rows 4g..4g+3: gate g < 2
                else if constexpr (kFp8 && kKs)
                    tot[r][c] += (sbuf[d][r] * ks) * acc[c];
                else if constexpr (kFp8)
                    tot[r][c] += sbuf[d][r] * acc[c];
                else if constexpr (kKs)
                    tot[r][c] += ks * acc[c];
                else
                    tot[r][c] += acc[c];
            }
        }
    };

    if constexpr (D == 1) {
        // depth 1: load a column block, compute it (the compiler schedules the
        // loads; measured as fast as any explicit pipeline for the FP8 launches).
        // Wave w takes blocks w, w + KSPLIT, ...: at any moment the workgroup reads
        // KSPLIT adjacent tiles per row-tile (1-3% faster than contiguous runs)
        // (with NP > 1 partials per wave, its j-th block goes to partial j % NP)
        if constexpr (kKs) {
            for (int kb0 = s_begin + wave; kb0 < s_end; kb0 += KSPLIT * NP) {
#pragma unroll
                for (int q = 0; q < NP; ++q) {
                    const int kb = kb0 + q * KSPLIT;
                    if (q == 0 || kb < s_end) {
                        const float4 qs = block_sums(kb);
                        const float4 qs1 = NCT > 1 ? block_sums(kb, NCT - 1) : qs;
                        load(0, kb, true);
                        compute(0, kb, block_scale(qs), q, block_scale(qs1));
                    }
                }
            }
        } else {
            for (int kb0 = s_begin + wave; kb0 < s_end; kb0 += KSPLIT * NP) {
#pragma unroll
                for (int q = 0; q < NP; ++q) {
                    const int kb = kb0 + q * KSPLIT;
                    if (q == 0 || kb < s_end) {
                        load(0, kb, true);
                        compute(0, kb, 1.f, q);
                    }
                }
            }
        }
    } else if (kb_begin < kb_end) {
        // software pipeline, D stages
#pragma unroll
        for (int d = 0; d < D; ++d) load(d, kb_begin + d, kb_begin + d < kb_end);
        // Phase order pinned (compiler memory barrier + scheduling barrier): no
        // load may move past a compute phase, or the in-order load counter would
        // make that compute wait for the loads queued behind its own.
        if constexpr (D > 1) asm volatile("" ::: "memory");
        for (int kb = kb_begin; kb < kb_end; kb += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                if constexpr (D > 1) __builtin_amdgcn_sched_barrier(0);
                if (kb + d < kb_end) compute(d, kb + d);
                if constexpr (D > 1) {
                    asm volatile("" ::: "memory");
                    __builtin_amdgcn_sched_barrier(0);
                }
                load(d, kb + d + D, kb + d + D < kb_end);
                if constexpr (D > 1) asm volatile("" ::: "memory");
            }
        }
    }

    // Cross-wave reduction in a fixed order.  red[w][r][lane] holds C rows
    // 4*(lane/16)+v, column lane%16.
#pragma unroll
    for (int q = 0; q < NP; ++q)
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int c = 0; c < NCT; ++c) red[wave + q * KSPLIT][r][c][lane] = tots[q][r][c];
    reduce_ss();
    __syncthreads();

    // items: (r, t, row); value = hi column + mid column, summed over waves
    const int items = RT * T * kTileRows;
    auto wg_value = [&](int r, int t, int row) {
        const int src_lane = (row >> 2) * 16;
        const int v = row & 3;
        const int ch = t, cm = T + t;  // B columns of the token's hi and mid parts
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < KP; ++w)
            s += red[w][r][NCT > 1 ? ch >> 4 : 0][src_lane + (ch & 15)][v] +
                 red[w][r][NCT > 1 ? cm >> 4 : 0][src_lane + (cm & 15)][v];
        return s;
    };

    auto final_value = [&](int r, int t, int row) -> float {
        const float v = wg_value(r, t, row);
        return has_ss ? v * s_inv[t] : v;
    };

    if (kGuh && epilogue == kSwiGLU) {
        // half tiles: rows j and 8 + j of a tile are gate and up of output 8k + j
        for (int it = threadIdx.x; it < RT * T * 8; it += 64 * KSPLIT) {
            const int j = it % 8, t = (it / 8) % T, r = it / (8 * T);
            const int orow = (rt0 + r) * 8 + j;
            if (rt0 + r < m_tiles && orow < m_valid) {
                const float gv = final_value(r, t, j);
                const float uv = final_value(r, t, 8 + j);
                const float h = gv / (1.f + __expf(-gv)) * uv;
                if (Y) Y[static_cast<size_t>(t) * ldy + orow] = h;
                if (frag_out) {
                    uint16_t hi, mid;
                    split_bf16(h, hi, mid);
                    uint16_t* f16 = reinterpret_cast<uint16_t*>(frag_out);
                    const size_t u = frag_unit(orow >> 3, t, T);
                    f16[u * 8 + (orow & 7)] = hi;
                    f16[(u + T) * 8 + (orow & 7)] = mid;
                }
            }
        }
    } else if (epilogue == kSwiGLU) {
        // interleaved tiles: even = gate rows, odd = up rows of the same 16 outputs.
        // h = silu(g) * u goes to Y (fp32, if given) and, if frag_out is given, to the
        // bf16 hi/mid fragments of the next linear (input column = output row), each
        // thread storing its element's two halves directly.
        for (int it = threadIdx.x; it < (RT / 2) * T * kTileRows; it += 64 * KSPLIT) {
            const int row = it % kTileRows, t = (it / kTileRows) % T, r = it / (kTileRows * T);
            const int orow = ((rt0 + 2 * r) / 2) * kTileRows + row;
            if (rt0 + 2 * r + 1 < m_tiles && orow < m_valid) {
                const float gv = final_value(2 * r, t, row);
                const float uv = final_value(2 * r + 1, t, row);
                const float h = gv / (1.f + __expf(-gv)) * uv;
                if (Y) Y[static_cast<size_t>(t) * ldy + orow] = h;
                if (frag_out) {
                    uint16_t hi, mid;
                    split_bf16(h, hi, mid);
                    uint16_t* f16 = reinterpret_cast<uint16_t*>(frag_out);
                    const size_t u = frag_unit(orow >> 3, t, T);
                    f16[u * 8 + (orow & 7)] = hi;
                    f16[(u + T) * 8 + (orow & 7)] = mid;
                }
            }
        }
    } else if (epilogue == kAddNorm) {
        // Residual add fused with the next RMSNorm's data movement (one writer per
        // row): x += W.a in place; this thread's element of the next linear's input
        // fragments, x * (1 + gamma), written as its two bf16 halves; and the group's
        // sum of x^2 per token, reduced over the token's RT*16 lanes in a fixed
        // butterfly order (double), stored as float (io.ss_out[group][t]).
        const bool an_item = static_cast<int>(threadIdx.x) < RT * T * kTileRows;
        const int an_t = threadIdx.x / (RT * kTileRows);
        const int an_r = (threadIdx.x / kTileRows) % RT;
        const int an_row = threadIdx.x % kTileRows;
        const int an_orow = an_orow_of();
        if (an_item) {
            double sq = 0.0;
            if (an_valid_of()) {
                const float x = xpre + final_value(an_r, an_t, an_row);
                Y[static_cast<size_t>(an_t) * ldy + an_orow] = x;
                uint16_t hi, mid;
                split_bf16(x * gpre, hi, mid);
                uint16_t* f16 = reinterpret_cast<uint16_t*>(frag_out);
                const size_t u = frag_unit(an_orow >> 3, an_t, T);
                f16[u * 8 + (an_orow & 7)] = hi;
                f16[(u + T) * 8 + (an_orow & 7)] = mid;
                sq = static_cast<double>(x) * x;
            }
#pragma unroll
            for (int o = 1; o < RT * kTileRows; o <<= 1) sq += __shfl_xor(sq, o, 64);
            if (threadIdx.x % (RT * kTileRows) == 0)
                io.ss_out[static_cast<size_t>(blockIdx.x) * T + an_t] = static_cast<float>(sq);
        }
    } else {
        for (int it = threadIdx.x; it < items; it += 64 * KSPLIT) {
            const int row = it % kTileRows, t = (it / kTileRows) % T, r = it / (kTileRows * T);
            const int orow = (rt0 + r) * kTileRows + row;
            if (orow < m_valid) {
                const float val = final_value(r, t, row);
                float* dst = Y + (static_cast<size_t>(slice) * T + t) * ldy + orow;
                if (epilogue == kAdd)
                    *dst += val;
                else
                    *dst = val;
            }
        }
    }

    // overflow row tiles (NormIO::xpart): workgroup u < (tiles) * x_slices computes
    // K-slice u % x_slices of tile x_tile0 + u / x_slices, one column block per wave
    if (io.xpart && static_cast<int>(blockIdx.x) < (io.x_rows / kTileRows) * io.x_slices) {
        const int u = blockIdx.x;
        const int xt = io.x_tile0 + u / io.x_slices, sl = u % io.x_slices;
        const int per = (n_kb + io.x_slices - 1) / io.x_slices;
        const int kb = sl * per + wave;
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            wbase[r] = W + static_cast<size_t>(xt) * n_kb * kTileBytes;
            sbase[r] = kFp8 ? tscale + static_cast<size_t>(xt) * n_kb : nullptr;
#pragma unroll
            for (int c = 0; c < NCT; ++c) tot[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        if (wave < per && kb < n_kb) {
            load(0, kb, true);
            compute(0, kb);
        }
        __syncthreads();  // the row epilogue above has read red
#pragma unroll
        for (int c = 0; c < NCT; ++c) red[wave][0][c][lane] = tot[0][c];
        __syncthreads();
        if (static_cast<int>(threadIdx.x) < kTileRows * T) {
            const int row = threadIdx.x % kTileRows, t = threadIdx.x / kTileRows;
            io.xpart[(static_cast<size_t>(sl) * T + t) * io.x_rows + (xt - io.x_tile0) * kTileRows + row] =
                final_value(0, t, row);
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
                                uint8_t* __restrict__ out, float* __restrict__ tscale, int m, int n, int n_kb,
                                int rt_stride, int rt_offset) {
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
    const size_t drt = static_cast<size_t>(rt) * rt_stride + rt_offset;  // destination tile row
    uint8_t* tile = out + (drt * n_kb + kb) * 2048;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        tile[16 * lane + e] = b[e];
        tile[1024 + 16 * lane + e] = b[16 + e];
    }
    if (lane == 0) {
        const int sb_cols = (n + 127) / 128;
        tscale[drt * n_kb + kb] = scale[static_cast<size_t>((rt * kTileRows) / 128) * sb_cols + kb];
    }
}

// Gate or up (half = 0 / 1) [I][n] into the half-tile gate/up layout: tile k rows
// 8*half .. 8*half+7 take source rows 8k .. 8k+7; scale [tile][kb][2].  Each lane
// owns tile row (lane & 15), as in pack_fp8_kernel.
__global__ void pack_fp8_guh_kernel(const uint8_t* __restrict__ w, const float* __restrict__ scale,
                                    uint8_t* __restrict__ out, float* __restrict__ tscale, int I, int n, int n_kb,
                                    int half) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int tiles = (I + 7) / 8;
    if (idx >= static_cast<size_t>(tiles) * n_kb * 64) return;
    const int lane = idx & 63;
    const int kb = (idx >> 6) % n_kb;
    const int rt = static_cast<int>((idx >> 6) / n_kb);
    const int r16 = lane & 15;
    if ((r16 >= 8) != (half != 0)) return;
    const int row = rt * 8 + (r16 & 7);
    const int c0 = kb * kBlockCols + 32 * (lane >> 4);
    uint8_t b[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) b[e] = (row < I && c0 + e < n) ? w[static_cast<size_t>(row) * n + c0 + e] : 0;
    uint8_t* tile = out + (static_cast<size_t>(rt) * n_kb + kb) * 2048;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        tile[16 * lane + e] = b[e];
        tile[1024 + 16 * lane + e] = b[16 + e];
    }
    if (r16 == 8 * half) {
        const int sb_cols = (n + 127) / 128;
        tscale[(static_cast<size_t>(rt) * n_kb + kb) * 2 + half] = scale[static_cast<size_t>((rt * 8) / 128) * sb_cols + kb];
    }
}

__global__ void pack_bf16_guh_kernel(const uint16_t* __restrict__ w, uint16_t* __restrict__ out, int I, int n,
                                     int n_kb, int half) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int tiles = (I + 7) / 8;
    if (idx >= static_cast<size_t>(tiles) * n_kb * 64) return;
    const int lane = idx & 63;
    const int kb = (idx >> 6) % n_kb;
    const int rt = static_cast<int>((idx >> 6) / n_kb);
    const int r16 = lane & 15;
    if ((r16 >= 8) != (half != 0)) return;
    const int row = rt * 8 + (r16 & 7);
    const int c0 = kb * kBlockCols + 32 * (lane >> 4);
    uint16_t* tile = out + (static_cast<size_t>(rt) * n_kb + kb) * 2048;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int c = c0 + 8 * q + e;
            tile[q * 512 + 8 * lane + e] = (row < I && c < n) ? w[static_cast<size_t>(row) * n + c] : 0;
        }
}

__global__ void pack_bf16_kernel(const uint16_t* __restrict__ w, uint16_t* __restrict__ out, int m, int n,
                                 int n_kb, int rt_stride, int rt_offset) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int m_tiles = (m + kTileRows - 1) / kTileRows;
    if (idx >= static_cast<size_t>(m_tiles) * n_kb * 64) return;
    const int lane = idx & 63;
    const int kb = (idx >> 6) % n_kb;
    const int rt = static_cast<int>((idx >> 6) / n_kb);
    const int row = rt * kTileRows + (lane & 15);
    const int c0 = kb * kBlockCols + 32 * (lane >> 4);
    const size_t drt = static_cast<size_t>(rt) * rt_stride + rt_offset;
    uint16_t* tile = out + (drt * n_kb + kb) * 2048;  // 4096 B = 2048 halves
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

// Work split per launch: row-tiles per workgroup (RT), waves per workgroup along K
// (KS), load pipeline depth (D).  Measured on MI355X with weights cold in HBM
// (16480/34816 x 5120, 5120 x 17408/6144, T=1..4): RT=2 with 8 waves is best when
// there are >= 256 workgroups; short m (fewer workgroups than CUs) does better
// with 16 waves per workgroup.
struct GemmCfg {
    int rt, ks, d;
};
static GemmCfg g_force{0, 0, 0};
// RL_GEMM_BPERM=0 keeps the per-lane B operand loads (A/B measurement)
inline bool bperm_enabled() {
    static const bool on = [] {
        const char* v = std::getenv("RL_GEMM_BPERM");
        return !(v && v[0] == '0');
    }();
    return on;
}

// Row tiles per workgroup of the store and half-tile SwiGLU launches at T = 5..8
// (RL_GEMM_RT8 = 1, 2 or 4 overrides it for measurement)
inline int rt_wide() {
    static const int rt = [] {
        const char* v = std::getenv("RL_GEMM_RT8");
        const int r = v ? std::atoi(v) : 0;
        return r == 1 || r == 2 || r == 4 ? r : 2;
    }();
    return rt;
}

// Row tiles per workgroup of the store and half-tile SwiGLU launches at T = 9..16
// (RL_GEMM_RT16 = 2 or 4 overrides it for measurement)
inline int rt_batch() {
    static const int rt = [] {
        const char* v = std::getenv("RL_GEMM_RT16");
        const int r = v ? std::atoi(v) : 0;
        return r == 2 || r == 4 ? r : 4;
    }();
    return rt;
}

// RL_ADDNORM16=0: the T = 1 residual add-norm launches keep 8 waves (A/B measurement)
inline bool addnorm16_enabled() {
    static const bool on = [] {
        const char* v = std::getenv("RL_ADDNORM16");
        return !(v && v[0] == '0');
    }();
    return on;
}

template <bool kFp8, int RT, int KS, int D, bool kKs, int TT, int EPI = -1, int SSIN = -1, bool kGuh = false>
void launch_gemm_tt(const void* W, const float* tscale, const void* frag, float* Y, int m, int n_kb, int T,
                    int epilogue, int ldy, int m_valid, int S, void* frag_out, const NormIO& io, hipStream_t s) {
    const int groups = (m_tiles_of(m) + RT - 1) / RT;
    hipLaunchKernelGGL((gemm_frag_kernel<RT, KS, D, kFp8, kKs, TT, EPI, SSIN, kGuh>), dim3(groups * S),
                       dim3(64 * KS), 0, s, static_cast<const uint8_t*>(W), tscale, static_cast<const i32x4*>(frag),
                       Y, m, n_kb, T, epilogue, ldy, m_valid, S, static_cast<i32x4*>(frag_out), io);
}

// The permuted-B kernel for (RT, KS) with the epilogue and folded-norm input as
// compile-time parameters (the combinations the decode step uses; others run the
// kernel with runtime ones).
template <bool kFp8, int RT, int KS, bool kKs, int TT, bool kGuh = false>
void launch_gemm_spec(const void* W, const float* tscale, const void* frag, float* Y, int m, int n_kb, int T,
                      int epilogue, int ldy, int m_valid, int S, void* frag_out, const NormIO& io, hipStream_t s) {
    const bool ss = io.ss_in != nullptr;
#define RL_SPEC(E, SS)                                                                                              \
    if (epilogue == E && ss == static_cast<bool>(SS)) {                                                             \
        launch_gemm_tt<kFp8, RT, KS, 1, kKs, TT, E, SS, kGuh>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, \
                                                             S, frag_out, io, s);                                 \
        return;                                                                                                     \
    }
    if constexpr (kGuh) {
        RL_SPEC(kSwiGLU, 0) RL_SPEC(kSwiGLU, 1)
    } else if constexpr (RT == 1) {
        RL_SPEC(kStore, 0) RL_SPEC(kStore, 1) RL_SPEC(kAdd, 0) RL_SPEC(kAdd, 1)
    } else if constexpr (kKs) {
        RL_SPEC(kAddNorm, 0)
    } else {
        RL_SPEC(kSwiGLU, 0) RL_SPEC(kSwiGLU, 1) RL_SPEC(kAddNorm, 0)
    }
#undef RL_SPEC
    launch_gemm_tt<kFp8, RT, KS, 1, kKs, TT, -1, -1, kGuh>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, S,
                                                         frag_out, io, s);
}

// Depth-1 launches take the compile-time-T kernels (permuted B operand for T <= 4).
template <bool kFp8, int RT, int KS, int D, bool kKs = false, bool kGuh = false>
void launch_gemm_cfg(const void* W, const float* tscale, const void* frag, float* Y, int m, int n_kb, int T,
                     int epilogue, int ldy, int m_valid, int S, void* frag_out, const NormIO& io, hipStream_t s) {
    if constexpr (D == 1) {
        if (bperm_enabled()) {
            switch (T) {
            case 1: launch_gemm_spec<kFp8, RT, KS, kKs, 1, kGuh>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, S, frag_out, io, s); return;
            case 2: launch_gemm_spec<kFp8, RT, KS, kKs, 2, kGuh>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, S, frag_out, io, s); return;
            case 3: launch_gemm_spec<kFp8, RT, KS, kKs, 3, kGuh>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, S, frag_out, io, s); return;
            case 4: launch_gemm_spec<kFp8, RT, KS, kKs, 4, kGuh>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, S, frag_out, io, s); return;
            case 5: launch_gemm_spec<kFp8, RT, KS, kKs, 5, kGuh>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, S, frag_out, io, s); return;
            case 6: launch_gemm_spec<kFp8, RT, KS, kKs, 6, kGuh>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, S, frag_out, io, s); return;
            case 7: launch_gemm_spec<kFp8, RT, KS, kKs, 7, kGuh>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, S, frag_out, io, s); return;
            case 8: launch_gemm_spec<kFp8, RT, KS, kKs, 8, kGuh>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, S, frag_out, io, s); return;
            default: break;
            }
            // T = 9..16 (batch steps of up to 16 rows): the 16-wave splits
            if constexpr (KS == 16) {
#define RL_T16(TN)                                                                                                      case TN:                                                                                                                launch_gemm_spec<kFp8, RT, KS, kKs, TN, kGuh>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, S,                                                        frag_out, io, s);                                                   return;
                switch (T) {
                    RL_T16(9) RL_T16(10) RL_T16(11) RL_T16(12) RL_T16(13) RL_T16(14) RL_T16(15) RL_T16(16)
                default: break;
                }
#undef RL_T16
            }
        }
    }
    RL_REQUIRE(T <= 8, RL_ERR_UNSUPPORTED, "gemm: more than 8 rows need the batch work split");
    launch_gemm_tt<kFp8, RT, KS, D, kKs, 0, -1, -1, kGuh>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, S,
                                                         frag_out, io, s);
}

// m = rows of the (tiled) weight; outputs go to Y[t * ldy + row] for row < m_valid
// (for kSwiGLU, output rows are m/2 and m_valid bounds those).
template <bool kFp8>
void launch_gemm(const void* W, const float* tscale, const void* frag, float* Y, int m, int n, int T, int epilogue,
                 int ldy, int m_valid, hipStream_t s, int S = 1, void* frag_out = nullptr,
                 const NormIO* norm = nullptr) {
    const NormIO io = norm ? *norm : NormIO{};
    RL_REQUIRE(m > 0 && n > 0, RL_ERR_RANGE, "gemm: empty shape");
    RL_REQUIRE(T >= 1 && T <= 16, RL_ERR_RANGE, "gemm: T must be in 1..16");
    RL_REQUIRE(W && frag && (Y || frag_out), RL_ERR_RANGE, "gemm: null pointer");
    RL_REQUIRE(!frag_out || epilogue == kSwiGLU || epilogue == kSwiGLUH || epilogue == kAddNorm, RL_ERR_RANGE,
               "gemm: fragment output only with the SwiGLU / add-norm epilogues");
    RL_REQUIRE(epilogue != kAddNorm || (Y && frag_out && io.gamma_out && io.ss_out && S == 1), RL_ERR_RANGE,
               "gemm add-norm: needs Y, fragment output, gamma and the sum-of-squares output, no split");
    RL_REQUIRE(!io.ss_in || (io.groups_in >= 1 && io.groups_in <= 256 && io.n_norm > 0), RL_ERR_RANGE,
               "gemm: folded RMSNorm needs 1..256 partial groups");
    RL_REQUIRE(!frag_out || frag_out != frag, RL_ERR_RANGE, "gemm: fragment output must not alias the input");
    RL_REQUIRE(!kFp8 || tscale, RL_ERR_RANGE, "gemm: FP8 weights need tile scales");
    const int n_kb = n_kb_of(n);
    const int m_tiles = m_tiles_of(m);
    if (epilogue == kSwiGLUH) {
        // half-tile gate/up: one row tile per 16-wave workgroup (34816 x 5120: 27.5 us
        // vs 29.6 us for the whole-tile interleave at two tiles per workgroup)
        RL_REQUIRE(m % 16 == 0 && S == 1 && !io.kss && !io.xpart, RL_ERR_RANGE,
                   "gemm swiglu (half tiles): rows a multiple of 16, no split or block scale");
        const int rtw = T > 4 ? rt_wide() : 1;
        if (T > 8 && rt_batch() == 4)
            launch_gemm_cfg<kFp8, 4, 16, 1, false, true>(W, tscale, frag, Y, m, n_kb, T, kSwiGLU, ldy, m_valid, S,
                                                         frag_out, io, s);
        else if (T > 8)
            launch_gemm_cfg<kFp8, 2, 16, 1, false, true>(W, tscale, frag, Y, m, n_kb, T, kSwiGLU, ldy, m_valid, S,
                                                         frag_out, io, s);
        else if (rtw == 4)
            launch_gemm_cfg<kFp8, 4, 16, 1, false, true>(W, tscale, frag, Y, m, n_kb, T, kSwiGLU, ldy, m_valid, S,
                                                         frag_out, io, s);
        else if (rtw == 2)
            launch_gemm_cfg<kFp8, 2, 16, 1, false, true>(W, tscale, frag, Y, m, n_kb, T, kSwiGLU, ldy, m_valid, S,
                                                         frag_out, io, s);
        else
            launch_gemm_cfg<kFp8, 1, 16, 1, false, true>(W, tscale, frag, Y, m, n_kb, T, kSwiGLU, ldy, m_valid, S,
                                                         frag_out, io, s);
        check_launch("gemm_frag_kernel");
        return;
    }
    if (epilogue == kSwiGLU)
        RL_REQUIRE(m % 32 == 0, RL_ERR_RANGE, "gemm swiglu: interleaved rows must be a multiple of 32");
    RL_REQUIRE(S >= 1 && (S == 1 || epilogue == kPartial), RL_ERR_RANGE, "gemm: split-K needs the partial epilogue");
    // FP8 launches are one round of workgroups (all resident); depth 1 (loads
    // scheduled by the compiler) measured best there: 19.3 us vs 24.2 us (depth 2)
    // for 16480x5120 with weights cold in HBM.  BF16 (lm_head: many rounds) keeps
    // depth 2 (6.4 TB/s).
    GemmCfg c{2, (m_tiles + 1) / 2 * S >= 256 ? 8 : 16, kFp8 ? 1 : 2};
    if (kFp8 && bperm_enabled() && S == 1) {
        // compile-time-T kernels, measured cold (T = 1 / 4): stores one row tile per
        // 16-wave workgroup (16480 x 5120: 15.6 / 17.7 us vs 17.7 / 18.7 with two row
        // tiles per 8 waves), SwiGLU two (gate and up) per 16 waves (34816 x 5120:
        // 29.6 / 30.2 us vs 30.8 / 31.1)
        if (epilogue == kStore || epilogue == kAdd) c = GemmCfg{T > 8 ? 2 : T > 4 ? rt_wide() : 1, 16, 1};
        if (epilogue == kSwiGLU) c = GemmCfg{2, 16, 1};
    }
    // BF16 stores (the lm_head: 248320 x 5120, 2.54 GB) take the same split: 370 / 360 us
    // at T = 1 / 4 against 392 / 398 us for two row tiles per 8 waves at depth 2
    // (weights in HBM; every T uses this split, so rows of a verify or batch step
    // equal the T = 1 rows bit for bit)
    if (!kFp8 && bperm_enabled() && S == 1 && (epilogue == kStore || epilogue == kAdd))
        c = GemmCfg{T > 8 ? 2 : T > 4 ? rt_wide() : 1, 16, 1};
    if (g_force.rt) c = g_force;
    if (epilogue == kSwiGLU && c.rt == 1) c.rt = 2;
    // residual GEMMs (m = hidden: 160 groups): 8 waves measured faster than 16 there
    // (5120x17408: 21.2 vs 22.8 us cold); the sum-of-squares groups are 2 row tiles
    // At T = 1 (permuted-B kernels) 16 waves: 5120 x 17408 19.1 vs 20.1 us, 5120 x 6144
    // 8.2 vs 8.4 us cold; at T = 4 they are slower (24.6 vs 22.3 us).  Both splits
    // add the same 16 partial sums in the same order (gemm_frag_kernel's KP), so a
    // T = 1 row equals the same row of a verify or batch step bit for bit.
    if (epilogue == kAddNorm && !g_force.rt)
        c = GemmCfg{2, kFp8 && bperm_enabled() && T == 1 && addnorm16_enabled() ? 16 : 8, kFp8 ? 1 : 2};
    // 9..16 rows: the compile-time-T kernels with 16 waves at depth 1 (the same K split
    // as T = 1, so a batch row equals the single-sequence row bit for bit).  The
    // activation fragments of 16 tokens (8 KiB per column block) outweigh a row tile's
    // weights (2 KiB), so stores take several row tiles per workgroup: at T = 16
    // 34816 x 5120 SwiGLU 77.8 / 57.7 / 50.5 us with one / two / four, 14336 x 5120
    // 26.6 / 21.0 us with two / four
    if (T > 8) {
        RL_REQUIRE(bperm_enabled() && !g_force.rt, RL_ERR_UNSUPPORTED,
                   "gemm: more than 8 rows need the default work splits");
        c = GemmCfg{epilogue == kStore || epilogue == kAdd ? rt_batch() : 2, 16, 1};
    }
    if (epilogue == kAddNorm)
        RL_REQUIRE(c.rt * T * kTileRows <= 64 * c.ks, RL_ERR_RANGE, "gemm add-norm: a thread per output item");
    if (io.kss) {
        // folded gated norm (out_proj): the residual configuration only
        RL_REQUIRE(!io.ss_in && io.kss_n > 0 && S == 1, RL_ERR_RANGE, "gemm: bad block input scale");
        RL_REQUIRE(!g_force.rt, RL_ERR_UNSUPPORTED, "gemm: block input scale uses the residual work split");
        if (c.ks == 16)
            launch_gemm_cfg<kFp8, 2, 16, 1, true>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, S,
                                                  frag_out, io, s);
        else
            launch_gemm_cfg<kFp8, 2, 8, 1, true>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, S,
                                                 frag_out, io, s);
        check_launch("gemm_frag_kernel");
        return;
    }
    if (io.xpart) {
        // the rows from x_tile0 on as K-slices run by the first workgroups
        // (the store work split: two row tiles per 8 waves, or one per 16 waves with
        // the permuted-B kernels; one column block per wave in a slice)
        RL_REQUIRE(epilogue == kStore && S == 1 && !g_force.rt && !io.kss, RL_ERR_RANGE,
                   "gemm: overflow slices need a plain store launch");
        const int rpw = gemm_store_rows_per_wg(), waves = gemm_store_waves();
        RL_REQUIRE(kFp8 || rpw == 2, RL_ERR_UNSUPPORTED, "gemm: overflow slices with BF16 need the paired split");
        RL_REQUIRE(io.x_tile0 > 0 && io.x_tile0 % rpw == 0 && io.x_tile0 < m_tiles && io.x_slices >= 1 &&
                       io.x_rows == (m_tiles - io.x_tile0) * kTileRows &&
                       (n_kb + io.x_slices - 1) / io.x_slices <= waves &&
                       (m_tiles - io.x_tile0) * io.x_slices <= io.x_tile0 / rpw,
                   RL_ERR_RANGE, "gemm: bad overflow slices");
        if (rpw == 2)
            launch_gemm_cfg<kFp8, 2, 8, 1>(W, tscale, frag, Y, io.x_tile0 * kTileRows, n_kb, T, epilogue, ldy,
                                           std::min(m_valid, io.x_tile0 * kTileRows), S, frag_out, io, s);
        else
            launch_gemm_cfg<kFp8, 1, 16, 1>(W, tscale, frag, Y, io.x_tile0 * kTileRows, n_kb, T, epilogue, ldy,
                                            std::min(m_valid, io.x_tile0 * kTileRows), S, frag_out, io, s);
        check_launch("gemm_frag_kernel");
        return;
    }
#define RL_GEMM_CASE(R, K, DD)                                                            \
    if (c.rt == R && c.ks == K && c.d == DD) {                                            \
        launch_gemm_cfg<kFp8, R, K, DD>(W, tscale, frag, Y, m, n_kb, T, epilogue, ldy, m_valid, S, frag_out, io, s); \
        check_launch("gemm_frag_kernel");                                                 \
        return;                                                                           \
    }
    RL_GEMM_CASE(2, 8, 1) RL_GEMM_CASE(2, 16, 1) RL_GEMM_CASE(2, 8, 2) RL_GEMM_CASE(2, 16, 2)
    RL_GEMM_CASE(2, 4, 1) RL_GEMM_CASE(2, 4, 2) RL_GEMM_CASE(1, 8, 1) RL_GEMM_CASE(1, 16, 1)
    RL_GEMM_CASE(4, 16, 1)
#undef RL_GEMM_CASE
    throw Error(RL_ERR_UNSUPPORTED, "gemm: unsupported work split");
}

void launch_pack_act(const float* X, void* frag, int n, int T, hipStream_t s) {
    RL_REQUIRE(n > 0 && T >= 1 && T <= 65536, RL_ERR_RANGE, "pack_act: bad shape");
    const int n_kb = n_kb_of(n);
    const int total = n_kb * 16 * T;
    hipLaunchKernelGGL(pack_act_kernel, dim3((total + 255) / 256), dim3(256), 0, s, X, static_cast<i32x4*>(frag), n,
                       n_kb, T);
    check_launch("pack_act_kernel");
}

}  // namespace

namespace rl {
size_t act_frag_bytes(int n, int T) { return static_cast<size_t>(n_kb_of(n)) * 16 * 2 * T * 16; }
// Internal entry points shared with the engine.
void gemm_fp8_frag(const uint8_t* W, const float* ts, const void* frag, float* Y, int m, int n, int T, int epi,
                   int ldy, int m_valid, hipStream_t s, int S, void* frag_out, const NormIO* norm) {
    launch_gemm<true>(W, ts, frag, Y, m, n, T, epi, ldy, m_valid, s, S, frag_out, norm);
}
void gemm_bf16_frag(const uint16_t* W, const void* frag, float* Y, int m, int n, int T, int epi, int ldy, int m_valid,
                    hipStream_t s, int S, void* frag_out, const NormIO* norm) {
    launch_gemm<false>(W, nullptr, frag, Y, m, n, T, epi, ldy, m_valid, s, S, frag_out, norm);
}
int add_norm_groups(int m) { return (m_tiles_of(m) + 1) / 2; }
int norm_group_rows() { return 2 * kTileRows; }
static bool store_pairs_rows() { return !(bperm_enabled() && !g_force.rt); }
int gemm_store_rows_per_wg() { return store_pairs_rows() ? 2 : 1; }
int gemm_store_waves() { return store_pairs_rows() ? 8 : 16; }
int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    RL_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) RL_HIP(hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev));
    return cus[dev];
}
void pack_fp8_rows(const uint8_t* w, const float* scale, uint8_t* dst, float* tscale, int m, int n, int rt_stride,
                   int rt_offset, hipStream_t s) {
    const size_t total = static_cast<size_t>(m_tiles_of(m)) * n_kb_of(n) * 64;
    hipLaunchKernelGGL(pack_fp8_kernel, dim3((total + 255) / 256), dim3(256), 0, s, w, scale, dst, tscale, m, n,
                       n_kb_of(n), rt_stride, rt_offset);
    check_launch("pack_fp8_kernel");
}
void pack_fp8_gate_up(const uint8_t* gw, const float* gs, const uint8_t* uw, const float* us, uint8_t* dst,
                      float* tscale, int I, int n, hipStream_t s) {
    RL_REQUIRE(I > 0 && I % 8 == 0 && n > 0, RL_ERR_RANGE, "pack gate/up: I must be a positive multiple of 8");
    const size_t total = static_cast<size_t>(I / 8) * n_kb_of(n) * 64;
    for (int half = 0; half < 2; ++half)
        hipLaunchKernelGGL(pack_fp8_guh_kernel, dim3((total + 255) / 256), dim3(256), 0, s, half ? uw : gw,
                           half ? us : gs, dst, tscale, I, n, n_kb_of(n), half);
    check_launch("pack_fp8_guh_kernel");
}
void pack_bf16_gate_up(const uint16_t* gw, const uint16_t* uw, uint16_t* dst, int I, int n, hipStream_t s) {
    RL_REQUIRE(I > 0 && I % 8 == 0 && n > 0, RL_ERR_RANGE, "pack gate/up: I must be a positive multiple of 8");
    const size_t total = static_cast<size_t>(I / 8) * n_kb_of(n) * 64;
    for (int half = 0; half < 2; ++half)
        hipLaunchKernelGGL(pack_bf16_guh_kernel, dim3((total + 255) / 256), dim3(256), 0, s, half ? uw : gw, dst, I,
                           n, n_kb_of(n), half);
    check_launch("pack_bf16_guh_kernel");
}
void pack_bf16_rows(const uint16_t* w, uint16_t* dst, int m, int n, int rt_stride, int rt_offset, hipStream_t s) {
    const size_t total = static_cast<size_t>(m_tiles_of(m)) * n_kb_of(n) * 64;
    hipLaunchKernelGGL(pack_bf16_kernel, dim3((total + 255) / 256), dim3(256), 0, s, w, dst, m, n, n_kb_of(n),
                       rt_stride, rt_offset);
    check_launch("pack_bf16_kernel");
}
void pack_act(const float* X, void* frag, int n, int T, hipStream_t s) { launch_pack_act(X, frag, n, T, s); }
}  // namespace rl

using namespace rl;

extern "C" {

int rl_hip_set_gemm_config(int row_tiles, int k_waves, int depth) {
    g_force = GemmCfg{row_tiles, k_waves, depth > 0 ? depth : 2};
    return RL_OK;
}


size_t rl_hip_fp8_packed_bytes(int m, int n) { return static_cast<size_t>(m_tiles_of(m)) * n_kb_of(n) * 2048; }
size_t rl_hip_fp8_tile_scales(int m, int n) { return static_cast<size_t>(m_tiles_of(m)) * n_kb_of(n); }
size_t rl_hip_bf16_packed_bytes(int m, int n) { return static_cast<size_t>(m_tiles_of(m)) * n_kb_of(n) * 4096; }
size_t rl_hip_act_frag_bytes(int n, int T) { return static_cast<size_t>(n_kb_of(n)) * 16 * 2 * T * 16; }

int rl_hip_pack_fp8(const uint8_t* w, const float* scale, uint8_t* w_tiled, float* tile_scale, int m, int n,
                    void* stream) {
    return guard([&] {
        RL_REQUIRE(m > 0 && n > 0 && w && scale && w_tiled && tile_scale, RL_ERR_RANGE, "pack_fp8: bad args");
        rl::pack_fp8_rows(w, scale, w_tiled, tile_scale, m, n, 1, 0, S(stream));
    });
}

size_t rl_hip_fp8_gate_up_tile_scales(int I, int n) {
    return I > 0 && n > 0 ? static_cast<size_t>((I + 7) / 8) * n_kb_of(n) * 2 : 0;
}

int rl_hip_pack_fp8_gate_up(const uint8_t* gate_w, const float* gate_scale, const uint8_t* up_w, const float* up_scale,
                            uint8_t* w_tiled, float* tile_scale, int I, int n, void* stream) {
    return guard([&] {
        RL_REQUIRE(gate_w && gate_scale && up_w && up_scale && w_tiled && tile_scale, RL_ERR_RANGE,
                   "pack_fp8_gate_up: null pointer");
        rl::pack_fp8_gate_up(gate_w, gate_scale, up_w, up_scale, w_tiled, tile_scale, I, n, S(stream));
    });
}

int rl_hip_pack_bf16_gate_up(const uint16_t* gate_w, const uint16_t* up_w, uint16_t* w_tiled, int I, int n,
                             void* stream) {
    return guard([&] {
        RL_REQUIRE(gate_w && up_w && w_tiled, RL_ERR_RANGE, "pack_bf16_gate_up: null pointer");
        rl::pack_bf16_gate_up(gate_w, up_w, w_tiled, I, n, S(stream));
    });
}

int rl_hip_pack_bf16(const uint16_t* w, uint16_t* w_tiled, int m, int n, void* stream) {
    return guard([&] {
        RL_REQUIRE(m > 0 && n > 0 && w && w_tiled, RL_ERR_RANGE, "pack_bf16: bad args");
        rl::pack_bf16_rows(w, w_tiled, m, n, 1, 0, S(stream));
    });
}

int rl_hip_pack_act(const float* X, void* frag, int n, int T, void* stream) {
    return guard([&] { launch_pack_act(X, frag, n, T, S(stream)); });
}

int rl_hip_gemm_fp8_frag(const uint8_t* w_tiled, const float* tile_scale, const void* frag, float* Y, int m, int n,
                         int T, int accumulate, void* stream) {
    return guard([&] { launch_gemm<true>(w_tiled, tile_scale, frag, Y, m, n, T, accumulate ? kAdd : kStore, m, m, S(stream)); });
}

int rl_hip_gemm_bf16_frag(const uint16_t* w_tiled, const void* frag, float* Y, int m, int n, int T, int accumulate,
                          void* stream) {
    return guard([&] { launch_gemm<false>(w_tiled, nullptr, frag, Y, m, n, T, accumulate ? kAdd : kStore, m, m, S(stream)); });
}

int rl_hip_gemm_fp8(const uint8_t* w_tiled, const float* tile_scale, const float* X, float* Y, void* frag_scratch,
                    int m, int n, int T, void* stream) {
    return guard([&] {
        launch_pack_act(X, frag_scratch, n, T, S(stream));
        launch_gemm<true>(w_tiled, tile_scale, frag_scratch, Y, m, n, T, kStore, m, m, S(stream));
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
