// attn.hip -- gated GQA attention decode over an fp16 KV cache, T = 1..4 tokens.
//
// Reference semantics (CPU, src/kernels/ops_fused.cpp:137-184; src/runtime/
// session.cpp:271-323): per head [q | gate] split of the q projection (hd >= 64),
// Qwen RMSNorm with (1 + gamma) on q and k heads (ops.cpp:107-127), partial RoPE
// rotate-half over the first rotary_dim dims (ops.cpp:470-493), append K/V at
// pos, softmax(q.k / sqrt(hd)) over positions 0..pos (ops.cpp:575-605), output
// times sigmoid(gate).  The cache holds K (after RoPE) and V rounded to fp16 with
// round-to-nearest-even, as the reference's GPU engine keeps it
// (src/kernels/cuda/cuda_engine.cu:20122-20123).
//
// Kernels:
//  qk_prep     one wave per (head, token): norm + RoPE + fp16 cache write; q is
//              written as fp16 hi + lo fragments (hi + lo carries ~22 bits).
//  attn_part   one workgroup per (kv head, 256-position chunk), 4 waves.  Scores
//              S^T = K . Q^T on v_mfma_f32_16x16x32_f16 with A = K rows straight
//              from the cache and B = the fragments of all G*T query rows of the
//              kv group (hi and lo in two column tiles, summed per lane); chunk
//              softmax; P (fp16) staged in LDS by position; O^T = V^T . P^T.  Every
//              K and V byte of the chunk is read once for all heads and tokens.
//  attn_comb   merges the chunk partials (max, sum, O) per query row, applies
//              sigmoid(gate) and writes fp32 and/or the o_proj GEMM fragments.
//
// Cache layouts: K and V fp16 [n_kv][ctx * hd] in MFMA fragment order (k_off / v_off
// below); ctx % 256 == 0.
#include "internal.h"

using namespace rl;

namespace {

constexpr int kHD = 256;
constexpr int kChunk = 256;
constexpr int kMaxPairs = 32;  // G * T query rows per kv head (<= 2 tiles of 16)
#ifndef ATTN_UNROLL
#define ATTN_UNROLL 2
#endif

typedef _Float16 half4 __attribute__((ext_vector_type(4)));

__device__ inline float sigmoid_f(float x) { return 1.f / (1.f + expf(-x)); }

struct AttnArgs {
    const float* Y;  // fused q(+gate)/k/v projection output, [T][ld_y]
    int ld_y;
    const float* q_norm;
    const float* k_norm;
    uint16_t* kc;  // [nkv][ctx][hd]
    uint16_t* vt;  // [nkv][hd][ctx]
    int ctx;
    const int* pos;  // device: position of token 0
    int T, nq, nkv, G, rot;
    int t_off, T_out;  // outputs: token t goes to column t_off + t of T_out
    float theta, eps;
    i32x4* qf;     // [nkv][8 s][4 g][2*PT ct][16 col] x 16 B
    float* part_o; // [nkv][chunks][kMaxPairs][hd]
    float* part_m; // [nkv][chunks][kMaxPairs]
    float* part_l;
    int max_chunks;
    float* out;     // optional [T][nq*hd]
    i32x4* frag;    // optional o_proj fragments (n = nq*hd)
    // batch decode: nb sequences ("slots") in one launch set.  Slot b's token t is
    // row b*T + t of Y and output column t_off + b*T + t; its cache, position and
    // workspace (qf, partials) sit kv_bstride elements, pos_stride ints and ws_slot
    // bytes after slot b-1's.
    int nb;
    size_t kv_bstride;
    int pos_stride;
    size_t ws_slot;
};

// Arguments of slot b (uniform per workgroup: the offsets stay in scalar registers).
__device__ inline void to_slot(AttnArgs& p, int b) {
    p.kc += b * p.kv_bstride;
    p.vt += b * p.kv_bstride;
    p.pos += b * p.pos_stride;
    p.Y += static_cast<size_t>(b) * p.T * p.ld_y;
    p.qf = reinterpret_cast<i32x4*>(reinterpret_cast<char*>(p.qf) + b * p.ws_slot);
    p.part_o = reinterpret_cast<float*>(reinterpret_cast<char*>(p.part_o) + b * p.ws_slot);
    p.part_m = reinterpret_cast<float*>(reinterpret_cast<char*>(p.part_m) + b * p.ws_slot);
    p.part_l = reinterpret_cast<float*>(reinterpret_cast<char*>(p.part_l) + b * p.ws_slot);
    p.t_off += b * p.T;
}

__host__ __device__ inline int pair_tiles(int G, int T) { return (G * T + 15) / 16; }

// Cache layouts (per kv head, ctx * 256 fp16), in MFMA fragment order so that every
// wave load is one contiguous 1 KiB run (lane l reads 16 B at 16 l), and the 4 waves
// of a chunk workgroup read adjacent runs at every step (one 16 KiB stretch):
//   K: [pos/256][d/32][(pos/16)%16][(d/8)%4][pos%16][d%8] -- A operand of S^T = K . Q^T
//   V: [pos/32][d/16][(pos/8)%4][d%16][pos%8]              -- A operand of O^T = V^T . P^T
__host__ __device__ inline size_t k_off(int pos, int d) {
    return ((((static_cast<size_t>(pos >> 8) * 8 + (d >> 5)) * 16 + ((pos >> 4) & 15)) * 4 + ((d >> 3) & 3)) * 16 +
            (pos & 15)) * 8 +
           (d & 7);
}
__host__ __device__ inline size_t v_off(int pos, int d) {
    return (((static_cast<size_t>(pos >> 5) * 16 + (d >> 4)) * 4 + ((pos >> 3) & 3)) * 16 + (d & 15)) * 8 + (pos & 7);
}

// grid (nq + 2*nkv, T, slots), 64 threads.  Heads [0,nq): q; [nq, nq+nkv): k; then v.
__global__ __launch_bounds__(64) void qk_prep_kernel(AttnArgs p) {
    __shared__ float vec[kHD];
    to_slot(p, blockIdx.z);
    const int head = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int pos = *p.pos + t;
    const float* row = p.Y + static_cast<size_t>(t) * p.ld_y;
    const int qcols = p.nq * kHD * 2;
    if (head >= p.nq + p.nkv) {  // v: straight to the transposed cache
        const int kv = head - p.nq - p.nkv;
        const float* src = row + qcols + p.nkv * kHD + kv * kHD;
        uint16_t* vb = p.vt + static_cast<size_t>(kv) * p.ctx * kHD;
        for (int d = lane; d < kHD; d += 64) vb[v_off(pos, d)] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(src[d]));
        return;
    }
    const bool is_q = head < p.nq;
    const float* src = is_q ? row + static_cast<size_t>(head) * 2 * kHD : row + qcols + (head - p.nq) * kHD;
    const float* gam = is_q ? p.q_norm : p.k_norm;
    double ss = 0.0;
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        x[r] = src[lane + 64 * r];
        ss += static_cast<double>(x[r]) * x[r];
    }
    ss = wave_sum_d(ss);
    const float inv = 1.f / sqrtf(static_cast<float>(ss / kHD) + p.eps);
#pragma unroll
    for (int r = 0; r < 4; ++r) vec[lane + 64 * r] = x[r] * inv * (gam ? 1.f + gam[lane + 64 * r] : 1.f);
    __syncthreads();
    const int half = p.rot / 2;
    for (int i = lane; i < half; i += 64) {
        const float freq = 1.f / powf(p.theta, static_cast<float>(i) / static_cast<float>(half));
        const float ang = static_cast<float>(pos) * freq;
        const float c = cosf(ang), s = sinf(ang);
        const float x0 = vec[i], x1 = vec[i + half];
        vec[i] = x0 * c - x1 * s;
        vec[i + half] = x0 * s + x1 * c;
    }
    __syncthreads();
    if (!is_q) {
        const int kv = head - p.nq;
        uint16_t* kb = p.kc + static_cast<size_t>(kv) * p.ctx * kHD;
        for (int d = lane; d < kHD; d += 64) kb[k_off(pos, d)] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(vec[d]));
        return;
    }
    // q -> fp16 hi/lo fragments: dim d = 32 s + 8 g + e; pair k = t*G + head%G
    const int kv = head / p.G;
    const int k = t * p.G + head % p.G;
    const int PT = pair_tiles(p.G, p.T);
    const int pt = k >> 4, col = k & 15;
    _Float16* qf = reinterpret_cast<_Float16*>(p.qf);
    for (int d = lane; d < kHD; d += 64) {
        const int s = d >> 5, g = (d >> 3) & 3, e = d & 7;
        const _Float16 hi = static_cast<_Float16>(vec[d]);
        const _Float16 lo = static_cast<_Float16>(vec[d] - static_cast<float>(hi));
        const size_t base = (((static_cast<size_t>(kv) * 8 + s) * 4 + g) * (2 * PT));
        qf[((base + 2 * pt) * 16 + col) * 8 + e] = hi;
        qf[((base + 2 * pt + 1) * 16 + col) * 8 + e] = lo;
    }
}

union H8 {
    f16x8 v;
    i32x4 i;
    _Float16 h[8];
};

template <int PT>
__global__ __launch_bounds__(256) void attn_part_kernel(AttnArgs p) {
    // chunk-major dispatch order (kv head fastest, then slot): the chunks past the
    // current position (early exit) come last, so the active workgroups spread
    // evenly over the CUs
    const int kv = blockIdx.x % p.nkv;
    const int chunk = blockIdx.x / p.nkv / p.nb;
    to_slot(p, (blockIdx.x / p.nkv) % p.nb);
    const int p0 = *p.pos;
    const int L = p0 + p.T;  // keys 0 .. L-1 exist after this step's writes
    const int c0 = chunk * kChunk;
    if (c0 >= L) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, col = lane & 15;
    const int npairs = p.G * p.T;
    const float scale = 1.f / sqrtf(static_cast<float>(kHD));

    // [u][pair tile][pair col][32 positions + 8 pad]: the 80-byte row stride puts the
    // 16 pair columns of a write instruction on distinct banks
    __shared__ _Float16 P_lds[8][PT][16][40];
    __shared__ float max_s[4][PT][16];
    __shared__ float sum_s[4][PT][16];

    // ---- scores for positions c0 + 64*wave + 16*ptile + row
    // S^T = K . (Q_hi + Q_lo).  One pair tile: hi and lo in separate accumulators
    // (independent MFMA chains); two pair tiles: both parts accumulate into the
    // same tile (half the accumulator registers, keeping 4 waves per SIMD).
    constexpr int NA = PT == 1 ? 2 : 1;
    f32x4 acc[4][PT * NA];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < PT * NA; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint16_t* kbase = p.kc + static_cast<size_t>(kv) * p.ctx * kHD;
    const i32x4* qbase = p.qf + static_cast<size_t>(kv) * 8 * 4 * (2 * PT) * 16;
#pragma unroll ATTN_UNROLL
    for (int s = 0; s < 8; ++s) {
        H8 bq[2 * PT];
#pragma unroll
        for (int ct = 0; ct < 2 * PT; ++ct) bq[ct].i = qbase[((s * 4 + g) * (2 * PT) + ct) * 16 + col];
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) {
            // tiles past the last key (masked) re-read the chunk's first tile, which
            // is cached: the partial last chunk costs about what it holds in HBM reads
            const int ptile = c0 + 16 * (4 * wave + pt) < L ? 4 * wave + pt : 0;
            H8 a;
            a.i = reinterpret_cast<const i32x4*>(kbase + ((static_cast<size_t>(chunk) * 8 + s) * 16 + ptile) * 512)[lane];
#pragma unroll
            for (int q = 0; q < PT; ++q) {
                acc[pt][NA * q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.v, bq[2 * q].v, acc[pt][NA * q], 0, 0, 0);
                acc[pt][NA * q + NA - 1] =
                    __builtin_amdgcn_mfma_f32_16x16x32_f16(a.v, bq[2 * q + 1].v, acc[pt][NA * q + NA - 1], 0, 0, 0);
            }
        }
    }

    // ---- V of the chunk's first 64 positions requested now, so the loads are in flight
    // across the softmax (the V loop below keeps two steps ahead)
    const uint16_t* vbase = p.vt + static_cast<size_t>(kv) * kHD * p.ctx;  // fragment-ordered V
    H8 va[3][4];
    auto vload = [&](int u, H8* dst) {
        // positions past the last key have P = 0: their group re-reads the first one
        const int grp = 32 * ((c0 >> 5) + u) < L ? (c0 >> 5) + u : (c0 >> 5);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
            dst[dt].i = reinterpret_cast<const i32x4*>(vbase + (static_cast<size_t>(grp) * 16 + 4 * wave + dt) * 512)[lane];
    };
    vload(0, va[0]);
    vload(1, va[1]);

    // ---- masked scores, chunk max (lane: query row `col` of pair tile, 4 rows each)
    float sc[4][PT][4];
    float mx[PT];
#pragma unroll
    for (int q = 0; q < PT; ++q) mx[q] = -INFINITY;
#pragma unroll
    for (int pt = 0; pt < 4; ++pt)
#pragma unroll
        for (int q = 0; q < PT; ++q) {
            const int k = q * 16 + col;
            const int t = k / p.G;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int pos = c0 + 64 * wave + 16 * pt + 4 * g + v;
                const bool ok = k < npairs && pos <= p0 + t;
                const float val = (NA == 2 ? acc[pt][2 * q][v] + acc[pt][2 * q + 1][v] : acc[pt][q][v]) * scale;
                sc[pt][q][v] = ok ? val : -INFINITY;
                mx[q] = fmaxf(mx[q], sc[pt][q][v]);
            }
        }
#pragma unroll
    for (int q = 0; q < PT; ++q) {
        mx[q] = fmaxf(mx[q], __shfl_xor(mx[q], 16, 64));
        mx[q] = fmaxf(mx[q], __shfl_xor(mx[q], 32, 64));
        if (g == 0) max_s[wave][q][col] = mx[q];
    }
    __syncthreads();
    float M[PT], sum[PT];
#pragma unroll
    for (int q = 0; q < PT; ++q) {
        M[q] = fmaxf(fmaxf(max_s[0][q][col], max_s[1][q][col]), fmaxf(max_s[2][q][col], max_s[3][q][col]));
        sum[q] = 0.f;
    }
    // P = exp(s - M) (0 where masked), staged as fp16 by chunk position:
    // P_lds[u][q][pair col][j] holds position 32u + j
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) {
#pragma unroll
        for (int q = 0; q < PT; ++q) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int pl = 64 * wave + 16 * pt + 4 * g + v;
                const float e = M[q] == -INFINITY ? 0.f : expf(sc[pt][q][v] - M[q]);
                sum[q] += e;
                P_lds[pl >> 5][q][col][pl & 31] = static_cast<_Float16>(e);
            }
        }
    }
#pragma unroll
    for (int q = 0; q < PT; ++q) {
        sum[q] += __shfl_xor(sum[q], 16, 64);
        sum[q] += __shfl_xor(sum[q], 32, 64);
        if (g == 0) sum_s[wave][q][col] = sum[q];
    }
    __syncthreads();

    // ---- O^T[d][pair] for d in [64*wave, 64*wave+64)
    f32x4 o[4][PT];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int q = 0; q < PT; ++q) o[a][q] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        if (u + 2 < 8) vload(u + 2, va[(u + 2) % 3]);
        H8 bp[PT];
#pragma unroll
        for (int q = 0; q < PT; ++q) bp[q].i = *reinterpret_cast<const i32x4*>(&P_lds[u][q][col][8 * g]);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int q = 0; q < PT; ++q)
                o[dt][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[u % 3][dt].v, bp[q].v, o[dt][q], 0, 0, 0);
    }

    // ---- partials: O^T lane (pair col, g) holds d = 64*wave + 16*dt + 4g + v
    const size_t cbase = static_cast<size_t>(kv) * p.max_chunks + chunk;
#pragma unroll
    for (int q = 0; q < PT; ++q) {
        const int k = q * 16 + col;
        if (k >= npairs) continue;
        float* dst = p.part_o + (cbase * kMaxPairs + k) * kHD;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
            *reinterpret_cast<float4*>(dst + 64 * wave + 16 * dt + 4 * g) =
                make_float4(o[dt][q][0], o[dt][q][1], o[dt][q][2], o[dt][q][3]);
        if (wave == 0 && g == 0) {
            p.part_m[cbase * kMaxPairs + k] = M[q];
            p.part_l[cbase * kMaxPairs + k] = sum_s[0][q][col] + sum_s[1][q][col] + sum_s[2][q][col] + sum_s[3][q][col];
        }
    }
}

// grid (G*T pairs, nkv, slots * hd/64), 1024 threads = 16 chunk groups x 64 dims
// (at 32K context each thread's chunk loop is 8 loads, issued together).
// Chunk weights w_c = exp(m_c - M) are computed once into LDS; each thread sums
// its chunk group's O_c[d] * w_c, the 16 groups are added in a fixed order.
constexpr int kMaxChunksLds = 4096;  // 1M positions

constexpr int kCombG = 16;  // chunk groups (waves) per workgroup
__global__ __launch_bounds__(64 * kCombG) void attn_comb_kernel(AttnArgs p) {
    const int k = blockIdx.x, kv = blockIdx.y;
    const int dz = blockIdx.z % (kHD / 64);
    to_slot(p, blockIdx.z / (kHD / 64));
    const int tid = threadIdx.x, q = tid >> 6, dl = tid & 63;
    const int d = dz * 64 + dl;
    const int t = k / p.G;
    const int h = kv * p.G + k % p.G;
    const int L = *p.pos + p.T;
    const int nch = (L + kChunk - 1) / kChunk;
    const size_t base = static_cast<size_t>(kv) * p.max_chunks;
    __shared__ float w_s[kMaxChunksLds];
    __shared__ float red[kCombG][64];
    __shared__ float sh[2 * kCombG];
    // chunk max
    float mx = -INFINITY;
    for (int c = tid; c < nch; c += 64 * kCombG) mx = fmaxf(mx, p.part_m[(base + c) * kMaxPairs + k]);
    mx = wave_max(mx);
    if ((tid & 63) == 0) sh[tid >> 6] = mx;
    __syncthreads();
    float M = sh[0];
#pragma unroll
    for (int w = 1; w < kCombG; ++w) M = fmaxf(M, sh[w]);
    // weights and the softmax denominator
    float ls = 0.f;
    for (int c = tid; c < nch; c += 64 * kCombG) {
        const float m = p.part_m[(base + c) * kMaxPairs + k];
        const float w = m == -INFINITY ? 0.f : expf(m - M);
        w_s[c] = w;
        ls += p.part_l[(base + c) * kMaxPairs + k] * w;
    }
    ls = wave_sum(ls);
    __syncthreads();
    if ((tid & 63) == 0) sh[kCombG + (tid >> 6)] = ls;
    __syncthreads();
    float Ls = 0.f;
#pragma unroll
    for (int w = 0; w < kCombG; ++w) Ls += sh[kCombG + w];  // fixed order
    // weighted sum of the chunk outputs for dim d over chunks c = q (mod 4)
    float acc = 0.f;
    const float* po = p.part_o + (base * kMaxPairs + k) * kHD + d;
    const size_t cstride = static_cast<size_t>(kMaxPairs) * kHD;
#pragma unroll 8
    for (int c = q; c < nch; c += kCombG) acc += po[c * cstride] * w_s[c];
    red[q][dl] = acc;
    __syncthreads();
    if (q != 0) return;
    float os = 0.f;
#pragma unroll
    for (int w = 0; w < kCombG; ++w) os += red[w][dl];  // fixed order
    const float o = os / Ls;
    const float gate = p.Y[static_cast<size_t>(t) * p.ld_y + static_cast<size_t>(h) * 2 * kHD + kHD + d];
    const float val = o * sigmoid_f(gate);
    const int n = p.nq * kHD;
    const int j = h * kHD + d;
    if (p.out) p.out[static_cast<size_t>(p.t_off + t) * n + j] = val;
    if (p.frag) {
        red[1][dl] = val;  // wave 0 only from here on: reuse a row of red
        __builtin_amdgcn_wave_barrier();
        if (dl < 8) {  // 8 units of 8 columns cover this workgroup's 64 dims
            const int unit = (h * kHD + dz * 64) / 8 + dl;
            union {
                uint16_t hh[8];
                i32x4 v;
            } hi, mid;
#pragma unroll
            for (int e = 0; e < 8; ++e) split_bf16(red[1][8 * dl + e], hi.hh[e], mid.hh[e]);
            const int kb = unit >> 4, jb = (unit & 15) * 8;
            const int gg = jb >> 5, i = (jb >> 3) & 3;
            const size_t u = ((static_cast<size_t>(kb) * 4 + i) * 4 + gg) * (2 * p.T_out) + p.t_off + t;
            p.frag[u] = hi.v;
            p.frag[u + p.T_out] = mid.v;
        }
    }
}

// ------------------------------------------------------------------ prefill
// Prompt prefill over T tokens at positions p0 .. p0+T-1 (the reference's prefill
// attention, cuda_engine.cu:18338-18590, causal GQA over the cache): one
// workgroup per (block of 16 tokens, kv head, group of up to 3 of its G heads)
// streams the kv head's cache for those heads x 16 tokens, keeping a running max / sum / O per
// query row across 256-position chunks (online softmax) -- no partials to combine.
// Per chunk: S^T = K . Q^T (wave w: positions 64w .. 64w+63, hi and lo parts of q
// in one accumulator), the chunk max and the rescale of O through LDS, P staged
// as fp16 by position, O^T += V^T . P^T (wave w: dims 64w .. 64w+63).

// grid (nq + 2*nkv, T), 64 threads: norm + RoPE + cache write as qk_prep_kernel; q
// goes to qp[kv][tb][s][g][q][hi/lo][16 col] (16 B each; col = token % 16).
__global__ __launch_bounds__(64) void qk_prep_pf_kernel(AttnArgs p, i32x4* __restrict__ qp) {
    __shared__ float vec[kHD];
    const int head = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int pos = *p.pos + t;
    const float* row = p.Y + static_cast<size_t>(t) * p.ld_y;
    const int qcols = p.nq * kHD * 2;
    if (head >= p.nq + p.nkv) {
        const int kv = head - p.nq - p.nkv;
        const float* src = row + qcols + p.nkv * kHD + kv * kHD;
        uint16_t* vb = p.vt + static_cast<size_t>(kv) * p.ctx * kHD;
        for (int d = lane; d < kHD; d += 64) vb[v_off(pos, d)] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(src[d]));
        return;
    }
    const bool is_q = head < p.nq;
    const float* src = is_q ? row + static_cast<size_t>(head) * 2 * kHD : row + qcols + (head - p.nq) * kHD;
    const float* gam = is_q ? p.q_norm : p.k_norm;
    double ss = 0.0;
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        x[r] = src[lane + 64 * r];
        ss += static_cast<double>(x[r]) * x[r];
    }
    ss = wave_sum_d(ss);
    const float inv = 1.f / sqrtf(static_cast<float>(ss / kHD) + p.eps);
#pragma unroll
    for (int r = 0; r < 4; ++r) vec[lane + 64 * r] = x[r] * inv * (gam ? 1.f + gam[lane + 64 * r] : 1.f);
    __syncthreads();
    const int half = p.rot / 2;
    for (int i = lane; i < half; i += 64) {
        const float freq = 1.f / powf(p.theta, static_cast<float>(i) / static_cast<float>(half));
        const float ang = static_cast<float>(pos) * freq;
        const float c = cosf(ang), s = sinf(ang);
        const float x0 = vec[i], x1 = vec[i + half];
        vec[i] = x0 * c - x1 * s;
        vec[i + half] = x0 * s + x1 * c;
    }
    __syncthreads();
    if (!is_q) {
        const int kv = head - p.nq;
        uint16_t* kb = p.kc + static_cast<size_t>(kv) * p.ctx * kHD;
        for (int d = lane; d < kHD; d += 64) kb[k_off(pos, d)] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(vec[d]));
        return;
    }
    const int kv = head / p.G, q = head % p.G;
    const int ntb = (p.T + 15) / 16, tb = t >> 4, col = t & 15;
    _Float16* qh = reinterpret_cast<_Float16*>(qp);
    for (int d = lane; d < kHD; d += 64) {
        const int s = d >> 5, g = (d >> 3) & 3, e = d & 7;
        const _Float16 hi = static_cast<_Float16>(vec[d]);
        const _Float16 lo = static_cast<_Float16>(vec[d] - static_cast<float>(hi));
        const size_t base = ((((static_cast<size_t>(kv) * ntb + tb) * 8 + s) * 4 + g) * p.G + q) * 2;
        qh[((base + 0) * 16 + col) * 8 + e] = hi;
        qh[((base + 1) * 16 + col) * 8 + e] = lo;
    }
}

// grid (token blocks, nkv, G / QT), 256 threads.  QT query tiles of 16 tokens per
// workgroup: tile q = head kv*G + blockIdx.z*QT + q (at most 3, so the score and
// output accumulators stay in registers).
// Output o[t][h*hd + d] = softmax(q.K/sqrt(hd)) V * sigmoid(gate).
template <int QT>
__global__ __launch_bounds__(256) void attn_prefill_kernel(AttnArgs p, const i32x4* __restrict__ qp,
                                                            float* __restrict__ out) {
    const int tb = blockIdx.x, kv = blockIdx.y, q0 = blockIdx.z * QT;
    const int G = p.G;
    const int ntb = (p.T + 15) / 16;
    const int p0 = *p.pos;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, col = lane & 15;
    const float scale = 1.f / sqrtf(static_cast<float>(kHD));
    const int t_last = min(p.T, 16 * tb + 16) - 1;  // last token of the block
    const int L = p0 + t_last + 1;                   // keys 0 .. L-1 seen by this block
    const int tcol = 16 * tb + col;                  // token of query column `col`
    const int qpos = p0 + min(tcol, p.T - 1);        // its position (masked cols: any)

    __shared__ _Float16 P_lds[8][QT][16][40];
    __shared__ float max_s[4][QT][16];
    __shared__ float sum_s[4][QT][16];

    const uint16_t* kbase = p.kc + static_cast<size_t>(kv) * p.ctx * kHD;
    const uint16_t* vbase = p.vt + static_cast<size_t>(kv) * kHD * p.ctx;
    const i32x4* qbase = qp + (static_cast<size_t>(kv) * ntb + tb) * 8 * 4 * G * 2 * 16;

    f32x4 o[4][QT];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int q = 0; q < QT; ++q) o[a][q] = f32x4{0.f, 0.f, 0.f, 0.f};
    float Mrun[QT], Lrun[QT];
#pragma unroll
    for (int q = 0; q < QT; ++q) {
        Mrun[q] = -INFINITY;
        Lrun[q] = 0.f;
    }

    const int nch = (L + kChunk - 1) / kChunk;
    for (int chunk = 0; chunk < nch; ++chunk) {
        const int c0 = chunk * kChunk;
        f32x4 acc[4][QT];
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int q = 0; q < QT; ++q) acc[a][q] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < 8; ++s) {
            H8 a4[4];
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) {
                const int ptile = c0 + 16 * (4 * wave + pt) < L ? 4 * wave + pt : 0;
                a4[pt].i = reinterpret_cast<const i32x4*>(kbase + ((static_cast<size_t>(chunk) * 8 + s) * 16 + ptile) * 512)[lane];
            }
#pragma unroll
            for (int q = 0; q < QT; ++q) {
                H8 bh, bl;
                const i32x4* qq = qbase + ((static_cast<size_t>(s) * 4 + g) * G + q0 + q) * 2 * 16 + col;
                bh.i = qq[0];
                bl.i = qq[16];
#pragma unroll
                for (int pt = 0; pt < 4; ++pt) {
                    acc[pt][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a4[pt].v, bh.v, acc[pt][q], 0, 0, 0);
                    acc[pt][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a4[pt].v, bl.v, acc[pt][q], 0, 0, 0);
                }
            }
        }
        // masked scores and this wave's max per query column
        float mx[QT];
#pragma unroll
        for (int q = 0; q < QT; ++q) mx[q] = -INFINITY;
#pragma unroll
        for (int pt = 0; pt < 4; ++pt)
#pragma unroll
            for (int q = 0; q < QT; ++q)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int pos = c0 + 64 * wave + 16 * pt + 4 * g + v;
                    const float val = pos <= qpos ? acc[pt][q][v] * scale : -INFINITY;
                    acc[pt][q][v] = val;
                    mx[q] = fmaxf(mx[q], val);
                }
#pragma unroll
        for (int q = 0; q < QT; ++q) {
            mx[q] = fmaxf(mx[q], __shfl_xor(mx[q], 16, 64));
            mx[q] = fmaxf(mx[q], __shfl_xor(mx[q], 32, 64));
            if (g == 0) max_s[wave][q][col] = mx[q];
        }
        __syncthreads();
        float Mn[QT], alpha[QT], sum[QT];
#pragma unroll
        for (int q = 0; q < QT; ++q) {
            const float mc = fmaxf(fmaxf(max_s[0][q][col], max_s[1][q][col]), fmaxf(max_s[2][q][col], max_s[3][q][col]));
            Mn[q] = fmaxf(Mrun[q], mc);
            alpha[q] = Mn[q] == -INFINITY ? 1.f : expf(Mrun[q] - Mn[q]);
            sum[q] = 0.f;
        }
#pragma unroll
        for (int pt = 0; pt < 4; ++pt)
#pragma unroll
            for (int q = 0; q < QT; ++q)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int pl = 64 * wave + 16 * pt + 4 * g + v;
                    const float e = Mn[q] == -INFINITY ? 0.f : expf(acc[pt][q][v] - Mn[q]);
                    sum[q] += e;
                    P_lds[pl >> 5][q][col][pl & 31] = static_cast<_Float16>(e);
                }
#pragma unroll
        for (int q = 0; q < QT; ++q) {
            sum[q] += __shfl_xor(sum[q], 16, 64);
            sum[q] += __shfl_xor(sum[q], 32, 64);
            if (g == 0) sum_s[wave][q][col] = sum[q];
        }
        __syncthreads();
        // rescale the running output and sum, then O^T += V^T . P^T
#pragma unroll
        for (int q = 0; q < QT; ++q) {
            Lrun[q] = Lrun[q] * alpha[q] + ((sum_s[0][q][col] + sum_s[1][q][col]) + (sum_s[2][q][col] + sum_s[3][q][col]));
            Mrun[q] = Mn[q];
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) o[dt][q] *= alpha[q];
        }
        for (int u = 0; u < 8; ++u) {
            const int grp = 32 * ((c0 >> 5) + u) < L ? (c0 >> 5) + u : (c0 >> 5);
            H8 va[4];
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
                va[dt].i = reinterpret_cast<const i32x4*>(vbase + (static_cast<size_t>(grp) * 16 + 4 * wave + dt) * 512)[lane];
#pragma unroll
            for (int q = 0; q < QT; ++q) {
                H8 bp;
                bp.i = *reinterpret_cast<const i32x4*>(&P_lds[u][q][col][8 * g]);
#pragma unroll
                for (int dt = 0; dt < 4; ++dt)
                    o[dt][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[dt].v, bp.v, o[dt][q], 0, 0, 0);
            }
        }
        __syncthreads();  // P_lds / max_s / sum_s are rewritten by the next chunk
    }

    // lane (g, col) holds dims 64*wave + 16*dt + 4g + v of query column col
    if (tcol >= p.T) return;
    const int n = p.nq * kHD;
#pragma unroll
    for (int q = 0; q < QT; ++q) {
        const int h = kv * G + q0 + q;
        const float inv = 1.f / Lrun[q];
        const float* gate = p.Y + static_cast<size_t>(tcol) * p.ld_y + static_cast<size_t>(h) * 2 * kHD + kHD;
        float* dst = out + static_cast<size_t>(tcol) * n + static_cast<size_t>(h) * kHD;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const int d0 = 64 * wave + 16 * dt + 4 * g;
            float4 r;
            r.x = o[dt][q][0] * inv * sigmoid_f(gate[d0]);
            r.y = o[dt][q][1] * inv * sigmoid_f(gate[d0 + 1]);
            r.z = o[dt][q][2] * inv * sigmoid_f(gate[d0 + 2]);
            r.w = o[dt][q][3] * inv * sigmoid_f(gate[d0 + 3]);
            *reinterpret_cast<float4*>(dst + d0) = r;
        }
    }
}

}  // namespace

namespace rl {

size_t attn_workspace_bytes(int nkv, int ctx) {
    const size_t chunks = static_cast<size_t>(ctx) / kChunk;
    const size_t qf = static_cast<size_t>(nkv) * 8 * 4 * 4 * 16 * 16;  // PT <= 2
    return (qf + static_cast<size_t>(nkv) * chunks * kMaxPairs * (kHD + 2) * 4 + 256 + 255) / 256 * 256;
}

void attn_decode_layer(const float* Y, int ld_y, const float* q_norm, const float* k_norm, uint16_t* kc, uint16_t* vt,
                       int ctx, const int* pos_dev, int T, int nq, int nkv, int hd, int rot, float theta, float eps,
                       void* ws, size_t ws_bytes, float* out, void* frag, hipStream_t s, int t_off, int T_out, int nb,
                       size_t kv_bstride, int pos_stride) {
    RL_REQUIRE(hd == kHD, RL_ERR_UNSUPPORTED, "attn: head_dim must be 256");
    RL_REQUIRE(nb >= 1 && nb <= 64, RL_ERR_RANGE, "attn: slot count must be in 1..64");
    if (T_out <= 0) T_out = T * nb;
    RL_REQUIRE(t_off >= 0 && t_off + nb * T <= T_out && T_out <= 16, RL_ERR_RANGE, "attn: bad output columns");
    RL_REQUIRE(nb == 1 || (kv_bstride >= static_cast<size_t>(nkv) * ctx * kHD && pos_stride >= 1), RL_ERR_RANGE,
               "attn: slot strides must separate the slots' caches and positions");
    RL_REQUIRE(nkv > 0 && nq % nkv == 0, RL_ERR_RANGE, "attn: n_q must be a multiple of n_kv");
    const int G = nq / nkv;
    RL_REQUIRE(T >= 1 && G * T <= kMaxPairs, RL_ERR_RANGE, "attn: (n_q/n_kv) * T must be <= 32");
    RL_REQUIRE(ctx > 0 && ctx % kChunk == 0, RL_ERR_RANGE, "attn: cache capacity must be a multiple of 256");
    RL_REQUIRE(ctx / kChunk <= kMaxChunksLds, RL_ERR_RANGE, "attn: cache capacity above 1M positions");
    RL_REQUIRE(rot >= 2 && rot % 2 == 0 && rot <= hd, RL_ERR_RANGE, "attn: bad rotary dim");
    RL_REQUIRE(Y && kc && vt && pos_dev && ws && (out || frag), RL_ERR_RANGE, "attn: null pointer");
    RL_REQUIRE(ws_bytes >= nb * attn_workspace_bytes(nkv, ctx), RL_ERR_RANGE, "attn: workspace too small");
    const int chunks = ctx / kChunk;
    char* w = static_cast<char*>(ws);
    AttnArgs p{};
    p.Y = Y;
    p.ld_y = ld_y;
    p.q_norm = q_norm;
    p.k_norm = k_norm;
    p.kc = kc;
    p.vt = vt;
    p.ctx = ctx;
    p.pos = pos_dev;
    p.T = T;
    p.nq = nq;
    p.nkv = nkv;
    p.G = G;
    p.rot = rot;
    p.theta = theta;
    p.eps = eps;
    p.qf = reinterpret_cast<i32x4*>(w);
    w += static_cast<size_t>(nkv) * 8 * 4 * 4 * 16 * 16;
    p.part_o = reinterpret_cast<float*>(w);
    w += static_cast<size_t>(nkv) * chunks * kMaxPairs * kHD * 4;
    p.part_m = reinterpret_cast<float*>(w);
    w += static_cast<size_t>(nkv) * chunks * kMaxPairs * 4;
    p.part_l = reinterpret_cast<float*>(w);
    p.max_chunks = chunks;
    p.out = out;
    p.frag = static_cast<i32x4*>(frag);
    p.t_off = t_off;
    p.T_out = T_out;
    p.nb = nb;
    p.kv_bstride = kv_bstride;
    p.pos_stride = pos_stride;
    p.ws_slot = attn_workspace_bytes(nkv, ctx);
    hipLaunchKernelGGL(qk_prep_kernel, dim3(nq + 2 * nkv, T, nb), dim3(64), 0, s, p);
    check_launch("qk_prep_kernel");
    if (pair_tiles(G, T) == 1)
        hipLaunchKernelGGL(attn_part_kernel<1>, dim3(chunks * nkv * nb), dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL(attn_part_kernel<2>, dim3(chunks * nkv * nb), dim3(256), 0, s, p);
    check_launch("attn_part_kernel");
    hipLaunchKernelGGL(attn_comb_kernel, dim3(G * T, nkv, (kHD / 64) * nb), dim3(64 * kCombG), 0, s, p);
    check_launch("attn_comb_kernel");
}


size_t attn_prefill_workspace_bytes(int nq, int T) {
    return static_cast<size_t>(nq) * ((T + 15) / 16) * 16 * kHD * 2 * 2 + 256;
}

void attn_prefill_layer(const float* Y, int ld_y, const float* q_norm, const float* k_norm, uint16_t* kc,
                        uint16_t* vt, int ctx, const int* pos_dev, int T, int nq, int nkv, int hd, int rot,
                        float theta, float eps, void* ws, size_t ws_bytes, float* out, hipStream_t s) {
    RL_REQUIRE(hd == kHD, RL_ERR_UNSUPPORTED, "attn prefill: head_dim must be 256");
    RL_REQUIRE(nkv > 0 && nq % nkv == 0, RL_ERR_RANGE, "attn prefill: n_q must be a multiple of n_kv");
    const int G = nq / nkv;
    RL_REQUIRE(G >= 1 && G <= 8, RL_ERR_UNSUPPORTED, "attn prefill: n_q/n_kv must be in 1..8");
    RL_REQUIRE(T >= 1 && T <= 65535 * 16, RL_ERR_RANGE, "attn prefill: bad token count");
    RL_REQUIRE(ctx > 0 && ctx % kChunk == 0, RL_ERR_RANGE, "attn prefill: cache capacity must be a multiple of 256");
    RL_REQUIRE(rot >= 2 && rot % 2 == 0 && rot <= hd, RL_ERR_RANGE, "attn prefill: bad rotary dim");
    RL_REQUIRE(Y && kc && vt && pos_dev && ws && out, RL_ERR_RANGE, "attn prefill: null pointer");
    RL_REQUIRE(ws_bytes >= attn_prefill_workspace_bytes(nq, T), RL_ERR_RANGE, "attn prefill: workspace too small");
    AttnArgs p{};
    p.Y = Y;
    p.ld_y = ld_y;
    p.q_norm = q_norm;
    p.k_norm = k_norm;
    p.kc = kc;
    p.vt = vt;
    p.ctx = ctx;
    p.pos = pos_dev;
    p.T = T;
    p.nq = nq;
    p.nkv = nkv;
    p.G = G;
    p.rot = rot;
    p.theta = theta;
    p.eps = eps;
    i32x4* qp = static_cast<i32x4*>(ws);
    hipLaunchKernelGGL(qk_prep_pf_kernel, dim3(nq + 2 * nkv, T), dim3(64), 0, s, p, qp);
    check_launch("qk_prep_pf_kernel");
    // query tiles per workgroup: 3, 2 or 1 (a divisor of G; four spill registers)
    const int QT = G % 3 == 0 ? 3 : G % 2 == 0 ? 2 : 1;
    const dim3 grid((T + 15) / 16, nkv, G / QT);
    switch (QT) {
    case 3: hipLaunchKernelGGL(attn_prefill_kernel<3>, grid, dim3(256), 0, s, p, qp, out); break;
    case 2: hipLaunchKernelGGL(attn_prefill_kernel<2>, grid, dim3(256), 0, s, p, qp, out); break;
    default: hipLaunchKernelGGL(attn_prefill_kernel<1>, grid, dim3(256), 0, s, p, qp, out); break;
    }
    check_launch("attn_prefill_kernel");
}

}  // namespace rl

extern "C" {

size_t rl_hip_attn_workspace_bytes(int n_kv, int ctx) { return rl::attn_workspace_bytes(n_kv, ctx); }

int rl_hip_attn_decode_layer(const float* Y, int ld_y, const float* q_norm, const float* k_norm, uint16_t* k_cache,
                             uint16_t* vt_cache, int ctx, const int* pos_dev, int T, int n_q, int n_kv, int head_dim,
                             int rotary_dim, float theta, float eps, void* workspace, size_t workspace_bytes,
                             float* out, void* frag, void* stream) {
    return guard([&] {
        rl::attn_decode_layer(Y, ld_y, q_norm, k_norm, k_cache, vt_cache, ctx, pos_dev, T, n_q, n_kv, head_dim,
                              rotary_dim, theta, eps, workspace, workspace_bytes, out, frag, S(stream));
    });
}

size_t rl_hip_attn_prefill_workspace_bytes(int n_q, int T) { return rl::attn_prefill_workspace_bytes(n_q, T); }

int rl_hip_attn_prefill_layer(const float* Y, int ld_y, const float* q_norm, const float* k_norm, uint16_t* k_cache,
                              uint16_t* vt_cache, int ctx, const int* pos_dev, int T, int n_q, int n_kv, int head_dim,
                              int rotary_dim, float theta, float eps, void* workspace, size_t workspace_bytes,
                              float* out, void* stream) {
    return guard([&] {
        rl::attn_prefill_layer(Y, ld_y, q_norm, k_norm, k_cache, vt_cache, ctx, pos_dev, T, n_q, n_kv, head_dim,
                               rotary_dim, theta, eps, workspace, workspace_bytes, out, S(stream));
    });
}

}  // extern "C"
