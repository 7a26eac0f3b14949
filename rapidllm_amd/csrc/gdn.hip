// gdn.hip -- Gated DeltaNet recurrent decode for T = 1..8 tokens, fused:
//   causal conv1d window update (+SiLU), head map, q/k L2 norm (q * 1/sqrt(dk)),
//   gates beta = sigmoid(b), g = exp(-exp(A_log) * softplus(a + dt_bias)),
//   delta rule per token on the fp32 state.
// Arithmetic follows the reference CPU path: conv1d_update (src/kernels/ops.cpp:
// 458-468), gates (src/kernels/ops_fused.cpp:111-123), l2norm (ops.cpp:158-163),
// delta_recurrent_step (ops.cpp:495-534).  Output o is the raw recurrent output;
// the gated RMSNorm is fused into the packing kernel of the next linear (norms.hip).
//
// Two kernels.  gdn_decode_kernel (any dv multiple of 32, state ring for the
// unfused engine path): one workgroup per (v-head h, 16 value columns), thread
// (c, jj) keeps S[h][8c .. 8c+7][16*cg + jj] in registers.  gdn_fused_kernel (below;
// dk 128, dv multiple of 32): one workgroup per (v-head, 32 value columns), the gated
// norm's elementwise part and the out_proj packing fused, speculative records
// instead of a state ring.  Column j of S evolves independently given k, q, g, beta
// and v_j, so the only cross-thread work per token is two lane-group sums
// (k^T S and q^T S).  The state is read once and written once for all T tokens.
//
// State layout in HBM (transposed per head): St[h][j][i] = S[h][i][j], so each
// thread's 8 values are 32 contiguous bytes and a wave reads 2 KiB contiguously.
// Conv window layout is the reference's [channel][tap] (tap 0 oldest).
#include <cstdlib>
#include <algorithm>

#include "internal.h"

using namespace rl;

namespace {

constexpr int kDK = 128;    // key head dim (rows of S)
constexpr int kCols = 16;   // value columns per workgroup
constexpr int kRowChunks = 16;  // threads per column (8 rows each)
constexpr int kRowsPer = kDK / kRowChunks;
constexpr int kMaxT = 8;
constexpr int kConvK = 4;   // conv taps (Qwen3.6/3.8: 4)

__device__ inline float silu_f(float x) { return x / (1.f + expf(-x)); }
// The fused kernel's SiLU and inverse square roots on the per-token path use the
// hardware approximations (exp2, reciprocal, rsq: about 1 ulp) instead of the
// correctly rounded sequences, which were the longest stretches of each token's
// dependent chain.
__device__ inline float silu_fast(float x) {
    return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * 1.44269504088896341f));
}
__device__ inline float rsqrt_fast(float x) { return __builtin_amdgcn_rsqf(x); }
__device__ inline float sigmoid_f(float x) { return 1.f / (1.f + expf(-x)); }
__device__ inline float softplus_f(float x) { return log1pf(expf(-fabsf(x))) + fmaxf(x, 0.f); }

struct GdnArgs {
    const float* qkv;   // [T][ld_in]: raw in_proj qkv channels at offset 0
    const float* a;     // [T][ld_in]: a at this pointer (nv values per token)
    const float* b;     // [T][ld_in]
    int ld_in;          // row stride (floats) of qkv/a/b
    const float* A_log; // [nv]
    const float* dt_bias;
    const float* conv_w;  // [conv_dim][K]
    // Direct mode (cur == nullptr): read conv_in / S_in, write the state after the
    // last token to conv_out / S_out.  S_out may alias S_in (each thread owns its
    // slice); conv_out must not alias conv_in (q/k windows are read by several
    // workgroups).
    // Ring mode (cur != nullptr): R slots of conv_slot / s_slot floats at conv_in /
    // S_in; read slot *cur, write the state after token t to slot (*cur + 1 + t) % R
    // (R > T), so a speculative verify can keep any prefix without recomputation.
    const float* conv_in;
    float* conv_out;
    const float* S_in;    // [nv][dv][dk] (transposed)
    float* S_out;
    const int* cur;
    size_t conv_slot, s_slot;
    int R;
    float* o;             // [T][nv*dv]
    int T, nk, nv, dv, K, v_tiled;
    // fused kernel: a and b are the sums of ab_slices partials,
    // a[(s * T + t) * ab_ld + h] (1 slice with ab_ld = ld_in: the plain layout)
    int ab_slices = 1, ab_ld = 0;
};

__global__ __launch_bounds__(256) void gdn_decode_kernel(GdnArgs p) {
    const int tid = threadIdx.x;
    const int c = tid & (kRowChunks - 1);  // row chunk: rows 8c .. 8c+7
    const int jj = tid / kRowChunks;       // column within the group
    const int groups_per_head = p.dv / kCols;
    const int h = blockIdx.x / groups_per_head;
    const int cg = blockIdx.x % groups_per_head;
    const int j = cg * kCols + jj;
    const int rep = p.nv / p.nk;
    const int src = p.v_tiled ? (h % p.nk) : (h / rep);
    const int qdim = p.nk * kDK;
    const int T = p.T;
    constexpr int K = kConvK;

    __shared__ float q_s[kMaxT][kDK];
    __shared__ float k_s[kMaxT][kDK];
    __shared__ float v_s[kMaxT][kCols];
    __shared__ float gate_s[kMaxT][2];  // decay g, beta
    __shared__ double red_s[2][kMaxT][4];

    const int slot0 = p.cur ? *p.cur : 0;
    const float* S_in = p.cur ? p.S_in + static_cast<size_t>(slot0) * p.s_slot : p.S_in;
    const float* conv_in = p.cur ? p.conv_in + static_cast<size_t>(slot0) * p.conv_slot : p.conv_in;
    auto s_dst = [&](int t) -> float* {
        return p.cur ? const_cast<float*>(p.S_in) + static_cast<size_t>((slot0 + 1 + t) % p.R) * p.s_slot : p.S_out;
    };
    auto conv_dst = [&](int t) -> float* {
        return p.cur ? const_cast<float*>(p.conv_in) + static_cast<size_t>((slot0 + 1 + t) % p.R) * p.conv_slot
                     : p.conv_out;
    };
    const bool per_token = p.cur != nullptr;

    // ---- state: 8 rows of column j, contiguous in the transposed layout
    const size_t s_off = (static_cast<size_t>(h) * p.dv + j) * kDK + kRowsPer * c;
    float S[kRowsPer];
    {
        const float4* sp = reinterpret_cast<const float4*>(S_in + s_off);
#pragma unroll
        for (int r = 0; r < kRowsPer / 4; ++r) {
            const float4 v = sp[r];
            S[4 * r] = v.x;
            S[4 * r + 1] = v.y;
            S[4 * r + 2] = v.z;
            S[4 * r + 3] = v.w;
        }
    }

    // gate inputs of token tid, loaded with the state (before any store of this
    // thread, whose completion a later wait would otherwise include)
    float gin_a = 0.f, gin_b = 0.f, gin_A = 0.f, gin_dt = 0.f;
    if (tid < T) {
        gin_a = p.a[static_cast<size_t>(tid) * p.ld_in + h];
        gin_b = p.b[static_cast<size_t>(tid) * p.ld_in + h];
        gin_A = p.A_log[h];
        gin_dt = p.dt_bias[h];
    }

    // ---- conv1d over T tokens for the 2*128 q/k channels of the source k-head and
    // the 32 v channels of this workgroup (288 channels, 256 threads).
    // The q/k window state is written back only by one workgroup per source head.
    const bool owns_qk = cg == 0 && (p.v_tiled ? (h == src) : (h == src * rep));
    for (int ch = tid; ch < 2 * kDK + kCols; ch += 256) {
        int chan;
        if (ch < kDK)
            chan = src * kDK + ch;
        else if (ch < 2 * kDK)
            chan = qdim + src * kDK + (ch - kDK);
        else
            chan = 2 * qdim + h * p.dv + cg * kCols + (ch - 2 * kDK);
        const bool write_state = ch >= 2 * kDK || owns_qk;
        float win[K];
        {
            const float4 wv = *reinterpret_cast<const float4*>(conv_in + static_cast<size_t>(chan) * K);
            win[0] = wv.x;
            win[1] = wv.y;
            win[2] = wv.z;
            win[3] = wv.w;
        }
        // taps in registers: the per-token window stores below could alias conv_w
        // as far as the compiler knows, which would reload it after every store
        float w[K];
        {
            const float4 w4 = *reinterpret_cast<const float4*>(p.conv_w + static_cast<size_t>(chan) * K);
            w[0] = w4.x;
            w[1] = w4.y;
            w[2] = w4.z;
            w[3] = w4.w;
        }
        // every token's input for this channel, loaded together (one memory round
        // trip instead of T dependent ones)
        float xin[kMaxT];
#pragma unroll
        for (int t = 0; t < kMaxT; ++t) xin[t] = t < T ? p.qkv[static_cast<size_t>(t) * p.ld_in + chan] : 0.f;
#pragma unroll
        for (int t = 0; t < kMaxT; ++t) {
            if (t >= T) break;
#pragma unroll
            for (int q = 0; q + 1 < K; ++q) win[q] = win[q + 1];
            win[K - 1] = xin[t];
            double acc = 0.0;
#pragma unroll
            for (int q = 0; q < K; ++q) acc += static_cast<double>(w[q]) * win[q];
            const float y = silu_f(static_cast<float>(acc));
            if (ch < kDK)
                q_s[t][ch] = y;
            else if (ch < 2 * kDK)
                k_s[t][ch - kDK] = y;
            else
                v_s[t][ch - 2 * kDK] = y;
            if (write_state && (per_token || t == T - 1)) {
                *reinterpret_cast<float4*>(conv_dst(t) + static_cast<size_t>(chan) * K) =
                    make_float4(win[0], win[1], win[2], win[3]);
            }
        }
    }
    if (tid < T) {
        const float beta = sigmoid_f(gin_b);
        const float g_log = -expf(gin_A) * softplus_f(gin_a + gin_dt);
        gate_s[tid][0] = expf(g_log);
        gate_s[tid][1] = beta;
    }
    __syncthreads();

    // ---- L2 norms (double sums over 128): waves 0/1 take q/k of every token
    {
        const int wave = tid >> 6, lane = tid & 63;
        if (wave < 2) {
            float(*vec)[kDK] = wave == 0 ? q_s : k_s;
            for (int t = 0; t < T; ++t) {
                const double a0 = vec[t][lane], a1 = vec[t][lane + 64];
                const double ss = wave_sum_d(a0 * a0 + a1 * a1);
                if (lane == 0) red_s[wave][t][0] = ss;
            }
        }
    }
    __syncthreads();
    const float qscale = 1.f / sqrtf(static_cast<float>(kDK));
    for (int e = tid; e < T * kDK; e += 256) {
        const int t = e / kDK, i = e % kDK;
        const float iq = 1.f / sqrtf(static_cast<float>(red_s[0][t][0]) + 1e-6f);
        const float ik = 1.f / sqrtf(static_cast<float>(red_s[1][t][0]) + 1e-6f);
        q_s[t][i] = (q_s[t][i] * iq) * qscale;
        k_s[t][i] = k_s[t][i] * ik;
    }
    __syncthreads();

    // ---- delta rule, token by token
    for (int t = 0; t < T; ++t) {
        const float g = gate_s[t][0], beta = gate_s[t][1];
        float kv = 0.f;
#pragma unroll
        for (int r = 0; r < kRowsPer; ++r) {
            S[r] *= g;
            kv += S[r] * k_s[t][kRowsPer * c + r];
        }
        kv = group16_sum(kv);
        const float delta = (v_s[t][jj] - kv) * beta;
        float ov = 0.f;
#pragma unroll
        for (int r = 0; r < kRowsPer; ++r) {
            S[r] += k_s[t][kRowsPer * c + r] * delta;
            ov += S[r] * q_s[t][kRowsPer * c + r];
        }
        ov = group16_sum(ov);
        if (c == 0) p.o[static_cast<size_t>(t) * p.nv * p.dv + static_cast<size_t>(h) * p.dv + j] = ov;
        if (per_token || t == T - 1) {
            float4* dp = reinterpret_cast<float4*>(s_dst(t) + s_off);
#pragma unroll
            for (int r = 0; r < kRowsPer / 4; ++r)
                dp[r] = make_float4(S[4 * r], S[4 * r + 1], S[4 * r + 2], S[4 * r + 3]);
        }
    }
}

// ------------------------------------------------------- (head, 32 columns) per WG
// Same arithmetic as gdn_decode_kernel with 32 value columns per workgroup
// (nv * dv / 32 workgroups: the state slices stream through that many CUs) and
// thread (c, jj) keeping S rows 16c .. 16c+15 of column j = 32*cc + jj.  The gated
// RMSNorm of the head (reference ops.cpp:129-156, per head of dv, eps 1e-6, double
// sum) is split: this kernel packs y = gamma * o * silu(z) into the out_proj input
// fragments and writes the chunk's sum of o^2 per token; out_proj scales the
// head's column block by 1/rms (NormIO::kss).
// The recurrent state is not kept in the ring: with the conv ring the kernel keeps
// one committed S and the per-token records of GdnRecords.
constexpr int kCW = 32;                  // value columns per workgroup
constexpr int kCChunks = 16;             // threads per column
constexpr int kCRows = kDK / kCChunks;   // 8 rows per thread
constexpr int kCT = kCW * kCChunks;      // 512 threads (8 waves)
constexpr int kCRecPer = kMaxT * kDK / kCT;  // replayed k values per thread
static_assert(kCT >= 2 * kDK, "the q/k conv channels need a thread each");
// the kCChunks threads of a column sum their rows' products (fixed DPP order)
__device__ inline float column_sum(float v) { return kCChunks == 8 ? group8_sum(v) : group16_sum(v); }
constexpr int kMaxAbSlices = 8;
constexpr int kRing = 5;  // conv / record ring of the engine's T <= 4 steps

struct GdnFusedArgs {
    GdnArgs g;
    const float* z;      // [T][ld_in] at the head-0 z column (gated norm gate)
    const float* gamma;  // [dv]
    i32x4* frag;         // out_proj input fragments (may be null)
    float* gss;          // [nv][T][4] partial sums of o^2 (with frag or y32)
    float* y32;          // [T][nv * dv] fp32 rows of y (may be null)
    GdnRecords rec;      // rec.rec == nullptr: no records (direct mode)
    GdnBatch batch;
    // token rows: this call's tokens are rows row_off .. row_off + T - 1 of T_rows
    // (prompt prefill: sub-chunks of a chunk; 0: B * T rows, sequence b at b * T)
    int row_off = 0, T_rows = 0;
};

// TT > 0: the token count as a compile-time constant (the per-token loops then have
// no branches, so the compiler overlaps a token's independent work -- LDS reads,
// norms, gates, conv -- with the previous token's state chain); 0: runtime p.T.
template <int TT>
__global__ __launch_bounds__(kCT) void gdn_fused_kernel(GdnFusedArgs a) {
    const GdnArgs& p = a.g;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int c = tid & (kCChunks - 1);
    const int jj = tid / kCChunks;  // column within the chunk
    const int dv = p.dv;
    const int chunks = dv / kCW;
    const int rep = p.nv / p.nk;
    // XCD-aware order: workgroups are dispatched to the 8 XCDs round-robin
    // (blockIdx % 8), each XCD with its own L2.  With n_k a multiple of 8, XCD x
    // takes whole k-heads (all rep v-heads x chunks workgroups of each), so a
    // k-head's q/k conv window, weights and inputs are fetched into one L2 and
    // shared by its workgroups; otherwise workgroup = (v-head, chunk) in order.
    int h, cc;
    if (p.nk % 8 == 0) {
        const int M = rep * chunks;  // workgroups per k-head
        const int x = blockIdx.x % 8, jx = blockIdx.x / 8;
        const int g = x * (p.nk / 8) + jx / M, m = jx % M;
        const int r = m / chunks;
        cc = m % chunks;
        h = p.v_tiled ? g + r * p.nk : g * rep + r;
    } else {
        h = blockIdx.x / chunks;
        cc = blockIdx.x % chunks;
    }
    const int j = cc * kCW + jj;
    const int src = p.v_tiled ? (h % p.nk) : (h / rep);
    const int qdim = p.nk * kDK;
    const int T = TT > 0 ? TT : p.T;
    constexpr int K = kConvK;
    // sequence of the batch: state / ring / records / scalars at its strides, its
    // tokens are rows row0 .. row0 + T - 1 of T_tot
    const int bs = blockIdx.y;
    const int T_tot = a.T_rows ? a.T_rows : a.batch.B * T, row0 = a.row_off + bs * T;
    const float* S_in = p.S_in + bs * a.batch.s_stride;
    float* S_out = p.S_out + bs * a.batch.s_stride;
    const float* conv_base = p.conv_in + bs * a.batch.conv_stride;
    const int* cur = p.cur ? p.cur + bs * a.batch.scal_stride : nullptr;

    __shared__ float q_s[kMaxT][kDK];   // conv outputs (q, k not yet normalised)
    __shared__ float k_s[kMaxT][kDK];
    __shared__ float v_s[kMaxT][kCW];
    __shared__ float o_s[kMaxT][kCW];
    __shared__ float y_s[kMaxT][kCW];
    __shared__ float gate_s[kMaxT][2];
    __shared__ double red_s[4][kMaxT];  // sums of squares: q lanes 0-63, 64-127, k 0-63, 64-127
    __shared__ float rk_s[kMaxT][kDK];  // replayed records: k, delta, g
    __shared__ float rd_s[kMaxT][kCW];
    __shared__ float rg_s[kMaxT];

    const int slot0 = cur ? *cur : 0;
    const float* conv_in = cur ? conv_base + static_cast<size_t>(slot0) * p.conv_slot : conv_base;
    auto conv_dst = [&](int t) -> float* {
        return cur ? const_cast<float*>(conv_base) + static_cast<size_t>((slot0 + 1 + t) % p.R) * p.conv_slot
                   : p.conv_out + bs * a.batch.conv_stride;
    };
    const bool per_token = cur != nullptr;

    // ---- loads, in the order they are needed (vector loads complete in order):
    // conv inputs of this thread's channels (tid: q/k channel; tid < 32 also v
    // channel 256 + tid), gate inputs, gated-norm operands, then the state slice and
    // the previous call's records, which are first needed after the barrier.
    auto chan_of = [&](int ch) {
        if (ch < kDK) return src * kDK + ch;
        if (ch < 2 * kDK) return qdim + src * kDK + (ch - kDK);
        return 2 * qdim + h * dv + cc * kCW + (ch - 2 * kDK);
    };
    const bool has_v = tid < kCW;
    const bool qk_lane = tid < 2 * kDK;  // thread tid < 256 owns q/k conv channel tid
    const int chan0 = chan_of(qk_lane ? tid : 0), chan1 = chan_of(2 * kDK + (has_v ? tid : 0));
    float win0[K], win1[K], w0[K], w1[K], xin0[kMaxT], xin1[kMaxT];
    // With a ring of kRing slots the windows of every slot are requested at once and
    // the current one picked when the slot index has arrived: no dependent memory
    // round trip before the conv
    const bool ring_all = cur && p.R == kRing;
    {
        float4 a0, a1;
        if (ring_all) {
            float4 c0[kRing], c1[kRing];
#pragma unroll
            for (int q = 0; q < kRing; ++q) {
                c0[q] = *reinterpret_cast<const float4*>(conv_base + q * p.conv_slot + static_cast<size_t>(chan0) * K);
                c1[q] = *reinterpret_cast<const float4*>(conv_base + q * p.conv_slot + static_cast<size_t>(chan1) * K);
            }
            a0 = c0[0];
            a1 = c1[0];
#pragma unroll
            for (int q = 1; q < kRing; ++q)
                if (slot0 == q) {
                    a0 = c0[q];
                    a1 = c1[q];
                }
        } else {
            a0 = *reinterpret_cast<const float4*>(conv_in + static_cast<size_t>(chan0) * K);
            a1 = *reinterpret_cast<const float4*>(conv_in + static_cast<size_t>(chan1) * K);
        }
        const float4 b0 = *reinterpret_cast<const float4*>(p.conv_w + static_cast<size_t>(chan0) * K);
        const float4 b1 = *reinterpret_cast<const float4*>(p.conv_w + static_cast<size_t>(chan1) * K);
        win0[0] = a0.x, win0[1] = a0.y, win0[2] = a0.z, win0[3] = a0.w;
        win1[0] = a1.x, win1[1] = a1.y, win1[2] = a1.z, win1[3] = a1.w;
        w0[0] = b0.x, w0[1] = b0.y, w0[2] = b0.z, w0[3] = b0.w;
        w1[0] = b1.x, w1[1] = b1.y, w1[2] = b1.z, w1[3] = b1.w;
#pragma unroll
        for (int t = 0; t < kMaxT; ++t) {
            xin0[t] = t < T ? p.qkv[static_cast<size_t>(row0 + t) * p.ld_in + chan0] : 0.f;
            xin1[t] = t < T ? p.qkv[static_cast<size_t>(row0 + t) * p.ld_in + chan1] : 0.f;
        }
    }
    // gate inputs: lane e = 16t + 8(b) + s holds slice s of a (or b) of token t; the 8
    // slices are summed by a DPP 8-lane reduction (fixed order)
    float gin = 0.f, gin_A = 0.f, gin_dt = 0.f;
    const bool gate_lane = tid < 16 * T;
    if (gate_lane) {
        const int t = tid >> 4, sl = tid & 7;
        const float* src = (tid & 8) ? p.b : p.a;
        if (sl < p.ab_slices) gin = src[(static_cast<size_t>(sl) * T_tot + row0 + t) * p.ab_ld + h];
        gin_A = p.A_log[h];
        gin_dt = p.dt_bias[h];
    }
    float zt[kMaxT];
    float gam = 0.f;
    const bool gn = (a.frag != nullptr || a.y32 != nullptr) && c == 0;
    if (gn) {
        gam = a.gamma[j];
#pragma unroll
        for (int t = 0; t < kMaxT; ++t)
            zt[t] = t < T ? a.z[static_cast<size_t>(row0 + t) * p.ld_in + h * dv + j] : 0.f;
    }
    // state: 16 rows of column j (64 contiguous bytes of the transposed layout)
    const size_t s_off = (static_cast<size_t>(h) * dv + j) * kDK + kCRows * c;
    float S[kCRows];
    {
        // non-temporal (as the stores below): the state lines are not kept in the
        // caches, so the stores stream out instead of dirtying cached lines that a
        // later kernel's loads would have to evict (measured: the following
        // attention kernel ran ~4 us slower with cached state lines)
        const f32x4* sp = reinterpret_cast<const f32x4*>(S_in + s_off);
#pragma unroll
        for (int r = 0; r < kCRows / 4; ++r) {
            const f32x4 v = __builtin_nontemporal_load(sp + r);
            S[4 * r] = v[0];
            S[4 * r + 1] = v[1];
            S[4 * r + 2] = v[2];
            S[4 * r + 3] = v[3];
        }
    }
    // records: bank *cur is written, the previous call's bank is read
    const bool records = a.rec.rec != nullptr;
    const bool keep = records && a.rec.keep;
    float* rec_base = records ? a.rec.rec + bs * a.batch.rec_stride : nullptr;
    int* count = records ? a.rec.count + bs * a.batch.count_stride : nullptr;
    const int n_cons = records ? a.rec.n_cons[bs * a.batch.scal_stride] : 0;
    const int rbank = records ? ((slot0 - n_cons) % p.R + p.R) % p.R : 0;
    int cnt = 0;
    if (records && ring_all) {
        // every bank's count requested together, the bank picked afterwards
        int cq[kRing];
#pragma unroll
        for (int q = 0; q < kRing; ++q) cq[q] = count[q * p.nv + h];
        cnt = cq[0];
#pragma unroll
        for (int q = 1; q < kRing; ++q)
            if (rbank == q) cnt = cq[q];
    } else if (records) {
        cnt = count[rbank * p.nv + h];
    }
    const int n_rep = records ? min(min(n_cons, cnt), kMaxT) : 0;
    const size_t rec_t = static_cast<size_t>(p.nv) * kGdnRecFloats;  // token stride
    const size_t bank = static_cast<size_t>(a.rec.max_t) * rec_t;
    const float* rec_r = records ? rec_base + rbank * bank + static_cast<size_t>(h) * kGdnRecFloats : nullptr;
    float* rec_w = records ? rec_base + slot0 * bank + static_cast<size_t>(h) * kGdnRecFloats : nullptr;
    float rk[kCRecPer], rd = 0.f, rg = 0.f;  // record values e = tid + q * kCT (token e / 128)
#pragma unroll
    for (int q = 0; q < kCRecPer; ++q) {
        const int e = tid + q * kCT;
        rk[q] = e < n_rep * kDK ? rec_r[(e / kDK) * rec_t + e % kDK] : 0.f;
    }
    if (tid < n_rep * kCW) rd = rec_r[(tid / kCW) * rec_t + kDK + cc * kCW + tid % kCW];
    if (tid < n_rep) rg = rec_r[tid * rec_t + 2 * kDK];

    // ---- conv1d over T tokens (+ SiLU); q/k lanes also sum their squares per token
    // (double), reduced per wave: the L2 norms need no pass of their own.  The
    // q/k window state is written back by one workgroup per source k-head.
    const bool owns_qk = cc == 0 && (p.v_tiled ? (h == src) : (h == src * rep));
    double sq[kMaxT];
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
        sq[t] = 0.0;
        if (t >= T) continue;
#pragma unroll
        for (int q = 0; q + 1 < K; ++q) {
            win0[q] = win0[q + 1];
            win1[q] = win1[q + 1];
        }
        win0[K - 1] = xin0[t];
        win1[K - 1] = xin1[t];
        double acc0 = 0.0, acc1 = 0.0;
#pragma unroll
        for (int q = 0; q < K; ++q) {
            acc0 += static_cast<double>(w0[q]) * win0[q];
            acc1 += static_cast<double>(w1[q]) * win1[q];
        }
        const float y0 = silu_fast(static_cast<float>(acc0));
        if (tid < kDK)
            q_s[t][tid] = y0;
        else if (qk_lane)
            k_s[t][tid - kDK] = y0;
        sq[t] = qk_lane ? static_cast<double>(y0) * y0 : 0.0;
        if (owns_qk && qk_lane && (per_token || t == T - 1))
            *reinterpret_cast<float4*>(conv_dst(t) + static_cast<size_t>(chan0) * K) =
                make_float4(win0[0], win0[1], win0[2], win0[3]);
        if (has_v) {
            v_s[t][tid] = silu_fast(static_cast<float>(acc1));
            if (per_token || t == T - 1)
                *reinterpret_cast<float4*>(conv_dst(t) + static_cast<size_t>(chan1) * K) =
                    make_float4(win1[0], win1[1], win1[2], win1[3]);
        }
    }
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
        if (t >= T) break;
        if (wave < 4) {  // the q/k waves
            const double ws = wave_sum_d(sq[t]);
            if (lane == 0) red_s[wave][t] = ws;
        }
    }
    if (wave * 4 < T) {  // waves holding gate lanes (all lanes take part in the DPP sums)
        const float sum = group8_sum(gin);
        const float bsum = __shfl_down(sum, 8, 64);  // b of the same token, 8 lanes up
        if (gate_lane && (tid & 15) == 0) {
            const int t = tid >> 4;
            const float beta = sigmoid_f(bsum);
            const float g_log = -expf(gin_A) * softplus_f(sum + gin_dt);
            gate_s[t][0] = expf(g_log);
            gate_s[t][1] = beta;
        }
    }
#pragma unroll
    for (int q = 0; q < kCRecPer; ++q) {
        const int e = tid + q * kCT;
        if (e < n_rep * kDK) rk_s[e / kDK][e % kDK] = rk[q];
    }
    if (tid < n_rep * kCW) rd_s[tid / kCW][tid % kCW] = rd;
    if (tid < n_rep) rg_s[tid] = rg;
    __syncthreads();

    // ---- replay the consumed records of the previous call (same operations as the
    // update below)
    for (int t = 0; t < n_rep; ++t) {
        const float g = rg_s[t];
        const float delta = rd_s[t][jj];
#pragma unroll
        for (int r = 0; r < kCRows; ++r) S[r] = __fmaf_rn(rk_s[t][kCRows * c + r], delta, __fmul_rn(S[r], g));
    }
    auto store_state = [&] {
        f32x4* dp = reinterpret_cast<f32x4*>(S_out + s_off);
#pragma unroll
        for (int r = 0; r < kCRows / 4; ++r)
            __builtin_nontemporal_store(f32x4{S[4 * r], S[4 * r + 1], S[4 * r + 2], S[4 * r + 3]}, dp + r);
    };
    if (keep && n_rep > 0) store_state();

    // ---- delta rule, token by token; q and k normalised as read:
    // q = (q * 1/|q|) * 1/sqrt(dk), k = k * 1/|k| (eps 1e-6 inside the root)
    const float qscale = 1.f / sqrtf(static_cast<float>(kDK));
    const bool rec_k = keep && cc == 0 && jj == 0;  // one writer of the per-head k and g records
    // unrolled over the token bound: the next token's LDS reads, norms and gates and
    // the previous token's output work are independent of the state chain, and the
    // compiler interleaves them with it
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
        if (t >= T) break;
        const float iq = rsqrt_fast(static_cast<float>(red_s[0][t] + red_s[1][t]) + 1e-6f);
        const float ik = rsqrt_fast(static_cast<float>(red_s[2][t] + red_s[3][t]) + 1e-6f);
        const float g = gate_s[t][0], beta = gate_s[t][1];
        float kn[kCRows];
#pragma unroll
        for (int r = 0; r < kCRows; ++r) kn[r] = k_s[t][kCRows * c + r] * ik;
        if (rec_k) {
            float4* kp = reinterpret_cast<float4*>(rec_w + t * rec_t + kCRows * c);
#pragma unroll
            for (int r = 0; r < kCRows / 4; ++r) kp[r] = make_float4(kn[4 * r], kn[4 * r + 1], kn[4 * r + 2], kn[4 * r + 3]);
            if (c == 0) rec_w[t * rec_t + 2 * kDK] = g;
        }
        float kv4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < kCRows; ++r) {
            S[r] = __fmul_rn(S[r], g);
            kv4[r & 3] = __fmaf_rn(S[r], kn[r], kv4[r & 3]);
        }
        const float kv = column_sum((kv4[0] + kv4[1]) + (kv4[2] + kv4[3]));
        const float delta = (v_s[t][jj] - kv) * beta;
        float ov4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < kCRows; ++r) {
            S[r] = __fmaf_rn(kn[r], delta, S[r]);
            ov4[r & 3] = __fmaf_rn(S[r], (q_s[t][kCRows * c + r] * iq) * qscale, ov4[r & 3]);
        }
        const float ov = column_sum((ov4[0] + ov4[1]) + (ov4[2] + ov4[3]));
        if (c == 0) {
            if (p.o) p.o[static_cast<size_t>(row0 + t) * p.nv * dv + static_cast<size_t>(h) * dv + j] = ov;
            if (keep) rec_w[t * rec_t + kDK + j] = delta;
            if (gn) {
                o_s[t][jj] = ov;
                y_s[t][jj] = gam * ov * silu_fast(zt[t]);
            }
        }
    }
    if (!keep) store_state();
    if (records && cc == 0 && tid == 0) count[slot0 * p.nv + h] = keep ? T : 0;
    if (!a.frag && !a.y32) return;

    // ---- per token: the chunk's sum of o^2 (double; 16-lane rows, then the row
    // pair) and y: fragments (thread t*4 + u packs columns 8u .. 8u+7) or fp32 rows
    __syncthreads();
    if (wave * 2 < T) {  // wave w: tokens 2w (lanes 0-31) and 2w + 1 (lanes 32-63)
        const int t = 2 * wave + (lane >> 5), i = lane & 31;
        const double v = t < T ? static_cast<double>(o_s[t][i]) * o_s[t][i] : 0.0;
        const double r = group16_sum_d(v);
        const double s0 = readlane_d(r, 0) + readlane_d(r, 16), s1 = readlane_d(r, 32) + readlane_d(r, 48);
        if (lane == 0) a.gss[(static_cast<size_t>(h) * T_tot + row0 + t) * 4 + cc] = static_cast<float>(s0);
        if (lane == 32 && t < T) a.gss[(static_cast<size_t>(h) * T_tot + row0 + t) * 4 + cc] = static_cast<float>(s1);
    }
    if (a.y32 && tid < T * kCW) {
        const int t = tid / kCW, i = tid % kCW;
        a.y32[static_cast<size_t>(row0 + t) * p.nv * dv + h * dv + cc * kCW + i] = y_s[t][i];
    }
    if (a.frag && tid < T * (kCW / 8)) {
        const int t = tid / (kCW / 8), u = tid % (kCW / 8);
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = y_s[t][8 * u + e];
        write_frag8(a.frag, (h * dv + cc * kCW) / 8 + u, row0 + t, T_tot, v);
    }
}

// ------------------------------------------------------------------ prefill
// Prompt prefill over T tokens (the reference's chunked prefill,
// cuda_engine.cu:18338-18590: conv1d_prefill / conv1d_upd_seq then the recurrent
// scan; CPU: per token conv1d_update + delta_recurrent_step, ops.cpp:458-534).
// Two kernels per layer instead of one launch per 8 tokens:
//   gdn_pf_conv: one thread per (token, channel): conv + SiLU from the token's
//                4-tap window (double accumulation as conv1d_update), the final
//                window, and the gates of (t, head);
//   gdn_pf_rec:  one workgroup per (v-head, 32 value columns) keeps its slice of S
//                in registers for all T tokens: per token the q/k L2 norms, decay,
//                delta rule and output, the tokens' inputs staged through LDS in
//                blocks of 32 (the next block loading during the current one).
struct GdnPfArgs {
    const float* y;      // in_proj rows [T][ld]: qkv channels at 0, a at off_a, b at off_b
    int ld, off_a, off_b;
    const float* A_log;
    const float* dt_bias;
    const float* conv_w;  // [conv_dim][4]
    const float* conv_in;
    float* conv_out;      // window after the last token (must not alias conv_in)
    float* xc;            // [T][conv_dim] conv outputs (after SiLU)
    float* gates;         // [T][nv][2]: decay g = exp(g_log), beta
    float* S;             // [nv][dv][dk] transposed, updated in place
    float* o;             // [T][nv*dv]
    int T, nk, nv, dv, conv_dim, v_tiled;
};

// One thread per (channel, kPfConvTok consecutive tokens): the conv output of token t
// only needs the inputs of tokens t-3 .. t (the window before the chunk for t < 3),
// so token blocks are independent; within a block the 4-tap window slides in
// registers (each input read once, the weights and incoming window once per block).
// Grid (channel blocks, token blocks); the thread holding token T-1 also writes the
// final window; threads past the conv channels form the gates of (t, head).
constexpr int kPfConvTok = 16;

__global__ __launch_bounds__(256) void gdn_pf_conv_kernel(GdnPfArgs p) {
    const int t0 = blockIdx.y * kPfConvTok, ch = blockIdx.x * blockDim.x + threadIdx.x;
    const int nt = min(kPfConvTok, p.T - t0);
    constexpr int K = kConvK;
    if (ch < p.conv_dim) {
        const float4 w4 = *reinterpret_cast<const float4*>(p.conv_w + static_cast<size_t>(ch) * K);
        // window before token t0: inputs of tokens t0-4 .. t0-1 (taps of the incoming
        // window for tokens before the chunk)
        float win[K];
        {
            const float4 s4 = *reinterpret_cast<const float4*>(p.conv_in + static_cast<size_t>(ch) * K);
            const float st[K] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
            for (int q = 0; q < K; ++q) {
                const int tt = t0 - K + q;
                win[q] = tt >= 0 ? p.y[static_cast<size_t>(tt) * p.ld + ch] : st[q];
            }
        }
        float in[kPfConvTok];
#pragma unroll
        for (int j = 0; j < kPfConvTok; ++j) in[j] = j < nt ? p.y[static_cast<size_t>(t0 + j) * p.ld + ch] : 0.f;
        const float w[K] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int j = 0; j < kPfConvTok; ++j) {
            if (j >= nt) break;
            // window after token t0 + j: taps q hold inputs of tokens t0+j-3+q
            win[0] = win[1], win[1] = win[2], win[2] = win[3], win[3] = in[j];
            double acc = 0.0;
#pragma unroll
            for (int q = 0; q < K; ++q) acc += static_cast<double>(w[q]) * win[q];
            p.xc[static_cast<size_t>(t0 + j) * p.conv_dim + ch] = silu_f(static_cast<float>(acc));
            if (t0 + j == p.T - 1)
                *reinterpret_cast<float4*>(p.conv_out + static_cast<size_t>(ch) * K) =
                    make_float4(win[0], win[1], win[2], win[3]);
        }
    } else if (ch < p.conv_dim + p.nv) {
        const int h = ch - p.conv_dim;
        for (int j = 0; j < nt; ++j) {
            const int t = t0 + j;
            const size_t k = static_cast<size_t>(t) * p.nv + h;
            const float av = p.y[static_cast<size_t>(t) * p.ld + p.off_a + h];
            const float bv = p.y[static_cast<size_t>(t) * p.ld + p.off_b + h];
            const float g_log = -expf(p.A_log[h]) * softplus_f(av + p.dt_bias[h]);
            p.gates[2 * k] = expf(g_log);
            p.gates[2 * k + 1] = sigmoid_f(bv);
        }
    }
}

// Tokens are staged through LDS in blocks of kPfTB (q and k of the head's k-head,
// the workgroup's 32 v columns, the gates): the next block's loads are in flight
// while the current block's tokens run, so the per-token chain reads LDS only.
constexpr int kPfTB = 32;
constexpr int kPfTokFloats = 2 * kDK + kCW + 2;  // q | k | v | g, beta
// 16 threads per value column (8 state rows each): 8 waves per workgroup, twice the
// waves of the decode layout, so the per-token chains of two waves share a SIMD
constexpr int kPfCh = 16;
constexpr int kPfRows = kDK / kPfCh;
constexpr int kPfCT = kCW * kPfCh;

__global__ __launch_bounds__(kPfCT) void gdn_pf_rec_kernel(GdnPfArgs p) {
    const int tid = threadIdx.x;
    const int c = tid & (kPfCh - 1);
    const int jj = tid / kPfCh;
    const int chunks = p.dv / kCW;
    const int h = blockIdx.x / chunks, cc = blockIdx.x % chunks;
    const int j = cc * kCW + jj;
    const int rep = p.nv / p.nk;
    const int src = p.v_tiled ? (h % p.nk) : (h / rep);
    const int qdim = p.nk * kDK;
    const float qscale = 1.f / sqrtf(static_cast<float>(kDK));

    __shared__ __align__(16) float blk[2][kPfTB][kPfTokFloats];
    // per-token scales of the block, computed once per block off the recurrence's
    // dependency chain: 1/|q| * 1/sqrt(dk) and 1/|k| (eps 1e-6 inside the root)
    __shared__ float inv_s[2][kPfTB][2];
    // staging: element e of a block = (token, float index); 16-byte units where possible
    constexpr int kUnits = kPfTB * (2 * kDK + kCW) / 4;  // q, k, v as float4 units
    constexpr int kPer = (kUnits + kPfCT - 1) / kPfCT;
    float4 stg[kPer];
    float2 stg_g = make_float2(0.f, 0.f);
    auto stage_load = [&](int t0) {
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int u = tid + q * kPfCT;
            stg[q] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (u < kUnits) {
                const int tt = u / ((2 * kDK + kCW) / 4), f = (u % ((2 * kDK + kCW) / 4)) * 4;
                const int t = t0 + tt;
                if (t < p.T) {
                    const float* row = p.xc + static_cast<size_t>(t) * p.conv_dim;
                    const float* src_p = f < kDK ? row + src * kDK + f
                                                 : f < 2 * kDK ? row + qdim + src * kDK + (f - kDK)
                                                               : row + 2 * qdim + h * p.dv + cc * kCW + (f - 2 * kDK);
                    stg[q] = *reinterpret_cast<const float4*>(src_p);
                }
            }
        }
        if (tid < kPfTB && t0 + tid < p.T)
            stg_g = reinterpret_cast<const float2*>(p.gates)[static_cast<size_t>(t0 + tid) * p.nv + h];
    };
    auto stage_store = [&](int buf) {
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int u = tid + q * kPfCT;
            if (u < kUnits) {
                const int tt = u / ((2 * kDK + kCW) / 4), f = (u % ((2 * kDK + kCW) / 4)) * 4;
                *reinterpret_cast<float4*>(&blk[buf][tt][f]) = stg[q];
            }
        }
        if (tid < kPfTB) {
            blk[buf][tid][2 * kDK + kCW] = stg_g.x;
            blk[buf][tid][2 * kDK + kCW + 1] = stg_g.y;
        }
    };
    // after a block is in LDS: 8 lanes per (token, q|k) vector, 16 values each
    auto block_norms = [&](int buf) {
        const int v = tid >> 3, part = tid & 7;  // v = 2 * token + (0: q, 1: k)
        const float* x = &blk[buf][v >> 1][(v & 1) * kDK + 16 * part];
        float a4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < 16; ++r) a4[r & 3] = fmaf(x[r], x[r], a4[r & 3]);
        const float sum = group8_sum((a4[0] + a4[1]) + (a4[2] + a4[3]));
        if (part == 0) inv_s[buf][v >> 1][v & 1] = (v & 1) ? 1.f / sqrtf(sum + 1e-6f) : 1.f / sqrtf(sum + 1e-6f) * qscale;
    };

    const size_t s_off = (static_cast<size_t>(h) * p.dv + j) * kDK + kPfRows * c;
    float S[kPfRows];
    {
        const f32x4* sp = reinterpret_cast<const f32x4*>(p.S + s_off);
#pragma unroll
        for (int r = 0; r < kPfRows / 4; ++r) {
            const f32x4 v = sp[r];
            S[4 * r] = v[0];
            S[4 * r + 1] = v[1];
            S[4 * r + 2] = v[2];
            S[4 * r + 3] = v[3];
        }
    }
    stage_load(0);
    stage_store(0);
    __syncthreads();
    block_norms(0);
    __syncthreads();
    for (int t0 = 0; t0 < p.T; t0 += kPfTB) {
        const int buf = (t0 / kPfTB) & 1;
        const bool more = t0 + kPfTB < p.T;
        if (more) stage_load(t0 + kPfTB);
        const int nt = min(kPfTB, p.T - t0);
        for (int tt = 0; tt < nt; ++tt) {
            const float* tk = blk[buf][tt];
            float q[kPfRows], k[kPfRows];
#pragma unroll
            for (int r = 0; r < kPfRows / 4; ++r) {
                const float4 a4 = *reinterpret_cast<const float4*>(tk + kPfRows * c + 4 * r);
                const float4 b4 = *reinterpret_cast<const float4*>(tk + kDK + kPfRows * c + 4 * r);
                q[4 * r] = a4.x, q[4 * r + 1] = a4.y, q[4 * r + 2] = a4.z, q[4 * r + 3] = a4.w;
                k[4 * r] = b4.x, k[4 * r + 1] = b4.y, k[4 * r + 2] = b4.z, k[4 * r + 3] = b4.w;
            }
            const float v = tk[2 * kDK + jj];
            const float g = tk[2 * kDK + kCW], beta = tk[2 * kDK + kCW + 1];
            const float iq = inv_s[buf][tt][0], ik = inv_s[buf][tt][1];
            float kv4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int r = 0; r < kPfRows; ++r) {
                k[r] *= ik;
                S[r] *= g;
                kv4[r & 3] = fmaf(S[r], k[r], kv4[r & 3]);
            }
            const float kv = group16_sum((kv4[0] + kv4[1]) + (kv4[2] + kv4[3]));
            const float delta = (v - kv) * beta;
            float ov4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int r = 0; r < kPfRows; ++r) {
                S[r] = fmaf(k[r], delta, S[r]);
                ov4[r & 3] = fmaf(S[r], q[r] * iq, ov4[r & 3]);
            }
            const float ov = group16_sum((ov4[0] + ov4[1]) + (ov4[2] + ov4[3]));
            if (c == 0)
                p.o[static_cast<size_t>(t0 + tt) * p.nv * p.dv + static_cast<size_t>(h) * p.dv + j] = ov;
        }
        if (more) stage_store(buf ^ 1);
        __syncthreads();
        if (more) {
            block_norms(buf ^ 1);
            __syncthreads();
        }
    }
    f32x4* dp = reinterpret_cast<f32x4*>(p.S + s_off);
#pragma unroll
    for (int r = 0; r < kPfRows / 4; ++r) dp[r] = f32x4{S[4 * r], S[4 * r + 1], S[4 * r + 2], S[4 * r + 3]};
}


// ---- chunked prefill scan (gated delta rule in WY form over chunks of 64 tokens)
// Within a chunk with cumulative log decays la_t = sum_{s<=t} log g_s, the per-token
// recurrence (decay, delta rule, output) is the same as
//   (I + A) X = diag(beta) [V | diag(gamma) K],  A[t][i] = beta_t G[t][i] k_t.k_i (i < t),
//   X = [U~ | W~],  U = U~ - W~ S0,
//   O = diag(gamma) Q S0 + (M o U),  M[t][i] = G[t][i] q_t.k_i (i <= t),
//   S  = gamma_C S0 + K~^T U,         K~ = diag(gamma_C / gamma_i) K,
// with gamma_t = exp(la_t), G[t][i] = exp(la_t - la_i) (never a division, so no
// overflow however strong the decay).  gdn_pf_chunk_prep builds everything that
// does not depend on S0 for all chunks at once (one workgroup per (v-head, chunk));
// gdn_pf_chunk_scan then runs the chunks in order, one workgroup per (v-head,
// 16 value columns), the state block in MFMA accumulators (fp32 16x16x4: exact
// fp32 products, fp32 sums).
constexpr int kCk = 64;          // tokens per chunk
constexpr int kCkStride = kDK + 4;  // LDS row stride of q / k (floats)
constexpr int kCkA = kCk + 4;       // LDS row stride of A
// one (v-head, chunk) block of the workspace: U~ [64][128] | W~ [64][128] |
// gamma Q [64][128] | K~^T [128][64] | M [64][64]
constexpr size_t kCkFloats = 4 * static_cast<size_t>(kCk) * kDK + static_cast<size_t>(kCk) * kCk;

__device__ inline f32x4 mfma_f32_4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Tile pairs (t block, i block) of the 64 x 64 chunk matrices in 16 x 16 tiles:
// the ten on or below the diagonal first, so that wave w's jobs w, w+4, w+8, w+12
// hold two or three of them.
__constant__ unsigned char kCkPairs[16][2] = {{0, 0}, {1, 0}, {1, 1}, {2, 0}, {2, 1}, {2, 2}, {3, 0}, {3, 1},
                                              {3, 2}, {3, 3}, {0, 1}, {0, 2}, {0, 3}, {1, 2}, {1, 3}, {2, 3}};

__global__ __launch_bounds__(256, 2) void gdn_pf_chunk_prep_kernel(GdnPfArgs p, float* ws, float* gc, int nch) {
    const int h = blockIdx.x, c = blockIdx.y, tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63, r = lane & 15, g = lane >> 4;
    const int t0 = c * kCk, n = min(kCk, p.T - t0);
    const int rep = p.nv / p.nk;
    const int src = p.v_tiled ? (h % p.nk) : (h / rep);
    const int qdim = p.nk * kDK;
    const float qscale = 1.f / sqrtf(static_cast<float>(kDK));
    __shared__ __align__(16) float q_s[kCk][kCkStride];  // after the products: A [64][kCkA]
    __shared__ __align__(16) float k_s[kCk][kCkStride];
    __shared__ double la_s[kCk];
    __shared__ float beta_s[kCk];
    float(*a_s)[kCkA] = reinterpret_cast<float(*)[kCkA]>(&q_s[0][0]);
    static_assert(kCk * kCkA <= kCk * kCkStride, "A fits in the q buffer");

    float* blk = ws + (static_cast<size_t>(h) * nch + c) * kCkFloats;
    float* ut = blk;
    float* wt = ut + kCk * kDK;
    float* qg = wt + kCk * kDK;
    float* ktT = qg + kCk * kDK;
    float* m = ktT + kDK * kCk;

    // q and k of the chunk's tokens (zeros past the last token), gates
    for (int u = tid; u < kCk * (2 * kDK / 4); u += 256) {
        const int tt = u / (2 * kDK / 4), f = (u % (2 * kDK / 4)) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (tt < n) {
            const float* row = p.xc + static_cast<size_t>(t0 + tt) * p.conv_dim;
            v = *reinterpret_cast<const float4*>(f < kDK ? row + src * kDK + f : row + qdim + src * kDK + (f - kDK));
        }
        *reinterpret_cast<float4*>(f < kDK ? &q_s[tt][f] : &k_s[tt][f - kDK]) = v;
    }
    // each thread's value column of V (threads 128 .. 255: the W~ columns, later)
    float x[kCk];
    const int col = tid;
    if (col < kDK) {
        const float* vp = p.xc + static_cast<size_t>(t0) * p.conv_dim + 2 * qdim + h * p.dv + col;
#pragma unroll
        for (int t = 0; t < kCk; ++t) x[t] = t < n ? vp[static_cast<size_t>(t) * p.conv_dim] : 0.f;
    }
    if (w == 0) {
        // log of the decay the recurrence multiplies by (a decay that underflowed to
        // 0 becomes exp(-150), itself 0 in fp32), summed over the chunk in double
        float2 gb = make_float2(1.f, 0.f);
        if (lane < n) gb = reinterpret_cast<const float2*>(p.gates)[static_cast<size_t>(t0 + lane) * p.nv + h];
        double la = gb.x > 0.f ? static_cast<double>(fmaxf(logf(gb.x), -150.f)) : -150.0;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const double o = __shfl_up(la, d);
            if (lane >= d) la += o;
        }
        la_s[lane] = la;
        beta_s[lane] = gb.y;
    }
    __syncthreads();
    // L2 norms: two threads per vector (q of token v, or k of token v - 64)
    {
        const int v = tid >> 1, half = tid & 1;
        float* xv = v < kCk ? &q_s[v][64 * half] : &k_s[v - kCk][64 * half];
        float a4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 64; ++i) a4[i & 3] = fmaf(xv[i], xv[i], a4[i & 3]);
        float sum = (a4[0] + a4[1]) + (a4[2] + a4[3]);
        sum += __shfl_xor(sum, 1);
        const float inv = v < kCk ? 1.f / sqrtf(sum + 1e-6f) * qscale : 1.f / sqrtf(sum + 1e-6f);
#pragma unroll
        for (int i = 0; i < 64; ++i) xv[i] *= inv;
    }
    __syncthreads();
    // gamma Q rows (q is not needed after the products below)
    for (int u = tid; u < kCk * kDK / 4; u += 256) {
        const int t = u / (kDK / 4), d = (u % (kDK / 4)) * 4;
        const float gm = expf(static_cast<float>(la_s[t]));
        const float4 qv = *reinterpret_cast<const float4*>(&q_s[t][d]);
        *reinterpret_cast<float4*>(qg + t * kDK + d) = make_float4(gm * qv.x, gm * qv.y, gm * qv.z, gm * qv.w);
    }
    // K K^T and Q K^T by 16 x 16 tiles on MFMA; M to memory, A kept until q is free
    f32x4 at[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
        const int job = w + 4 * jb;
        const int tb = kCkPairs[job][0], ib = kCkPairs[job][1];
        f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = {0.f, 0.f, 0.f, 0.f};
        if (job < 10) {
#pragma unroll
            for (int s = 0; s < kDK / 16; ++s) {
                const float4 ka = *reinterpret_cast<const float4*>(&k_s[16 * tb + r][16 * s + 4 * g]);
                const float4 qa = *reinterpret_cast<const float4*>(&q_s[16 * tb + r][16 * s + 4 * g]);
                const float4 kb = *reinterpret_cast<const float4*>(&k_s[16 * ib + r][16 * s + 4 * g]);
                kk = mfma_f32_4(ka.x, kb.x, kk);
                qk = mfma_f32_4(qa.x, kb.x, qk);
                kk = mfma_f32_4(ka.y, kb.y, kk);
                qk = mfma_f32_4(qa.y, kb.y, qk);
                kk = mfma_f32_4(ka.z, kb.z, kk);
                qk = mfma_f32_4(qa.z, kb.z, qk);
                kk = mfma_f32_4(ka.w, kb.w, kk);
                qk = mfma_f32_4(qa.w, kb.w, qk);
            }
        }
        const int i = 16 * ib + r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = 16 * tb + 4 * g + e;
            const float G = i <= t ? expf(static_cast<float>(la_s[t] - la_s[i])) : 0.f;
            at[jb][e] = i < t ? beta_s[t] * G * kk[e] : 0.f;
            m[t * kCk + i] = G * qk[e];
        }
    }
    __syncthreads();
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
        const int job = w + 4 * jb;
        const int tb = kCkPairs[job][0], ib = kCkPairs[job][1];
#pragma unroll
        for (int e = 0; e < 4; ++e) a_s[16 * tb + 4 * g + e][16 * ib + r] = at[jb][e];
    }
    __syncthreads();

    // forward substitution, one right-hand column per thread: V (U~) or gamma K (W~)
    if (col >= kDK) {
#pragma unroll
        for (int t = 0; t < kCk; ++t) x[t] = expf(static_cast<float>(la_s[t])) * k_s[t][col - kDK];
    }
#pragma unroll
    for (int t = 0; t < kCk; ++t) {
        float s4[4] = {beta_s[t] * x[t], 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < t; ++i) s4[i & 3] = fmaf(-a_s[t][i], x[i], s4[i & 3]);
        x[t] = (s4[0] + s4[1]) + (s4[2] + s4[3]);
    }
    {
        float* dst = col < kDK ? ut + col : wt + (col - kDK);
#pragma unroll
        for (int t = 0; t < kCk; ++t) dst[t * kDK] = x[t];
    }
    // K~ transposed
    for (int u = tid; u < kDK * kCk / 4; u += 256) {
        const int d = u / (kCk / 4), t = (u % (kCk / 4)) * 4;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            v[e] = expf(static_cast<float>(la_s[n - 1] - la_s[t + e])) * k_s[t + e][d];
        *reinterpret_cast<float4*>(ktT + d * kCk + t) = make_float4(v[0], v[1], v[2], v[3]);
    }
    if (tid == 0) gc[static_cast<size_t>(h) * nch + c] = expf(static_cast<float>(la_s[n - 1]));
}


// Barrier for LDS hand-offs only: waits for this wave's LDS traffic, not for its
// global loads (a __syncthreads drains those too, which would stall the next
// chunk's prefetch).
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// A-operand registers of one chunk for one lane (row r = lane % 16, k group
// g = lane / 16), in two sets loaded at different points of the previous chunk so
// that at most three sets are live: first W~ and gamma Q rows of the wave's tokens
// and U~ at the lane's four output rows of each column tile, then the M row and
// K~^T rows of the wave's two state tiles.
template <int NCT>
struct CkOpsA {
    float4 wa[kDK / 16], qa[kDK / 16];
    float uu[NCT][4];
};
struct CkOpsB {
    float4 ma[kCk / 16], ka[2][kCk / 16];
    float gC;
};

// One workgroup per (v-head, 16 NCT value columns), 4 waves.  Wave w owns token
// rows 16w .. 16w+15 of U and O, and state rows 32w .. 32w+31 (two 16 x 16 MFMA
// tiles per 16-column tile, lane l holding rows 4(l/16) .. +3 of column l%16);
// each A operand feeds NCT MFMAs.  LDS holds the state block and U transposed,
// the B operands every wave reads.  The next chunk's A operands load while the
// current chunk computes.
template <int NCT>
__global__ __launch_bounds__(256, 3 - NCT) void gdn_pf_chunk_scan_kernel(GdnPfArgs p, const float* ws,
                                                                         const float* gc, int nch) {
    constexpr int NC = 16 * NCT;  // value columns per workgroup
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, r = lane & 15, g = lane >> 4;
    // consecutive workgroups take different heads, so the column blocks of one head
    // (which read the same chunk data) share an XCD when nv is a multiple of 8
    const int h = blockIdx.x % p.nv, j0 = (blockIdx.x / p.nv) * NC;
    __shared__ __align__(16) float st_s[NC][kDK + 4];  // state block transposed: [column][key row]
    __shared__ __align__(16) float ut_s[NC][kCk + 4];  // U transposed: [column][token]
    const int row = 16 * w + r;
    auto blk = [&](int c) { return ws + (static_cast<size_t>(h) * nch + c) * kCkFloats; };
    auto load_a = [&](int c, CkOpsA<NCT>& o) {
        const float* ut = blk(c);
        const float* wt = ut + kCk * kDK;
        const float* qg = wt + kCk * kDK;
#pragma unroll
        for (int s = 0; s < kDK / 16; ++s) {
            o.wa[s] = *reinterpret_cast<const float4*>(wt + row * kDK + 16 * s + 4 * g);
            o.qa[s] = *reinterpret_cast<const float4*>(qg + row * kDK + 16 * s + 4 * g);
        }
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
            for (int e = 0; e < 4; ++e) o.uu[ct][e] = ut[(16 * w + 4 * g + e) * kDK + j0 + 16 * ct + r];
    };
    auto load_b = [&](int c, CkOpsB& o) {
        const float* ktT = blk(c) + 3 * kCk * kDK;
        const float* m = ktT + kDK * kCk;
#pragma unroll
        for (int s = 0; s < kCk / 16; ++s) {
            o.ma[s] = *reinterpret_cast<const float4*>(m + row * kCk + 16 * s + 4 * g);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
                o.ka[tt][s] = *reinterpret_cast<const float4*>(ktT + (32 * w + 16 * tt + r) * kCk + 16 * s + 4 * g);
        }
        o.gC = gc[static_cast<size_t>(h) * nch + c];
    };
    f32x4 sreg[NCT][2];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int i0 = 32 * w + 16 * tt + 4 * g;
            sreg[ct][tt] = *reinterpret_cast<const f32x4*>(p.S + (static_cast<size_t>(h) * p.dv + j0 + 16 * ct + r) *
                                                                       kDK + i0);
            *reinterpret_cast<f32x4*>(&st_s[16 * ct + r][i0]) = sreg[ct][tt];
        }
    const size_t ldo = static_cast<size_t>(p.nv) * p.dv;
    // chunk c from operands (ac, bc); loads chunk c + 1's into (an, bn) on the way
    // (the last chunk reloads itself: no branch, nothing read out of bounds)
    auto chunk = [&](int c, const CkOpsA<NCT>& ac, const CkOpsB& bc, CkOpsA<NCT>& an, CkOpsB& bn)
        __attribute__((always_inline)) {
        const int cn = min(c + 1, nch - 1);
        load_b(cn, bn);
        const int n = min(kCk, p.T - c * kCk);
        // W~ S and gamma Q S for the wave's 16 tokens (K = 128 key rows)
        const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
        f32x4 au[NCT], ao[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) au[ct] = ao[ct] = z4;
#pragma unroll
        for (int s = 0; s < kDK / 16; ++s) {
            const float4 wa = ac.wa[s], qa = ac.qa[s];
            float4 sb[NCT];
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) sb[ct] = *reinterpret_cast<const float4*>(&st_s[16 * ct + r][16 * s + 4 * g]);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
                au[ct] = mfma_f32_4(wa.x, sb[ct].x, au[ct]);
                ao[ct] = mfma_f32_4(qa.x, sb[ct].x, ao[ct]);
                au[ct] = mfma_f32_4(wa.y, sb[ct].y, au[ct]);
                ao[ct] = mfma_f32_4(qa.y, sb[ct].y, ao[ct]);
                au[ct] = mfma_f32_4(wa.z, sb[ct].z, au[ct]);
                ao[ct] = mfma_f32_4(qa.z, sb[ct].z, ao[ct]);
                au[ct] = mfma_f32_4(wa.w, sb[ct].w, au[ct]);
                ao[ct] = mfma_f32_4(qa.w, sb[ct].w, ao[ct]);
            }
        }
        // U = U~ - W~ S (rows 16w + 4g + e, column 16 ct + r)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
            f32x4 u;
#pragma unroll
            for (int e = 0; e < 4; ++e) u[e] = ac.uu[ct][e] - au[ct][e];
            *reinterpret_cast<f32x4*>(&ut_s[16 * ct + r][16 * w + 4 * g]) = u;
        }
        load_a(cn, an);
        lds_barrier();
        // O += M U over tokens 0 .. 16w+15 (M is zero above the diagonal)
#pragma unroll
        for (int s = 0; s < kCk / 16; ++s) {
            if (s > w) break;
            const float4 ma = bc.ma[s];
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
                const float4 ub = *reinterpret_cast<const float4*>(&ut_s[16 * ct + r][16 * s + 4 * g]);
                ao[ct] = mfma_f32_4(ma.x, ub.x, ao[ct]);
                ao[ct] = mfma_f32_4(ma.y, ub.y, ao[ct]);
                ao[ct] = mfma_f32_4(ma.z, ub.z, ao[ct]);
                ao[ct] = mfma_f32_4(ma.w, ub.w, ao[ct]);
            }
        }
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = 16 * w + 4 * g + e;
                if (t < n)
                    p.o[static_cast<size_t>(c * kCk + t) * ldo + static_cast<size_t>(h) * p.dv + j0 + 16 * ct + r] =
                        ao[ct][e];
            }
        // S = gamma_C S + K~^T U (2 NCT independent accumulator chains)
        f32x4 acc[NCT][2];
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) acc[ct][0] = sreg[ct][0] * bc.gC, acc[ct][1] = sreg[ct][1] * bc.gC;
#pragma unroll
        for (int s = 0; s < kCk / 16; ++s) {
            float4 ub[NCT];
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) ub[ct] = *reinterpret_cast<const float4*>(&ut_s[16 * ct + r][16 * s + 4 * g]);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                    for (int ct = 0; ct < NCT; ++ct) {
                        const float4 ka = bc.ka[tt][s];
                        const float av = q == 0 ? ka.x : q == 1 ? ka.y : q == 2 ? ka.z : ka.w;
                        const float bv = q == 0 ? ub[ct].x : q == 1 ? ub[ct].y : q == 2 ? ub[ct].z : ub[ct].w;
                        acc[ct][tt] = mfma_f32_4(av, bv, acc[ct][tt]);
                    }
        }
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                sreg[ct][tt] = acc[ct][tt];
                *reinterpret_cast<f32x4*>(&st_s[16 * ct + r][32 * w + 16 * tt + 4 * g]) = acc[ct][tt];
            }
        lds_barrier();
    };
    // two operand sets in turn (no register copies between chunks, which would
    // wait for the prefetch)
    CkOpsA<NCT> a0, a1;
    CkOpsB b0, b1;
    load_a(0, a0);
    load_b(0, b0);
    lds_barrier();
    int c = 0;
    for (; c + 1 < nch; c += 2) {
        chunk(c, a0, b0, a1, b1);
        chunk(c + 1, a1, b1, a0, b0);
    }
    if (c < nch) chunk(c, a0, b0, a1, b1);
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
            *reinterpret_cast<f32x4*>(p.S + (static_cast<size_t>(h) * p.dv + j0 + 16 * ct + r) * kDK + 32 * w +
                                      16 * tt + 4 * g) = sreg[ct][tt];
}

}  // namespace

namespace rl {

bool gdn_fused_supported(int dk, int dv, int K) { return dk == kDK && dv % kCW == 0 && dv > 0 && K == kConvK; }

void gdn_decode_fused(const float* qkv, const float* a, const float* b, int ld_in, const float* A_log,
                      const float* dt_bias, const float* conv_w, const float* conv_in, float* conv_out,
                      const float* S_in, float* S_out, const int* cur, size_t conv_slot, int R,
                      const GdnRecords* rec, float* o, const float* z, const float* gamma, void* frag, float* gss,
                      int T, int nk, int nv, int dk, int dv, int K, int v_tiled, hipStream_t s, int ab_slices,
                      int ab_ld, const GdnBatch* batch, int row_off, int T_rows, float* y32) {
    RL_REQUIRE(gdn_fused_supported(dk, dv, K), RL_ERR_UNSUPPORTED,
               "gdn_decode_fused: dk 128, dv a multiple of 32, conv 4");
    RL_REQUIRE(T >= 1 && T <= kMaxT, RL_ERR_RANGE, "gdn_decode_fused: T must be in 1..8");
    RL_REQUIRE(nk > 0 && nv > 0 && nv % nk == 0, RL_ERR_RANGE, "gdn_decode_fused: nv must be a multiple of nk");
    RL_REQUIRE(qkv && a && b && A_log && dt_bias && conv_w && conv_in && S_in && S_out && (o || frag || y32),
               RL_ERR_RANGE, "gdn_decode_fused: null pointer");
    RL_REQUIRE((!frag && !y32) || (z && gamma && gss && dv == 4 * kCW), RL_ERR_RANGE,
               "gdn_decode_fused: the gated norm needs z, gamma, gss and dv 128");
    if (cur) {
        RL_REQUIRE(R > T, RL_ERR_RANGE, "gdn_decode_fused: ring needs more slots than tokens");
        RL_REQUIRE(rec && rec->rec && rec->count && rec->n_cons && rec->max_t >= T && S_out == S_in, RL_ERR_RANGE,
                   "gdn_decode_fused: the conv ring needs records and one committed state");
    } else {
        RL_REQUIRE(!rec && conv_out && conv_out != conv_in, RL_ERR_RANGE, "gdn_decode_fused: bad conv output");
    }
    RL_REQUIRE(ab_slices >= 1 && ab_slices <= kMaxAbSlices, RL_ERR_RANGE, "gdn_decode_fused: 1..8 a/b slices");
    GdnFusedArgs p{{qkv, a, b, ld_in, A_log, dt_bias, conv_w, conv_in, conv_out, S_in, S_out, cur, conv_slot, 0, R,
                    o, T, nk, nv, dv, K, v_tiled, ab_slices, ab_slices > 1 ? ab_ld : ld_in},
                   z,
                   gamma,
                   static_cast<i32x4*>(frag),
                   gss,
                   y32,
                   rec ? *rec : GdnRecords{nullptr, nullptr, nullptr, 0, 0},
                   batch ? *batch : GdnBatch{},
                   row_off,
                   T_rows};
    RL_REQUIRE(T_rows == 0 || (p.batch.B == 1 && row_off >= 0 && row_off + T <= T_rows), RL_ERR_RANGE,
               "gdn_decode_fused: token rows out of range");
    // T tokens per sequence (its per-token arrays), B sequences as grid rows; the
    // token rows of all sequences (B x T) are only indexed in the global buffers
    RL_REQUIRE(p.batch.B >= 1 && p.batch.B <= 16 && T <= kMaxT && p.batch.B * T <= 16, RL_ERR_RANGE,
               "gdn_decode_fused: T <= 8 tokens and B x T <= 16 rows");
    RL_REQUIRE(p.batch.B == 1 || cur, RL_ERR_RANGE, "gdn_decode_fused: a batch needs the conv ring");
    const dim3 grid(nv * (dv / kCW), p.batch.B);
    switch (T) {
    case 1: hipLaunchKernelGGL(gdn_fused_kernel<1>, grid, dim3(kCT), 0, s, p); break;
    case 2: hipLaunchKernelGGL(gdn_fused_kernel<2>, grid, dim3(kCT), 0, s, p); break;
    case 3: hipLaunchKernelGGL(gdn_fused_kernel<3>, grid, dim3(kCT), 0, s, p); break;
    case 4: hipLaunchKernelGGL(gdn_fused_kernel<4>, grid, dim3(kCT), 0, s, p); break;
    default: hipLaunchKernelGGL(gdn_fused_kernel<0>, grid, dim3(kCT), 0, s, p); break;
    }
    check_launch("gdn_fused_kernel");
}

void gdn_decode(const float* qkv, const float* a, const float* b, int ld_in, const float* A_log, const float* dt_bias,
                const float* conv_w, const float* conv_in, float* conv_out, const float* S_in, float* S_out,
                const int* cur, size_t conv_slot, size_t s_slot, int R, float* o, int T, int nk, int nv, int dk,
                int dv, int K, int v_tiled, hipStream_t s) {
    RL_REQUIRE(dk == kDK, RL_ERR_UNSUPPORTED, "gdn_decode: key head dim must be 128");
    RL_REQUIRE(dv % 32 == 0 && dv > 0, RL_ERR_UNSUPPORTED, "gdn_decode: value head dim must be a multiple of 32");
    RL_REQUIRE(T >= 1 && T <= kMaxT, RL_ERR_RANGE, "gdn_decode: T must be in 1..8");
    RL_REQUIRE(K == kConvK, RL_ERR_UNSUPPORTED, "gdn_decode: conv width must be 4");
    RL_REQUIRE(nk > 0 && nv > 0 && nv % nk == 0, RL_ERR_RANGE, "gdn_decode: nv must be a multiple of nk");
    RL_REQUIRE(qkv && a && b && A_log && dt_bias && conv_w && conv_in && S_in && o, RL_ERR_RANGE,
               "gdn_decode: null pointer");
    if (cur) {
        RL_REQUIRE(R > T, RL_ERR_RANGE, "gdn_decode: ring needs more slots than tokens");
    } else {
        RL_REQUIRE(conv_out && S_out, RL_ERR_RANGE, "gdn_decode: null output state");
        RL_REQUIRE(conv_out != conv_in, RL_ERR_RANGE, "gdn_decode: conv_out must not alias conv_in");
    }
    GdnArgs p{qkv, a, b, ld_in, A_log, dt_bias, conv_w, conv_in, conv_out, S_in, S_out, cur, conv_slot, s_slot, R,
              o, T, nk, nv, dv, K, v_tiled};
    hipLaunchKernelGGL(gdn_decode_kernel, dim3(nv * (dv / kCols)), dim3(256), 0, s, p);
    check_launch("gdn_decode_kernel");
}


void gdn_prefill(const float* y, int ld, int off_a, int off_b, const float* A_log, const float* dt_bias,
                 const float* conv_w, const float* conv_in, float* conv_out, float* xc, float* gates, float* S,
                 float* o, int T, int nk, int nv, int dk, int dv, int K, int v_tiled, hipStream_t s, float* ck) {
    RL_REQUIRE(gdn_fused_supported(dk, dv, K), RL_ERR_UNSUPPORTED, "gdn_prefill: dk 128, dv a multiple of 32, conv 4");
    RL_REQUIRE(T >= 1 && nk > 0 && nv > 0 && nv % nk == 0, RL_ERR_RANGE, "gdn_prefill: bad shape");
    RL_REQUIRE(y && A_log && dt_bias && conv_w && conv_in && conv_out && xc && gates && S && o, RL_ERR_RANGE,
               "gdn_prefill: null pointer");
    RL_REQUIRE(conv_out != conv_in, RL_ERR_RANGE, "gdn_prefill: conv_out must not alias conv_in");
    const int conv_dim = 2 * nk * dk + nv * dv;
    GdnPfArgs p{y, ld, off_a, off_b, A_log, dt_bias, conv_w, conv_in, conv_out, xc, gates, S, o,
                T, nk, nv, dv, conv_dim, v_tiled};
    RL_REQUIRE(T <= 65535, RL_ERR_RANGE, "gdn_prefill: at most 65535 tokens per call");
    hipLaunchKernelGGL(gdn_pf_conv_kernel, dim3((conv_dim + nv + 255) / 256, (T + kPfConvTok - 1) / kPfConvTok),
                       dim3(256), 0, s, p);
    check_launch("gdn_pf_conv_kernel");
    if (ck && gdn_prefill_chunk_floats(T, nv, dk, dv) > 0) {
        const int nch = (T + kCk - 1) / kCk;
        float* gc = ck + static_cast<size_t>(nv) * nch * kCkFloats;
        hipLaunchKernelGGL(gdn_pf_chunk_prep_kernel, dim3(nv, nch), dim3(256), 0, s, p, ck, gc, nch);
        check_launch("gdn_pf_chunk_prep_kernel");
        static const int nct = [] {
            const char* e = std::getenv("RL_PF_GDN_NCT");  // measurement override
            return e && e[0] == '1' ? 1 : 2;
        }();
        if (nct == 2)
            hipLaunchKernelGGL(gdn_pf_chunk_scan_kernel<2>, dim3(nv * (dv / 32)), dim3(256), 0, s, p,
                               static_cast<const float*>(ck), static_cast<const float*>(gc), nch);
        else
            hipLaunchKernelGGL(gdn_pf_chunk_scan_kernel<1>, dim3(nv * (dv / 16)), dim3(256), 0, s, p,
                               static_cast<const float*>(ck), static_cast<const float*>(gc), nch);
        check_launch("gdn_pf_chunk_scan_kernel");
        return;
    }
    hipLaunchKernelGGL(gdn_pf_rec_kernel, dim3(nv * (dv / kCW)), dim3(kPfCT), 0, s, p);
    check_launch("gdn_pf_rec_kernel");
}

bool gdn_prefill_chunked() {
    const char* env = std::getenv("RL_PF_GDN_CHUNK");  // measurement override, read per call
    return !(env && env[0] == '0');
}

size_t gdn_prefill_chunk_floats(int T, int nv, int dk, int dv) {
    if (dk != kDK || dv != kDK || T < 1 || nv < 1) return 0;
    const size_t nch = static_cast<size_t>((T + kCk - 1) / kCk);
    return static_cast<size_t>(nv) * nch * (kCkFloats + 1);
}

}  // namespace rl

extern "C" {

int rl_hip_gdn_decode(const float* qkv, const float* a, const float* b, int ld_in, const float* A_log,
                      const float* dt_bias, const float* conv_w, const float* conv_in, float* conv_out,
                      const float* S_in, float* S_out, float* o, int T, int nk, int nv, int dk, int dv, int conv_k,
                      int v_tiled, void* stream) {
    return guard([&] {
        if (rl::gdn_fused_supported(dk, dv, conv_k))
            rl::gdn_decode_fused(qkv, a, b, ld_in, A_log, dt_bias, conv_w, conv_in, conv_out, S_in, S_out, nullptr,
                                 0, 0, nullptr, o, nullptr, nullptr, nullptr, nullptr, T, nk, nv, dk, dv, conv_k,
                                 v_tiled, S(stream));
        else
            rl::gdn_decode(qkv, a, b, ld_in, A_log, dt_bias, conv_w, conv_in, conv_out, S_in, S_out, nullptr, 0, 0,
                           0, o, T, nk, nv, dk, dv, conv_k, v_tiled, S(stream));
    });
}

size_t rl_hip_gdn_prefill_workspace_bytes(int T, int nk, int nv, int dk, int dv) {
    return (static_cast<size_t>(T) * (2 * nk * dk + nv * dv) + static_cast<size_t>(T) * nv * 2 +
            rl::gdn_prefill_chunk_floats(T, nv, dk, dv)) * sizeof(float) + 256;
}

int rl_hip_gdn_prefill(const float* y, int ld, int off_a, int off_b, const float* A_log, const float* dt_bias,
                       const float* conv_w, const float* conv_in, float* conv_out, float* S_state, float* o,
                       void* workspace, size_t workspace_bytes, int T, int nk, int nv, int dk, int dv, int conv_k,
                       int v_tiled, void* stream) {
    return guard([&] {
        RL_REQUIRE(workspace && workspace_bytes >= rl_hip_gdn_prefill_workspace_bytes(T, nk, nv, dk, dv),
                   RL_ERR_RANGE, "gdn_prefill: workspace too small");
        float* xc = static_cast<float*>(workspace);
        float* gates = xc + static_cast<size_t>(T) * (2 * nk * dk + nv * dv);
        float* ck = gates + static_cast<size_t>(T) * nv * 2;
        rl::gdn_prefill(y, ld, off_a, off_b, A_log, dt_bias, conv_w, conv_in, conv_out, xc, gates, S_state, o, T, nk,
                        nv, dk, dv, conv_k, v_tiled, S(stream), rl::gdn_prefill_chunked() ? ck : nullptr);
    });
}

}  // extern "C"
