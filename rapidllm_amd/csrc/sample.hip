// sample.hip -- greedy argmax over logits rows and on-device speculative acceptance.
//
// argmax: first index wins ties, as greedy_sample (reference src/runtime/
// sampler.cpp:8-18) and the CUDA argmax_partial_rows_k / argmax_final_rows_k
// (src/kernels/cuda/cuda_engine.cu:9375-9433).  Two passes: per-chunk (value, index)
// partials, then one wave per row.
//
// accept: greedy prefix acceptance of the reference CPU session
// (src/runtime/session.cpp:802-825) and the contract of Engine::spec_verify
// (include/rapidllm/runtime/cuda_engine.h:69-77): toks = [t0, d1..d(T-1)],
// preds[i] = greedy after toks[i]; n = 1 + longest prefix with preds[i] == toks[i+1].
// It advances the device position and recurrent-state slot by n, so the next step
// runs without a host round trip.
#include <algorithm>

#include "internal.h"

using namespace rl;

namespace {

constexpr int kArgChunk = 1024;  // 4 values per thread, loaded together

__device__ inline bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ logits, int V,
                                                             float* __restrict__ pv, int* __restrict__ pi,
                                                             int nchunks) {
    const int row = blockIdx.y, chunk = blockIdx.x;
    const float* x = logits + static_cast<size_t>(row) * V;
    const int b = chunk * kArgChunk, e = min(V, b + kArgChunk);
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    float vals[kArgChunk / 256];
#pragma unroll
    for (int k = 0; k < kArgChunk / 256; ++k) {
        const int i = b + threadIdx.x + 256 * k;
        vals[k] = i < e ? x[i] : -INFINITY;
    }
#pragma unroll
    for (int k = 0; k < kArgChunk / 256; ++k) {
        const int i = b + threadIdx.x + 256 * k;
        if (i < e && better(vals[k], i, bv, bi)) {
            bv = vals[k];
            bi = i;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    __shared__ float sv[4];
    __shared__ int si[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w)
            if (better(sv[w], si[w], bv, bi)) {
                bv = sv[w];
                bi = si[w];
            }
        // a chunk of all -inf / NaN keeps its first index
        if (bi == 0x7fffffff) bi = b;
        pv[row * nchunks + chunk] = bv;
        pi[row * nchunks + chunk] = bi;
    }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ pv, const int* __restrict__ pi,
                                                          int nchunks, int* __restrict__ out,
                                                          float* __restrict__ out_val) {
    const int row = blockIdx.x;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int c = threadIdx.x; c < nchunks; c += 64) {
        const float v = pv[row * nchunks + c];
        const int i = pi[row * nchunks + c];
        if (better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (threadIdx.x == 0) {
        out[row] = bi == 0x7fffffff ? 0 : bi;
        if (out_val) out_val[row] = bv;
    }
}

struct AcceptArgs {
    const int* toks;   // [T]
    const int* preds;  // [T]
    int T;
    int force_all;     // prefill: consume every token
    int* pos;          // advanced by n
    int* slot;         // recurrent-state ring slot, advanced by n mod R (may be null)
    int R;
    int* n_out;        // n consumed
    int* next_tok;     // preds[n-1]: the next token to feed
    int* gen_ring;     // optional: appended accepted outputs (preds[0..n))
    int* gen_count;
    int gen_cap;
    const float* xout;  // optional [T][H] hidden after the layers
    float* h_last;      // MTP history: hidden of the last consumed token
    float* h_prev;      // and of the one before it
    int H;
};

// grid: one workgroup per 256 hidden elements (at least one).  Every workgroup
// derives n from toks / preds (loaded together, compared in order); workgroup 0
// also advances the device scalars.
constexpr int kAcceptMaxT = 8;

__global__ __launch_bounds__(256) void accept_kernel(AcceptArgs a) {
    int n = 1;
    if (a.force_all) {
        n = a.T;
    } else {
        int tk[kAcceptMaxT], pr[kAcceptMaxT];
#pragma unroll
        for (int i = 0; i < kAcceptMaxT; ++i) {
            tk[i] = i < a.T ? a.toks[i] : -1;
            pr[i] = i < a.T ? a.preds[i] : -2;
        }
#pragma unroll
        for (int i = 1; i < kAcceptMaxT; ++i)
            if (n == i && i < a.T && pr[i - 1] == tk[i]) n = i + 1;
    }
    if (a.h_last && a.xout) {
        // h_prev <- hidden of token n-2 (or the previous h_last), h_last <- token n-1
        const int i = blockIdx.x * blockDim.x + threadIdx.x;
        if (i < a.H) {
            const float last = a.xout[static_cast<size_t>(n - 1) * a.H + i];
            const float prev = n >= 2 ? a.xout[static_cast<size_t>(n - 2) * a.H + i] : a.h_last[i];
            a.h_prev[i] = prev;
            a.h_last[i] = last;
        }
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *a.n_out = n;
        *a.pos += n;
        if (a.slot) *a.slot = (*a.slot + n) % a.R;
        *a.next_tok = a.preds[n - 1];
        if (a.gen_ring) {
            int c = *a.gen_count;
            for (int i = 0; i < n; ++i) {
                if (c < a.gen_cap) a.gen_ring[c] = a.preds[i];
                ++c;
            }
            *a.gen_count = c;
        }
    }
}

// Batch decode: every sequence consumed its one token.  Slot b's scalar block
// (stride ints): position += 1, conv-ring slot += 1 (mod R), consumed = 1.
__global__ void batch_advance_kernel(int* scal, int stride, int B, int R, int k_pos, int k_slot, int k_ncons) {
    const int b = threadIdx.x;
    if (b >= B) return;
    int* sb = scal + static_cast<size_t>(b) * stride;
    sb[k_pos] += 1;
    sb[k_slot] = (sb[k_slot] + 1) % R;
    sb[k_ncons] = 1;
}

}  // namespace

namespace rl {

void batch_advance(int* scal, int stride, int B, int R, int k_pos, int k_slot, int k_ncons, hipStream_t s) {
    RL_REQUIRE(B >= 1 && B <= 64, RL_ERR_RANGE, "batch_advance: bad batch");
    hipLaunchKernelGGL(batch_advance_kernel, dim3(1), dim3(64), 0, s, scal, stride, B, R, k_pos, k_slot, k_ncons);
    check_launch("batch_advance_kernel");
}

size_t argmax_workspace_bytes(int rows, int V) {
    const size_t nch = (static_cast<size_t>(V) + kArgChunk - 1) / kArgChunk;
    return static_cast<size_t>(rows) * nch * 8 + 64;
}

void argmax_rows(const float* logits, int rows, int V, int* out, float* out_val, void* ws, hipStream_t s) {
    RL_REQUIRE(rows >= 1 && V >= 1 && logits && out && ws, RL_ERR_RANGE, "argmax: bad arguments");
    const int nch = (V + kArgChunk - 1) / kArgChunk;
    float* pv = static_cast<float*>(ws);
    int* pi = reinterpret_cast<int*>(pv + static_cast<size_t>(rows) * nch);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(nch, rows), dim3(256), 0, s, logits, V, pv, pi, nch);
    check_launch("argmax_partial_kernel");
    hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(64), 0, s, pv, pi, nch, out, out_val);
    check_launch("argmax_final_kernel");
}

void accept(const int* toks, const int* preds, int T, int force_all, int* pos, int* slot, int R, int* n_out,
            int* next_tok, int* gen_ring, int* gen_count, int gen_cap, const float* xout, float* h_last,
            float* h_prev, int H, hipStream_t s) {
    RL_REQUIRE(T >= 1 && T <= kAcceptMaxT, RL_ERR_RANGE, "accept: T must be in 1..8");
    AcceptArgs a{toks, preds, T, force_all, pos, slot, R, n_out, next_tok, gen_ring, gen_count, gen_cap,
                 xout, h_last, h_prev, H};
    const int blocks = h_last && xout ? std::max(1, (H + 255) / 256) : 1;
    hipLaunchKernelGGL(accept_kernel, dim3(blocks), dim3(256), 0, s, a);
    check_launch("accept_kernel");
}

}  // namespace rl

extern "C" {

size_t rl_hip_argmax_workspace_bytes(int rows, int vocab) { return rl::argmax_workspace_bytes(rows, vocab); }

int rl_hip_argmax_rows(const float* logits, int rows, int vocab, int* out_idx, float* out_val, void* workspace,
                       void* stream) {
    return guard([&] { rl::argmax_rows(logits, rows, vocab, out_idx, out_val, workspace, S(stream)); });
}

int rl_hip_accept_prefix(const int* toks, const int* preds, int T, int* pos, int* n_consumed, int* next_tok,
                         void* stream) {
    return guard([&] {
        RL_REQUIRE(T >= 1 && toks && preds && pos && n_consumed && next_tok, RL_ERR_RANGE, "accept: bad arguments");
        rl::accept(toks, preds, T, 0, pos, nullptr, 1, n_consumed, next_tok, nullptr, nullptr, 0, nullptr, nullptr,
                   nullptr, 0, S(stream));
    });
}

}  // extern "C"
