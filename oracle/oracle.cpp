// oracle.cpp -- TEST INFRASTRUCTURE ONLY.
//
// A CPU restatement of RapidLLM's CPU decode path, used as the parity checker for
// the HIP backend.  Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg may load this library; the product (rapidllm_amd/) never does.
//
// Every function cites the reference file:line whose arithmetic it restates.  The
// arithmetic order (double vs float accumulators, separate roundings, no FMA) is
// kept identical because parity is judged against the reference's own CPU output:
// build with -ffp-contract=off and without -mfma (oracle/Makefile), as the
// reference's scalar TU is built (CMakeLists.txt:20-70: no ISA flags on ops.cpp).
//
// Pinning (tests/test_oracle_kernels.py, tests/test_golden_vectors.py):
//   e4m3/fp16 decode     exhaustive vs closed form + numpy float16 + oracle/_ref
//   fp8 GEMV             brute force in exact rational arithmetic (tiny) + _ref
//   Q4_K / Q6_K dequant  bit-exact vs _ref + hand-built blocks with known values
//   conv/delta/norms     _ref + closed-form special cases (zero state, identities)
//   attention            _ref + softmax closed forms (uniform keys, one-hot)
//   model forward / MTP  tiny-hybrid greedy tokens from the reference's golden
//                        generator (tests/golden/) + greedy invariant
//   committed vectors    tests/golden/ref_vectors.npz from the _ref kernels, so the
//                        oracle stays pinned where the reference tree is absent
#include "../include/rl_model.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <map>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

float silu_f(float x) { return x / (1.f + std::exp(-x)); }
float sigmoid_f(float x) { return 1.f / (1.f + std::exp(-x)); }
// softplus as log1p(exp(-|x|)) + max(x, 0)  (ops_fused.cpp:13)
float softplus_f(float x) { return std::log1p(std::exp(-std::fabs(x))) + std::max(x, 0.f); }

float bits_to_f(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

uint32_t f_to_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

void run_rows(int m, int nthreads, const std::function<void(int, int)>& fn);

}  // namespace

extern "C" {

// ---------------------------------------------------------------- conversions

// IEEE binary16 -> binary32, exact, subnormals renormalised (ops.cpp:15-40).
float orc_fp16_to_f32(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const int exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    if (exp == 31) return bits_to_f(sign | 0x7f800000u | (man << 13));
    if (exp != 0) return bits_to_f(sign | (static_cast<uint32_t>(exp + 112) << 23) | (man << 13));
    if (man == 0) return bits_to_f(sign);
    int e = 113;  // exponent field a normal with the implicit bit at 2^-14 would get
    while (!(man & 0x400u)) {
        man <<= 1;
        --e;
    }
    return bits_to_f(sign | (static_cast<uint32_t>(e) << 23) | ((man & 0x3ffu) << 13));
}

// binary32 -> binary16 with round-to-nearest-even.  Not in the reference CPU path
// (its f32_to_fp16, ops.cpp:42-55, truncates); used to give the oracle the same
// fp16-rounded K/V that the device KV cache holds (cuda_engine.cu:20122-20123 keeps
// an fp16 cache written with round-to-nearest).  Pinned exhaustively vs numpy.
uint16_t orc_f32_to_fp16(float f) {
    const uint32_t x = f_to_bits(f);
    const uint16_t sign = static_cast<uint16_t>((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return static_cast<uint16_t>(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);  // rounds to >= 65520
    if (ax < 0x38800000u) {                                                // result subnormal or zero
        const float a = bits_to_f(ax);
        // value / 2^-24, rounded to nearest even; exact in float for |a| < 2^-14.
        const float q = std::nearbyint(a * 16777216.f);
        return static_cast<uint16_t>(sign | static_cast<uint16_t>(q));
    }
    const uint32_t e = (ax >> 23) - 112;
    uint32_t m = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    const uint32_t rest = m & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;  // carry may bump the exponent: correct
    return static_cast<uint16_t>(sign | h);
}

// OCP e4m3fn -> fp32: bias 7, subnormal m/8 * 2^-6, S.1111.111 = NaN, no Inf
// (ops.cpp:57-71).
float orc_e4m3_to_f32(uint8_t b) {
    const bool neg = (b & 0x80) != 0;
    const int e = (b >> 3) & 0xf;
    const int m = b & 7;
    float v;
    if (e == 0xf && m == 7) return std::nanf("");
    if (e == 0)
        v = std::ldexp(static_cast<float>(m), -9);  // (m/8) * 2^-6
    else
        v = std::ldexp(static_cast<float>(8 + m), e - 10);  // (1 + m/8) * 2^(e-7)
    return neg ? -v : v;
}

float orc_bf16_to_f32(uint16_t h) { return bits_to_f(static_cast<uint32_t>(h) << 16); }

// ---------------------------------------------------------------- linears

// Block-FP8 GEMV: y[i] = sum_j e4m3(W[i,j]) * scale[i/B][j/B] * x[j] with a double
// accumulator, rounded to fp32 at the end (ops.cpp:182-194).  The product
// (double)w * s * x is exact in double (4 + 24 + 24 significant bits).
static void gemv_fp8_rows(const uint8_t* W, const float* scale, const float* x, float* y, int n, int block, int r0,
                          int r1) {
    const int sb_cols = (n + block - 1) / block;
    float lut[256];
    for (int c = 0; c < 256; ++c) lut[c] = orc_e4m3_to_f32(static_cast<uint8_t>(c));
    for (int i = r0; i < r1; ++i) {
        const uint8_t* row = W + static_cast<size_t>(i) * n;
        const float* srow = scale + static_cast<size_t>(i / block) * sb_cols;
        double acc = 0.0;
        for (int j = 0; j < n; ++j) acc += static_cast<double>(lut[row[j]]) * srow[j / block] * x[j];
        y[i] = static_cast<float>(acc);
    }
}

void orc_gemv_fp8(const uint8_t* W, const float* scale, const float* x, float* y, int m, int n, int block) {
    gemv_fp8_rows(W, scale, x, y, n, block, 0, m);
}

// T tokens through the same weights = T independent GEMVs (the reference CPU
// session verifies drafts one token at a time, session.cpp:816-824).
void orc_gemm_fp8(const uint8_t* W, const float* scale, const float* X, float* Y, int m, int n, int T) {
    for (int t = 0; t < T; ++t) orc_gemv_fp8(W, scale, X + static_cast<size_t>(t) * n, Y + static_cast<size_t>(t) * m, m, n, 128);
}

// 6-bit scale / min of sub-block j from the 12 packed bytes of a Q4_K block
// (ops.cpp:245-253): j<4 low 6 bits of bytes j / j+4; j>=4 a nibble of byte j+4
// plus the top two bits of bytes j-4 / j.
static void q4k_sub(const uint8_t* s12, int j, int* sc, int* mn) {
    if (j < 4) {
        *sc = s12[j] & 0x3f;
        *mn = s12[j + 4] & 0x3f;
    } else {
        *sc = (s12[j + 4] & 0x0f) | ((s12[j - 4] >> 6) << 4);
        *mn = (s12[j + 4] >> 4) | ((s12[j] >> 6) << 4);
    }
}

// Q4_K super-block (144 B): fp16 d @0, fp16 dmin @2, 12 scale bytes @4, 128 nibble
// bytes @16.  Group g of 64 weights: low nibbles of q[32g..32g+31] are sub-block 2g,
// high nibbles sub-block 2g+1; w = (d*sc)*q - (dmin*mn), each product rounded to
// fp32 separately (ops.cpp:255-284).
void orc_dequant_q4_k(const uint8_t* packed, float* out, int n) {
    const int nb = n / 256;
    for (int b = 0; b < nb; ++b) {
        const uint8_t* blk = packed + static_cast<size_t>(b) * 144;
        uint16_t dh, mh;
        std::memcpy(&dh, blk, 2);
        std::memcpy(&mh, blk + 2, 2);
        const float d = orc_fp16_to_f32(dh), dmin = orc_fp16_to_f32(mh);
        const uint8_t* q = blk + 16;
        float* o = out + static_cast<size_t>(b) * 256;
        for (int g = 0; g < 4; ++g) {
            int s_lo, m_lo, s_hi, m_hi;
            q4k_sub(blk + 4, 2 * g, &s_lo, &m_lo);
            q4k_sub(blk + 4, 2 * g + 1, &s_hi, &m_hi);
            const float dl = d * static_cast<float>(s_lo), ml = dmin * static_cast<float>(m_lo);
            const float dhh = d * static_cast<float>(s_hi), mhh = dmin * static_cast<float>(m_hi);
            for (int l = 0; l < 32; ++l) {
                const uint8_t byte = q[32 * g + l];
                o[64 * g + l] = dl * static_cast<float>(byte & 0xf) - ml;
                o[64 * g + 32 + l] = dhh * static_cast<float>(byte >> 4) - mhh;
            }
        }
    }
}

// Q6_K super-block (210 B): ql[128] @0, qh[64] @128, int8 sc[16] @192, fp16 d @208.
// Per 128-half h and l in [0,32): four 6-bit values (low nibble of ql[l] / ql[l+32],
// high nibble of ql[l] / ql[l+32], each with 2 bits of qh[l]) minus 32, written to
// l, l+32, l+64, l+96 with scale sc[l/16 + {0,2,4,6}]; w = (d*sc)*q (ops.cpp:357-387).
void orc_dequant_q6_k(const uint8_t* packed, float* out, int n) {
    const int nb = n / 256;
    for (int b = 0; b < nb; ++b) {
        const uint8_t* blk = packed + static_cast<size_t>(b) * 210;
        uint16_t dh;
        std::memcpy(&dh, blk + 208, 2);
        const float d = orc_fp16_to_f32(dh);
        for (int half = 0; half < 2; ++half) {
            const uint8_t* ql = blk + 64 * half;
            const uint8_t* qh = blk + 128 + 32 * half;
            const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192 + 8 * half);
            float* o = out + static_cast<size_t>(b) * 256 + 128 * half;
            for (int l = 0; l < 32; ++l) {
                const int hb = qh[l];
                const int v0 = ((ql[l] & 0xf) | ((hb & 3) << 4)) - 32;
                const int v1 = ((ql[l + 32] & 0xf) | (((hb >> 2) & 3) << 4)) - 32;
                const int v2 = ((ql[l] >> 4) | (((hb >> 4) & 3) << 4)) - 32;
                const int v3 = ((ql[l + 32] >> 4) | (((hb >> 6) & 3) << 4)) - 32;
                const int s = l / 16;
                o[l] = d * static_cast<float>(sc[s]) * static_cast<float>(v0);
                o[l + 32] = d * static_cast<float>(sc[s + 2]) * static_cast<float>(v1);
                o[l + 64] = d * static_cast<float>(sc[s + 4]) * static_cast<float>(v2);
                o[l + 96] = d * static_cast<float>(sc[s + 6]) * static_cast<float>(v3);
            }
        }
    }
}

// K-quant GEMV: per 256-weight super-block, dequantise then a sequential fp32 dot,
// summed into an fp32 row accumulator (ops.cpp:286-305, 389-402); rows split over
// threads as cpu_caps.cpp:124-131, 200-222 does (work m*n >= 2M).
static void gemv_kq(void (*deq)(const uint8_t*, float*, int), size_t bsz, const uint8_t* packed, const float* x,
                    float* y, int m, int n, int nthreads) {
    const int nb = n / 256;
    auto body = [&](int r0, int r1) {
        float tmp[256];
        for (int i = r0; i < r1; ++i) {
            const uint8_t* row = packed + static_cast<size_t>(i) * nb * bsz;
            float acc = 0.f;
            for (int b = 0; b < nb; ++b) {
                deq(row + b * bsz, tmp, 256);
                const float* xb = x + b * 256;
                float s = 0.f;
                for (int k = 0; k < 256; ++k) s += tmp[k] * xb[k];
                acc += s;
            }
            y[i] = acc;
        }
    };
    if (static_cast<long long>(m) * n < 2000000LL || nthreads <= 1)
        body(0, m);
    else
        run_rows(m, nthreads, body);
}

void orc_gemv_q4_k(const uint8_t* packed, const float* x, float* y, int m, int n, int nthreads) {
    gemv_kq(orc_dequant_q4_k, 144, packed, x, y, m, n, nthreads);
}

void orc_gemv_q6_k(const uint8_t* packed, const float* x, float* y, int m, int n, int nthreads) {
    gemv_kq(orc_dequant_q6_k, 210, packed, x, y, m, n, nthreads);
}

// Dense GEMVs with a float accumulator (cpu_caps.cpp:171-198 scalar branch;
// ops.cpp:235-242).  f32 weights accumulate in double (ops.cpp:165-172).
void orc_gemv_bf16(const uint16_t* W, const float* x, float* y, int m, int n, int nthreads) {
    auto body = [&](int r0, int r1) {
        for (int i = r0; i < r1; ++i) {
            const uint16_t* row = W + static_cast<size_t>(i) * n;
            float acc = 0.f;
            for (int j = 0; j < n; ++j) acc += orc_bf16_to_f32(row[j]) * x[j];
            y[i] = acc;
        }
    };
    if (static_cast<long long>(m) * n < 2000000LL || nthreads <= 1)
        body(0, m);
    else
        run_rows(m, nthreads, body);
}

void orc_gemv_f16(const uint16_t* W, const float* x, float* y, int m, int n) {
    for (int i = 0; i < m; ++i) {
        const uint16_t* row = W + static_cast<size_t>(i) * n;
        float acc = 0.f;
        for (int j = 0; j < n; ++j) acc += orc_fp16_to_f32(row[j]) * x[j];
        y[i] = acc;
    }
}

void orc_gemv_f32(const float* W, const float* x, float* y, int m, int n) {
    for (int i = 0; i < m; ++i) {
        const float* row = W + static_cast<size_t>(i) * n;
        double acc = 0.0;
        for (int j = 0; j < n; ++j) acc += static_cast<double>(row[j]) * x[j];
        y[i] = static_cast<float>(acc);
    }
}

// ops::linear dispatch by quant kind (ops.cpp:404-437).
int orc_linear(int quant, const void* w, const float* scale, const float* x, float* y, int m, int n, int nthreads) {
    switch (quant) {
    case RL_Q_F32: orc_gemv_f32(static_cast<const float*>(w), x, y, m, n); return 0;
    case RL_Q_F16: orc_gemv_f16(static_cast<const uint16_t*>(w), x, y, m, n); return 0;
    case RL_Q_BF16: orc_gemv_bf16(static_cast<const uint16_t*>(w), x, y, m, n, nthreads); return 0;
    case RL_Q_FP8_E4M3_B128:
        if (!scale) return -1;
        // rows are independent: splitting them over threads changes no result (the
        // reference's ops::gemv_fp8 runs them on one thread)
        if (static_cast<long long>(m) * n < 2000000LL || nthreads <= 1)
            orc_gemv_fp8(static_cast<const uint8_t*>(w), scale, x, y, m, n, 128);
        else
            run_rows(m, nthreads, [&](int r0, int r1) {
                gemv_fp8_rows(static_cast<const uint8_t*>(w), scale, x, y, n, 128, r0, r1);
            });
        return 0;
    case RL_Q_Q4_K: orc_gemv_q4_k(static_cast<const uint8_t*>(w), x, y, m, n, nthreads); return 0;
    case RL_Q_Q6_K: orc_gemv_q6_k(static_cast<const uint8_t*>(w), x, y, m, n, nthreads); return 0;
    default: return -2;
    }
}

// ---------------------------------------------------------------- norms

// Qwen3 RMSNorm with (1 + gamma): double sum of squares, fp32 inverse
// (ops.cpp:107-127, scalar branch).
void orc_qwen3_rmsnorm(const float* x, const float* gamma, float* y, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += static_cast<double>(x[i]) * x[i];
    const float inv = 1.f / std::sqrt(static_cast<float>(ss / n) + eps);
    for (int i = 0; i < n; ++i) y[i] = x[i] * inv * (gamma ? 1.f + gamma[i] : 1.f);
}

// gamma * (x / rms(x)) * silu(z); per head of gamma_n when gamma_n < n,
// n % gamma_n == 0 and n >= 256, else over the whole vector (ops.cpp:129-156).
void orc_gated_rmsnorm(const float* x, const float* z, const float* gamma, float* y, int n, float eps, int gamma_n) {
    if (gamma_n <= 0) gamma_n = n;
    const bool per_head = gamma_n < n && n % gamma_n == 0 && n >= 256;
    const int seg = per_head ? gamma_n : n;
    for (int h0 = 0; h0 < n; h0 += seg) {
        double ss = 0.0;
        for (int i = 0; i < seg; ++i) ss += static_cast<double>(x[h0 + i]) * x[h0 + i];
        const float inv = 1.f / std::sqrt(static_cast<float>(ss / seg) + eps);
        for (int i = 0; i < seg; ++i) {
            const float g = gamma ? gamma[per_head ? i : (h0 + i) % gamma_n] : 1.f;
            y[h0 + i] = g * (x[h0 + i] * inv) * silu_f(z[h0 + i]);
        }
    }
}

// x / sqrt(sum x^2 + eps), eps inside the root of the SUM (ops.cpp:158-163).
void orc_l2norm(const float* x, float* y, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += static_cast<double>(x[i]) * x[i];
    const float inv = 1.f / std::sqrt(static_cast<float>(ss) + eps);
    for (int i = 0; i < n; ++i) y[i] = x[i] * inv;
}

// ---------------------------------------------------------------- DeltaNet

// Causal conv1d decode step: state [dim][k] shifts one tap left, x_t enters at tap
// k-1 (tap 0 oldest); y = silu(sum_p w[c][p] * st[c][p]) with a double sum
// (ops.cpp:458-468).
void orc_conv1d_update(const float* x_t, const float* w, float* state, float* y, int dim, int k) {
    for (int c = 0; c < dim; ++c) {
        float* st = state + static_cast<size_t>(c) * k;
        std::memmove(st, st + 1, sizeof(float) * (k - 1));
        st[k - 1] = x_t[c];
        double acc = 0.0;
        for (int p = 0; p < k; ++p) acc += static_cast<double>(w[static_cast<size_t>(c) * k + p]) * st[p];
        y[c] = silu_f(static_cast<float>(acc));
    }
}

// beta = sigmoid(b), g_log = -exp(A_log) * softplus(a + dt_bias)
// (ops_fused.cpp:122-123; session.cpp:244-246).
void orc_gdn_gates(const float* a, const float* b, const float* A_log, const float* dt_bias, float* beta, float* g_log,
                   int nv) {
    for (int h = 0; h < nv; ++h) {
        beta[h] = sigmoid_f(b[h]);
        g_log[h] = -std::exp(A_log[h]) * softplus_f(a[h] + dt_bias[h]);
    }
}

// One gated delta-rule step per v-head, state S[h][i<dk][j<dv] fp32
// (ops.cpp:495-534): q,k <- l2norm; q *= 1/sqrt(dk); S *= exp(g_log);
// kv = S^T k; delta = (v - kv) * beta; S += k (x) delta; o = S^T q.
void orc_delta_step(float* S, const float* q_in, const float* k_in, const float* v, const float* beta,
                    const float* g_log, float* o, int nv, int dk, int dv, float eps) {
    std::vector<float> q(dk), k(dk), kv(dv), dl(dv);
    const float qscale = 1.f / std::sqrt(static_cast<float>(dk));
    for (int h = 0; h < nv; ++h) {
        orc_l2norm(q_in + static_cast<size_t>(h) * dk, q.data(), dk, eps);
        orc_l2norm(k_in + static_cast<size_t>(h) * dk, k.data(), dk, eps);
        for (int i = 0; i < dk; ++i) q[i] *= qscale;
        float* Sh = S + static_cast<size_t>(h) * dk * dv;
        const float decay = std::exp(g_log[h]);
        for (int t = 0; t < dk * dv; ++t) Sh[t] *= decay;
        std::fill(kv.begin(), kv.end(), 0.f);
        for (int i = 0; i < dk; ++i)
            for (int j = 0; j < dv; ++j) kv[j] += Sh[i * dv + j] * k[i];
        const float* vh = v + static_cast<size_t>(h) * dv;
        for (int j = 0; j < dv; ++j) dl[j] = (vh[j] - kv[j]) * beta[h];
        for (int i = 0; i < dk; ++i)
            for (int j = 0; j < dv; ++j) Sh[i * dv + j] += k[i] * dl[j];
        float* oh = o + static_cast<size_t>(h) * dv;
        std::fill(oh, oh + dv, 0.f);
        for (int i = 0; i < dk; ++i)
            for (int j = 0; j < dv; ++j) oh[j] += Sh[i * dv + j] * q[i];
    }
}

// ---------------------------------------------------------------- attention

// Partial RoPE: first rotary_dim dims, pair (i, i + rot/2) when head_dim >= 64
// ("rotate half"), adjacent pairs otherwise; freq = theta^(-i/(rot/2)) in fp32
// (ops.cpp:470-493).
void orc_rope_partial(float* q, float* k, int n_q, int n_kv, int head_dim, int rotary_dim, int pos, float theta) {
    const int pairs = rotary_dim / 2;
    for (int which = 0; which < 2; ++which) {
        float* base = which == 0 ? q : k;
        const int nh = which == 0 ? n_q : n_kv;
        for (int h = 0; h < nh; ++h) {
            float* v = base + static_cast<size_t>(h) * head_dim;
            for (int i = 0; i < pairs; ++i) {
                const float freq = 1.f / std::pow(theta, static_cast<float>(i) / static_cast<float>(pairs));
                const float ang = static_cast<float>(pos) * freq;
                const float c = std::cos(ang), s = std::sin(ang);
                const int a = head_dim >= 64 ? i : 2 * i;
                const int b = head_dim >= 64 ? i + pairs : 2 * i + 1;
                const float x0 = v[a], x1 = v[b];
                v[a] = x0 * c - x1 * s;
                v[b] = x0 * s + x1 * c;
            }
        }
    }
}

// GQA decode over positions 0..pos: scores in double rounded to fp32 then
// * 1/sqrt(hd); softmax with fp32 exp and a double normaliser; fp32 output sums
// (ops.cpp:575-605).  Caches are [pos][n_kv][hd] fp32.
void orc_attn_decode(const float* q, const float* kc, const float* vc, float* o, int pos, int n_q, int n_kv,
                     int head_dim) {
    const int len = pos + 1;
    const int rep = n_q / n_kv;
    const float scale = 1.f / std::sqrt(static_cast<float>(head_dim));
    std::vector<float> p(len);
    for (int hq = 0; hq < n_q; ++hq) {
        const int hk = hq / rep;
        const float* qh = q + static_cast<size_t>(hq) * head_dim;
        float mx = -1e30f;
        for (int s = 0; s < len; ++s) {
            const float* kr = kc + (static_cast<size_t>(s) * n_kv + hk) * head_dim;
            double dot = 0.0;
            for (int d = 0; d < head_dim; ++d) dot += static_cast<double>(qh[d]) * kr[d];
            p[s] = static_cast<float>(dot) * scale;
            mx = std::max(mx, p[s]);
        }
        double z = 0.0;
        for (int s = 0; s < len; ++s) {
            p[s] = std::exp(p[s] - mx);
            z += p[s];
        }
        float* oh = o + static_cast<size_t>(hq) * head_dim;
        std::fill(oh, oh + head_dim, 0.f);
        for (int s = 0; s < len; ++s) {
            const float w = static_cast<float>(p[s] / z);
            const float* vr = vc + (static_cast<size_t>(s) * n_kv + hk) * head_dim;
            for (int d = 0; d < head_dim; ++d) oh[d] += w * vr[d];
        }
    }
}

void orc_swiglu(const float* g, const float* u, float* y, int n) {
    for (int i = 0; i < n; ++i) y[i] = silu_f(g[i]) * u[i];
}

// argmax, first index wins ties (sampler.cpp:8-18).
int orc_greedy(const float* logits, int vocab) {
    int best = 0;
    for (int i = 1; i < vocab; ++i)
        if (logits[i] > logits[best]) best = i;
    return best;
}

// Rows of `rows` x `vocab` logits -> argmax each.
void orc_argmax_rows(const float* logits, int rows, int vocab, int* out) {
    for (int r = 0; r < rows; ++r) out[r] = orc_greedy(logits + static_cast<size_t>(r) * vocab, vocab);
}

// Greedy acceptance (session.cpp:802-825): toks = [t0, d1..dn], pred[i] is the
// greedy token after toks[0..i].  Accept the longest prefix with pred[i] == d_{i+1};
// returns n_consumed = 1 + accepted drafts.
int orc_accept_prefix(const int* toks, const int* preds, int T) {
    int k = 1;
    while (k < T && preds[k - 1] == toks[k]) ++k;
    return k;
}

}  // extern "C"

// ---------------------------------------------------------------- whole model

namespace {

void run_rows(int m, int nthreads, const std::function<void(int, int)>& fn) {
    nthreads = std::max(1, std::min(nthreads, m));
    std::vector<std::thread> th;
    const int chunk = (m + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; ++t) {
        const int r0 = t * chunk, r1 = std::min(m, r0 + chunk);
        if (r0 >= r1) break;
        th.emplace_back([&fn, r0, r1] { fn(r0, r1); });
    }
    for (auto& t : th) t.join();
}

struct W {
    int quant = RL_Q_F32;
    int64_t rows = 0, cols = 0;
    const void* data = nullptr;
    const float* scale = nullptr;
    const float* f32() const {
        if (quant != RL_Q_F32) throw std::runtime_error("expected f32 tensor");
        return static_cast<const float*>(data);
    }
};

// CPU decode model following Session's fused one-token path (session.cpp:325-411,
// 531-559; ops_fused.cpp:66-184) with DualCache layouts (dual_cache.cpp:5-36).
struct Model {
    RlModelConfig c{};
    std::map<std::string, W> w;
    int ctx = 0, pos = 0, nthreads = 1;
    bool kv_fp16 = false;  // round K (after RoPE) and V to fp16 before caching
    std::vector<std::vector<float>> S, conv, kc, vc;
    std::vector<int> slot;  // layer -> mixer slot within its kind (ModelDesc::mixer_slot)
    std::vector<float> logits, last_hidden;
    std::vector<float> hist_h;  // mtp_hh_: residual after the layers, per token
    std::vector<int> hist_ids;  // mtp_hids_
    int mtp_mode = 0;           // 0: stem (Session::mtp_draft), 1: stem + mtp.layers[0]
    mutable std::vector<float> mtp_h;  // the last draft's hidden before norm_mtp

    const W& get(const std::string& n) const {
        auto it = w.find(n);
        if (it == w.end()) throw std::runtime_error("missing weight " + n);
        return it->second;
    }
    void lin(const W& t, const float* x, float* y, int m, int n) const {
        if (orc_linear(t.quant, t.data, t.scale, x, y, m, n, nthreads) != 0) throw std::runtime_error("linear");
    }
    int qkv_dim() const { return 2 * c.n_k_heads * c.k_dim + c.n_v_heads * c.v_dim; }

    void reset() {
        const int nd = static_cast<int>(std::count(c.layer_kind, c.layer_kind + c.n_layers, RL_LAYER_DELTA));
        const int na = c.n_layers - nd;
        S.assign(nd, std::vector<float>(static_cast<size_t>(c.n_v_heads) * c.k_dim * c.v_dim, 0.f));
        conv.assign(nd, std::vector<float>(static_cast<size_t>(qkv_dim()) * c.conv_k, 0.f));
        kc.assign(na, std::vector<float>(static_cast<size_t>(ctx) * c.n_kv * c.head_dim, 0.f));
        vc.assign(na, std::vector<float>(static_cast<size_t>(ctx) * c.n_kv * c.head_dim, 0.f));
        slot.assign(c.n_layers, 0);
        int di = 0, ai = 0;
        for (int i = 0; i < c.n_layers; ++i) slot[i] = c.layer_kind[i] == RL_LAYER_DELTA ? di++ : ai++;
        pos = 0;
        logits.assign(c.vocab, 0.f);
        last_hidden.assign(c.hidden, 0.f);
        hist_h.clear();
        hist_ids.clear();
    }

    void embed(int id, float* out) const {
        const W& e = get("embed");
        const int H = c.hidden;
        if (id < 0 || id >= c.vocab) throw std::runtime_error("token out of range");
        if (e.quant == RL_Q_F32) {
            std::memcpy(out, e.f32() + static_cast<size_t>(id) * H, sizeof(float) * H);
        } else if (e.quant == RL_Q_BF16 || e.quant == RL_Q_F16) {
            const uint16_t* r = static_cast<const uint16_t*>(e.data) + static_cast<size_t>(id) * H;
            for (int i = 0; i < H; ++i) out[i] = e.quant == RL_Q_BF16 ? orc_bf16_to_f32(r[i]) : orc_fp16_to_f32(r[i]);
        } else if (e.quant == RL_Q_Q4_K || e.quant == RL_Q_Q6_K) {
            // block-quantised embedding row (cuda_engine.cu:19930-19955 dequantises the
            // table with ops::dequant_q4_k / dequant_q6_k)
            const size_t rowb = static_cast<size_t>(H / 256) * (e.quant == RL_Q_Q4_K ? 144 : 210);
            const uint8_t* r = static_cast<const uint8_t*>(e.data) + static_cast<size_t>(id) * rowb;
            if (e.quant == RL_Q_Q4_K) orc_dequant_q4_k(r, out, H);
            else orc_dequant_q6_k(r, out, H);
        } else {
            throw std::runtime_error("embed quant");
        }
    }

    // ops_fused.cpp:66-82
    void mlp(const std::string& p, float* x) const {
        const int H = c.hidden;
        const W& wd = get(p + "mlp.down");
        const int I = static_cast<int>(wd.cols);
        std::vector<float> xn(H), g(I), u(I), y(H);
        orc_qwen3_rmsnorm(x, get(p + "ffn_norm").f32(), xn.data(), H, c.rms_eps);
        lin(get(p + "mlp.gate"), xn.data(), g.data(), I, H);
        lin(get(p + "mlp.up"), xn.data(), u.data(), I, H);
        orc_swiglu(g.data(), u.data(), g.data(), I);
        lin(wd, g.data(), y.data(), H, I);
        for (int d = 0; d < H; ++d) x[d] += y[d];
    }

    // ops_fused.cpp:84-135
    void delta(const std::string& p, int sl, float* x) {
        const int H = c.hidden, nk = c.n_k_heads, nv = c.n_v_heads, dk = c.k_dim, dv = c.v_dim;
        const int qd = nk * dk, qkvd = qkv_dim(), zd = nv * dv;
        std::vector<float> xn(H), qkv(qkvd), z(zd), a(nv), b(nv), mix(qkvd);
        orc_qwen3_rmsnorm(x, get(p + "attn_norm").f32(), xn.data(), H, c.rms_eps);
        lin(get(p + "delta.gemm.in_proj_qkv"), xn.data(), qkv.data(), qkvd, H);
        lin(get(p + "delta.gemm.in_proj_z"), xn.data(), z.data(), zd, H);
        lin(get(p + "delta.leftover.in_proj_a"), xn.data(), a.data(), nv, H);
        lin(get(p + "delta.leftover.in_proj_b"), xn.data(), b.data(), nv, H);
        orc_conv1d_update(qkv.data(), get(p + "delta.leftover.conv1d").f32(), conv[sl].data(), mix.data(), qkvd,
                          c.conv_k);
        std::vector<float> qh(static_cast<size_t>(nv) * dk), kh(static_cast<size_t>(nv) * dk), beta(nv), gl(nv);
        const int rep = nv / nk;
        for (int h = 0; h < nv; ++h) {
            const int src = c.v_tiled ? h % nk : h / rep;
            std::memcpy(&qh[static_cast<size_t>(h) * dk], &mix[static_cast<size_t>(src) * dk], sizeof(float) * dk);
            std::memcpy(&kh[static_cast<size_t>(h) * dk], &mix[qd + static_cast<size_t>(src) * dk], sizeof(float) * dk);
        }
        orc_gdn_gates(a.data(), b.data(), get(p + "delta.leftover.a_log").f32(), get(p + "delta.leftover.dt_bias").f32(),
                      beta.data(), gl.data(), nv);
        std::vector<float> o(zd), og(zd), y(H);
        orc_delta_step(S[sl].data(), qh.data(), kh.data(), &mix[2 * qd], beta.data(), gl.data(), o.data(), nv, dk, dv,
                       1e-6f);
        const W& gn = get(p + "delta.leftover.norm");
        orc_gated_rmsnorm(o.data(), z.data(), gn.f32(), og.data(), zd, 1e-6f, static_cast<int>(gn.rows));
        lin(get(p + "delta.gemm.out_proj"), og.data(), y.data(), H, zd);
        for (int d = 0; d < H; ++d) x[d] += y[d];
    }

    // ops_fused.cpp:137-184 (+ DualCache::append_kv, dual_cache.cpp:72-78)
    void attn(const std::string& p, int sl, float* x, std::vector<float>& kcache, std::vector<float>& vcache,
              int at) const {
        const int H = c.hidden, nq = c.n_q, nkv = c.n_kv, hd = c.head_dim;
        const int qn = nq * hd, kn = nkv * hd;
        std::vector<float> xn(H), qg(2 * static_cast<size_t>(qn)), q(qn), gate(qn), k(kn), v(kn);
        orc_qwen3_rmsnorm(x, get(p + "attn_norm").f32(), xn.data(), H, c.rms_eps);
        lin(get(p + "attn.wq"), xn.data(), qg.data(), 2 * qn, H);
        lin(get(p + "attn.wk"), xn.data(), k.data(), kn, H);
        lin(get(p + "attn.wv"), xn.data(), v.data(), kn, H);
        for (int h = 0; h < nq; ++h)
            for (int d = 0; d < hd; ++d) {
                // hd >= 64: per head [q(hd) | gate(hd)]; else [all q | all gate]
                const size_t qi = hd >= 64 ? static_cast<size_t>(h) * 2 * hd + d : static_cast<size_t>(h) * hd + d;
                const size_t gi = hd >= 64 ? qi + hd : qi + qn;
                q[static_cast<size_t>(h) * hd + d] = qg[qi];
                gate[static_cast<size_t>(h) * hd + d] = qg[gi];
            }
        for (int h = 0; h < nq; ++h)
            orc_qwen3_rmsnorm(&q[static_cast<size_t>(h) * hd], get(p + "attn.q_norm").f32(), &q[static_cast<size_t>(h) * hd],
                              hd, c.rms_eps);
        for (int h = 0; h < nkv; ++h)
            orc_qwen3_rmsnorm(&k[static_cast<size_t>(h) * hd], get(p + "attn.k_norm").f32(), &k[static_cast<size_t>(h) * hd],
                              hd, c.rms_eps);
        orc_rope_partial(q.data(), k.data(), nq, nkv, hd, c.rotary_dim, at, c.rope_theta);
        if (kv_fp16) {
            for (auto& t : k) t = orc_fp16_to_f32(orc_f32_to_fp16(t));
            for (auto& t : v) t = orc_fp16_to_f32(orc_f32_to_fp16(t));
        }
        std::memcpy(&kcache[static_cast<size_t>(at) * kn], k.data(), sizeof(float) * kn);
        std::memcpy(&vcache[static_cast<size_t>(at) * kn], v.data(), sizeof(float) * kn);
        std::vector<float> o(qn), y(H);
        orc_attn_decode(q.data(), kcache.data(), vcache.data(), o.data(), at, nq, nkv, hd);
        for (int j = 0; j < qn; ++j) o[j] *= sigmoid_f(gate[j]);
        lin(get(p + "attn.wo"), o.data(), y.data(), H, qn);
        for (int d = 0; d < H; ++d) x[d] += y[d];
        (void)sl;
    }

    // Session::decode_token CPU branch (session.cpp:531-559)
    void decode(int token) {
        if (pos >= ctx) throw std::runtime_error("context full");
        const int H = c.hidden;
        std::vector<float> x(H);
        embed(token, x.data());
        for (int i = 0; i < c.n_layers; ++i) {
            const std::string p = "layers[" + std::to_string(i) + "].";
            if (c.layer_kind[i] == RL_LAYER_DELTA)
                delta(p, slot[i], x.data());
            else
                attn(p, slot[i], x.data(), kc[slot[i]], vc[slot[i]], pos);
            mlp(p, x.data());
        }
        std::vector<float> fn(H);
        orc_qwen3_rmsnorm(x.data(), get("final_norm").f32(), fn.data(), H, c.rms_eps);
        lin(get("lm_head"), fn.data(), logits.data(), c.vocab, H);
        last_hidden = x;
        hist_h.insert(hist_h.end(), x.begin(), x.end());
        hist_ids.push_back(token);
        ++pos;
    }

    // Session::mtp_draft CPU branch (session.cpp:619-681): stem draft, no MTP
    // decoder layer.  h' = fc([norm_e(embed tok) ; norm_h(h)]); tok = argmax(
    // lm_head(norm_mtp(h'))).  First draft from the last history hidden, later
    // drafts from the one before it.
    // mtp_mode 1 passes h' through the MTP decoder layer first, as
    // Session::mtp_layer_step(h', i) does (session.cpp:561-617): fused_attn_decode
    // with the mtp.layers[0] weights on the layer's own KV cache at draft position
    // i (zeroed per call, session.cpp:637-640), then fused_mlp_decode.
    int mtp_draft(int first, int n, int* out) const {
        if (!c.has_mtp || n <= 0) return 0;
        const int H = c.hidden;
        const int nh = std::min(static_cast<int>(hist_h.size()) / H, static_cast<int>(hist_ids.size()));
        const float* h_last = nh > 0 ? &hist_h[static_cast<size_t>(nh - 1) * H] : last_hidden.data();
        const float* h_prev = nh > 1 ? &hist_h[static_cast<size_t>(nh - 2) * H] : h_last;
        std::vector<float> eh(H), ee(H), er(H), cat(2 * static_cast<size_t>(H)), hp(H), hn(H), lg(c.vocab);
        const size_t kn = static_cast<size_t>(c.n_kv) * c.head_dim;
        std::vector<float> mkc(mtp_mode ? static_cast<size_t>(n) * kn : 0, 0.f), mvc(mkc.size(), 0.f);
        int tok = first;
        for (int i = 0; i < n; ++i) {
            const float* href = i == 0 ? h_last : h_prev;
            orc_qwen3_rmsnorm(href, get("mtp.pre_fc_norm_hidden").f32(), eh.data(), H, c.rms_eps);
            embed(tok, er.data());
            orc_qwen3_rmsnorm(er.data(), get("mtp.pre_fc_norm_embedding").f32(), ee.data(), H, c.rms_eps);
            std::memcpy(cat.data(), ee.data(), sizeof(float) * H);
            std::memcpy(cat.data() + H, eh.data(), sizeof(float) * H);
            lin(get("mtp.fc"), cat.data(), hp.data(), H, 2 * H);
            if (mtp_mode) {
                attn("mtp.layers[0].", 0, hp.data(), mkc, mvc, i);
                mlp("mtp.layers[0].", hp.data());
            }
            mtp_h = hp;
            orc_qwen3_rmsnorm(hp.data(), get("mtp.norm").f32(), hn.data(), H, c.rms_eps);
            lin(get("lm_head"), hn.data(), lg.data(), c.vocab, H);
            tok = orc_greedy(lg.data(), c.vocab);
            out[i] = tok;
        }
        return n;
    }
};

}  // namespace

extern "C" {

void* orc_model_create(const RlModelConfig* cfg, const RlTensor* t, int n, int ctx, int kv_fp16, int nthreads) {
    try {
        auto* m = new Model();
        m->c = *cfg;
        m->ctx = ctx;
        m->kv_fp16 = kv_fp16 != 0;
        m->nthreads = nthreads;
        for (int i = 0; i < n; ++i) m->w[t[i].name] = W{t[i].quant, t[i].rows, t[i].cols, t[i].data, t[i].scale};
        m->reset();
        return m;
    } catch (...) {
        return nullptr;
    }
}

void orc_model_free(void* h) { delete static_cast<Model*>(h); }
void orc_model_reset(void* h) { static_cast<Model*>(h)->reset(); }
int orc_model_pos(void* h) { return static_cast<Model*>(h)->pos; }

int orc_model_decode(void* h, int token, float* logits, float* hidden) {
    auto* m = static_cast<Model*>(h);
    try {
        m->decode(token);
    } catch (...) {
        return -1;
    }
    if (logits) std::memcpy(logits, m->logits.data(), sizeof(float) * m->c.vocab);
    if (hidden) std::memcpy(hidden, m->last_hidden.data(), sizeof(float) * m->c.hidden);
    return orc_greedy(m->logits.data(), m->c.vocab);
}

void orc_model_set_mtp_mode(void* h, int mode) { static_cast<Model*>(h)->mtp_mode = mode; }

int orc_model_mtp_hidden(void* h, float* out) {
    const auto* m = static_cast<Model*>(h);
    if (static_cast<int>(m->mtp_h.size()) != m->c.hidden) return -1;
    std::memcpy(out, m->mtp_h.data(), sizeof(float) * m->c.hidden);
    return 0;
}

int orc_model_mtp_draft(void* h, int first, int n, int* out) {
    try {
        return static_cast<Model*>(h)->mtp_draft(first, n, out);
    } catch (...) {
        return -1;
    }
}

// Session::generate CPU branch (session.cpp:687-829, prefill = sequential decode
// of the prompt, which is what the layer-wise prefill computes).  spec_n = 0 is
// spec off.  Returns produced; *accepted / *proposed are the spec stats.
int orc_model_generate(void* h, const int* prompt, int n, int max_new, int spec_n, int* out, int* proposed,
                       int* accepted) {
    auto* m = static_cast<Model*>(h);
    try {
        m->reset();
        for (int i = 0; i < n; ++i) m->decode(prompt[i]);
        int produced = 0, prop = 0, acc = 0;
        while (produced < max_new) {
            const int t0 = orc_greedy(m->logits.data(), m->c.vocab);
            out[produced++] = t0;
            int drafts[16];
            int nd = 0;
            if (spec_n > 0 && produced < max_new) {
                nd = m->mtp_draft(t0, std::min(spec_n, 16), drafts);
                prop += nd;
            }
            m->decode(t0);
            for (int i = 0; i < nd && produced < max_new; ++i) {
                if (orc_greedy(m->logits.data(), m->c.vocab) != drafts[i]) break;
                out[produced++] = drafts[i];
                ++acc;
                m->decode(drafts[i]);
            }
        }
        if (proposed) *proposed = prop;
        if (accepted) *accepted = acc;
        return produced;
    } catch (...) {
        return -1;
    }
}

// Layer-level entry points for the kernel parity tests: run one DeltaNet layer /
// attention layer / MLP of the model in place on x (ops_fused.cpp).
int orc_model_layer(void* h, int layer, float* x, int part) {
    auto* m = static_cast<Model*>(h);
    try {
        const std::string p = "layers[" + std::to_string(layer) + "].";
        if (part == 0) {
            if (m->c.layer_kind[layer] == RL_LAYER_DELTA)
                m->delta(p, m->slot[layer], x);
            else
                m->attn(p, m->slot[layer], x, m->kc[m->slot[layer]], m->vc[m->slot[layer]], m->pos);
        } else {
            m->mlp(p, x);
        }
        return 0;
    } catch (...) {
        return -1;
    }
}

// Direct access to the model's recurrent state / caches (for seeding and compare).
float* orc_model_state(void* h, int slot) { return static_cast<Model*>(h)->S[slot].data(); }
float* orc_model_conv(void* h, int slot) { return static_cast<Model*>(h)->conv[slot].data(); }
float* orc_model_kcache(void* h, int slot) { return static_cast<Model*>(h)->kc[slot].data(); }
float* orc_model_vcache(void* h, int slot) { return static_cast<Model*>(h)->vc[slot].data(); }
void orc_model_set_pos(void* h, int pos) { static_cast<Model*>(h)->pos = pos; }

}  // extern "C"
