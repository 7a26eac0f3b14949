// internal.h -- launchers shared between the kernel files and the engine.
#pragma once

#include "common.h"

namespace rl {

enum GemmEpilogue {
    kEpiStore = 0,
    kEpiAdd = 1,
    kEpiSwiGLU = 2,
    kEpiPartial = 3,
    kEpiAddNorm = 4,
    kEpiSwiGLUH = 5,
    // prefill only: SwiGLU over half tiles written straight as the next GEMM's bf16
    // hi + mid input fragments (Y is the fragment buffer; outputs a multiple of 128)
    kEpiSwiGLUHFrag = 6
};

// RMSNorm folded across a residual GEMM and the next linear (y = rmsnorm(x) * (1+g)
// never materialised):
//   producer (kEpiAddNorm): Y = x += W.a in place; frag_out = fragments of
//     x * (1 + gamma_out); ss_out[group][t] = sum of x^2 over the group's rows
//     (add_norm_groups(m) groups of 32 rows, summed in double, stored as float);
//   consumer (ss_in != null): its input fragments are x * (1 + gamma); outputs are
//     scaled by 1/sqrt(sum_groups ss_in / n_norm + eps) per token.
struct NormIO {
    const float* ss_in = nullptr;
    int groups_in = 0;
    int n_norm = 0;
    float eps = 0.f;
    const float* gamma_out = nullptr;
    float* ss_out = nullptr;
    // Gated RMSNorm folded into the consuming GEMM, one norm group per 128-column
    // block: kss[kb][t][4] holds four partial sums of squares of block kb's
    // un-normalised inputs for token t, and the block's products are scaled by
    // 1/sqrt(sum / kss_n + kss_eps).
    const float* kss = nullptr;
    int kss_n = 0;
    float kss_eps = 0.f;
    // Store launches: the row tiles from x_tile0 on are not given workgroups of their
    // own (so the launch fits two workgroups per CU); the first workgroups compute
    // them after their own rows as x_slices K-slices.  Slice s of token t, row r
    // (counted from row 16 * x_tile0) goes to xpart[(s * T + t) * x_rows + r]; the
    // consumer adds the slices in order.
    float* xpart = nullptr;
    int x_tile0 = 0;
    int x_slices = 0;
    int x_rows = 0;
};

// gemm.hip
// S > 1 (split-K) requires epi == kEpiPartial: slice s writes Y + (s*T + t)*ldy.
// frag_out (SwiGLU / add-norm): also write the next linear's input fragments.
void gemm_fp8_frag(const uint8_t* W, const float* ts, const void* frag, float* Y, int m, int n, int T, int epi,
                   int ldy, int m_valid, hipStream_t s, int S = 1, void* frag_out = nullptr,
                   const NormIO* norm = nullptr);
void gemm_bf16_frag(const uint16_t* W, const void* frag, float* Y, int m, int n, int T, int epi, int ldy, int m_valid,
                    hipStream_t s, int S = 1, void* frag_out = nullptr, const NormIO* norm = nullptr);
int add_norm_groups(int m);
int norm_group_rows();  // rows per add-norm sum-of-squares group
// FP8 store launches (T <= 4): row tiles and waves per workgroup (two workgroups
// per CU are resident either way)
int gemm_store_rows_per_wg();
int gemm_store_waves();

// prefill.hip: Y = W . X for T (any) tokens on MFMA; epi store / add / SwiGLU
// (interleaved gate/up tiles, m_valid = m/2 output rows).  frag: act fragments of T.
// wk 0: FP8 tiles (ts); 1: BF16 tiles; 2: BF16 W + W_lo tiles (16 significant bits)
void gemm_prefill_any(int wk, const uint8_t* W, const uint8_t* W_lo, const float* ts, const void* frag, float* Y,
                      int m, int n, int T, int epi, int ldy, int m_valid, hipStream_t s, const float* xscale = nullptr);
// K-quant tiles (qt 4 / 6, m rows in 16-row tiles) -> BF16 tiles hi and lo
void kq_to_bf16x2(int qt, const uint8_t* tiled, uint16_t* hi, uint16_t* lo, int m, int n, hipStream_t s);
// K-quant tiles -> fp16 in the BF16 tile layout, one power-of-two scale per (16-row
// tile, 128-column block) in tscale[m_tiles][n / 128]
void kq_to_f16(int qt, const uint8_t* tiled, void* w16, float* tscale, int m, int n, hipStream_t s);
// bf16 hi + mid activation fragments (T tokens, n columns) -> fp16 hi + lo fragments
// of x / xscale[kb][t], xscale a power of two per (128-column block, token)
void act_frag_to_f16(const void* frag, void* frag16, float* xscale, int n, int T, hipStream_t s);
void gemm_fp8_prefill(const uint8_t* W, const float* ts, const void* frag, float* Y, int m, int n, int T, int epi,
                      int ldy, int m_valid, hipStream_t s);
int device_cus();  // CUs of the current device
void pack_act(const float* X, void* frag, int n, int T, hipStream_t s);
void pack_fp8_rows(const uint8_t* w, const float* scale, uint8_t* dst, float* tscale, int m, int n, int rt_stride,
                   int rt_offset, hipStream_t s);
void pack_bf16_rows(const uint16_t* w, uint16_t* dst, int m, int n, int rt_stride, int rt_offset, hipStream_t s);
// Gate and up [I][n] into half tiles (tile k: gate rows 8k..8k+7, then up rows), 2*I
// tiled rows; FP8 tile scales [tile][kb][2].  The kEpiSwiGLUH epilogue reads this.
void pack_fp8_gate_up(const uint8_t* gw, const float* gs, const uint8_t* uw, const float* us, uint8_t* dst,
                      float* tscale, int I, int n, hipStream_t s);
void pack_bf16_gate_up(const uint16_t* gw, const uint16_t* uw, uint16_t* dst, int I, int n, hipStream_t s);

// kquant.hip
// RMSNorm folded across K-quant GEMVs (as NormIO for the FP8 path):
//   consumer (ss_in): x is the producer's x * (1 + gamma) rows; the outputs are
//     scaled by 1/sqrt(sum_groups ss_in / n_norm + eps);
//   producer (ss_out, with accumulate into the residual rows x [T][m]): x += W.a,
//     ss_out[group][t] = sum of x^2 over the row group's rows (kq_norm_groups(m)
//     groups, double, stored as float), xg_out [T][m] = x * (1 + gamma_out) and, if
//     frag_out, the same as the next FP8 / BF16 linear's input fragments.
struct KqNorm {
    const float* ss_in = nullptr;
    int groups_in = 0;
    int n_norm = 0;
    float eps = 0.f;
    float* ss_out = nullptr;
    const float* gamma_out = nullptr;
    float* xg_out = nullptr;
    void* frag_out = nullptr;
    // the rows are gate / up half tiles (rl_hip_pack_kquant_gate_up): the launch
    // writes h [T][m/2] = silu(gate) * up at stride ldy instead of the m rows
    int swiglu = 0;
    // with ss_out: the input's 128-column blocks are scaled per token by
    // 1/sqrt(sum / 128 + 1e-6), sum the four partial sums bss[(blk * T + t) * 4 + 0..3]
    // (the DeltaNet output's gated RMSNorm per head)
    const float* bss = nullptr;
    // Extra rows in BF16 (the DeltaNet in_proj a / b rows beside K-quant q|k|v, z):
    // ab_w is their tiled BF16 matrix (rl_hip_pack_bf16 layout, ab_rows rows, the
    // launch's n columns); extra workgroups compute them from the same x as
    // ab_slices K-slice partials, ab_out[(slice * T + t) * ab_ld + row], scaled like
    // the main rows (1/rms with ss_in).
    const uint16_t* ab_w = nullptr;
    int ab_rows = 0;
    int ab_slices = 0;
    float* ab_out = nullptr;
    int ab_ld = 0;
};
int kq_norm_groups(int m);
bool kq_fold_supported();  // the folded-norm variants run with the default work split
size_t kq_workspace_bytes(int m, int n, int T);
// Host dequantisation of row-major GGML blocks (Q8_0 / Q4_K / Q5_K / Q6_K) with the
// reference's rounding order (loader.cpp); n = number of values.
void dequant_host(int quant, const uint8_t* blocks, float* out, int64_t n);
void kq_gemm(int qt, const uint8_t* W, const float* x, float* Y, void* ws, size_t ws_bytes, int m, int n, int T,
             int accumulate, int ldy, hipStream_t s, const KqNorm* norm = nullptr);

// norms.hip
void rmsnorm_pack(const float* x, int ld_x, const float* gamma, float* y, void* frag, int n, int T, float eps,
                  hipStream_t s);
// Residual update fused with the next RMSNorm: x_out = x_in + sum_{s<S} P[s] (rows
// [T][n], slices P + s*T*n, added in slice order), then y / frag = rmsnorm(x_out).
// x_out must not alias x_in.  P may be NULL (S ignored).
void residual_rmsnorm_pack(const float* x_in, const float* P, int S, float* x_out, const float* gamma, float* y,
                           void* frag, int n, int T, float eps, hipStream_t s);
void gnorm_pack(const float* o, const float* z, int ld_z, const float* gamma, int gamma_n, float* y, void* frag,
                int n, int T, float eps, hipStream_t s);
void embed_rows(const void* table, int kind, const int* tokens, float* out, int H, int vocab, int T, hipStream_t s);
void swiglu(const float* g, int ldg, const float* u, int ldu, float* h, int n, int T, hipStream_t s);
void copy_int(const int* src, int* dst, hipStream_t s);

// gdn.hip
void gdn_decode(const float* qkv, const float* a, const float* b, int ld_in, const float* A_log, const float* dt_bias,
                const float* conv_w, const float* conv_in, float* conv_out, const float* S_in, float* S_out,
                const int* cur, size_t conv_slot, size_t s_slot, int R, float* o, int T, int nk, int nv, int dk,
                int dv, int K, int v_tiled, hipStream_t s);

// Fused DeltaNet decode (dk 128, dv a multiple of 32, conv 4) with the gated
// RMSNorm's elementwise part and the packing into out_proj fragments (gamma [dv],
// gate z at z[t*ld_in + h*dv + j]).
// Speculative bookkeeping of the fused DeltaNet kernel.  The state S is kept once,
// committed up to the last consumed token.  A call that may be partly rejected
// (keep = 1) stores, per head and token, the normalised k, the update
// delta = (v - S^T k) * beta and the decay g (kGdnRecFloats floats), and leaves S
// at the committed point; the next call first replays the first
// min(*n_cons, count) records onto S (the same float operations the update
// performs, so the result is bit-identical to having kept S after that token).
// Records live in R banks, one per conv-ring slot: a call writes bank *cur and
// reads bank (*cur - *n_cons) mod R, the previous call's (distinct, as
// 1 <= n_cons <= T < R), so workgroups of one call never read what others write.
constexpr int kGdnRecFloats = 264;  // k[128] | delta[dv <= 128] | g
struct GdnRecords {
    float* rec;          // [R][max_t][nv][kGdnRecFloats]
    int* count;          // [R][nv]: tokens recorded per head
    const int* n_cons;   // tokens the previous call consumed
    int max_t;           // token capacity of a bank
    int keep;            // record this call's tokens instead of committing them
};
// Batch of independent sequences (grid dimension y): sequence b's state, conv ring,
// records and scalars sit at the given strides from sequence 0's; its T tokens are
// input / output rows b * T + t of B * T.
struct GdnBatch {
    int B = 1;
    size_t s_stride = 0, conv_stride = 0, rec_stride = 0;  // floats
    int count_stride = 0, scal_stride = 0;                // ints
};
// Workgroup = (v-head, 32 value columns).  conv window: a ring of R slots when
// cur != nullptr (slot *cur read, slot (*cur + 1 + t) % R written after token t),
// else conv_in -> conv_out.  S: S_in -> S_out (may alias); with cur, rec must be
// given and S_out == S_in is the committed state.  Outputs: o [T][nv*dv] (may be
// null) and/or, with frag, the out_proj input fragments of
// y = gamma * o * silu(z) with the per-head norm left to the GEMM: gss[h][t][4]
// receives the four 32-column partial sums of o^2 (dv must be 128 then); y32
// (optional, same conditions) receives y as fp32 rows [T][nv * dv].
// a / b (per head h, token t): the sum over s < ab_slices of a[(s * T + t) * ab_ld + h]
// (ab_slices 1: a[t * ld_in + h]).
bool gdn_fused_supported(int dk, int dv, int K);
void gdn_decode_fused(const float* qkv, const float* a, const float* b, int ld_in, const float* A_log,
                      const float* dt_bias, const float* conv_w, const float* conv_in, float* conv_out,
                      const float* S_in, float* S_out, const int* cur, size_t conv_slot, int R,
                      const GdnRecords* rec, float* o, const float* z, const float* gamma, void* frag, float* gss,
                      int T, int nk, int nv, int dk, int dv, int K, int v_tiled, hipStream_t s, int ab_slices = 1,
                      int ab_ld = 0, const GdnBatch* batch = nullptr, int row_off = 0, int T_rows = 0,
                      float* y32 = nullptr);

// Prompt prefill of T tokens from the conv window conv_in (direct mode): conv +
// gates over all tokens (xc [T][conv_dim], gates [T][nv][2] scratch), then the
// recurrence with S (transposed, one copy) updated in place; o [T][nv*dv] raw
// recurrent output; conv_out = window after the last token.
void gdn_prefill(const float* y, int ld, int off_a, int off_b, const float* A_log, const float* dt_bias,
                 const float* conv_w, const float* conv_in, float* conv_out, float* xc, float* gates, float* S,
                 float* o, int T, int nk, int nv, int dk, int dv, int K, int v_tiled, hipStream_t s,
                 float* ck = nullptr);
// ck (when not null and dk = dv = 128): gdn_prefill_chunk_floats(T, nv, dk, dv)
// floats of scratch for the chunked scan; null, or other head sizes: the per-token
// scan.  0 where the chunked scan does not apply.
size_t gdn_prefill_chunk_floats(int T, int nv, int dk, int dv);
// The chunked scan unless RL_PF_GDN_CHUNK=0.
bool gdn_prefill_chunked();

// attn.hip
size_t attn_workspace_bytes(int nkv, int ctx);
// Outputs of token t go to column t_off + t of T_out (T_out 0: T), so one sequence
// of a batch can write its column of the next linear's input.
void attn_decode_layer(const float* Y, int ld_y, const float* q_norm, const float* k_norm, uint16_t* kc, uint16_t* vt,
                       int ctx, const int* pos_dev, int T, int nq, int nkv, int hd, int rot, float theta, float eps,
                       void* ws, size_t ws_bytes, float* out, void* frag, hipStream_t s, int t_off = 0,
                       int T_out = 0, int nb = 1, size_t kv_bstride = 0, int pos_stride = 0);

// Prompt prefill of T tokens at *pos_dev .. *pos_dev + T - 1: K/V of all T written to
// the cache, causal attention over the cache, out [T][nq*hd] fp32 (times sigmoid(gate)).
size_t attn_prefill_workspace_bytes(int nq, int T);
void attn_prefill_layer(const float* Y, int ld_y, const float* q_norm, const float* k_norm, uint16_t* kc,
                        uint16_t* vt, int ctx, const int* pos_dev, int T, int nq, int nkv, int hd, int rot,
                        float theta, float eps, void* ws, size_t ws_bytes, float* out, hipStream_t s);

// sample.hip
size_t argmax_workspace_bytes(int rows, int V);
void argmax_rows(const float* logits, int rows, int V, int* out, float* out_val, void* ws, hipStream_t s);
void batch_advance(int* scal, int stride, int B, int R, int k_pos, int k_slot, int k_ncons, hipStream_t s);
void accept(const int* toks, const int* preds, int T, int force_all, int* pos, int* slot, int R, int* n_out,
            int* next_tok, int* gen_ring, int* gen_count, int gen_cap, const float* xout, float* h_last,
            float* h_prev, int H, hipStream_t s);

// synth.hip
void fill_fp8(uint8_t* p, size_t n, uint64_t seed, hipStream_t s);
// random GGML Q4_K / Q6_K super-blocks (fp16 d, dmin log-uniform in [1e-4, 1e-2])
void fill_kquant(uint8_t* p, int type, size_t n_blocks, uint64_t seed, hipStream_t s);
void fill_loguniform(float* p, size_t n, float lo, float hi, uint64_t seed, hipStream_t s);
void fill_normal_f32(float* p, size_t n, float mean, float stdv, uint64_t seed, hipStream_t s);
void fill_normal_bf16(uint16_t* p, size_t n, float stdv, uint64_t seed, hipStream_t s);
void fill_normal_f16(uint16_t* p, size_t n, float stdv, uint64_t seed, hipStream_t s);

size_t act_frag_bytes(int n, int T);

}  // namespace rl
