/*
 * rapidllm_hip.h -- C ABI of the MI355X (gfx950) decode backend for RapidLLM.
 *
 * Plain pointers and sizes only; no C++ or torch types cross this boundary.  Every
 * function returns an RlStatus (values identical to RapidStatus,
 * include/rapidllm/api.h:11-19 of the reference) and leaves a message for
 * rl_hip_last_error() on failure; no exception crosses the ABI (the reference's C
 * layer does the same, src/api/rapidllm_c.cpp:46-50, 246-251).
 *
 * Device pointers are plain `void*` from rl_hip_malloc (or any hipMalloc'd
 * memory); `stream` is a hipStream_t passed as void* (NULL = the null stream).
 * Kernel entry points are asynchronous on `stream`.
 *
 * The reference interfaces each group replaces are cited per declaration.
 * Benchmark, tuning and calibration entry points (no reference counterpart) are
 * declared separately, in rapidllm_hip_bench.h.
 */
#ifndef RAPIDLLM_HIP_H
#define RAPIDLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "rl_model.h"

#ifdef __cplusplus
extern "C" {
#endif

#define RL_HIP_ABI_VERSION 1

typedef enum RlStatus {
    RL_OK = 0,
    RL_ERR_IO,
    RL_ERR_FORMAT,
    RL_ERR_NOMEM,
    RL_ERR_UNSUPPORTED,
    RL_ERR_DEVICE,
    RL_ERR_RANGE,
    RL_ERR_INTERNAL
} RlStatus;

/* ---- runtime ------------------------------------------------------------
 * Replaces: cuda_gen::available() (include/rapidllm/runtime/cuda_engine.h:11),
 * rapidllm::Device::{allocate, create_stream, memcpy} and Stream::synchronize
 * (include/rapidllm/backend/device.h:41-60). */
int rl_hip_abi_version(void);
int rl_hip_available(void); /* 1 when a gfx950 device is visible */
const char* rl_hip_last_error(void);
int rl_hip_device_info(char* arch, int cap, int* n_cu, size_t* hbm_bytes);
int rl_hip_malloc(void** ptr, size_t bytes);
int rl_hip_free(void* ptr);
int rl_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int rl_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int rl_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int rl_hip_memset(void* ptr, int value, size_t bytes, void* stream);
/* Pinned host memory the device can read and write (Device::allocate for
 * host-visible buffers, BufferDesc::host_visible, device.h:15-19). */
int rl_hip_host_alloc(void** ptr, size_t bytes);
int rl_hip_host_free(void* ptr);
int rl_hip_stream_create(void** stream);
int rl_hip_stream_destroy(void* stream);
int rl_hip_stream_synchronize(void* stream);
int rl_hip_device_synchronize(void);
/* Events time work on the stream it is recorded on. */
int rl_hip_event_create(void** ev);
int rl_hip_event_destroy(void* ev);
int rl_hip_event_record(void* ev, void* stream);
int rl_hip_event_elapsed_ms(void* start, void* stop, float* ms);

/* ---- e4m3 decode -----------------------------------------------------------
 * Replaces: ops::e4m3_to_f32 (src/kernels/ops.cpp:57-71).  Decodes with the same
 * hardware conversion the GEMM uses (to bf16, then widened), so its bit-exactness
 * test covers the GEMM's weight decode. */
int rl_hip_e4m3_to_f32(const uint8_t* in, float* out, size_t n, void* stream);

/* ---- block-FP8 / BF16 linears ---------------------------------------------
 * Replaces: ops::gemv_fp8 / ops::linear(FP8_E4M3_B128) (src/kernels/ops.cpp:182-194,
 * 404-418), the CUDA launch_linear / launch_gemm_fp8 T<=4 family
 * (src/kernels/cuda/cuda_engine.cu:10656-10672, 11964-12030), and
 * Device::launch("gemv_fp8", GemvFp8Params) (include/rapidllm/backend/params.h:6).
 *
 * Weights live on the device in an MFMA-tiled layout (16 rows x 128 columns per
 * tile, lane-ordered); rl_hip_pack_* converts the on-disk row-major bytes.
 * rows are padded to 16 and columns to 128 with zeros.
 *   packed FP8 bytes  = rl_hip_fp8_packed_bytes(m, n)
 *   tile scales (f32) = rl_hip_fp8_tile_scales(m, n) floats, one per 16x128 tile,
 *                       copied from the [ceil(m/128)][ceil(n/128)] block scales.
 * Activations are fp32 [T][n]; they are split into bf16 hi + mid terms (16
 * significant bits, fp32 range) in a fragment buffer of rl_hip_act_frag_bytes(n, T). */
size_t rl_hip_fp8_packed_bytes(int m, int n);
size_t rl_hip_fp8_tile_scales(int m, int n);
size_t rl_hip_bf16_packed_bytes(int m, int n);
size_t rl_hip_act_frag_bytes(int n, int T);
int rl_hip_pack_fp8(const uint8_t* w_dev_rowmajor, const float* scale_dev, uint8_t* w_tiled, float* tile_scale,
                    int m, int n, void* stream);
int rl_hip_pack_bf16(const uint16_t* w_dev_rowmajor, uint16_t* w_tiled, int m, int n, void* stream);
/* MLP gate and up ([I][n] each, I a multiple of 8) packed together for the SwiGLU
 * epilogue: tiled row tile k holds gate rows 8k..8k+7 then up rows 8k..8k+7, so the
 * packed matrix has 2*I rows (rl_hip_fp8_packed_bytes(2*I, n) bytes) and FP8 tile
 * scales [I/8][ceil(n/128)][2] (rl_hip_fp8_gate_up_tile_scales(I, n) floats; each
 * half keeps its own 128x128 block scale). */
size_t rl_hip_fp8_gate_up_tile_scales(int I, int n);
int rl_hip_pack_fp8_gate_up(const uint8_t* gate_w, const float* gate_scale, const uint8_t* up_w, const float* up_scale,
                            uint8_t* w_tiled, float* tile_scale, int I, int n, void* stream);
int rl_hip_pack_bf16_gate_up(const uint16_t* gate_w, const uint16_t* up_w, uint16_t* w_tiled, int I, int n,
                             void* stream);
int rl_hip_pack_act(const float* X, void* frag, int n, int T, void* stream);
/* Y[T][m] (=, or += when accumulate) W . X for T in 1..16 using a packed fragment
 * buffer.  Deterministic: partial sums are combined in a fixed order, and token t's
 * result does not depend on T. */
/* Prompt prefill: Y[t][ldy] (=, +=) W . x_t for T (any) tokens of rl_hip_pack_act
 * fragments, on the matrix cores (128 rows x 64 tokens per workgroup).  epilogue:
 * 0 store, 1 add, 2 SwiGLU over interleaved gate/up 16-row tiles (m/2 output rows),
 * 5 SwiGLU over the rl_hip_pack_fp8_gate_up half tiles (m/2 output rows), 6 the same
 * written as rl_hip_pack_act fragments of the m/2 outputs (Y is then the fragment
 * buffer, bit-identical to epilogue 5 followed by rl_hip_pack_act; m/2 a multiple of
 * 128).  ldy <= 0: m (m/2 for SwiGLU).  Replaces the reference's prefill linears
 * (cuda_engine.cu:18338-18590 -> launch_linear for T > 8, :12008-12016). */
int rl_hip_gemm_fp8_prefill(const uint8_t* w_tiled, const float* tile_scale, const void* frag, float* Y, int m, int n,
                            int T, int epilogue, int ldy, void* stream);
/* The same over BF16 tiles (rl_hip_pack_bf16 layout): W, or W_hi + W_lo when
 * w_lo_tiled is given (a weight split into 16 significant bits, as
 * rl_hip_kquant_to_bf16x2 writes a K-quant matrix).  The K-quant models' prefill
 * linears (the reference runs them through its multi-token K-quant GEMVs,
 * cuda_engine.cu:12076-12260). */
int rl_hip_gemm_bf16_prefill(const uint16_t* w_tiled, const uint16_t* w_lo_tiled, const void* frag, float* Y, int m,
                             int n, int T, int epilogue, int ldy, void* stream);
/* A tiled Q4_K / Q6_K matrix (rl_hip_pack_kquant, or the gate / up half tiles) as
 * two BF16 tiled matrices W_hi + W_lo of the same row order: each weight dequantised
 * exactly as ops::dequant_q4_k / dequant_q6_k (ops.cpp:245-402), then split into
 * its top 16 bits (hi) and the top 16 bits of the remainder (lo). */
int rl_hip_kquant_to_bf16x2(int type, const uint8_t* tiled, uint16_t* w_hi, uint16_t* w_lo, int m, int n,
                            void* stream);
/* The K-quant prefill linears' form: a tiled Q4_K / Q6_K matrix as fp16 tiles in
 * the BF16 tile layout (w16: 2 bytes per weight), each weight dequantised exactly,
 * divided by its (16-row tile, 128-column block)'s power-of-two scale tile_scale
 * [m/16][n/128] (which puts the block's largest |w| in [2^14, 2^15)) and rounded to
 * fp16 (11 significant bits). */
int rl_hip_kquant_to_f16(int type, const uint8_t* tiled, void* w16, float* tile_scale, int m, int n, void* stream);
/* rl_hip_pack_act fragments (bf16 hi + mid) -> fp16 hi + lo fragments of
 * x / xscale, xscale [n/128][T] a power of two per (128-column block, token). */
int rl_hip_act_frag_to_f16(const void* frag, void* frag16, float* xscale, int n, int T, void* stream);
/* Prompt prefill over fp16 tiles: Y[t][ldy] (=, +=, SwiGLU) sum over blocks of
 * tile_scale * xscale * (W16 . x16) (two fp16 MFMAs per step, hi and lo of x). */
int rl_hip_gemm_f16_prefill(const void* w16, const float* tile_scale, const void* frag16, const float* xscale,
                            float* Y, int m, int n, int T, int epilogue, int ldy, void* stream);

int rl_hip_gemm_fp8_frag(const uint8_t* w_tiled, const float* tile_scale, const void* frag, float* Y, int m, int n,
                         int T, int accumulate, void* stream);
int rl_hip_gemm_bf16_frag(const uint16_t* w_tiled, const void* frag, float* Y, int m, int n, int T, int accumulate,
                          void* stream);
/* Convenience: pack X into `frag_scratch` then GEMM (two launches). */
int rl_hip_gemm_fp8(const uint8_t* w_tiled, const float* tile_scale, const float* X, float* Y, void* frag_scratch,
                    int m, int n, int T, void* stream);

/* ---- GGUF K-quant linears -------------------------------------------------
 * Replaces: ops::dequant_q4_k / dequant_q6_k (src/kernels/ops.cpp:255-284, 357-387),
 * ops::gemv_q4_k / gemv_q6_k (ops.cpp:292-305, 389-402; threaded in
 * src/kernels/cpu_caps.cpp:200-222), the CUDA K-quant T=1..4 families
 * (src/kernels/cuda/cuda_engine.cu:2347-2647, gemv_t4_pipe.cu, gemv_t4_q6_t12tile.cu)
 * and Device::launch("gemv_q4k" / "gemv_q6k", GemvKQuantParams) (params.h:7).
 * `type` is RL_Q_Q4_K or RL_Q_Q6_K.  Blocks are the GGUF bytes (144 B / 210 B per
 * 256 weights, rows contiguous); rl_hip_pack_kquant moves them (bytes only) into
 * the device layout.  X is fp32 [T][n], T in 1..16 (one weight pass for all T rows;
 * the noalloc variant below takes 1..4), n a multiple of 256.
 * rl_hip_dequant_kquant decodes row-major blocks bit-exactly like the reference.
 * workspace (rl_hip_kquant_workspace_bytes): split-K tickets then partial sums.
 * Zero-fill it once after allocation (rl_hip_memset); every launch leaves the
 * tickets at zero again.  Launches sharing one workspace must not overlap in time:
 * give each stream its own workspace. */
size_t rl_hip_kquant_tiled_bytes(int type, int m, int n);
size_t rl_hip_kquant_workspace_bytes(int m, int n, int T);
int rl_hip_pack_kquant(int type, const uint8_t* blocks, uint8_t* tiled, int m, int n, void* stream);
int rl_hip_gemm_kquant(int type, const uint8_t* tiled, const float* X, float* Y, void* workspace,
                       size_t workspace_bytes, int m, int n, int T, int accumulate, void* stream);
int rl_hip_dequant_kquant(int type, const uint8_t* blocks, float* out, size_t n_blocks, void* stream);

/* Fused MLP gate / up projection with SwiGLU.  Replaces the pair gemv_q4_k /
 * gemv_q6_k over mlp.gate and mlp.up plus ops::swiglu (ops.cpp:607-609) of the
 * reference's MLP block (the CUDA engine's fused gate/up + SwiGLU family,
 * cuda_engine.cu:2347-2647).  rl_hip_pack_kquant_gate_up packs the I x n gate and up
 * blocks (one type) as half tiles: tiled = rl_hip_kquant_tiled_bytes(type, 2 I, n)
 * bytes, I a multiple of 8.  rl_hip_gemm_kquant_swiglu writes
 * H [T][I] = silu(gate . x) * (up . x) with the workspace of a 2 I x n launch
 * (rl_hip_kquant_workspace_bytes(2 I, n, T)). */
int rl_hip_pack_kquant_gate_up(int type, const uint8_t* gate_blocks, const uint8_t* up_blocks, uint8_t* tiled,
                               int I, int n, void* stream);
int rl_hip_gemm_kquant_swiglu(int type, const uint8_t* tiled, const float* X, float* H, void* workspace,
                              size_t workspace_bytes, int I, int n, int T, void* stream);

/* Allocation-free variant of rl_hip_gemm_kquant.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same arguments
 * and result as rl_hip_gemm_kquant without the workspace: the split-K tickets and
 * partial sums live in a fixed device array of the library
 * (rl_hip_gemm_kquant_noalloc_max_scratch() bytes = 4 MiB per device, held until
 * the process ends), set up on the first call on each device.  Shapes whose
 * workspace (rl_hip_kquant_workspace_bytes) exceeds it return RL_ERR_RANGE.  It
 * calls no allocating routine.  The first call on a device clears the array on its
 * stream; calls on other streams issued before that clear is seen complete wait for
 * it on the device (hipStreamWaitEvent), so first uses on several streams are safe.
 * After that, every call on one device shares the array: calls that overlap in
 * time on one device (two streams, two threads) race, so serialise them (one
 * stream per device) or use rl_hip_gemm_kquant with a workspace per stream. */
int rl_hip_gemm_kquant_noalloc(int type, const uint8_t* tiled, const float* X, float* Y, int m, int n, int T,
                               int accumulate, void* stream);
size_t rl_hip_gemm_kquant_noalloc_max_scratch(void);

/* ---- Gated DeltaNet recurrent decode -----------------------------------------
 * Replaces: ops::conv1d_update (src/kernels/ops.cpp:458-468), the gate math of
 * ops::fused_delta_decode (src/kernels/ops_fused.cpp:111-123), ops::l2norm and
 * ops::delta_recurrent_step{,_simd} (ops.cpp:158-163, 495-540; cpu_caps.cpp:236-265),
 * the CUDA gdn_decode_t1_k / gdn_decode_tn_k (cuda_engine.cu:5166-5410) and
 * Device::launch("conv1d_update" / "delta_recurrent", Conv1dParams /
 * DeltaRecurrentParams) (params.h:17-18).
 * For T tokens: qkv/a/b are rows t*ld_in of the in_proj output (raw, before conv);
 * conv state [conv_dim][conv_k] (tap 0 oldest), conv_dim = 2*nk*dk + nv*dv;
 * S fp32 per v-head TRANSPOSED: S_dev[h][j][i] = S[h][i][j] (i < dk, j < dv).
 * o = [T][nv*dv] raw recurrent output (before the gated RMSNorm).
 * dk must be 128, dv a multiple of 32, T <= 8.  S_out may alias S_in;
 * conv_out must not alias conv_in. */
int rl_hip_gdn_decode(const float* qkv, const float* a, const float* b, int ld_in, const float* A_log,
                      const float* dt_bias, const float* conv_w, const float* conv_in, float* conv_out,
                      const float* S_in, float* S_out, float* o, int T, int nk, int nv, int dk, int dv, int conv_k,
                      int v_tiled, void* stream);

/* Prompt prefill of T tokens (1..65535) for one DeltaNet layer, from the in_proj rows y
 * [T][ld] (qkv channels at 0, a at off_a, b at off_b): conv window conv_in ->
 * conv_out (window after the last token; must not alias), S (transposed, as
 * rl_hip_gdn_decode) updated in place, o [T][nv*dv] raw recurrent output.  Workspace
 * rl_hip_gdn_prefill_workspace_bytes(T, ...).  dk 128, dv a multiple of 32, conv 4.
 * With dk = dv = 128 the scan runs in chunks of 64 tokens (gated delta rule in WY
 * form, fp32; the workspace then also holds the chunks' matrices, about 147 KB per
 * head and chunk); other shapes, or RL_PF_GDN_CHUNK=0 in the environment, step the
 * state token by token.  Both follow the same per-token recurrence to fp32 rounding.
 * Replaces the reference's prefill conv + scan (cuda_engine.cu:18338-18590;
 * CPU: per token ops::conv1d_update + delta_recurrent_step, ops.cpp:458-534). */
size_t rl_hip_gdn_prefill_workspace_bytes(int T, int nk, int nv, int dk, int dv);
int rl_hip_gdn_prefill(const float* y, int ld, int off_a, int off_b, const float* A_log, const float* dt_bias,
                       const float* conv_w, const float* conv_in, float* conv_out, float* S, float* o, void* workspace,
                       size_t workspace_bytes, int T, int nk, int nv, int dk, int dv, int conv_k, int v_tiled,
                       void* stream);

/* ---- norms fused with GEMM input packing; embedding --------------------------
 * Replaces: ops::qwen3_rmsnorm (src/kernels/ops.cpp:107-127), ops::gated_rmsnorm
 * (ops.cpp:129-156), the CUDA rmsnorm_k / gated_rms_k families
 * (cuda_engine.cu:4293-4450), Device::launch("rmsnorm" / "gated_rmsnorm",
 * RmsNormParams) (params.h:5) and embed_row (src/runtime/session.cpp:122-140).
 * Either output may be NULL: y = fp32 [T][n]; frag = GEMM fragments for n columns
 * (rl_hip_act_frag_bytes(n, T) bytes).  gamma NULL = no weight.  rmsnorm uses
 * (1 + gamma); the gated norm is per head when gamma_n < n, n % gamma_n == 0 and
 * n >= 256 (the reference rule), with z rows at stride ld_z. */
int rl_hip_rmsnorm_pack(const float* x, int ld_x, const float* gamma, float* y, void* frag, int n, int T, float eps,
                        void* stream);
int rl_hip_gated_rmsnorm_pack(const float* o, const float* z, int ld_z, const float* gamma, int gamma_n, float* y,
                              void* frag, int n, int T, float eps, void* stream);
int rl_hip_embed_rows(const void* table, int kind, const int* tokens_dev, float* out, int H, int vocab, int T,
                      void* stream);

/* ---- gated GQA attention decode over an fp16 KV cache -----------------------
 * Replaces: the attention half of ops::fused_attn_decode (src/kernels/ops_fused.cpp:
 * 137-184: q/gate split, q/k head RMSNorm, rope_partial, KV append, attn_decode,
 * sigmoid gate), ops::attn_decode (ops.cpp:575-605), the CUDA qk_prep_store_k /
 * qk_attn_decode_gqa_k (cuda_engine.cu:5696-5866) and Device::launch("attn_decode",
 * AttnDecodeParams) (params.h:16).
 * Y: rows t*ld_y of the fused projection [q0|gate0|q1|gate1|...| k | v] (per head
 * q then gate, hd each).  Token t sits at position *pos_dev + t; its K (after RoPE)
 * and V are stored as fp16 (round to nearest even) and it attends to positions
 * 0 .. *pos_dev + t.  Caches (n_kv * ctx * hd fp16 each, ctx a multiple of 256,
 * zero-filled at allocation) in MFMA fragment order, per kv head:
 *   k_cache element (pos, d): [pos/256][d/32][(pos/16)%16][(d/8)%4][pos%16][d%8]
 *   vt_cache element (pos, d): [pos/32][d/16][(pos/8)%4][d%16][pos%8].  head_dim 256,
 * (n_q/n_kv)*T <= 32.  Outputs o * sigmoid(gate): fp32 `out` [T][n_q*hd] and/or
 * o_proj fragments `frag`.  *pos_dev is not modified. */
/* Prompt prefill of T tokens at positions *pos_dev .. *pos_dev + T - 1: the T tokens'
 * K (after norm + RoPE) and V are written to the caches, then causal attention of
 * every token over positions 0 .. its own, out = [T][n_q*256] fp32 times
 * sigmoid(gate).  One workgroup per (16 tokens, kv head) with an online softmax over
 * 256-position chunks.  Replaces the reference's prefill attention
 * (cuda_engine.cu:18338-18590; CPU: per token ops::attn_decode, ops.cpp:575-605). */
size_t rl_hip_attn_prefill_workspace_bytes(int n_q, int T);
int rl_hip_attn_prefill_layer(const float* Y, int ld_y, const float* q_norm, const float* k_norm, uint16_t* k_cache,
                              uint16_t* vt_cache, int ctx, const int* pos_dev, int T, int n_q, int n_kv, int head_dim,
                              int rotary_dim, float theta, float eps, void* workspace, size_t workspace_bytes,
                              float* out, void* stream);

size_t rl_hip_attn_workspace_bytes(int n_kv, int ctx);
int rl_hip_attn_decode_layer(const float* Y, int ld_y, const float* q_norm, const float* k_norm, uint16_t* k_cache,
                             uint16_t* vt_cache, int ctx, const int* pos_dev, int T, int n_q, int n_kv, int head_dim,
                             int rotary_dim, float theta, float eps, void* workspace, size_t workspace_bytes,
                             float* out, void* frag, void* stream);

/* ---- single ops of the kernel-name device seam -----------------------------
 * Replaces: Device::launch("conv1d_update" / "delta_recurrent" / "attn_decode")
 * (include/rapidllm/backend/device.h:49-60, params Conv1dParams /
 * DeltaRecurrentParams / AttnDecodeParams, params.h:16-18) over the reference CPU
 * path's own layouts, with the arguments of ops::conv1d_update (ops.cpp:458-468),
 * ops::delta_recurrent_step (ops.cpp:495-540) and ops::attn_decode (ops.cpp:575-605):
 *   conv1d_update:   state [dim][k] (tap 0 oldest) updated in place, y [dim];
 *   delta_recurrent: S [n_v][dk][dv] row-major (the CPU Session's layout) updated
 *                    in place; q, k [n_v][dk] raw (l2-normalised here, q scaled by
 *                    1/sqrt(dk)); v, o [n_v][dv]; beta, g_log [n_v]; dk <= 256;
 *   attn_decode_f32: fp32 caches [seq][n_kv][head_dim], q, o [n_q][head_dim],
 *                    softmax(q.k / sqrt(head_dim)) over positions 0..pos; head_dim
 *                    <= 256.
 * The decode engine does not use them (its step runs the fused kernels). */
int rl_hip_conv1d_update(const float* x_t, const float* w, float* state, float* y, int dim, int k, void* stream);
int rl_hip_delta_recurrent(float* S, const float* q, const float* k, const float* v, const float* beta,
                           const float* g_log, float* o, int n_v, int dk, int dv, float eps_l2, void* stream);
int rl_hip_attn_decode_f32(const float* q, const float* k_cache, const float* v_cache, float* o, int pos, int n_q,
                           int n_kv, int head_dim, void* stream);

/* ---- greedy argmax and speculative acceptance --------------------------------
 * Replaces: greedy_sample (src/runtime/sampler.cpp:8-18), the CUDA
 * argmax_partial_rows_k / argmax_final_rows_k (cuda_engine.cu:9375-9433) and the
 * host-side prefix compare of spec_verify (cuda_engine.cu:17053-17117;
 * src/runtime/session.cpp:802-825).  Ties go to the lowest index; NaN never wins.
 * accept: n = 1 + longest prefix with preds[i] == toks[i+1]; *pos += n;
 * *next_tok = preds[n-1].  All pointers are device pointers. */
size_t rl_hip_argmax_workspace_bytes(int rows, int vocab);
int rl_hip_argmax_rows(const float* logits, int rows, int vocab, int* out_idx, float* out_val, void* workspace,
                       void* stream);
int rl_hip_accept_prefix(const int* toks, const int* preds, int T, int* pos, int* n_consumed, int* next_tok,
                         void* stream);

/* ---- decode engine ----------------------------------------------------------
 * Replaces: cuda_gen::Engine (include/rapidllm/runtime/cuda_engine.h:13-83) and its
 * CUDA implementation's decode / verify / MTP paths (src/kernels/cuda/cuda_engine.cu:
 * 17053-17733 spec_verify, 18613-18997 launch_spec_chunk / launch_decode,
 * 15266-16300 MTP).  Numerics follow the reference CPU Session
 * (src/runtime/session.cpp:325-411, 531-559, 619-681, 799-829).
 * Weights: the reference IR names (see rl_model.h).  Linears may be
 * FP8_E4M3_B128, BF16, Q4_K or Q6_K; norms / A_log / dt_bias / conv1d F32;
 * embed F32 / F16 / BF16.  Tensor data is copied during create; the caller may free
 * it afterwards.  Limits: hidden % 128 == 0, DeltaNet k_dim 128 and v_dim % 32 == 0,
 * conv width 4, attention head_dim 256, (n_q/n_kv)*max_T <= 32, max_T <= 4.
 * The engine owns one HIP stream; calls on one engine must not overlap. */
typedef struct RlEngine RlEngine;
RlEngine* rl_hip_engine_create(const RlModelConfig* cfg, const RlTensor* tensors, int n_tensors, int ctx, int max_T,
                               int* status);
void rl_hip_engine_destroy(RlEngine* e);
int rl_hip_engine_reset(RlEngine* e);
int rl_hip_engine_prefill(RlEngine* e, const int32_t* ids, int n);                    /* cuda_engine.h:18 */
int rl_hip_engine_decode_token(RlEngine* e, int32_t token);                           /* :21 */
int rl_hip_engine_decode_steps(RlEngine* e, int n);                                   /* :24 */
int rl_hip_engine_copy_gen_tokens(RlEngine* e, int32_t* host, int n);                 /* :27 */
int rl_hip_engine_copy_logits(RlEngine* e, float* host);                              /* :31 */
int rl_hip_engine_copy_last_hidden(RlEngine* e, float* host);                         /* :33 */
int rl_hip_engine_mtp_draft(RlEngine* e, int32_t first, int n, int32_t* out, int* n_out); /* :36 */
int rl_hip_engine_spec_verify(RlEngine* e, const int32_t* toks, int T, int32_t* preds, int* n_consumed); /* :72 */
/* MTP draft mode.  RL_MTP_STEM (default): the stem only, as Session::mtp_draft's
 * CPU branch (src/runtime/session.cpp:619-681).  RL_MTP_LAYER: the stem's fc output
 * then passes through the MTP decoder layer mtp.layers[0] -- gated attention over
 * its own fp16 KV cache at draft positions 0, 1, ... of the call, then the MLP --
 * as Session::mtp_layer_step (session.cpp:561-617) composes fused_attn_decode and
 * fused_mlp_decode; the reference's CUDA engine drafts through that layer for
 * official and GGUF checkpoints (cuda_engine.cu:16304-16357, 16745-16778).
 * set_mtp_mode returns RL_ERR_UNSUPPORTED for LAYER when the weights have no
 * mtp.layers[0].  Applies to mtp_draft and mtp_spec. */
#define RL_MTP_STEM 0
#define RL_MTP_LAYER 1
int rl_hip_engine_set_mtp_mode(RlEngine* e, int mode);
int rl_hip_engine_mtp_mode(RlEngine* e, int* mode, int* layer_available);
/* The last draft's hidden state before the final MTP norm ([hidden] fp32; the
 * CUDA engine's d_mtp_h_, cuda_engine.cu:16304-16357). */
int rl_hip_engine_copy_mtp_hidden(RlEngine* e, float* out);
/* MTP stem draft of T-1 tokens after t0 and the T-token verify, one submission (:40). */
int rl_hip_engine_mtp_spec(RlEngine* e, int32_t t0, int T, int32_t* toks_out, int32_t* preds, int* n_consumed);
int rl_hip_engine_greedy(RlEngine* e, int32_t* tok);                                  /* :41 */
int rl_hip_engine_pos(RlEngine* e, int* pos);                                         /* :42 */
int rl_hip_engine_info(RlEngine* e, int* vocab, int* hidden, int* ctx_capacity, size_t* device_bytes);
void* rl_hip_engine_stream(RlEngine* e);

/* ---- continuous batch (cuda_engine.h:46-66) ------------------------------------
 * Replaces: Engine::max_batch / decode_tokens / copy_logits_n / copy_greedy_n /
 * replicate_slot0 / zero_slots / prefill_slot (include/rapidllm/runtime/
 * cuda_engine.h:46-66) and the CUDA launch_decode_batch (cuda_engine.cu:18999-19113)
 * that Session::generate_batch drives (src/runtime/session.cpp:832-964).
 * An engine created with max_batch > 1 keeps max_batch independent sequences
 * (slots): DeltaNet state, conv window, KV cache and position each.  Slot 0 is the
 * sequence every single-sequence call works on.  decode_tokens consumes tokens[b]
 * at position poss[b] for slots 0 .. B-1 in one weight pass (B = 1: set_pos +
 * decode_token, as the reference); copy_logits_n / copy_greedy_n return its B rows.
 * prefill_slot runs the prefill on slot `slot` (copy_logits then has its last row).
 * max_batch <= 16.  Every weight format takes all 16 rows in one weight pass.  Needs the folded path: FP8 / BF16 linears (v_dim 128), or K-quant
 * (Q4_K / Q6_K) linears with max_T <= 4; otherwise RL_ERR_UNSUPPORTED. */
RlEngine* rl_hip_engine_create_batch(const RlModelConfig* cfg, const RlTensor* tensors, int n_tensors, int ctx,
                                     int max_T, int max_batch, int* status);
int rl_hip_engine_max_batch(RlEngine* e, int* max_batch);                              /* :46 */
int rl_hip_engine_decode_tokens(RlEngine* e, const int32_t* tokens, const int* poss, int B); /* :48 */
int rl_hip_engine_copy_logits_n(RlEngine* e, float* host, int B);                      /* :53 */
int rl_hip_engine_copy_greedy_n(RlEngine* e, int32_t* host, int B);                    /* :57 */
int rl_hip_engine_replicate_slot0(RlEngine* e, int n_slots);                           /* :59 */
int rl_hip_engine_zero_slots(RlEngine* e, int n_slots);                                /* :60 */
int rl_hip_engine_prefill_slot(RlEngine* e, const int32_t* ids, int n, int slot);      /* :62 */
/* Equal-length prompts of B sequences (ids time-major [T][B]) into slots 0 .. B-1,
 * which the caller has zeroed (Session::generate_batch, session.cpp:882-893);
 * afterwards copy_logits_n / copy_greedy_n return each slot's row after its last
 * token.  Replaces Engine::prefill_eq_batch (cuda_engine.h:66-68,
 * cuda_engine.cu:16998-17010).  T <= B runs T batch steps (B rows per weight pass);
 * T > B runs each sequence's chunked prefill in its slot. */
int rl_hip_engine_prefill_eq_batch(RlEngine* e, const int32_t* ids, int T, int B);

/* ---- checkpoint loading ---------------------------------------------------
 * Replaces: rapidllm::make_loader + IWeightLoader::load + WeightStore::open
 * (include/rapidllm/frontend/weight_store.h:55-72, src/frontend/weight_store.cpp:
 * 125-155), the HF FP8 safetensors loader (src/frontend/hf_loader.cpp:87-251), the
 * GGUF loader (src/frontend/gguf_loader.cpp:128-397) and map_hf_name /
 * map_gguf_name (src/frontend/name_map.cpp:115-226).  Host code only (no GPU call).
 * `path` is an HF directory (config.json + *.safetensors, optionally sharded by
 * model.safetensors.index.json) or a *.gguf file; max_layers > 0 keeps layers
 * 0 .. max_layers-1.  The table holds the reference's IR names and the reference
 * WeightStore's conversions (FP8 block scales as fp32; F16/BF16 norms, A_log,
 * dt_bias, conv1d as F32; GGUF: quantised in_proj_a/b dequantised to F32, raw
 * Qwen RMSNorm scales shifted by -1, llama.cpp ssm_a = -exp(A_log) turned back into
 * A_log with cfg->v_tiled = 1).  Tensor data stays valid until rl_hip_weights_close
 * (most of it points into the mapped files); the table is what
 * rl_hip_engine_create takes.  Errors: RL_ERR_IO (missing files), RL_ERR_FORMAT
 * (bad or truncated files, FP8 weight without weight_scale_inv, quantised
 * DeltaNet leftovers), RL_ERR_UNSUPPORTED (unknown dtypes / ggml types). */
typedef struct RlWeights RlWeights;
RlWeights* rl_hip_weights_open(const char* path, int max_layers, int* status);
void rl_hip_weights_close(RlWeights* w);
/* source: 0 HF safetensors, 1 GGUF (SourceKind, weight_store.h:18) */
int rl_hip_weights_config(const RlWeights* w, RlModelConfig* cfg, int* source);
int rl_hip_weights_table(const RlWeights* w, const RlTensor** tensors, int* n);
/* Per-tensor file facts (TensorDesc::src_name / shape / ndim / gguf_type / nbytes,
 * weight_store.h:20-33) for table entry i; n_scale = number of fp32 block scales. */
int rl_hip_weights_info(const RlWeights* w, int i, const char** src_name, int* ndim, int64_t* shape4, int* gguf_type,
                        uint64_t* nbytes, int* n_scale);
/* IR name of a source tensor name (gguf = 0: HF, 1: GGUF); "" when the path does not
 * use the tensor (vision tower, unknown names). */
int rl_hip_map_name(int gguf, const char* src, char* out, int cap);

#ifdef __cplusplus
}
#endif

#endif
