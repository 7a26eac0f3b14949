/*
 * rapidllm_hip_bench.h -- benchmark, tuning and calibration entry points of the
 * MI355X decode backend.  None has a counterpart in the reference: they serve
 * bench.py and the roofline / profiler measurements, not the engine seam
 * (rapidllm_hip.h), and a RapidLLM integration does not need them.
 *
 * rl_hip_set_gemm_config changes process-wide state (the GEMM work split every
 * later launch uses); the timing functions launch back-to-back kernels on the given
 * stream.  Status codes and error reporting as in rapidllm_hip.h.
 */
#ifndef RAPIDLLM_HIP_BENCH_H
#define RAPIDLLM_HIP_BENCH_H

#include "rapidllm_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Tuning hook: force the work split (row-tiles per workgroup, waves per workgroup
 * along K, load pipeline depth); row_tiles = 0 restores the shape-based choice. */
int rl_hip_set_gemm_config(int row_tiles, int k_waves, int depth);

/* Random-init weights of cfg's architecture generated on the device (benchmark). */
RlEngine* rl_hip_engine_create_synthetic(const RlModelConfig* cfg, uint64_t seed, int ctx, int max_T, int* status);

/* Benchmark support: set the position, or fill the KV cache rows [0, n) with fp16
 * N(0,1) and the recurrent states with random values, then set pos = n; time
 * `iters` graph replays of the T-token step (mtp_drafts > 0: of the MTP draft). */
int rl_hip_engine_set_pos(RlEngine* e, int pos);
int rl_hip_engine_synthetic_context(RlEngine* e, int n, uint64_t seed);
int rl_hip_engine_time_steps(RlEngine* e, int T, int iters, int mtp_drafts, float* ms);
/* Average graph-replayed time (ms) of one layer's launches alone (layer 0 ..
 * n_layers-1) or of the step's head and tail alone (layer = n_layers: embedding,
 * first norm, lm_head, argmax, acceptance), T tokens, on whatever the layer's input
 * buffers hold; folded-norm engines only.  Where a step's time goes under graph
 * replay, which kernel traces cannot follow.  No counterpart in the reference. */
int rl_hip_engine_time_layer(RlEngine* e, int layer, int T, int iters, float* ms);

RlEngine* rl_hip_engine_create_synthetic_batch(const RlModelConfig* cfg, uint64_t seed, int ctx, int max_T,
                                               int max_batch, int* status);

/* Benchmark support: time `iters` graph replays of the B-sequence batch step (the
 * slots' positions advance; the tokens in place are re-fed). */
int rl_hip_engine_time_batch(RlEngine* e, int B, int iters, float* ms);

/* ---- bandwidth calibration ------------------------------------------------
 * No counterpart in the reference.  A streaming copy / read of `bytes` (multiple of
 * 16) that measures the achievable HBM rate and calibrates rocprof's FETCH_SIZE /
 * WRITE_SIZE counters against bytes known to be moved. */
int rl_hip_copy_probe(const void* src, void* dst, size_t bytes, void* stream);
int rl_hip_read_probe(const void* src, size_t bytes, void* out4, void* stream);

/* Rows per partial sum-of-squares group written by the add-norm epilogue (the
 * residual GEMM's rows per workgroup).  No counterpart in the reference. */
int rl_hip_norm_group_rows(void);

/* GEMM timing (no counterpart in the reference): `iters` back-to-back launches of the
 * block-FP8 GEMM on `stream`, launch i reading weight copy i % n_copies (so weights
 * come from HBM, not from the Infinity Cache), with one event pair around the loop;
 * *avg_ms = average launch duration.  epilogue: 0 store (Y [T][m]), 3 split-K
 * partials (Y [split][T][m]), 2 SwiGLU over interleaved gate/up tiles writing the
 * next linear's fragments to frag_out (act_frag_bytes(m/2, T)), 5 the same over the
 * rl_hip_pack_fp8_gate_up half tiles (tile scales [m/16][kb][2]), 4 residual add with
 * the next RMSNorm's data (Y [T][m] += result; frag_out = fragments of Y * (1 + gamma),
 * act_frag_bytes(m, T); sumsq [ceil(m/G)][T] = sums of squares per G rows,
 * G = rl_hip_norm_group_rows()).
 * block_sumsq (add-norm only, may be null): [n/128][T][4] partial sums of squares of
 * the input per 128-column block, each block's products then scaled per token by
 * 1/sqrt(sum/128 + 1e-6) (the DeltaNet out_proj's folded gated RMSNorm).
 * sumsq_in (store / SwiGLU only, may be null): the input's sums of squares as an
 * add-norm launch writes them for an n-row output ([ceil(n/G)][T]); the products
 * are then scaled per token by 1/sqrt(sum/n + 1e-6) (the folded RMSNorm of the
 * GEMMs that read the residual stream). */
int rl_hip_time_gemm_fp8(const void* const* w_copies, int n_copies, const float* tile_scales, const void* frag,
                         float* Y, void* frag_out, const float* gamma, float* sumsq, const float* block_sumsq,
                         const float* sumsq_in, int m, int n, int T, int epilogue, int split, int iters,
                         void* stream, float* avg_ms);

/* T=1 block-FP8 GEMV on the VALU (e4m3 -> fp32 conversion, FMA, shuffle sums) over
 * the rl_hip_pack_fp8 layout, for comparison with the matrix-core GEMM: Y [m] =
 * W . X (X fp32 [n], n a multiple of 128, at most 16384); `iters` launches cycling
 * over n_copies weight copies, *avg_ms their average duration.  No counterpart in
 * the reference (measurement only; the engine never calls it). */
int rl_hip_time_gemv_fp8_valu(const void* const* w_copies, int n_copies, const float* tile_scales, const float* X,
                              float* Y, int m, int n, int iters, void* stream, float* avg_ms);

/* Average duration of `iters` back-to-back rl_hip_gemm_kquant launches (store),
 * cycling over n_copies packed weight copies.  No counterpart in the reference
 * (bench / roofline measurement). */
int rl_hip_time_gemm_kquant(int type, const void* const* w_copies, int n_copies, const float* X, float* Y,
                            void* workspace, size_t workspace_bytes, int m, int n, int T, int iters, void* stream,
                            float* avg_ms);

/* Average duration of one DeltaNet decode launch (rl_hip_gdn_decode semantics with
 * S updated in place) over `iters` passes across n_layers layer states.  No
 * counterpart in the reference (bench / roofline measurement). */
int rl_hip_time_gdn(float* const* S_layers, int n_layers, const float* qkv, const float* a, const float* b, int ld_in,
                    const float* A_log, const float* dt_bias, const float* conv_w, const float* conv_in,
                    float* conv_out, float* o, int T, int nk, int nv, int dk, int dv, int conv_k, int v_tiled,
                    int iters, void* stream, float* avg_ms);

#ifdef __cplusplus
}
#endif

#endif
