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
int rl_hip_pack_act(const float* X, void* frag, int n, int T, void* stream);
/* Y[T][m] (=, or += when accumulate) W . X for T in 1..8 using a packed fragment
 * buffer.  Deterministic: partial sums are combined in a fixed order, and token t's
 * result does not depend on T. */
int rl_hip_gemm_fp8_frag(const uint8_t* w_tiled, const float* tile_scale, const void* frag, float* Y, int m, int n,
                         int T, int accumulate, void* stream);
int rl_hip_gemm_bf16_frag(const uint16_t* w_tiled, const void* frag, float* Y, int m, int n, int T, int accumulate,
                          void* stream);
/* Tuning hook: force the work split (row-tiles per workgroup, waves per workgroup
 * along K, load pipeline depth); row_tiles = 0 restores the shape-based choice. */
int rl_hip_set_gemm_config(int row_tiles, int k_waves, int depth);
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
 * the device layout.  X is fp32 [T][n], T in 1..4, n a multiple of 256.
 * rl_hip_dequant_kquant decodes row-major blocks bit-exactly like the reference. */
size_t rl_hip_kquant_tiled_bytes(int type, int m, int n);
size_t rl_hip_kquant_workspace_bytes(int m, int n, int T);
int rl_hip_pack_kquant(int type, const uint8_t* blocks, uint8_t* tiled, int m, int n, void* stream);
int rl_hip_gemm_kquant(int type, const uint8_t* tiled, const float* X, float* Y, void* workspace,
                       size_t workspace_bytes, int m, int n, int T, int accumulate, void* stream);
int rl_hip_dequant_kquant(int type, const uint8_t* blocks, float* out, size_t n_blocks, void* stream);

/* ---- bandwidth calibration ------------------------------------------------
 * No counterpart in the reference.  A streaming copy / read of `bytes` (multiple of
 * 16) that measures the achievable HBM rate and calibrates rocprof's FETCH_SIZE /
 * WRITE_SIZE counters against bytes known to be moved. */
int rl_hip_copy_probe(const void* src, void* dst, size_t bytes, void* stream);
int rl_hip_read_probe(const void* src, size_t bytes, void* out4, void* stream);

#ifdef __cplusplus
}
#endif

#endif
