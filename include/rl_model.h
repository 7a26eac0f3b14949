/*
 * rl_model.h -- plain-C description of a Qwen3.6/3.8-27B-style hybrid decoder and
 * of the weight table that feeds it.  Shared by the HIP engine (rapidllm_hip.h)
 * and by the CPU oracle under oracle/, so that both consume byte-identical weights.
 *
 * Mirrors, in C, the pieces of the reference that describe a model to its engine:
 *   - QuantKind ordering            include/rapidllm/ir/model_desc.h:14-25
 *   - ModelDesc / DeltaNetDesc /
 *     GatedAttnDesc defaults        include/rapidllm/ir/model_desc.h:55-147
 *   - TensorDesc {data, scale, quant}
 *     as held by the WeightStore    include/rapidllm/frontend/weight_store.h:20-72
 * Tensor names are the reference's IR names (src/runtime/session.cpp:144-160,
 * 183-196, 271-279, 633-638): "embed", "lm_head", "final_norm",
 * "layers[i].attn_norm", "layers[i].delta.gemm.in_proj_qkv", ... , "mtp.fc".
 */
#ifndef RL_MODEL_H
#define RL_MODEL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same order as rapidllm::QuantKind (model_desc.h:14-25). */
typedef enum RlQuant {
    RL_Q_F32 = 0,
    RL_Q_F16 = 1,
    RL_Q_BF16 = 2,
    RL_Q_FP8_E4M3_B128 = 3,
    RL_Q_PACKED_INT4 = 4,
    RL_Q_Q8_0 = 5,
    RL_Q_Q4_K = 6,
    RL_Q_Q5_K = 7,
    RL_Q_Q6_K = 8
} RlQuant;

/* Layer mixer kinds (rapidllm::LayerKind, model_desc.h:11). */
enum { RL_LAYER_DELTA = 0, RL_LAYER_ATTN = 1 };

#define RL_MAX_LAYERS 256

typedef struct RlModelConfig {
    int vocab, hidden, n_layers, intermediate;
    /* Gated DeltaNet (DeltaNetDesc) */
    int n_k_heads, n_v_heads, k_dim, v_dim, conv_k;
    /* Gated attention (GatedAttnDesc) */
    int n_q, n_kv, head_dim, rotary_dim;
    float rope_theta;
    float rms_eps;
    int v_tiled;  /* ModelDesc::gdn_v_tiled: src head = h % nk instead of h / (nv/nk) */
    int has_mtp;  /* mtp.fc / mtp.norm / mtp.pre_fc_norm_{hidden,embedding} present */
    unsigned char layer_kind[RL_MAX_LAYERS];
} RlModelConfig;

/*
 * One weight.  2-D tensors are [rows][cols] row-major in the on-disk block format
 * named by `quant` (FP8: e4m3fn bytes + fp32 scale [ceil(rows/128)][ceil(cols/128)];
 * Q4_K: 144-byte super-blocks; Q6_K: 210-byte super-blocks; BF16/F16: 2-byte words).
 * 1-D tensors (norm weights, A_log, dt_bias) use rows = n, cols = 1, quant F32.
 * conv1d weight is [conv_dim][conv_k] F32.
 */
typedef struct RlTensor {
    const char* name;
    int quant;
    int64_t rows, cols;
    const void* data;
    const float* scale; /* FP8 block scales, NULL otherwise */
} RlTensor;

#ifdef __cplusplus
}
#endif

#endif
