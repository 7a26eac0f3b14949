// ref_shim.cpp -- TEST INFRASTRUCTURE ONLY.
//
// extern "C" entry points over the reference's own CPU kernels, so that tests can
// check the oracle restatement (oracle.cpp) against the real thing.  Compiled by
// oracle/Makefile together with the reference sources where they lie under
// /root/reference/src; the result goes to oracle/_ref/libref.so (never committed).
#include "rapidllm/kernels/ops.h"
#include "rapidllm/runtime/thread_pool.h"

#include <cstdint>

namespace rapidllm {
int32_t greedy_sample(const float* logits, int vocab);  // src/runtime/sampler.cpp:8
}

using namespace rapidllm;

extern "C" {
float ref_e4m3_to_f32(uint8_t b) { return ops::e4m3_to_f32(b); }
float ref_fp16_to_f32(uint16_t h) { return ops::fp16_to_f32(h); }
void ref_gemv_fp8(const uint8_t* W, const float* s, const float* x, float* y, int m, int n) {
    ops::gemv_fp8(W, s, x, y, m, n, 128);
}
void ref_dequant_q4_k(const uint8_t* p, float* out, int n) { ops::dequant_q4_k(p, out, n); }
void ref_dequant_q6_k(const uint8_t* p, float* out, int n) { ops::dequant_q6_k(p, out, n); }
void ref_gemv_q4_k(const uint8_t* p, const float* x, float* y, int m, int n) { ops::gemv_q4_k(p, x, y, m, n); }
void ref_gemv_q6_k(const uint8_t* p, const float* x, float* y, int m, int n) { ops::gemv_q6_k(p, x, y, m, n); }
void ref_gemv_bf16(const uint16_t* W, const float* x, float* y, int m, int n) { ops::gemv_bf16(W, x, y, m, n); }
void ref_qwen3_rmsnorm(const float* x, const float* g, float* y, int n, float eps) {
    ops::qwen3_rmsnorm(x, g, y, n, eps);
}
void ref_gated_rmsnorm(const float* x, const float* z, const float* g, float* y, int n, float eps, int gn) {
    ops::gated_rmsnorm(x, z, g, y, n, eps, gn);
}
void ref_l2norm(const float* x, float* y, int n, float eps) { ops::l2norm(x, y, n, eps); }
void ref_conv1d_update(const float* x, const float* w, float* st, float* y, int dim, int k) {
    ops::conv1d_update(x, w, st, y, dim, k);
}
void ref_delta_step_scalar(float* S, const float* q, const float* k, const float* v, const float* beta,
                           const float* gl, float* o, int nv, int dk, int dv, float eps) {
    ops::delta_recurrent_step_scalar(S, q, k, v, beta, gl, o, nv, dk, dv, eps);
}
void ref_delta_step_simd(float* S, const float* q, const float* k, const float* v, const float* beta,
                         const float* gl, float* o, int nv, int dk, int dv, float eps) {
    ops::delta_recurrent_step_simd(S, q, k, v, beta, gl, o, nv, dk, dv, eps);
}
void ref_rope_partial(float* q, float* k, int nq, int nkv, int hd, int rot, int pos, float theta) {
    ops::rope_partial(q, k, nq, nkv, hd, rot, pos, theta);
}
void ref_attn_decode(const float* q, const float* kc, const float* vc, float* o, int pos, int nq, int nkv, int hd) {
    ops::attn_decode(q, kc, vc, o, pos, nq, nkv, hd);
}
void ref_swiglu(const float* g, const float* u, float* y, int n) { ops::swiglu(g, u, y, n); }
int ref_greedy(const float* l, int v) { return greedy_sample(l, v); }
int ref_num_threads() { return num_threads(); }
const char* ref_simd_name() { return ops::simd_isa_name(); }

// One-token fused layers at full shape (ops_fused.cpp), for the CPU baseline timing.
void ref_fused_mlp(const float* rms_w, const uint8_t* wg, const float* sg, const uint8_t* wu, const float* su,
                   const uint8_t* wd, const float* sd, float* x, int hidden, int inter, float eps) {
    ops::FusedMlpArgs a{};
    a.x = x;
    a.x_inout = x;
    a.rms_w = rms_w;
    a.Wg = {wg, sg, QuantKind::FP8_E4M3_B128};
    a.Wu = {wu, su, QuantKind::FP8_E4M3_B128};
    a.Wd = {wd, sd, QuantKind::FP8_E4M3_B128};
    a.hidden = hidden;
    a.intermediate = inter;
    a.eps = eps;
    a.use_simd = true;
    ops::fused_mlp_decode(a);
}

// ops::fused_delta_decode (ops_fused.cpp:84-135) with block-FP8 projections (qkv, z,
// a, b, out): x += the DeltaNet layer's output; S and the conv window advance.
void ref_fused_delta(const float* rms_w, const uint8_t* wqkv, const float* sqkv, const uint8_t* wz, const float* sz,
                     const uint8_t* wa, const float* sa, const uint8_t* wb, const float* sb, const uint8_t* wo,
                     const float* so, const float* A_log, const float* dt_bias, const float* conv_w,
                     const float* gnorm, float* S, float* conv_state, float* x, int hidden, int nk, int nv, int dk,
                     int dv, int conv_k, int gnorm_n, float eps) {
    ops::FusedDeltaArgs a{};
    a.x = x;
    a.x_inout = x;
    a.rms_w = rms_w;
    a.Wqkv = {wqkv, sqkv, QuantKind::FP8_E4M3_B128};
    a.Wz = {wz, sz, QuantKind::FP8_E4M3_B128};
    a.Wa = {wa, sa, QuantKind::FP8_E4M3_B128};
    a.Wb = {wb, sb, QuantKind::FP8_E4M3_B128};
    a.Wo = {wo, so, QuantKind::FP8_E4M3_B128};
    a.A_log = A_log;
    a.dt_bias = dt_bias;
    a.conv_w = conv_w;
    a.gnorm = gnorm;
    a.S = S;
    a.conv_state = conv_state;
    a.hidden = hidden;
    a.nk = nk;
    a.nv = nv;
    a.dk = dk;
    a.dv = dv;
    a.conv_k = conv_k;
    a.gnorm_n = gnorm_n;
    a.eps = eps;
    a.use_simd = true;
    ops::fused_delta_decode(a);
}

// ops::fused_attn_decode (ops_fused.cpp:137-184) with block-FP8 projections: x += the
// gated attention output at position pos, K / V appended to the fp32 caches.
void ref_fused_attn(const float* rms_w, const uint8_t* wq, const float* sq, const uint8_t* wk, const float* sk,
                    const uint8_t* wv, const float* sv, const uint8_t* wo, const float* so, const float* q_norm,
                    const float* k_norm, float* k_cache, float* v_cache, float* x, int hidden, int n_q, int n_kv,
                    int head_dim, int rotary_dim, int pos, float theta, float eps) {
    ops::FusedAttnArgs a{};
    a.x = x;
    a.x_inout = x;
    a.rms_w = rms_w;
    a.Wq = {wq, sq, QuantKind::FP8_E4M3_B128};
    a.Wk = {wk, sk, QuantKind::FP8_E4M3_B128};
    a.Wv = {wv, sv, QuantKind::FP8_E4M3_B128};
    a.Wo = {wo, so, QuantKind::FP8_E4M3_B128};
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.hidden = hidden;
    a.n_q = n_q;
    a.n_kv = n_kv;
    a.head_dim = head_dim;
    a.rotary_dim = rotary_dim;
    a.pos = pos;
    a.theta = theta;
    a.eps = eps;
    a.use_simd = true;
    ops::fused_attn_decode(a);
}
}

// ---- the reference's checkpoint loaders (src/frontend/*.cpp), for cross-checking
// the loader of the HIP library on the same files.
#include "rapidllm/backend/device.h"
#include "rapidllm/frontend/weight_store.h"

#include <cstring>
#include <string>
#include <vector>

namespace {
// WeightStore::open takes a Device it does not use (weight_store.cpp:137); a device
// with no capabilities satisfies the signature.
class NoDevice final : public rapidllm::Device {
public:
    rapidllm::DeviceKind kind() const override { return rapidllm::DeviceKind::CPU; }
    const char* name() const override { return "none"; }
    std::unique_ptr<rapidllm::Buffer> allocate(const rapidllm::BufferDesc&) override { return nullptr; }
    std::unique_ptr<rapidllm::Stream> create_stream() override { return nullptr; }
    void memcpy(rapidllm::TensorView, rapidllm::TensorView, rapidllm::Stream&) override {}
    void launch(const char*, const rapidllm::TensorView*, int, const void*, size_t, rapidllm::Stream&) override {}
    bool has_kernel(const char*) const override { return false; }
};

struct RefWeights {
    rapidllm::WeightStore ws;
    std::vector<const rapidllm::TensorDesc*> v;
};
}  // namespace

extern "C" {
void* ref_weights_open(const char* path, char* err, int cap) {
    try {
        NoDevice dev;
        rapidllm::LoadOptions opt;
        auto* r = new RefWeights{rapidllm::WeightStore::open(path, dev, opt), {}};
        for (auto& [_, t] : r->ws.table().tensors) r->v.push_back(&t);
        return r;
    } catch (const std::exception& e) {
        std::snprintf(err, cap, "%s", e.what());
        return nullptr;
    }
}
void ref_weights_close(void* h) { delete static_cast<RefWeights*>(h); }
int ref_weights_count(void* h) { return static_cast<int>(static_cast<RefWeights*>(h)->v.size()); }
const char* ref_weights_name(void* h, int i) { return static_cast<RefWeights*>(h)->v[i]->ir_name.c_str(); }
const char* ref_weights_src(void* h, int i) { return static_cast<RefWeights*>(h)->v[i]->src_name.c_str(); }
int ref_weights_quant(void* h, int i) { return static_cast<int>(static_cast<RefWeights*>(h)->v[i]->quant); }
int ref_weights_shape(void* h, int i, int64_t* shape4) {
    const auto* t = static_cast<RefWeights*>(h)->v[i];
    for (int d = 0; d < 4; ++d) shape4[d] = t->shape[d];
    return t->ndim;
}
uint64_t ref_weights_nbytes(void* h, int i) { return static_cast<RefWeights*>(h)->v[i]->data.size(); }
const uint8_t* ref_weights_data(void* h, int i) { return static_cast<RefWeights*>(h)->v[i]->data.data(); }
int ref_weights_nscale(void* h, int i) { return static_cast<int>(static_cast<RefWeights*>(h)->v[i]->scale.size()); }
const float* ref_weights_scale(void* h, int i) { return static_cast<RefWeights*>(h)->v[i]->scale.data(); }
// n_layers, hidden, vocab, intermediate, gdn_v_tiled, has_mtp, source, tie_embed
void ref_weights_model(void* h, int* out8, unsigned char* kinds) {
    const auto& t = static_cast<RefWeights*>(h)->ws.table();
    const auto& m = t.model;
    out8[0] = m.n_layers;
    out8[1] = m.hidden;
    out8[2] = m.vocab;
    out8[3] = m.intermediate;
    out8[4] = m.gdn_v_tiled ? 1 : 0;
    out8[5] = m.has_mtp ? 1 : 0;
    out8[6] = t.source == rapidllm::SourceKind::GgufFile ? 1 : 0;
    out8[7] = m.tie_embed ? 1 : 0;
    for (int i = 0; i < m.n_layers; ++i) kinds[i] = static_cast<unsigned char>(m.layers[i].kind);
}
int ref_map_name(int gguf, const char* src, char* out, int cap) {
    const std::string s = gguf ? rapidllm::map_gguf_name(src) : rapidllm::map_hf_name(src);
    std::snprintf(out, cap, "%s", s.c_str());
    return static_cast<int>(s.size());
}
}
