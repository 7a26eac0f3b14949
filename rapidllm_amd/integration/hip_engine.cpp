// hip_engine.cpp -- cuda_gen::Engine (include/rapidllm/runtime/cuda_engine.h:13-83)
// implemented over the HIP backend's C ABI (include/rapidllm_hip.h).
//
// The Session (src/runtime/session.cpp:25, 487-501, 695-798) drives the GPU only
// through this interface, so a HIP build creates this engine where the reference
// creates its CUDA one.  The weight table's IR names, quant kinds and the
// ModelDesc fields pass through unchanged; data is copied to the device during
// construction (the host TensorDesc bytes may be freed afterwards, as
// cuda_engine.cu:20485-20493 does).
#include "hip_backend.h"

#include "rapidllm_hip.h"

#include <algorithm>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <vector>

namespace rapidllm::hip_gen {
namespace {

void check(int st) {
    if (st != RL_OK) throw std::runtime_error(std::string("hip backend: ") + rl_hip_last_error());
}

// RlQuant uses QuantKind's numbering (model_desc.h:14-25); checked here so that a
// reordering on either side fails the build instead of mislabelling weights.
static_assert(static_cast<int>(QuantKind::F32) == RL_Q_F32, "QuantKind::F32");
static_assert(static_cast<int>(QuantKind::F16) == RL_Q_F16, "QuantKind::F16");
static_assert(static_cast<int>(QuantKind::BF16) == RL_Q_BF16, "QuantKind::BF16");
static_assert(static_cast<int>(QuantKind::FP8_E4M3_B128) == RL_Q_FP8_E4M3_B128, "QuantKind::FP8_E4M3_B128");
static_assert(static_cast<int>(QuantKind::PackedInt4) == RL_Q_PACKED_INT4, "QuantKind::PackedInt4");
static_assert(static_cast<int>(QuantKind::Q8_0) == RL_Q_Q8_0, "QuantKind::Q8_0");
static_assert(static_cast<int>(QuantKind::Q4_K) == RL_Q_Q4_K, "QuantKind::Q4_K");
static_assert(static_cast<int>(QuantKind::Q5_K) == RL_Q_Q5_K, "QuantKind::Q5_K");
static_assert(static_cast<int>(QuantKind::Q6_K) == RL_Q_Q6_K, "QuantKind::Q6_K");
int quant_of(QuantKind q) { return static_cast<int>(q); }

RlModelConfig config_of(const ModelDesc& md) {
    RlModelConfig c{};
    c.vocab = md.vocab;
    c.hidden = md.hidden;
    c.n_layers = md.n_layers;
    c.intermediate = md.intermediate;
    c.rms_eps = md.rms_eps;
    c.rope_theta = md.rope.theta;
    c.v_tiled = md.gdn_v_tiled ? 1 : 0;
    c.has_mtp = md.has_mtp ? 1 : 0;
    if (md.n_layers < 1 || md.n_layers > RL_MAX_LAYERS || static_cast<int>(md.layers.size()) < md.n_layers)
        throw std::runtime_error("hip backend: bad layer count");
    const LayerDesc* d = nullptr;
    const LayerDesc* a = nullptr;
    for (int i = 0; i < md.n_layers; ++i) {
        const LayerKind k = md.kind_of(i);
        if (k == LayerKind::DenseAttn) throw std::runtime_error("hip backend: dense attention layers are not supported");
        const bool attn = k == LayerKind::GatedAttn;
        c.layer_kind[i] = attn ? RL_LAYER_ATTN : RL_LAYER_DELTA;
        (attn ? a : d) = &md.layers[static_cast<size_t>(i)];
    }
    const DeltaNetDesc dn = d ? d->delta : DeltaNetDesc{};
    const GatedAttnDesc at = a ? a->attn : GatedAttnDesc{};
    c.n_k_heads = dn.n_k_heads;
    c.n_v_heads = dn.n_v_heads;
    c.k_dim = dn.k_dim;
    c.v_dim = dn.v_dim;
    c.conv_k = dn.conv_k;
    c.n_q = at.n_q;
    c.n_kv = at.n_kv;
    c.head_dim = at.head_dim;
    // partial rotary: the first head_dim * partial_factor dims (Session's rope_partial)
    c.rotary_dim = static_cast<int>(static_cast<float>(at.head_dim) * md.rope.partial_factor);
    return c;
}

class HipEngine final : public cuda_gen::Engine {
public:
    HipEngine(const TensorTable& table, int ctx, int max_batch) {
        const RlModelConfig c = config_of(table.model);
        std::vector<RlTensor> t;
        t.reserve(table.tensors.size());
        for (const auto& [name, td] : table.tensors) {
            if (td.skipped || td.data.empty()) continue;
            RlTensor r{};
            r.name = name.c_str();
            r.quant = quant_of(td.quant);
            // row-major shape: the last dim is the row length (GGUF shapes are
            // reversed to this order by the loader, gguf_loader.cpp:187-189)
            int64_t numel = 1;
            for (int k = 0; k < td.ndim && k < 4; ++k) numel *= td.shape[k];
            r.cols = td.ndim >= 2 ? td.shape[td.ndim - 1] : 1;
            r.rows = td.ndim >= 2 ? numel / r.cols : numel;
            r.data = td.data.data();
            r.scale = td.scale.empty() ? nullptr : td.scale.data();
            t.push_back(r);
        }
        int st = RL_OK;
        e_ = rl_hip_engine_create_batch(&c, t.data(), static_cast<int>(t.size()), ctx, /*max_T=*/4,
                                        std::max(1, max_batch), &st);
        check(st);
        size_t bytes = 0;
        int cap = 0;
        check(rl_hip_engine_info(e_, &vocab_, &hidden_, &cap, &bytes));
        // RAPIDLLM_HIP_MTP_LAYER=1: draft through the MTP decoder layer
        // (mtp.layers[0], Session::mtp_layer_step) when the weights have it; the
        // default is the stem, as Session::mtp_draft's CPU branch
        const char* ml = std::getenv("RAPIDLLM_HIP_MTP_LAYER");
        int mode = RL_MTP_STEM, have_layer = 0;
        check(rl_hip_engine_mtp_mode(e_, &mode, &have_layer));
        if (ml && ml[0] == '1' && have_layer) check(rl_hip_engine_set_mtp_mode(e_, RL_MTP_LAYER));
    }
    ~HipEngine() override { rl_hip_engine_destroy(e_); }

    void prefill(const int32_t* ids, int n) override { check(rl_hip_engine_prefill(e_, ids, n)); }
    void decode_token(int32_t tok) override { check(rl_hip_engine_decode_token(e_, tok)); }
    void decode_steps(int n) override { check(rl_hip_engine_decode_steps(e_, n)); }
    void copy_gen_tokens(int32_t* h, int n) override { check(rl_hip_engine_copy_gen_tokens(e_, h, n)); }
    void copy_logits(float* h) const override { check(rl_hip_engine_copy_logits(e_, h)); }
    void copy_last_hidden(float* h) override { check(rl_hip_engine_copy_last_hidden(e_, h)); }
    int mtp_draft(int32_t first, int n, int32_t* out) override {
        int k = 0;
        check(rl_hip_engine_mtp_draft(e_, first, n, out, &k));
        return k;
    }
    // Session::generate reads the accepted drafts from pm[1 .. k-1] with pm[0] = t0
    // (session.cpp:736-745): the fed tokens [t0, d0, ...], not the predictions; the
    // bonus token is greedy() afterwards.
    int mtp_spec2(int32_t t0, int32_t* pm) override { return spec(t0, 2, pm); }
    int mtp_spec4(int32_t t0, int32_t* pm) override { return spec(t0, 4, pm); }
    int spec_verify(const int32_t* toks, int T, int32_t* preds) override {
        int n = 0;
        check(rl_hip_engine_spec_verify(e_, toks, T, preds, &n));
        return n;
    }
    int spec_verify_t0(int32_t t0, int32_t* preds) override {
        const int32_t toks[2] = {t0, greedy()};
        return spec_verify(toks, 2, preds);
    }
    int32_t greedy() const override {
        int32_t t = 0;
        check(rl_hip_engine_greedy(e_, &t));
        return t;
    }
    int pos() const override {
        int p = 0;
        check(rl_hip_engine_pos(e_, &p));
        return p;
    }
    int vocab() const override { return vocab_; }
    int hidden() const override { return hidden_; }
    // continuous batch (cuda_engine.h:46-66)
    int max_batch() const override {
        int b = 1;
        check(rl_hip_engine_max_batch(e_, &b));
        return b;
    }
    void decode_tokens(const int32_t* toks, const int* poss, int B) override {
        check(rl_hip_engine_decode_tokens(e_, toks, poss, B));
    }
    void copy_logits_n(float* h, int B) const override { check(rl_hip_engine_copy_logits_n(e_, h, B)); }
    void copy_greedy_n(int32_t* h, int B) override { check(rl_hip_engine_copy_greedy_n(e_, h, B)); }
    void replicate_slot0(int n) override { check(rl_hip_engine_replicate_slot0(e_, n)); }
    void zero_slots(int n) override { check(rl_hip_engine_zero_slots(e_, n)); }
    void prefill_slot(const int32_t* ids, int n, int slot) override {
        check(rl_hip_engine_prefill_slot(e_, ids, n, slot));
    }
    bool prefill_eq_batch(const int32_t* ids, int T, int B) override {
        if (!ids || T <= 0 || B <= 1 || B > max_batch()) return false;
        check(rl_hip_engine_prefill_eq_batch(e_, ids, T, B));
        return true;
    }

private:
    int spec(int32_t t0, int T, int32_t* pm) {
        int32_t preds[4] = {};
        int n = 0;
        check(rl_hip_engine_mtp_spec(e_, t0, T, pm, preds, &n));
        return n;
    }
    RlEngine* e_ = nullptr;
    int vocab_ = 0, hidden_ = 0;
};

}  // namespace

bool available() { return rl_hip_available() == 1; }

std::unique_ptr<cuda_gen::Engine> create_from_table(const TensorTable& table, int ctx, int max_batch) {
    return std::make_unique<HipEngine>(table, ctx, max_batch);
}

std::unique_ptr<cuda_gen::Engine> create(WeightStore& store, int ctx) {
    // slots for decode_tokens: RAPIDLLM_MAX_BATCH, as the reference engine reads it
    // (cuda_engine.cu:20057-20062)
    const char* mb = std::getenv("RAPIDLLM_MAX_BATCH");
    const int max_batch = mb ? std::max(1, std::min(16, std::atoi(mb))) : 1;
    return create_from_table(store.table(), ctx, max_batch);
}

}  // namespace rapidllm::hip_gen
