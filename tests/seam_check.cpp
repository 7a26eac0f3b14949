// seam_check.cpp -- GPU check of the reference-side adapters
// (rapidllm_amd/integration: hip_gen::HipEngine for cuda_gen::Engine,
// include/rapidllm/runtime/cuda_engine.h:13-83, and hip_gen::HipDevice for
// rapidllm::Device, include/rapidllm/backend/device.h:49-60), compiled against the
// reference's own headers and driven the way the reference drives them.
//
//  1. A small hybrid model (D D D A, head_dim 256, MTP head) described as the
//     reference describes it -- a ModelDesc and a TensorTable of TensorDescs with
//     IR names, shapes and QuantKinds -- is created through HipEngine and, from
//     an explicitly written RlModelConfig / RlTensor table, directly through the C
//     ABI: both give bit-identical logits, and both match the oracle model (the
//     reference CPU Session's decode, 1e-3 relative L2).
//  2. Session::generate's MTP loop (src/runtime/session.cpp:728-747: mtp_spec2,
//     accepted drafts read from pm[1 .. k-1]) through HipEngine produces the plain
//     greedy tokens (the greedy invariant of tests/test_spec.cpp:46-79).
//  3. Every HipDevice kernel name, launched with the reference's parameter structs
//     (params.h:5-22) on buffers from Device::allocate, matches the oracle's op.
// Test infrastructure: links the oracle (oracle/_build/liboracle.so) as the checker.
#include "../rapidllm_amd/integration/hip_backend.h"

#include "rapidllm/backend/params.h"
#include "rapidllm_hip.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

extern "C" {
float orc_e4m3_to_f32(uint8_t b);
void orc_gemv_fp8(const uint8_t* W, const float* scale, const float* x, float* y, int m, int n, int block);
void orc_gemv_q4_k(const uint8_t* packed, const float* x, float* y, int m, int n, int nthreads);
void orc_gemv_q6_k(const uint8_t* packed, const float* x, float* y, int m, int n, int nthreads);
void orc_qwen3_rmsnorm(const float* x, const float* gamma, float* y, int n, float eps);
void orc_gated_rmsnorm(const float* x, const float* z, const float* gamma, float* y, int n, float eps, int gamma_n);
void orc_conv1d_update(const float* x_t, const float* w, float* state, float* y, int dim, int k);
void orc_delta_step(float* S, const float* q, const float* k, const float* v, const float* beta, const float* g_log,
                    float* o, int nv, int dk, int dv, float eps);
void orc_attn_decode(const float* q, const float* kc, const float* vc, float* o, int pos, int n_q, int n_kv, int hd);
void* orc_model_create(const RlModelConfig* cfg, const RlTensor* t, int n, int ctx, int kv_fp16, int nthreads);
int orc_model_decode(void* h, int token, float* logits, float* hidden);
void orc_model_free(void* h);
}

using namespace rapidllm;

namespace {

int g_fail = 0;
void expect(bool ok, const std::string& what) {
    std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
    if (!ok) ++g_fail;
}

double rel_l2(const float* a, const float* b, size_t n) {
    double num = 0, den = 0;
    for (size_t i = 0; i < n; ++i) {
        num += (static_cast<double>(a[i]) - b[i]) * (static_cast<double>(a[i]) - b[i]);
        den += static_cast<double>(b[i]) * b[i];
    }
    return std::sqrt(num / (den > 0 ? den : 1e-300));
}

struct Rng {
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    float uni() { return static_cast<float>((next() >> 40) + 0.5) / 16777216.f; }
    float normal() {
        const float u = uni(), v = uni();
        return std::sqrt(-2.f * std::log(u)) * std::cos(6.2831853f * v);
    }
    uint8_t fp8() {
        for (;;) {
            const uint8_t b = static_cast<uint8_t>(next());
            if ((b & 0x7F) != 0x7F) return b;
        }
    }
};

// ---------------------------------------------------------------- the model
constexpr int V = 1000, H = 256, I = 512, NK = 2, NV = 4, DK = 128, DV = 128, NQ = 4, NKV = 2, HD = 256;
constexpr int CONV = 2 * NK * DK + NV * DV;
const int kKinds[4] = {0, 0, 0, 1};

ModelDesc model_desc() {
    ModelDesc md;
    md.vocab = V;
    md.hidden = H;
    md.n_layers = 4;
    md.intermediate = I;
    md.rms_eps = 1e-6f;
    md.rope.theta = 1e7f;
    md.rope.partial_factor = 0.25f;
    md.has_mtp = true;
    md.layers.resize(4);
    for (int i = 0; i < 4; ++i) {
        LayerDesc& L = md.layers[static_cast<size_t>(i)];
        L.kind = kKinds[i] ? LayerKind::GatedAttn : LayerKind::GatedDeltaNet;
        L.delta.n_k_heads = NK;
        L.delta.n_v_heads = NV;
        L.delta.k_dim = DK;
        L.delta.v_dim = DV;
        L.delta.conv_k = 4;
        L.attn.n_q = NQ;
        L.attn.n_kv = NKV;
        L.attn.head_dim = HD;
    }
    return md;
}

void add(TensorTable& t, const std::string& name, QuantKind q, int64_t r, int64_t c, std::vector<uint8_t> data,
         std::vector<float> scale = {}) {
    TensorDesc d;
    d.ir_name = name;
    d.quant = q;
    d.ndim = c > 1 ? 2 : 1;
    d.shape[0] = r;
    if (c > 1) d.shape[1] = c;
    d.nbytes = data.size();
    d.data = std::move(data);
    d.scale = std::move(scale);
    t.tensors.emplace(name, std::move(d));
}

std::vector<uint8_t> f32_bytes(const std::vector<float>& v) {
    std::vector<uint8_t> b(v.size() * 4);
    std::memcpy(b.data(), v.data(), b.size());
    return b;
}

void add_vec(TensorTable& t, Rng& r, const std::string& name, int n, float mean, float sd, int cols = 1) {
    std::vector<float> v(static_cast<size_t>(n) * cols);
    for (float& x : v) x = mean + sd * r.normal();
    add(t, name, QuantKind::F32, n, cols, f32_bytes(v));
}

void add_fp8(TensorTable& t, Rng& r, const std::string& name, int m, int n) {
    std::vector<uint8_t> w(static_cast<size_t>(m) * n);
    for (auto& b : w) b = r.fp8();
    std::vector<float> s(static_cast<size_t>((m + 127) / 128) * ((n + 127) / 128));
    for (float& x : s) x = std::exp(std::log(1e-3f) + r.uni() * std::log(10.f));
    add(t, name, QuantKind::FP8_E4M3_B128, m, n, std::move(w), std::move(s));
}

void add_bf16(TensorTable& t, Rng& r, const std::string& name, int m, int n) {
    std::vector<uint8_t> w(static_cast<size_t>(m) * n * 2);
    for (size_t i = 0; i < w.size() / 2; ++i) {
        float x = 0.02f * r.normal();
        uint32_t u;
        std::memcpy(&u, &x, 4);
        const uint16_t h = static_cast<uint16_t>((u + 0x7FFF + ((u >> 16) & 1)) >> 16);
        std::memcpy(&w[2 * i], &h, 2);
    }
    add(t, name, QuantKind::BF16, m, n, std::move(w));
}

TensorTable make_table() {
    TensorTable t;
    t.model = model_desc();
    Rng r{42};
    add_bf16(t, r, "embed", V, H);
    add_bf16(t, r, "lm_head", V, H);
    add_vec(t, r, "final_norm", H, 0.f, 0.1f);
    for (int i = 0; i < 4; ++i) {
        const std::string p = "layers[" + std::to_string(i) + "].";
        add_vec(t, r, p + "attn_norm", H, 0.f, 0.1f);
        add_vec(t, r, p + "ffn_norm", H, 0.f, 0.1f);
        if (!kKinds[i]) {
            add_fp8(t, r, p + "delta.gemm.in_proj_qkv", CONV, H);
            add_fp8(t, r, p + "delta.gemm.in_proj_z", NV * DV, H);
            add_fp8(t, r, p + "delta.leftover.in_proj_a", NV, H);
            add_fp8(t, r, p + "delta.leftover.in_proj_b", NV, H);
            add_fp8(t, r, p + "delta.gemm.out_proj", H, NV * DV);
            add_vec(t, r, p + "delta.leftover.a_log", NV, 0.f, 0.5f);
            add_vec(t, r, p + "delta.leftover.dt_bias", NV, 0.f, 0.5f);
            add_vec(t, r, p + "delta.leftover.conv1d", CONV, 0.f, 0.5f, 4);
            add_vec(t, r, p + "delta.leftover.norm", DV, 1.f, 0.1f);
        } else {
            add_fp8(t, r, p + "attn.wq", 2 * NQ * HD, H);
            add_fp8(t, r, p + "attn.wk", NKV * HD, H);
            add_fp8(t, r, p + "attn.wv", NKV * HD, H);
            add_fp8(t, r, p + "attn.wo", H, NQ * HD);
            add_vec(t, r, p + "attn.q_norm", HD, 0.f, 0.1f);
            add_vec(t, r, p + "attn.k_norm", HD, 0.f, 0.1f);
        }
        add_fp8(t, r, p + "mlp.gate", I, H);
        add_fp8(t, r, p + "mlp.up", I, H);
        add_fp8(t, r, p + "mlp.down", H, I);
    }
    add_fp8(t, r, "mtp.fc", H, 2 * H);
    add_vec(t, r, "mtp.pre_fc_norm_hidden", H, 0.f, 0.1f);
    add_vec(t, r, "mtp.pre_fc_norm_embedding", H, 0.f, 0.1f);
    add_vec(t, r, "mtp.norm", H, 0.f, 0.1f);
    return t;
}

// The same model written out by hand for the C ABI (explicit rows / cols and an
// explicit rotary dimension: what the adapter must derive).
struct Direct {
    RlModelConfig cfg{};
    std::vector<RlTensor> ts;
};
Direct direct_of(const TensorTable& t) {
    Direct d;
    RlModelConfig& c = d.cfg;
    c.vocab = V, c.hidden = H, c.n_layers = 4, c.intermediate = I;
    c.n_k_heads = NK, c.n_v_heads = NV, c.k_dim = DK, c.v_dim = DV, c.conv_k = 4;
    c.n_q = NQ, c.n_kv = NKV, c.head_dim = HD, c.rotary_dim = 64;
    c.rope_theta = 1e7f, c.rms_eps = 1e-6f, c.v_tiled = 0, c.has_mtp = 1;
    for (int i = 0; i < 4; ++i) c.layer_kind[i] = static_cast<unsigned char>(kKinds[i]);
    for (const auto& [name, td] : t.tensors) {
        RlTensor r{};
        r.name = name.c_str();
        r.quant = static_cast<int>(td.quant);
        r.rows = td.shape[0];
        r.cols = td.ndim == 2 ? td.shape[1] : 1;
        r.data = td.data.data();
        r.scale = td.scale.empty() ? nullptr : td.scale.data();
        d.ts.push_back(r);
    }
    return d;
}

void check_engine() {
    const TensorTable table = make_table();
    const Direct dir = direct_of(table);
    auto eng = hip_gen::create_from_table(table, 512, 2);
    int st = 0;
    RlEngine* raw = rl_hip_engine_create_batch(&dir.cfg, dir.ts.data(), static_cast<int>(dir.ts.size()), 512, 4, 2, &st);
    expect(raw != nullptr && st == RL_OK, "direct C-ABI engine created");
    void* orc = orc_model_create(&dir.cfg, dir.ts.data(), static_cast<int>(dir.ts.size()), 512, 1, 8);
    expect(orc != nullptr, "oracle model created");
    if (!raw || !orc) return;
    expect(eng->vocab() == V && eng->hidden() == H && eng->max_batch() == 2, "HipEngine vocab / hidden / max_batch");

    std::vector<float> la(V), lb(V), lo(V), hid(H);
    const int32_t prompt[5] = {5, 9, 13, 2, 7};
    eng->prefill(prompt, 5);
    rl_hip_engine_prefill(raw, prompt, 5);
    int g = 0;
    for (int32_t tok : prompt) g = orc_model_decode(orc, tok, lo.data(), hid.data());
    int step_ok = 1;
    double worst = 0;
    for (int step = 0; step < 5; ++step) {
        eng->copy_logits(la.data());
        rl_hip_engine_copy_logits(raw, lb.data());
        step_ok &= std::memcmp(la.data(), lb.data(), V * 4) == 0;
        worst = std::max(worst, rel_l2(la.data(), lo.data(), V));
        int32_t tok = eng->greedy();
        eng->decode_token(tok);
        rl_hip_engine_decode_token(raw, tok);
        orc_model_decode(orc, tok, lo.data(), hid.data());
    }
    (void)g;
    expect(step_ok, "HipEngine logits == direct C-ABI engine logits (bit for bit, 5 steps)");
    expect(worst < 1e-3, "HipEngine logits vs oracle model: rel L2 " + std::to_string(worst) + " < 1e-3");
    expect(eng->pos() == 10, "HipEngine pos after prefill + 5 decodes");

    // Session::generate, MTP branch (session.cpp:728-747) vs plain greedy decoding
    const int want = 12;
    std::vector<int32_t> plain;
    eng->prefill(prompt, 5);
    plain.push_back(eng->greedy());
    while (static_cast<int>(plain.size()) < want) {
        eng->decode_token(plain.back());
        plain.push_back(eng->greedy());
    }
    std::vector<int32_t> spec;
    eng->prefill(prompt, 5);
    int steps = 0;
    while (static_cast<int>(spec.size()) < want) {
        const int32_t t0 = eng->greedy();
        spec.push_back(t0);
        if (static_cast<int>(spec.size()) >= want) break;
        int32_t pm[16];
        const int k2 = eng->mtp_spec2(t0, pm);
        ++steps;
        expect(k2 >= 1 && k2 <= 2 && pm[0] == t0, "mtp_spec2 returns the fed tokens [t0, d0] and n_consumed");
        for (int i = 0; i + 1 < k2 && static_cast<int>(spec.size()) < want; ++i) spec.push_back(pm[i + 1]);
    }
    expect(spec == plain, "Session MTP loop through HipEngine == plain greedy tokens (" + std::to_string(steps) +
                              " verify steps)");

    // continuous batch through the adapter == the direct engine
    const int32_t pa[3] = {1, 2, 3}, pb[4] = {9, 8, 7, 6};
    eng->prefill_slot(pa, 3, 0);
    eng->prefill_slot(pb, 4, 1);
    rl_hip_engine_prefill_slot(raw, pa, 3, 0);
    rl_hip_engine_prefill_slot(raw, pb, 4, 1);
    const int32_t toks[2] = {11, 12};
    const int poss[2] = {3, 4};
    eng->decode_tokens(toks, poss, 2);
    rl_hip_engine_decode_tokens(raw, toks, poss, 2);
    std::vector<float> na(2 * V), nb(2 * V);
    eng->copy_logits_n(na.data(), 2);
    rl_hip_engine_copy_logits_n(raw, nb.data(), 2);
    expect(std::memcmp(na.data(), nb.data(), na.size() * 4) == 0, "decode_tokens (B = 2) through HipEngine == direct");
    rl_hip_engine_destroy(raw);
    orc_model_free(orc);
}

// ---------------------------------------------------------------- the device
struct Buf {
    std::unique_ptr<Buffer> b;
    TensorView v;
};
Buf host_buf(Device& dev, DType dt, std::vector<int64_t> shape, const void* src, size_t bytes) {
    BufferDesc d;
    d.bytes = bytes;
    d.host_visible = true;
    Buf r{dev.allocate(d), {}};
    if (src) std::memcpy(r.b->host_ptr(), src, bytes);
    r.v.buf = r.b.get();
    r.v.dtype = dt;
    r.v.ndim = static_cast<int32_t>(shape.size());
    for (size_t i = 0; i < shape.size(); ++i) r.v.shape[i] = shape[i];
    return r;
}
Buf dev_buf(Device& dev, DType dt, std::vector<int64_t> shape, size_t bytes) {
    BufferDesc d;
    d.bytes = bytes;
    d.usage = BufferDesc::Usage::Weight;
    Buf r{dev.allocate(d), {}};
    r.v.buf = r.b.get();
    r.v.dtype = dt;
    r.v.ndim = static_cast<int32_t>(shape.size());
    for (size_t i = 0; i < shape.size(); ++i) r.v.shape[i] = shape[i];
    return r;
}
std::vector<float> normals(Rng& r, size_t n, float sd = 1.f) {
    std::vector<float> v(n);
    for (float& x : v) x = sd * r.normal();
    return v;
}
const float* F(Buf& b) { return static_cast<const float*>(b.b->host_ptr()); }

void check_device() {
    auto dev = hip_gen::create_device();
    auto stream = dev->create_stream();
    Rng r{7};
    expect(std::strcmp(dev->name(), "hip") == 0 && dev->has_kernel("gemv_fp8") && !dev->has_kernel("gemv_f32"),
           "HipDevice name / has_kernel");
    {  // rmsnorm (Session::dev_rms: args {x, gamma, y}, params {n, eps})
        const int n = 256;
        auto x = normals(r, n, 3.f), g = normals(r, n, 0.1f);
        Buf bx = host_buf(*dev, DType::F32, {n}, x.data(), n * 4), bg = host_buf(*dev, DType::F32, {n}, g.data(), n * 4);
        Buf by = host_buf(*dev, DType::F32, {n}, nullptr, n * 4);
        const TensorView a[3] = {bx.v, bg.v, by.v};
        const RmsNormParams p{n, 1e-6f};
        dev->launch("rmsnorm", a, 3, &p, sizeof(p), *stream);
        stream->synchronize();
        std::vector<float> want(n);
        orc_qwen3_rmsnorm(x.data(), g.data(), want.data(), n, 1e-6f);
        expect(rel_l2(F(by), want.data(), n) < 1e-6, "launch(\"rmsnorm\") vs ops::qwen3_rmsnorm");
    }
    {  // gated_rmsnorm, per head of 128
        const int n = 512, gn = 128;
        auto x = normals(r, n), z = normals(r, n), g = normals(r, gn);
        Buf bx = host_buf(*dev, DType::F32, {n}, x.data(), n * 4), bz = host_buf(*dev, DType::F32, {n}, z.data(), n * 4);
        Buf bg = host_buf(*dev, DType::F32, {gn}, g.data(), gn * 4), by = host_buf(*dev, DType::F32, {n}, nullptr, n * 4);
        const TensorView a[4] = {bx.v, bz.v, bg.v, by.v};
        const RmsNormParams p{n, 1e-6f};
        dev->launch("gated_rmsnorm", a, 4, &p, sizeof(p), *stream);
        stream->synchronize();
        std::vector<float> want(n);
        orc_gated_rmsnorm(x.data(), z.data(), g.data(), want.data(), n, 1e-6f, gn);
        expect(rel_l2(F(by), want.data(), n) < 1e-5, "launch(\"gated_rmsnorm\") vs ops::gated_rmsnorm");
    }
    {  // gemv_fp8: weights in device memory (Device::memcpy from a staging buffer), twice
        const int m = 300, n = 640;
        std::vector<uint8_t> w(static_cast<size_t>(m) * n);
        for (auto& b : w) b = r.fp8();
        std::vector<float> s(static_cast<size_t>((m + 127) / 128) * ((n + 127) / 128));
        for (float& v : s) v = 1e-3f + 1e-2f * r.uni();
        auto x = normals(r, n);
        Buf stage = host_buf(*dev, DType::I8, {m, n}, w.data(), w.size());
        Buf bw = dev_buf(*dev, DType::I8, {m, n}, w.size());
        dev->memcpy(bw.v, stage.v, *stream);
        Buf bs = host_buf(*dev, DType::F32, {static_cast<int64_t>(s.size())}, s.data(), s.size() * 4);
        Buf bx = host_buf(*dev, DType::F32, {n}, x.data(), n * 4), by = host_buf(*dev, DType::F32, {m}, nullptr, m * 4);
        const TensorView a[4] = {bw.v, bs.v, bx.v, by.v};
        GemvFp8Params p;
        p.m = m;
        p.n = n;
        std::vector<float> want(m), first(m);
        orc_gemv_fp8(w.data(), s.data(), x.data(), want.data(), m, n, 128);
        dev->launch("gemv_fp8", a, 4, &p, sizeof(p), *stream);
        stream->synchronize();
        std::memcpy(first.data(), F(by), m * 4);
        dev->launch("gemv_fp8", a, 4, &p, sizeof(p), *stream);  // packed weights from the cache
        stream->synchronize();
        expect(rel_l2(first.data(), want.data(), m) < 1e-3, "launch(\"gemv_fp8\") vs ops::gemv_fp8");
        expect(std::memcmp(first.data(), F(by), m * 4) == 0, "gemv_fp8 second launch (cached packing) identical");
        // a new weight buffer after the old one is freed (the allocator may hand out
        // the same address): the packed cache must not serve the old weights
        bw.b.reset();
        for (auto& b : w) b = r.fp8();
        std::memcpy(stage.b->host_ptr(), w.data(), w.size());
        Buf bw2 = dev_buf(*dev, DType::I8, {m, n}, w.size());
        dev->memcpy(bw2.v, stage.v, *stream);
        const TensorView a2[4] = {bw2.v, bs.v, bx.v, by.v};
        orc_gemv_fp8(w.data(), s.data(), x.data(), want.data(), m, n, 128);
        dev->launch("gemv_fp8", a2, 4, &p, sizeof(p), *stream);
        stream->synchronize();
        expect(rel_l2(F(by), want.data(), m) < 1e-3, "gemv_fp8 on a reallocated weight buffer uses the new weights");
    }
    for (int q6 = 0; q6 < 2; ++q6) {  // gemv_q4k / gemv_q6k on kquant_gemv_selftest's bytes (cuda_engine.cu:11295)
        const int m = 64, n = 512, bsz = q6 ? 210 : 144;
        std::vector<uint8_t> w(static_cast<size_t>(m) * (n / 256) * bsz);
        for (size_t i = 0; i < w.size(); ++i) w[i] = static_cast<uint8_t>((i * 17 + 11) & 0xff);
        const uint16_t d05 = 0x2A66, d01 = 0x211F;  // fp16 0.05, 0.01
        for (size_t b = 0; b < w.size() / bsz; ++b) {
            uint8_t* blk = w.data() + b * bsz;
            if (q6) {
                std::memcpy(blk + 208, &d05, 2);
                for (int s2 = 0; s2 < 16; ++s2) blk[192 + s2] = static_cast<uint8_t>(static_cast<int8_t>((s2 & 7) - 3));
            } else {
                std::memcpy(blk, &d05, 2);
                std::memcpy(blk + 2, &d01, 2);
            }
        }
        std::vector<float> x(n);
        for (int i = 0; i < n; ++i) x[i] = 0.02f * static_cast<float>((i % 17) - 8);
        Buf bw = host_buf(*dev, DType::I8, {static_cast<int64_t>(w.size())}, w.data(), w.size());
        Buf bx = host_buf(*dev, DType::F32, {n}, x.data(), n * 4), by = host_buf(*dev, DType::F32, {m}, nullptr, m * 4);
        const TensorView a[3] = {bw.v, bx.v, by.v};
        const GemvKQuantParams p{m, n, q6 ? 8 : 6};
        dev->launch(q6 ? "gemv_q6k" : "gemv_q4k", a, 3, &p, sizeof(p), *stream);
        stream->synchronize();
        std::vector<float> want(m);
        (q6 ? orc_gemv_q6_k : orc_gemv_q4_k)(w.data(), x.data(), want.data(), m, n, 1);
        expect(rel_l2(F(by), want.data(), m) < 1e-3,
               std::string("launch(\"") + (q6 ? "gemv_q6k" : "gemv_q4k") + "\") vs ops::gemv_q" + (q6 ? "6" : "4") + "_k");
    }
    {  // conv1d_update
        const int dim = 1000, k = 4;
        auto x = normals(r, dim), w = normals(r, static_cast<size_t>(dim) * k, 0.5f), s0 = normals(r, static_cast<size_t>(dim) * k);
        Buf bx = host_buf(*dev, DType::F32, {dim}, x.data(), dim * 4);
        Buf bw = host_buf(*dev, DType::F32, {dim, k}, w.data(), w.size() * 4);
        Buf bs = host_buf(*dev, DType::F32, {dim, k}, s0.data(), s0.size() * 4);
        Buf by = host_buf(*dev, DType::F32, {dim}, nullptr, dim * 4);
        const TensorView a[4] = {bx.v, bw.v, bs.v, by.v};
        const Conv1dParams p{dim, k, 1};
        dev->launch("conv1d_update", a, 4, &p, sizeof(p), *stream);
        stream->synchronize();
        std::vector<float> want(dim), ws = s0;
        orc_conv1d_update(x.data(), w.data(), ws.data(), want.data(), dim, k);
        expect(std::memcmp(F(bs), ws.data(), ws.size() * 4) == 0 && rel_l2(F(by), want.data(), dim) < 1e-6,
               "launch(\"conv1d_update\") vs ops::conv1d_update");
    }
    {  // delta_recurrent, two tokens
        const int nv = 4, dk = 128, dv = 128;
        auto S = normals(r, static_cast<size_t>(nv) * dk * dv, 0.02f), q = normals(r, nv * dk), k = normals(r, nv * dk),
             v = normals(r, nv * dv);
        std::vector<float> beta(nv), gl(nv);
        for (int h = 0; h < nv; ++h) beta[h] = 1.f / (1.f + std::exp(-r.normal())), gl[h] = -std::log1p(std::exp(r.normal()));
        Buf bS = host_buf(*dev, DType::F32, {nv, dk, dv}, S.data(), S.size() * 4);
        Buf bq = host_buf(*dev, DType::F32, {nv, dk}, q.data(), q.size() * 4);
        Buf bk = host_buf(*dev, DType::F32, {nv, dk}, k.data(), k.size() * 4);
        Buf bv = host_buf(*dev, DType::F32, {nv, dv}, v.data(), v.size() * 4);
        Buf bb = host_buf(*dev, DType::F32, {nv}, beta.data(), nv * 4), bg = host_buf(*dev, DType::F32, {nv}, gl.data(), nv * 4);
        Buf bo = host_buf(*dev, DType::F32, {nv, dv}, nullptr, nv * dv * 4);
        const TensorView a[7] = {bS.v, bq.v, bk.v, bv.v, bb.v, bg.v, bo.v};
        const DeltaRecurrentParams p{nv, dk, dv, 1e-6f};
        std::vector<float> o(static_cast<size_t>(nv) * dv);
        double worst = 0;
        for (int t = 0; t < 2; ++t) {
            dev->launch("delta_recurrent", a, 7, &p, sizeof(p), *stream);
            stream->synchronize();
            orc_delta_step(S.data(), q.data(), k.data(), v.data(), beta.data(), gl.data(), o.data(), nv, dk, dv, 1e-6f);
            worst = std::max(worst, rel_l2(F(bo), o.data(), o.size()));
        }
        expect(worst < 1e-3 && rel_l2(F(bS), S.data(), S.size()) < 1e-4,
               "launch(\"delta_recurrent\") vs ops::delta_recurrent_step (2 tokens)");
    }
    {  // attn_decode over fp32 caches
        const int pos = 50, nq = 8, nkv = 2, hd = 128;
        auto q = normals(r, nq * hd), kc = normals(r, static_cast<size_t>(pos + 1) * nkv * hd),
             vc = normals(r, static_cast<size_t>(pos + 1) * nkv * hd);
        Buf bq = host_buf(*dev, DType::F32, {nq, hd}, q.data(), q.size() * 4);
        Buf bk = host_buf(*dev, DType::F32, {pos + 1, nkv, hd}, kc.data(), kc.size() * 4);
        Buf bv = host_buf(*dev, DType::F32, {pos + 1, nkv, hd}, vc.data(), vc.size() * 4);
        Buf bo = host_buf(*dev, DType::F32, {nq, hd}, nullptr, q.size() * 4);
        const TensorView a[4] = {bq.v, bk.v, bv.v, bo.v};
        const AttnDecodeParams p{nq, nkv, hd, pos + 1, pos, static_cast<int>(DType::F32), 1e-6f};
        dev->launch("attn_decode", a, 4, &p, sizeof(p), *stream);
        stream->synchronize();
        std::vector<float> want(q.size());
        orc_attn_decode(q.data(), kc.data(), vc.data(), want.data(), pos, nq, nkv, hd);
        expect(rel_l2(F(bo), want.data(), want.size()) < 1e-3, "launch(\"attn_decode\") vs ops::attn_decode");
    }
}

}  // namespace

int main() {
    if (!hip_gen::available()) {
        std::printf("no gfx950 device\n");
        return 2;
    }
    try {
        check_device();
        check_engine();
    } catch (const std::exception& e) {
        std::printf("FAIL exception: %s\n", e.what());
        return 1;
    }
    std::printf(g_fail ? "seam_check FAILED (%d)\n" : "seam_check ok\n", g_fail);
    return g_fail ? 1 : 0;
}
