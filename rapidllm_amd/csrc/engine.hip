// engine.hip -- the MI355X decode engine: one forward step over T = 1..Tmax tokens of
// the Qwen3.6/3.8-27B hybrid stack, the MTP stem draft, greedy acceptance and
// speculative verify, captured as HIP graphs.
//
// It implements the surface of the reference's GPU engine seam, cuda_gen::Engine
// (include/rapidllm/runtime/cuda_engine.h:13-83): prefill, decode_token,
// decode_steps (self-feeding), copy_gen_tokens, copy_logits, copy_last_hidden,
// mtp_draft, spec_verify, greedy, pos, vocab, hidden; plus mtp_spec (draft + verify
// in one submission, the role of mtp_spec4, cuda_engine.h:40).  Numerics follow the
// reference CPU session (src/runtime/session.cpp:325-411, 531-559, 619-681,
// 799-829): the oracle for every parity test.
//
// Per step (T tokens), per layer:
//   rmsnorm_pack -> fused in_proj GEMM [qkv;z;a;b] -> gdn_decode -> gnorm_pack ->
//   out_proj GEMM (+= residual)                                   (DeltaNet layer)
//   rmsnorm_pack -> fused [q|gate;k;v] GEMM -> attention (qk_prep, chunk partials,
//   combine+gate+pack) -> o_proj GEMM (+= residual)              (attention layer)
//   rmsnorm_pack -> interleaved gate/up GEMM with SwiGLU epilogue -> pack ->
//   down GEMM (+= residual)                                       (MLP)
// then final norm -> lm_head -> argmax -> accept.  Every dynamic quantity (token
// ids, position, recurrent-state slot) lives in device memory, so a step is a fixed
// launch sequence and is captured once per T.
//
// Speculative rollback: recurrent states (S and the conv window) live in rings of
// R = Tmax + 1 slots; the DeltaNet kernel writes the state after every token of a
// verify step to its own slot and acceptance just advances the slot index by the
// number of tokens kept.  KV rows of rejected tokens are overwritten later and are
// never read (attention masks positions past each query).
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "internal.h"

using namespace rl;

namespace rl {

namespace {

inline int align16(int v) { return (v + 15) / 16 * 16; }

// Device allocations of one engine, zero-filled on the engine's stream: the stream
// is non-blocking, so a null-stream memset would not be ordered before the kernels
// that fill the buffer (weight packing) and could land after them.
struct DevAlloc {
    std::vector<void*> ptrs;
    size_t total = 0;
    hipStream_t st = nullptr;
    void* get(size_t bytes) {
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, bytes ? bytes : 256);
        if (e == hipErrorOutOfMemory) throw Error(RL_ERR_NOMEM, "engine: out of device memory");
        RL_HIP(e);
        RL_HIP(hipMemsetAsync(p, 0, bytes ? bytes : 256, st));
        ptrs.push_back(p);
        total += bytes;
        return p;
    }
    template <class T>
    T* get_n(size_t n) {
        return static_cast<T*>(get(n * sizeof(T)));
    }
    ~DevAlloc() {
        for (void* p : ptrs) (void)hipFree(p);
    }
};

// A linear on the device.  FP8 / BF16: MFMA-tiled (16-row tiles), possibly several
// source matrices fused along rows.  Q4_K / Q6_K: K-tiled, one matrix.
struct Lin {
    int kind = -1;
    int m = 0;  // rows of the device weight (FP8/BF16: padded to 16-row tiles)
    int n = 0;
    uint8_t* w = nullptr;
    float* ts = nullptr;
    bool guh = false;  // FP8/BF16 gate/up in half tiles (SwiGLU epilogue kEpiSwiGLUH)
    int swiglu_epi() const { return guh ? kEpiSwiGLUH : kEpiSwiGLU; }
};

struct Layer {
    int kind = RL_LAYER_DELTA;
    const float* attn_norm = nullptr;
    const float* ffn_norm = nullptr;
    // DeltaNet
    std::vector<Lin> in_parts;  // fused [qkv|z|a|b] (one Lin) or separate K-quant parts
    std::vector<int> in_offs;   // output column offset of each part
    int in_width = 0, off_z = 0, off_a = 0, off_b = 0;
    Lin out_proj;
    const float *A_log = nullptr, *dt_bias = nullptr, *conv_w = nullptr, *gnorm = nullptr;
    int gnorm_n = 0;
    int dslot = 0;  // index among DeltaNet layers
    // attention
    std::vector<Lin> qkv_parts;
    std::vector<int> qkv_offs;
    int qkv_width = 0;
    Lin o_proj;
    const float *q_norm = nullptr, *k_norm = nullptr;
    int aslot = 0;
    // MLP
    Lin gate_up;  // FP8/BF16: interleaved gate/up tiles, SwiGLU epilogue
    Lin gate, up; // K-quant: separate, or gate_cat: gate / up half tiles in `gate` (SwiGLU launch)
    bool gate_cat = false;
    Lin down;
};

}  // namespace

class Engine {
   public:
    Engine(const RlModelConfig& cfg, int ctx, int tmax, int max_batch = 1) : c_(cfg), tmax_(tmax), mb_(max_batch) {
        RL_REQUIRE(tmax >= 1 && tmax <= 4, RL_ERR_RANGE, "engine: max_T must be in 1..4");
        RL_REQUIRE(max_batch >= 1 && max_batch <= kMaxSlots, RL_ERR_RANGE, "engine: max_batch must be in 1..16");
        tcap_ = std::max(tmax_, std::min(mb_, kGroupRows));
        RL_REQUIRE(c_.n_layers >= 1 && c_.n_layers <= RL_MAX_LAYERS, RL_ERR_RANGE, "engine: bad layer count");
        RL_REQUIRE(c_.hidden % 128 == 0, RL_ERR_UNSUPPORTED, "engine: hidden must be a multiple of 128");
        RL_REQUIRE(c_.k_dim == 128 && c_.v_dim % 32 == 0, RL_ERR_UNSUPPORTED, "engine: DeltaNet dims 128 / 32k");
        RL_REQUIRE(c_.conv_k == 4, RL_ERR_UNSUPPORTED, "engine: conv width must be 4");
        RL_REQUIRE(c_.head_dim == 256, RL_ERR_UNSUPPORTED, "engine: attention head_dim must be 256");
        RL_REQUIRE(c_.n_kv > 0 && c_.n_q % c_.n_kv == 0 && (c_.n_q / c_.n_kv) * tmax <= 32, RL_ERR_UNSUPPORTED,
                   "engine: (n_q/n_kv) * max_T must be <= 32");
        ctx_ = (ctx + 255) / 256 * 256 + 256;  // room for a verify chunk past the last position
        R_ = tmax + 1;
        RL_HIP(hipStreamCreateWithFlags(&st_, hipStreamNonBlocking));
        mem_.st = st_;
    }

    ~Engine() {
        for (auto& g : graphs_)
            if (g.second) (void)hipGraphExecDestroy(g.second);
        if (st_) (void)hipStreamDestroy(st_);
        if (host_rb_) (void)hipHostFree(host_rb_);
        if (host_in_) (void)hipHostFree(host_in_);
    }

    // ------------------------------------------------------------ weights
    void load(const RlTensor* t, int n) {
        for (int i = 0; i < n; ++i) tab_[t[i].name] = &t[i];
        build([&](const std::string& name) -> const RlTensor* {
            auto it = tab_.find(name);
            return it == tab_.end() ? nullptr : it->second;
        });
    }

    // Synthetic random-init weights of the configured architecture, generated on the
    // device (benchmark configs: e4m3 bytes uniform without NaN codes, 128x128 fp32
    // scales log-uniform in [1e-3, 1e-1], bf16 embedding / lm_head, small norms).
    // RL_SYNTH_LINEAR=q4_k / q6_k: the layer linears and the MTP fc as GGML
    // K-quant blocks instead (in_proj a/b BF16, lm_head Q6_K, as in a Q4_K_M file).
    void load_synthetic(uint64_t seed) {
        synth_seed_ = seed;
        synthetic_ = true;
        if (const char* e = std::getenv("RL_SYNTH_LINEAR")) {
            if (std::strcmp(e, "q4_k") == 0) synth_quant_ = RL_Q_Q4_K;
            else if (std::strcmp(e, "q6_k") == 0) synth_quant_ = RL_Q_Q6_K;
        }
        build([&](const std::string&) -> const RlTensor* { return nullptr; });
    }

    // ------------------------------------------------------------ API
    int vocab() const { return c_.vocab; }
    int hidden() const { return c_.hidden; }
    int ctx_capacity() const { return ctx_ - 256; }
    int max_t() const { return tmax_; }
    size_t device_bytes() const { return mem_.total; }

    // Clear the current slot's sequence state (slot 0 outside prefill_slot).
    void reset() {
        sync_graph_state();
        zero_slot_state(cs_);
        RL_HIP(hipStreamSynchronize(st_));
        RL_HIP(hipMemsetAsync(h_last_, 0, c_.hidden * sizeof(float), st_));
        RL_HIP(hipMemsetAsync(h_prev_, 0, c_.hidden * sizeof(float), st_));
        RL_HIP(hipStreamSynchronize(st_));
        pos_ = 0;
        greedy_ = 0;
        n_last_ = 0;
    }

    // Stage n ints in pinned memory and enqueue their upload to dst (stream order).
    // Every public call ends with a stream synchronisation, so the stage is free.
    void upload_ints(int* dst, const int32_t* src, int n) {
        std::memcpy(host_in_, src, static_cast<size_t>(n) * sizeof(int));
        RL_HIP(hipMemcpyAsync(dst, host_in_, static_cast<size_t>(n) * sizeof(int), hipMemcpyHostToDevice, st_));
    }

    void prefill(const int32_t* ids, int n) {
        RL_REQUIRE(n >= 1 && ids, RL_ERR_RANGE, "prefill: empty prompt");
        RL_REQUIRE(n <= ctx_capacity(), RL_ERR_RANGE, "prefill: prompt longer than the context");
        check_ids(ids, n);
        reset();
        upload_ints(tok_all_, ids, n);
        // all but the last (up to max_T) tokens through the chunked prefill path; the
        // tail runs as a decode step, which leaves the logits, the next token, the MTP
        // history and the speculative bookkeeping exactly as decoding would
        int done = 0;
        const int tail = std::min(tmax_, n);
        if (n - tail >= kPfMinTokens && can_prefill_chunked()) {
            prefill_chunks(n - tail);
            done = n - tail;
        }
        for (int i = done; i < n; i += tmax_) {
            const int T = std::min(tmax_, n - i);
            RL_HIP(hipMemcpyAsync(tok_, tok_all_ + i, T * sizeof(int), hipMemcpyDeviceToDevice, st_));
            step(T, /*force_all=*/1, /*feed=*/false);
        }
        readback();
    }

    // ---------------------------------------------------------------- prefill
    // Chunked prompt prefill (the reference's launch_prefill_chunk,
    // cuda_engine.cu:18338-18590): per chunk of up to kPfChunk tokens, layer by
    // layer, the block-FP8 linears run over all chunk tokens on the matrix cores
    // (gemm_fp8_prefill), the DeltaNet conv runs over the chunk and the recurrence
    // steps the committed state through it in registers (gdn_prefill; the conv
    // window ping-pongs between ring slots 0 and 1), attention is the causal prefill kernel (which
    // also writes the chunk's K/V).  RMSNorms are explicit (norm + pack kernels).
    static constexpr int kPfChunk = 4096;
    static constexpr int kPfMinTokens = 16;
    int pf_cap_ = 0;
    float *pf_x_ = nullptr, *pf_y_ = nullptr, *pf_o_ = nullptr, *pf_h_ = nullptr, *pf_xc_ = nullptr,
          *pf_gates_ = nullptr, *pf_gdn_ck_ = nullptr;
    void *pf_frag_ = nullptr, *pf_frag_h_ = nullptr, *pf_attn_ws_ = nullptr;
    // K-quant prefill (fp16 form): the tiles' block scales, the input converted to
    // fp16 hi + lo fragments and its block scales, and which fragments that input is
    float* pf_ts_ = nullptr;
    void* pf_frag16_ = nullptr;
    float* pf_xs_ = nullptr;
    const void* pf_f16_src_ = nullptr;
    size_t pf_attn_ws_bytes_ = 0;
    int* pf_pos_ = nullptr;
    uint16_t *pf_whi_ = nullptr, *pf_wlo_ = nullptr;  // a K-quant linear as BF16 hi + lo tiles
    float* pf_u_ = nullptr;                          // up rows of separate K-quant gate / up
    std::unique_ptr<DevAlloc> pf_mem_;

    // RL_PREFILL_CHUNK: 0 = every prompt token through decode steps (T <= max_T);
    // n > 0 = chunk size (default kPfChunk)
    // read once per engine (at its first prefill)
    mutable int pf_chunk_ = -1;
    int pf_chunk_setting() const {
        if (pf_chunk_ < 0) {
            const char* e = std::getenv("RL_PREFILL_CHUNK");
            pf_chunk_ = e ? std::max(0, std::atoi(e)) : kPfChunk;
        }
        return pf_chunk_;
    }

    // Every layer linear FP8, BF16 or Q4_K / Q6_K (K-quant ones are dequantised to
    // BF16 hi + lo tiles per chunk), and the DeltaNet layers on the fused kernel's
    // state (one committed S, the conv ring), which the prefill recurrence writes.
    bool can_prefill_chunked() const {
        if (pf_chunk_setting() == 0) return false;
        for (const Layer& Ly : L_) {
            for (const Lin& L : Ly.kind == RL_LAYER_DELTA ? Ly.in_parts : Ly.qkv_parts)
                if (!known_kind(L)) return false;
            if (Ly.kind == RL_LAYER_DELTA && (!gdn_fused_ || !known_kind(Ly.out_proj))) return false;
            if (Ly.kind != RL_LAYER_DELTA && !known_kind(Ly.o_proj)) return false;
            if (Ly.gate_up.kind >= 0 ? !frag_kind(Ly.gate_up)
                                     : (!known_kind(Ly.gate) || (!Ly.gate_cat && !known_kind(Ly.up))))
                return false;
            if (!known_kind(Ly.down)) return false;
        }
        return c_.hidden % 8 == 0;
    }

    // elements of the largest K-quant layer linear (its BF16 hi / lo scratch)
    size_t kq_prefill_elems() const {
        size_t e = 0;
        auto see = [&](const Lin& L) {
            if (is_kq(L)) e = std::max(e, static_cast<size_t>((L.m + 15) / 16) * 16 * L.n);
        };
        for (const Layer& Ly : L_) {
            for (const Lin& L : Ly.kind == RL_LAYER_DELTA ? Ly.in_parts : Ly.qkv_parts) see(L);
            see(Ly.out_proj);
            see(Ly.o_proj);
            see(Ly.gate);
            see(Ly.up);
            see(Ly.down);
        }
        return e;
    }

    // One prefill linear over T tokens of fragments: Y (=, +=, SwiGLU) W . x.
    void pf_linear(const Lin& L, const void* frag, float* Y, int ldy, int m_valid, int T, int epi) {
        if (L.kind == RL_Q_FP8_E4M3_B128) {
            gemm_prefill_any(0, L.w, nullptr, L.ts, frag, Y, L.m, L.n, T, epi, ldy, m_valid, st_);
        } else if (L.kind == RL_Q_BF16) {
            gemm_prefill_any(1, L.w, nullptr, nullptr, frag, Y, L.m, L.n, T, epi, ldy, m_valid, st_);
        } else if (kq_f16()) {
            // fp16 tiles with a power-of-two scale per block, the input fragments as
            // fp16 hi + lo (converted once per input: the cache is cleared whenever a
            // producer writes the fragments)
            if (frag != pf_f16_src_) {
                act_frag_to_f16(frag, pf_frag16_, pf_xs_, L.n, T, st_);
                pf_f16_src_ = frag;
            }
            kq_to_f16(L.kind == RL_Q_Q4_K ? 4 : 6, L.w, pf_whi_, pf_ts_, L.m, L.n, st_);
            gemm_prefill_any(3, reinterpret_cast<const uint8_t*>(pf_whi_), nullptr, pf_ts_, pf_frag16_, Y, L.m, L.n, T,
                             epi, ldy, m_valid, st_, pf_xs_);
        } else {
            kq_to_bf16x2(L.kind == RL_Q_Q4_K ? 4 : 6, L.w, pf_whi_, pf_wlo_, L.m, L.n, st_);
            gemm_prefill_any(2, reinterpret_cast<const uint8_t*>(pf_whi_), reinterpret_cast<const uint8_t*>(pf_wlo_),
                             nullptr, frag, Y, L.m, L.n, T, epi, ldy, m_valid, st_);
        }
    }
    // K-quant prefill linears as fp16 tiles (RL_PF_KQ16=0: the BF16 hi + lo tiles)
    static bool kq_f16() {
        static const bool on = [] {
            const char* v = std::getenv("RL_PF_KQ16");
            return !(v && v[0] == '0');
        }();
        return on;
    }
    void pf_parts(const std::vector<Lin>& parts, const std::vector<int>& offs, float* Y, int ldy, int T) {
        for (size_t k = 0; k < parts.size(); ++k) pf_linear(parts[k], pf_frag_, Y + offs[k], ldy, parts[k].m, T, kEpiStore);
    }

    void ensure_pf_buffers(int C) {
        if (pf_cap_ >= C) return;
        pf_mem_ = std::make_unique<DevAlloc>();
        pf_mem_->st = st_;
        const int H = c_.hidden, I = c_.intermediate;
        int wy = 16, wo = 16, wf = H;
        for (const Layer& Ly : L_) {
            wy = std::max(wy, Ly.kind == RL_LAYER_DELTA ? Ly.in_width : Ly.qkv_width);
            wo = std::max(wo, Ly.kind == RL_LAYER_DELTA ? c_.n_v_heads * c_.v_dim : c_.n_q * c_.head_dim);
        }
        wf = std::max(wf, wo);
        pf_x_ = pf_mem_->get_n<float>(static_cast<size_t>(C) * H);
        pf_y_ = pf_mem_->get_n<float>(static_cast<size_t>(C) * wy);
        pf_o_ = pf_mem_->get_n<float>(static_cast<size_t>(C) * wo);
        pf_h_ = pf_mem_->get_n<float>(static_cast<size_t>(C) * I);
        pf_xc_ = pf_mem_->get_n<float>(static_cast<size_t>(C) * std::max(2 * c_.n_k_heads * c_.k_dim + c_.n_v_heads * c_.v_dim, 1));
        pf_gates_ = pf_mem_->get_n<float>(static_cast<size_t>(C) * std::max(c_.n_v_heads, 1) * 2);
        {
            const size_t ckf = gdn_prefill_chunked() ? gdn_prefill_chunk_floats(C, c_.n_v_heads, c_.k_dim, c_.v_dim) : 0;
            pf_gdn_ck_ = ckf ? pf_mem_->get_n<float>(ckf) : nullptr;
        }
        pf_frag_ = pf_mem_->get(act_frag_bytes(wf, C));
        pf_frag_h_ = pf_mem_->get(act_frag_bytes(I, C));
        pf_attn_ws_bytes_ = attn_prefill_workspace_bytes(std::max(c_.n_q, 1), C);
        pf_attn_ws_ = pf_mem_->get(pf_attn_ws_bytes_);
        pf_pos_ = pf_mem_->get_n<int>(64);
        const size_t kqe = kq_prefill_elems();
        if (kqe) {
            pf_whi_ = pf_mem_->get_n<uint16_t>(kqe);
            if (kq_f16()) {
                const int wmax = std::max(wf, I);
                pf_ts_ = pf_mem_->get_n<float>(kqe / 2048 + 1);  // one per 16 x 128 block
                pf_frag16_ = pf_mem_->get(act_frag_bytes(wmax, C));
                pf_xs_ = pf_mem_->get_n<float>(static_cast<size_t>((wmax + 127) / 128) * C);
            } else {
                pf_wlo_ = pf_mem_->get_n<uint16_t>(kqe);
            }
            pf_u_ = pf_mem_->get_n<float>(static_cast<size_t>(C) * I);
        }
        pf_f16_src_ = nullptr;
        pf_cap_ = C;
    }

    // Tokens tok_all_[0 .. N) at positions 0 .. N-1 from the reset state; leaves the
    // KV caches, the DeltaNet states and conv windows after token N-1, and the
    // position / ring slot scalars for the next step.
    void prefill_chunks(int N) {
        const int H = c_.hidden, nk = c_.n_k_heads, nv = c_.n_v_heads, dv = c_.v_dim, I = c_.intermediate;
        const int zdim = nv * dv, nq = c_.n_q, nkv = c_.n_kv, hd = c_.head_dim;
        const float eps = c_.rms_eps;
        const int C = std::min(pf_chunk_setting(), N);
        ensure_pf_buffers(C);
        // the prompt's upload reads the pinned stage that the positions below reuse
        RL_HIP(hipStreamSynchronize(st_));
        int slot = 0;  // conv ring slot holding the window (reset: 0)
        for (int c0 = 0; c0 < N; c0 += C) {
            const int T = std::min(C, N - c0);
            upload_ints(pf_pos_, &c0, 1);
            embed_rows(embed_, embed_kind_, tok_all_ + c0, pf_x_, H, c_.vocab, T, st_);
            for (int i = 0; i < c_.n_layers; ++i) {
                Layer& Ly = L_[i];
                rmsnorm_pack(pf_x_, H, Ly.attn_norm, nullptr, pf_frag_, H, T, eps, st_);
                pf_f16_src_ = nullptr;
                if (Ly.kind == RL_LAYER_DELTA) {
                    pf_parts(Ly.in_parts, Ly.in_offs, pf_y_, Ly.in_width, T);
                    float* ring = slot_conv(Ly.dslot);
                    gdn_prefill(pf_y_, Ly.in_width, Ly.off_a, Ly.off_b, Ly.A_log, Ly.dt_bias, Ly.conv_w,
                                ring + slot * conv_slot_, ring + (slot ^ 1) * conv_slot_, pf_xc_, pf_gates_,
                                slot_S(Ly.dslot), pf_o_, T, nk, nv, c_.k_dim, dv, c_.conv_k, c_.v_tiled, st_,
                                pf_gdn_ck_);
                    gnorm_pack(pf_o_, pf_y_ + Ly.off_z, Ly.in_width, Ly.gnorm, Ly.gnorm_n, nullptr, pf_frag_, zdim, T,
                               1e-6f, st_);
                    pf_f16_src_ = nullptr;
                    pf_linear(Ly.out_proj, pf_frag_, pf_x_, H, H, T, kEpiAdd);
                } else {
                    pf_parts(Ly.qkv_parts, Ly.qkv_offs, pf_y_, Ly.qkv_width, T);
                    attn_prefill_layer(pf_y_, Ly.qkv_width, Ly.q_norm, Ly.k_norm, slot_kc(Ly.aslot), slot_vt(Ly.aslot),
                                       ctx_, pf_pos_, T, nq, nkv, hd, c_.rotary_dim, c_.rope_theta, eps, pf_attn_ws_,
                                       pf_attn_ws_bytes_, pf_o_, st_);
                    pack_act(pf_o_, pf_frag_, nq * hd, T, st_);
                    pf_f16_src_ = nullptr;
                    pf_linear(Ly.o_proj, pf_frag_, pf_x_, H, H, T, kEpiAdd);
                }
                rmsnorm_pack(pf_x_, H, Ly.ffn_norm, nullptr, pf_frag_, H, T, eps, st_);
                pf_f16_src_ = nullptr;
                // half-tile gate / up pairs write the down projection's input
                // fragments directly when I fills whole 128-column blocks
                const bool h_frag = I % 128 == 0;
                float* hy = h_frag ? static_cast<float*>(pf_frag_h_) : pf_h_;
                const int he = h_frag ? kEpiSwiGLUHFrag : kEpiSwiGLUH;
                bool packed = false;
                if (Ly.gate_up.kind >= 0 && Ly.gate_up.guh) {
                    pf_linear(Ly.gate_up, pf_frag_, hy, I, I, T, he);
                    packed = h_frag;
                } else if (Ly.gate_up.kind >= 0) {
                    pf_linear(Ly.gate_up, pf_frag_, pf_h_, I, I, T, Ly.gate_up.swiglu_epi());
                } else if (Ly.gate_cat) {
                    pf_linear(Ly.gate, pf_frag_, hy, I, I, T, he);
                    packed = h_frag;
                } else {
                    pf_linear(Ly.gate, pf_frag_, pf_h_, I, I, T, kEpiStore);
                    pf_linear(Ly.up, pf_frag_, pf_u_, I, I, T, kEpiStore);
                    swiglu(pf_h_, I, pf_u_, I, pf_h_, I, T, st_);
                }
                if (!packed) pack_act(pf_h_, pf_frag_h_, I, T, st_);
                pf_f16_src_ = nullptr;
                pf_linear(Ly.down, pf_frag_h_, pf_x_, H, H, T, kEpiAdd);
            }
            slot ^= 1;
            RL_HIP(hipStreamSynchronize(st_));  // the pinned position stage is reused by the next chunk
        }
        const int scal[2] = {N, slot};  // kPos, kSlot
        upload_ints(sc() + kPos, scal, 2);
        RL_HIP(hipStreamSynchronize(st_));
        pos_ = N;
    }

    void decode_token(int32_t token) {
        check_ids(&token, 1);
        RL_REQUIRE(pos_ + 1 <= ctx_capacity(), RL_ERR_RANGE, "decode: context full");
        upload_ints(sc() + kNextTok, &token, 1);
        run_graph(1);
        readback();
    }

    // n self-fed T=1 steps, one host sync at the end (cuda_engine.h:22-26).
    void decode_steps(int n) {
        RL_REQUIRE(n >= 0, RL_ERR_RANGE, "decode_steps: n < 0");
        RL_REQUIRE(pos_ + n <= ctx_capacity(), RL_ERR_RANGE, "decode_steps: context full");
        RL_HIP(hipMemsetAsync(sc() + kGenCount, 0, sizeof(int), st_));
        for (int i = 0; i < n; ++i) run_graph(1);
        readback();
    }

    void copy_gen_tokens(int32_t* host, int n) {
        RL_REQUIRE(n >= 0 && n <= kGenCap, RL_ERR_RANGE, "copy_gen_tokens: n out of range");
        RL_HIP(hipMemcpyAsync(host, gen_, n * sizeof(int), hipMemcpyDeviceToHost, st_));
        RL_HIP(hipStreamSynchronize(st_));
    }

    // logits of the last consumed token
    void copy_logits(float* host) {
        const int row = n_last_ > 0 ? n_last_ - 1 : 0;
        RL_HIP(hipMemcpyAsync(host, logits_ + static_cast<size_t>(row) * c_.vocab, c_.vocab * sizeof(float),
                              hipMemcpyDeviceToHost, st_));
        RL_HIP(hipStreamSynchronize(st_));
    }

    void copy_last_hidden(float* host) {
        RL_HIP(hipMemcpyAsync(host, h_last_, c_.hidden * sizeof(float), hipMemcpyDeviceToHost, st_));
        RL_HIP(hipStreamSynchronize(st_));
    }

    // Draft mode: RL_MTP_STEM (Session::mtp_draft) or RL_MTP_LAYER (stem + the
    // mtp.layers[0] decoder layer, Session::mtp_layer_step).
    void set_mtp_mode(int mode) {
        RL_REQUIRE(mode == RL_MTP_STEM || mode == RL_MTP_LAYER, RL_ERR_RANGE, "mtp mode must be STEM or LAYER");
        RL_REQUIRE(mode == RL_MTP_STEM || has_mtp_layer_, RL_ERR_UNSUPPORTED,
                   "mtp mode LAYER: the model has no MTP decoder layer (mtp.layers[0].*)");
        mtp_mode_ = mode;
    }
    int mtp_mode() const { return mtp_mode_; }
    // the last draft's hidden before the final MTP norm
    void copy_mtp_hidden(float* out) {
        RL_REQUIRE(has_mtp_, RL_ERR_UNSUPPORTED, "model has no MTP head");
        RL_HIP(hipMemcpyAsync(out, mtp_hp_, c_.hidden * sizeof(float), hipMemcpyDeviceToHost, st_));
        RL_HIP(hipStreamSynchronize(st_));
    }
    bool has_mtp_layer() const { return has_mtp_layer_; }

    // Draft after the last consumed token (session.cpp:619-681).
    int mtp_draft(int32_t first, int n, int32_t* out) {
        if (!has_mtp_ || n <= 0) return 0;
        RL_REQUIRE(n <= 7, RL_ERR_RANGE, "mtp_draft: at most 7 drafts");
        check_ids(&first, 1);
        upload_ints(sc() + kNextTok, &first, 1);
        run_mtp(n);
        RL_HIP(hipMemcpyAsync(out, tok_ + 1, n * sizeof(int), hipMemcpyDeviceToHost, st_));
        RL_HIP(hipStreamSynchronize(st_));
        return n;
    }

    // Verify toks[0..T) in one weight pass (cuda_engine.h:69-77).  Returns n consumed.
    int spec_verify(const int32_t* toks, int T, int32_t* preds) {
        RL_REQUIRE(T >= 1 && T <= tmax_ && toks, RL_ERR_RANGE, "spec_verify: T out of range");
        RL_REQUIRE(pos_ + T <= ctx_capacity(), RL_ERR_RANGE, "spec_verify: context full");
        check_ids(toks, T);
        if (T == 1)  // the T = 1 step feeds the device's next token
            upload_ints(sc() + kNextTok, toks, 1);
        else
            upload_ints(tok_, toks, T);
        run_graph(T, /*from_host=*/true);
        readback();
        if (preds) std::memcpy(preds, host_rb_ + kRbPreds, T * sizeof(int));
        return n_last_;
    }

    // MTP draft of T-1 tokens after t0, then verify [t0, drafts] at T, one sync.
    int mtp_spec(int32_t t0, int T, int32_t* toks_out, int32_t* preds) {
        RL_REQUIRE(has_mtp_, RL_ERR_UNSUPPORTED, "mtp_spec: model has no MTP head");
        RL_REQUIRE(T >= 2 && T <= tmax_, RL_ERR_RANGE, "mtp_spec: T out of range");
        RL_REQUIRE(pos_ + T <= ctx_capacity(), RL_ERR_RANGE, "mtp_spec: context full");
        check_ids(&t0, 1);
        upload_ints(sc() + kNextTok, &t0, 1);
        run_mtp(T - 1);
        run_graph(T, /*from_host=*/true);
        readback();
        if (toks_out) std::memcpy(toks_out, host_rb_ + kRbToks, T * sizeof(int));
        if (preds) std::memcpy(preds, host_rb_ + kRbPreds, T * sizeof(int));
        return n_last_;
    }

    int32_t greedy() const { return greedy_; }
    int pos() const { return pos_; }

    // Benchmark support: claim `pos` positions of context as already filled (the KV
    // rows below pos are whatever the cache holds: zeros or synthetic values).
    void set_pos(int pos) {
        RL_REQUIRE(pos >= 0 && pos <= ctx_capacity(), RL_ERR_RANGE, "set_pos: out of range");
        upload_ints(sc() + kPos, &pos, 1);
        RL_HIP(hipStreamSynchronize(st_));
        pos_ = pos;
    }

    // Fill KV rows [0, n) with fp16 N(0,1) and recurrent states with their benchmark
    // distributions (S ~ N(0, 0.02), conv window ~ N(0,1)), then set pos = n.
    void synthetic_context(int n, uint64_t seed) {
        RL_REQUIRE(n >= 0 && n <= ctx_capacity(), RL_ERR_RANGE, "synthetic_context: out of range");
        reset();
        const size_t kv = static_cast<size_t>(c_.n_kv) * ctx_ * c_.head_dim;
        for (int l = 0; l < static_cast<int>(kc_.size()); ++l) {
            fill_normal_f16(slot_kc(l), kv, 1.f, seed + 11 * l + 1, st_);
            fill_normal_f16(slot_vt(l), kv, 1.f, seed + 11 * l + 2, st_);
        }
        for (int l = 0; l < static_cast<int>(S_.size()); ++l) {
            fill_normal_f32(slot_S(l), s_slot_, 0.f, 0.02f, seed + 13 * l + 3, st_);
            fill_normal_f32(slot_conv(l), conv_slot_, 0.f, 1.f, seed + 13 * l + 4, st_);
        }
        RL_HIP(hipStreamSynchronize(st_));
        set_pos(n);
    }

    // Time `iters` replays of the T-token step graph (or of the MTP draft graph when
    // mtp_drafts > 0) with events on the engine stream; state advances as in decode.
    float time_steps(int T, int iters, int mtp_drafts) {
        hipEvent_t a, b;
        RL_HIP(hipEventCreate(&a));
        RL_HIP(hipEventCreate(&b));
        RL_HIP(hipEventRecord(a, st_));
        for (int i = 0; i < iters; ++i) {
            if (mtp_drafts > 0)
                run_mtp(mtp_drafts);
            else
                run_graph(T, /*from_host=*/T > 1);
        }
        RL_HIP(hipEventRecord(b, st_));
        RL_HIP(hipEventSynchronize(b));
        float ms = 0.f;
        RL_HIP(hipEventElapsedTime(&ms, a, b));
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        readback();
        return ms;
    }

    // Graph-replayed time of one layer's launches alone (layer = 0 .. n_layers - 1) or
    // of the step's head and tail alone (layer = n_layers), T tokens: the layer runs
    // on whatever its input buffers hold (bench: where a step's time goes under
    // graph replay, which kernel traces cannot follow).
    float time_layer(int layer, int T, int iters) {
        RL_REQUIRE(layer >= 0 && layer <= c_.n_layers && iters >= 1 && T >= 1 && T <= tmax_, RL_ERR_RANGE,
                   "time_layer: layer in 0..n_layers, T in 1..max_T");
        RL_REQUIRE(fold_norm_ || kq_fold_, RL_ERR_UNSUPPORTED, "time_layer: folded-norm steps only");
        struct Reset {
            int& v;
            ~Reset() { v = -1; }
        } reset{only_layer_};
        only_layer_ = layer;
        hipEvent_t a, b;
        RL_HIP(hipEventCreate(&a));
        RL_HIP(hipEventCreate(&b));
        const int key = kKeyLayer + layer * 16 + T;
        launch_captured(key, [&] { step(T, T == 1 ? 1 : 0, false); });  // recorded outside the timing
        RL_HIP(hipEventRecord(a, st_));
        for (int i = 0; i < iters; ++i) launch_captured(key, [&] { step(T, T == 1 ? 1 : 0, false); });
        RL_HIP(hipEventRecord(b, st_));
        RL_HIP(hipEventSynchronize(b));
        float ms = 0.f;
        RL_HIP(hipEventElapsedTime(&ms, a, b));
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        return ms / static_cast<float>(iters);
    }

    void* stream() const { return st_; }

    float time_batch(int B, int iters) {
        RL_REQUIRE(B >= 2 && B <= mb_, RL_ERR_RANGE, "time_batch: B must be in 2..max_batch");
        hipEvent_t a, b;
        RL_HIP(hipEventCreate(&a));
        RL_HIP(hipEventCreate(&b));
        RL_HIP(hipEventRecord(a, st_));
        for (int i = 0; i < iters; ++i) launch_captured(kKeyBatch + B, [&] { batch_groups(B); });
        RL_HIP(hipEventRecord(b, st_));
        RL_HIP(hipEventSynchronize(b));
        float ms = 0.f;
        RL_HIP(hipEventElapsedTime(&ms, a, b));
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        return ms;
    }

    // ------------------------------------------------------------ batch decode
    // Slots 0 .. max_batch-1 each hold one sequence (DeltaNet state, conv ring,
    // records, KV cache, scalars); slot 0 is the single-sequence state
    // (cuda_engine.h:46-66).
    int max_batch() const { return mb_; }

    // One token for each of B sequences (slot b at position poss[b]) in one weight
    // pass: the linears run with B rows, DeltaNet and attention over the B slots'
    // states and caches.
    void decode_tokens(const int32_t* tokens, const int* poss, int B) {
        RL_REQUIRE(B >= 1 && B <= mb_ && tokens && poss, RL_ERR_RANGE, "decode_tokens: B out of range");
        check_ids(tokens, B);
        for (int b = 0; b < B; ++b)
            RL_REQUIRE(poss[b] >= 0 && poss[b] < ctx_capacity(), RL_ERR_RANGE, "decode_tokens: position out of range");
        if (B == 1) {  // the single-sequence step, as the reference does
            set_pos(poss[0]);
            decode_token(tokens[0]);
            batch_rows_ = 1;
            return;
        }
        // one staging of tokens and positions (every call ends with a sync)
        std::memcpy(host_in_, tokens, static_cast<size_t>(B) * sizeof(int));
        std::memcpy(host_in_ + kMaxSlots, poss, static_cast<size_t>(B) * sizeof(int));
        RL_HIP(hipMemcpyAsync(tok_, host_in_, static_cast<size_t>(B) * sizeof(int), hipMemcpyHostToDevice, st_));
        for (int b = 0; b < B; ++b)
            RL_HIP(hipMemcpyAsync(scal_ + b * kScalars + kPos, host_in_ + kMaxSlots + b, sizeof(int), hipMemcpyHostToDevice,
                                  st_));
        launch_captured(kKeyBatch + B, [&] { batch_groups(B); });
        RL_HIP(hipMemcpyAsync(host_rb_ + kRbPreds, preds_, kMaxSlots * sizeof(int), hipMemcpyDeviceToHost, st_));
        RL_HIP(hipStreamSynchronize(st_));
        batch_rows_ = B;
    }

    // logits rows of the last decode_tokens (row b = slot b)
    void copy_logits_n(float* host, int B) {
        RL_REQUIRE(host && B >= 1 && B <= batch_rows_, RL_ERR_RANGE, "copy_logits_n: B out of range");
        if (batch_rows_ == 1) {
            copy_logits(host);
            return;
        }
        RL_HIP(hipMemcpyAsync(host, logits_, static_cast<size_t>(B) * c_.vocab * sizeof(float), hipMemcpyDeviceToHost,
                              st_));
        RL_HIP(hipStreamSynchronize(st_));
    }

    void copy_greedy_n(int32_t* host, int B) {
        RL_REQUIRE(host && B >= 1 && B <= batch_rows_, RL_ERR_RANGE, "copy_greedy_n: B out of range");
        if (batch_rows_ == 1) {
            host[0] = greedy_;
            return;
        }
        std::memcpy(host, host_rb_ + kRbPreds, static_cast<size_t>(B) * sizeof(int));
    }

    // Copy slot 0's sequence state into slots 1 .. n_slots-1 (same-prompt batch).
    void replicate_slot0(int n_slots) {
        RL_REQUIRE(n_slots >= 1 && n_slots <= mb_, RL_ERR_RANGE, "replicate_slot0: n_slots out of range");
        sync_graph_state();
        auto copy = [&](void* dst, const void* src, size_t bytes) {
            RL_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, st_));
        };
        for (int b = 1; b < n_slots; ++b) {
            copy(scal_ + b * kScalars, scal_, kScalars * sizeof(int));
            for (size_t l = 0; l < S_.size(); ++l) {
                copy(S_[l] + b * s_bstride_, S_[l], s_bstride_ * sizeof(float));
                copy(conv_[l] + b * conv_bstride_, conv_[l], conv_bstride_ * sizeof(float));
            }
            for (size_t l = 0; l < rec_.size(); ++l) {
                copy(rec_[l] + b * rec_bstride_, rec_[l], rec_bstride_ * sizeof(float));
                copy(rec_n_[l] + b * recn_bstride_, rec_n_[l], recn_bstride_ * sizeof(int));
            }
            if (!kc_.empty()) copy(kc_[0] + b * kv_bstride_, kc_[0], kv_bstride_ * sizeof(uint16_t));
        }
        RL_HIP(hipStreamSynchronize(st_));
    }

    void zero_slots(int n_slots) {
        RL_REQUIRE(n_slots >= 1 && n_slots <= mb_, RL_ERR_RANGE, "zero_slots: n_slots out of range");
        sync_graph_state();
        for (int b = 0; b < n_slots; ++b) zero_slot_state(b);
        RL_HIP(hipStreamSynchronize(st_));
    }

    // Prefill one sequence into slot `slot` (the single-sequence prefill on that
    // slot's state); copy_logits then returns its last row.
    void prefill_slot(const int32_t* ids, int n, int slot) {
        RL_REQUIRE(slot >= 0 && slot < mb_, RL_ERR_RANGE, "prefill_slot: slot out of range");
        cs_ = slot;
        try {
            prefill(ids, n);
        } catch (...) {
            cs_ = 0;
            throw;
        }
        cs_ = 0;
    }

    // Equal-length prompts of B sequences into slots 0 .. B-1 (ids time-major
    // [T][B], the slots zeroed by the caller as Session::generate_batch does,
    // session.cpp:882-893); copy_logits_n / copy_greedy_n then return each slot's
    // row after its last token, and every slot is at position T.
    // T <= B: T batch steps of B rows (one weight pass each); T > B: the chunked
    // prefill of each sequence in its slot (B passes whose GEMMs are compute-bound
    // at prompt lengths: sharing the weight pass would save no arithmetic).
    void prefill_eq_batch(const int32_t* ids, int T, int B) {
        RL_REQUIRE(ids && B >= 2 && B <= mb_ && T >= 1 && T <= ctx_capacity(), RL_ERR_RANGE,
                   "prefill_eq_batch: B must be in 2..max_batch, T in 1..ctx");
        check_ids(ids, T * B);
        if (T <= B) {
            std::vector<int> poss(B);
            for (int t = 0; t < T; ++t) {
                for (int b = 0; b < B; ++b) poss[b] = t;
                decode_tokens(ids + static_cast<size_t>(t) * B, poss.data(), B);
            }
            return;
        }
        std::vector<int32_t> seq(T);
        std::vector<int32_t> preds(B);
        const size_t V = c_.vocab;
        for (int b = 0; b < B; ++b) {
            for (int t = 0; t < T; ++t) seq[t] = ids[static_cast<size_t>(t) * B + b];
            prefill_slot(seq.data(), T, b);
            const int row = n_last_ > 0 ? n_last_ - 1 : 0;
            RL_HIP(hipMemcpyAsync(eq_logits_ + b * V, logits_ + row * V, V * sizeof(float), hipMemcpyDeviceToDevice,
                                  st_));
            preds[b] = greedy_;
        }
        RL_HIP(hipMemcpyAsync(logits_, eq_logits_, B * V * sizeof(float), hipMemcpyDeviceToDevice, st_));
        RL_HIP(hipStreamSynchronize(st_));
        std::memcpy(host_rb_ + kRbPreds, preds.data(), static_cast<size_t>(B) * sizeof(int));
        batch_rows_ = B;
    }

   private:
    static constexpr int kMaxSlots = 16;   // batch slots
    static constexpr int kGroupRows = 16;  // rows of one batch step (FP8 / BF16 linears)
    static constexpr int kKqGroupRows = 16; // rows of one batch step (K-quant GEMV)
    // device scalar block
    enum { kPos = 0, kSlot = 1, kNCons = 2, kNextTok = 3, kGenCount = 4, kScalars = 8 };
    // host readback block (ints): scalars, then preds, then toks
    enum { kRbPreds = 8, kRbToks = 8 + kMaxSlots, kRbInts = 16 + kMaxSlots };
    static constexpr int kGenCap = 4096;
    // K-slices of the residual-add linears (o_proj, out_proj, down): their outputs
    // are partial sums that the next RMSNorm adds to the residual in slice order.
    static constexpr int kSplit = 4;

    RlModelConfig c_;
    int ctx_ = 0, tmax_ = 4, R_ = 5;
    int only_layer_ = -1;  // bench (time_layer): -1 the whole step, i layer i alone, n_layers head and tail
    int mb_ = 1;    // sequences (slots) for batch decode
    int tcap_ = 4;  // activation rows: max(tmax_, one slot group)
    // Batch slots: up to kMaxSlots; a batch step runs them in groups of at most
    // kGroupRows (FP8 / BF16 linears) or kKqGroupRows (K-quant GEMV) rows, one weight
    // pass per group, and gb_ is the first slot of the group being recorded.
    int gb_ = 0;
    int group_rows() const { return kq_fold_ ? kKqGroupRows : kGroupRows; }
    int cs_ = 0;    // slot the single-sequence calls work on (prefill_slot)
    int batch_rows_ = 1;  // rows of the last decode_tokens
    size_t s_bstride_ = 0, conv_bstride_ = 0, rec_bstride_ = 0, kv_bstride_ = 0;
    int recn_bstride_ = 0;
    int* sc() const { return scal_ + cs_ * kScalars; }
    float* slot_S(int l) const { return S_[l] + cs_ * s_bstride_; }
    float* slot_conv(int l) const { return conv_[l] + cs_ * conv_bstride_; }
    float* slot_rec(int l) const { return rec_[l] + cs_ * rec_bstride_; }
    int* slot_recn(int l) const { return rec_n_[l] + cs_ * recn_bstride_; }
    uint16_t* slot_kc(int l) const { return kc_[l] + cs_ * kv_bstride_; }
    uint16_t* slot_vt(int l) const { return vt_[l] + cs_ * kv_bstride_; }
    // the first slot of the batch group being recorded (gb_)
    int* b_scal() const { return scal_ + gb_ * kScalars; }
    float* b_S(int l) const { return S_[l] + gb_ * s_bstride_; }
    float* b_conv(int l) const { return conv_[l] + gb_ * conv_bstride_; }
    float* b_rec(int l) const { return rec_[l] + gb_ * rec_bstride_; }
    int* b_recn(int l) const { return rec_n_[l] + gb_ * recn_bstride_; }
    uint16_t* b_kc(int l) const { return kc_[l] + gb_ * kv_bstride_; }
    uint16_t* b_vt(int l) const { return vt_[l] + gb_ * kv_bstride_; }
    float* b_logits() const { return logits_ + static_cast<size_t>(gb_) * c_.vocab; }
    hipStream_t st_ = nullptr;
    DevAlloc mem_;
    std::map<std::string, const RlTensor*> tab_;
    bool synthetic_ = false;
    int synth_quant_ = RL_Q_FP8_E4M3_B128;  // synthetic layer-linear format
    uint64_t synth_seed_ = 0;
    uint64_t synth_ctr_ = 0;

    std::vector<Layer> L_;
    const void* embed_ = nullptr;
    int embed_kind_ = RL_Q_BF16;
    Lin lm_head_;
    const float* final_norm_ = nullptr;
    bool has_mtp_ = false;
    Lin mtp_fc_;
    const float *mtp_nh_ = nullptr, *mtp_ne_ = nullptr, *mtp_norm_ = nullptr;

    // states
    std::vector<float*> S_, conv_;
    size_t s_slot_ = 0, conv_slot_ = 0;
    std::vector<float*> rec_;   // DeltaNet replay records per layer (head kernel)
    std::vector<int*> rec_n_;
    float* gss_ = nullptr;      // per-head partial sums of o^2 for the folded gated norm
    // in_proj rows past two workgroups per CU (the a/b block) as K-slice partials
    static constexpr int kAbSlices = 8;
    float* abpart_ = nullptr;
    int ab_tile0_ = 0, ab_rows_ = 0;
    std::vector<uint16_t*> kc_, vt_;
    // activations / workspaces
    int* scal_ = nullptr;
    int* tok_ = nullptr;    // [Tmax]
    int* preds_ = nullptr;  // [Tmax]
    int* gen_ = nullptr;    // [kGenCap]
    float* xres_[2] = {nullptr, nullptr};  // [Tmax][H] residual stream (ping-pong)
    float* part_ = nullptr;  // [kSplit][Tmax][H] partial sums of the residual-add linears
    float* x_ = nullptr;     // residual after the last step (set by step())
    float* xn_ = nullptr;   // [Tmax][max_in] fp32 copy of the packed activation
    void* frag_ = nullptr;  // GEMM fragments
    void* frag_h_ = nullptr;  // fragments of the SwiGLU output (input of mlp.down)
    // RMSNorm folded into the GEMMs (all layer linears FP8 / BF16): the residual
    // GEMMs write x in place plus frag_x_ = fragments of x * (1 + next gamma) and
    // ss_ = per-group sums of x^2; the next GEMM scales its outputs by 1/rms.
    bool fold_norm_ = false;
    // K-quant models: the residual GEMVs (out_proj / o_proj / down) add into x and
    // write its per-row-group sums of squares and the next linear's fragments; the
    // consuming linears fold the RMSNorm (KqNorm / NormIO)
    bool kq_fold_ = false;
    float* kq_ss_ = nullptr;  // [kq_norm_groups(H)][Tmax]
    float* xg_ = nullptr;     // [Tmax][H]: x * (1 + gamma) of the next norm
    int kq_groups_ = 0;
    bool gdn_fused_norm_ = false;
    // K-quant models: the DeltaNet kernel writes y = gamma * o * silu(z) rows and the
    // per-head sums of o^2; out_proj applies the per-head 1/rms as it reads them
    bool kq_gnorm_ = false;
    // the fused DeltaNet kernel (one committed state + per-token records): FP8 / BF16
    // models with the gated norm in it (gdn_fused_norm_), K-quant models with it
    // writing o for gnorm_pack
    bool gdn_fused_ = false;
    float* kq_abpart_ = nullptr;  // K-quant models: in_proj a/b rows as K-slice partials
    void* frag_x_ = nullptr;
    float* ss_ = nullptr;  // [add_norm_groups(H)][Tmax]
    float* ybuf_ = nullptr; // [Tmax][max_width] fused projection outputs
    float* o_ = nullptr;    // [Tmax][zdim]
    float* h_ = nullptr;    // [Tmax][I]
    float* g_ = nullptr;    // [Tmax][I] (K-quant MLP)
    float* u_ = nullptr;
    float* logits_ = nullptr;
    float* mtp_logits_ = nullptr;  // [V] (keeps the verify logits intact)
    float* mtp_e_ = nullptr;   // [H]
    float* mtp_cat_ = nullptr; // [2H]
    float* mtp_hp_ = nullptr;  // [H]
    // MTP decoder layer (mtp.layers[0]) and its draft-position KV cache
    static constexpr int kMtpCtx = 256;  // draft positions the cache holds (one chunk)
    Layer mtp_layer_;
    bool has_mtp_layer_ = false;
    int mtp_mode_ = RL_MTP_STEM;
    uint16_t *mtp_kc_ = nullptr, *mtp_vt_ = nullptr;
    void* mtp_attn_ws_ = nullptr;
    size_t mtp_attn_ws_bytes_ = 0;
    int* mtp_pos_ = nullptr;    // [kMtpCtx] = 0, 1, 2, ... (device positions of the drafts)
    float* mtp_x1_ = nullptr;  // [H] residual between the layer's attention and MLP
    float* eq_logits_ = nullptr;  // [max_batch][V]: prefill_eq_batch's last rows
    float* h_last_ = nullptr;
    float* h_prev_ = nullptr;
    void* attn_ws_ = nullptr;
    size_t attn_ws_bytes_ = 0;
    void* arg_ws_ = nullptr;
    void* kq_ws_ = nullptr;
    size_t kq_ws_bytes_ = 0;
    size_t kq_need_ = 0;  // largest K-quant workspace over the loaded linears
    int kq_rows() const { return std::max(tmax_, std::min(mb_, kKqGroupRows)); }
    int max_in_ = 0;

    std::map<int, hipGraphExec_t> graphs_;  // key: T (1..Tmax), 100 + n for MTP drafts
    int* host_rb_ = nullptr;
    // Host inputs (token ids, positions) are staged in pinned memory and uploaded
    // with stream-ordered copies; a call rewrites host_in_ only after its previous
    // call's final stream synchronisation, and the prompt of a prefill is uploaded
    // once to tok_all_ (chunks are fed by device-to-device copies).
    int* host_in_ = nullptr;  // [ctx capacity + 16]
    int* tok_all_ = nullptr;  // device [ctx capacity]
    int pos_ = 0, n_last_ = 0;
    int32_t greedy_ = 0;

    // ---------------------------------------------------------------- build
    template <class Find>
    void build(Find find) {
        const int H = c_.hidden, nk = c_.n_k_heads, nv = c_.n_v_heads, dk = c_.k_dim, dv = c_.v_dim;
        const int conv_dim = 2 * nk * dk + nv * dv, zdim = nv * dv;
        const int nq = c_.n_q, nkv = c_.n_kv, hd = c_.head_dim;
        int I = c_.intermediate;

        // KV caches first, as one block
        {
            int n_attn = 0;
            for (int i = 0; i < c_.n_layers; ++i) n_attn += c_.layer_kind[i] == RL_LAYER_ATTN;
            const size_t kv = static_cast<size_t>(nkv) * ctx_ * hd;
            // slot b's caches follow slot 0's at kv_bstride_
            kv_bstride_ = 2 * kv * n_attn;
            uint16_t* blk = mem_.get_n<uint16_t>(kv_bstride_ * mb_);
            for (int l = 0; l < n_attn; ++l) {
                kc_.push_back(blk + 2 * l * kv);
                vt_.push_back(blk + (2 * l + 1) * kv);
            }
        }

        // embedding / head / final norm
        if (synthetic_) {
            embed_kind_ = RL_Q_BF16;
            uint16_t* e = mem_.get_n<uint16_t>(static_cast<size_t>(c_.vocab) * H);
            fill_normal_bf16(e, static_cast<size_t>(c_.vocab) * H, 0.02f, next_seed(), st_);
            embed_ = e;
            lm_head_ = synth_quant_ == RL_Q_FP8_E4M3_B128 ? synth_lin(RL_Q_BF16, c_.vocab, H)
                                                          : synth_kq(RL_Q_Q6_K, c_.vocab, H);
            final_norm_ = synth_vec(H, 0.f, 0.1f);
        } else {
            const RlTensor* e = need(find, "embed");
            RL_REQUIRE(e->rows == c_.vocab && e->cols == H, RL_ERR_FORMAT, "embed shape");
            if (e->quant == RL_Q_Q8_0 || e->quant == RL_Q_Q4_K || e->quant == RL_Q_Q5_K || e->quant == RL_Q_Q6_K) {
                // block-quantised embedding (GGUF token_embd): dequantised once to an
                // F32 table, exactly as the reference's CUDA engine stores it
                // (cuda_engine.cu:19930-19955); rows are staged through the host in chunks
                const int vals = e->quant == RL_Q_Q8_0 ? 32 : 256;
                const int bsz = e->quant == RL_Q_Q8_0 ? 34 : e->quant == RL_Q_Q4_K ? 144 : e->quant == RL_Q_Q5_K ? 176 : 210;
                RL_REQUIRE(H % vals == 0, RL_ERR_FORMAT, "embed: row length not a whole number of blocks");
                const size_t rowb = static_cast<size_t>(H / vals) * bsz;
                float* ed = mem_.get_n<float>(static_cast<size_t>(c_.vocab) * H);
                const int chunk = 2048;
                std::vector<float> stage(static_cast<size_t>(chunk) * H);
                for (int r0 = 0; r0 < c_.vocab; r0 += chunk) {
                    const int nr = std::min(chunk, c_.vocab - r0);
                    dequant_host(e->quant, static_cast<const uint8_t*>(e->data) + static_cast<size_t>(r0) * rowb,
                                 stage.data(), static_cast<int64_t>(nr) * H);
                    // on the engine stream, behind the zero-fill of `ed`; the stage is
                    // refilled only after the copy has drained
                    RL_HIP(hipMemcpyAsync(ed + static_cast<size_t>(r0) * H, stage.data(), sizeof(float) * nr * H,
                                          hipMemcpyHostToDevice, st_));
                    RL_HIP(hipStreamSynchronize(st_));
                }
                embed_kind_ = RL_Q_F32;
                embed_ = ed;
            } else {
                RL_REQUIRE(e->quant == RL_Q_F32 || e->quant == RL_Q_F16 || e->quant == RL_Q_BF16, RL_ERR_UNSUPPORTED,
                           "embed must be F32, F16, BF16, Q8_0, Q4_K, Q5_K or Q6_K");
                embed_kind_ = e->quant;
                const size_t eb = static_cast<size_t>(c_.vocab) * H * (e->quant == RL_Q_F32 ? 4 : 2);
                void* ed = mem_.get(eb);
                RL_HIP(hipMemcpyAsync(ed, e->data, eb, hipMemcpyHostToDevice, st_));
                embed_ = ed;
            }
            lm_head_ = upload_lin({need(find, "lm_head")}, c_.vocab, H);
            final_norm_ = upload_vec(need(find, "final_norm"), H);
        }

        int nd = 0, na = 0;
        L_.resize(c_.n_layers);
        int max_width = 0;
        for (int i = 0; i < c_.n_layers; ++i) {
            Layer& Ly = L_[i];
            const std::string p = "layers[" + std::to_string(i) + "].";
            Ly.kind = c_.layer_kind[i];
            Ly.attn_norm = synthetic_ ? synth_vec(H, 0.f, 0.1f) : upload_vec(need(find, p + "attn_norm"), H);
            Ly.ffn_norm = synthetic_ ? synth_vec(H, 0.f, 0.1f) : upload_vec(need(find, p + "ffn_norm"), H);
            if (Ly.kind == RL_LAYER_DELTA) {
                Ly.dslot = nd++;
                Ly.off_z = align16(conv_dim);
                Ly.off_a = Ly.off_z + align16(zdim);
                Ly.off_b = Ly.off_a + align16(nv);
                Ly.in_width = Ly.off_b + align16(nv);
                const std::vector<std::string> names = {p + "delta.gemm.in_proj_qkv", p + "delta.gemm.in_proj_z",
                                                        p + "delta.leftover.in_proj_a",
                                                        p + "delta.leftover.in_proj_b"};
                const std::vector<int> rows = {conv_dim, zdim, nv, nv};
                const std::vector<int> offs = {0, Ly.off_z, Ly.off_a, Ly.off_b};
                make_fused(find, names, rows, offs, H, Ly.in_parts, Ly.in_offs);
                Ly.out_proj = synthetic_ ? synth_layer_lin(H, zdim)
                                         : upload_lin({need(find, p + "delta.gemm.out_proj")}, H, zdim);
                if (synthetic_) {
                    Ly.A_log = synth_vec(nv, 0.f, 0.5f);
                    Ly.dt_bias = synth_vec(nv, 0.f, 0.5f);
                    Ly.conv_w = synth_vec(static_cast<size_t>(conv_dim) * c_.conv_k, 0.f, 0.5f);
                    Ly.gnorm = synth_vec(dv, 1.f, 0.1f);
                    Ly.gnorm_n = dv;
                } else {
                    Ly.A_log = upload_vec(need(find, p + "delta.leftover.a_log"), nv);
                    Ly.dt_bias = upload_vec(need(find, p + "delta.leftover.dt_bias"), nv);
                    Ly.conv_w = upload_vec(need(find, p + "delta.leftover.conv1d"),
                                           static_cast<size_t>(conv_dim) * c_.conv_k);
                    const RlTensor* gn = need(find, p + "delta.leftover.norm");
                    Ly.gnorm_n = static_cast<int>(gn->rows * gn->cols);
                    Ly.gnorm = upload_vec(gn, Ly.gnorm_n);
                }
                max_width = std::max(max_width, Ly.in_width);
            } else {
                Ly.aslot = na++;
                build_attn(Ly, p, find);
                max_width = std::max(max_width, Ly.qkv_width);
            }
            build_mlp(Ly, p, find);
        }

        // MTP stem head, and its decoder layer (mtp.layers[0]: attention with its own
        // KV cache + MLP, Session::mtp_layer_step) when the checkpoint has one
        if (c_.has_mtp) {
            has_mtp_ = true;
            if (synthetic_) {
                mtp_fc_ = synth_layer_lin(H, 2 * H);
                mtp_nh_ = synth_vec(H, 0.f, 0.1f);
                mtp_ne_ = synth_vec(H, 0.f, 0.1f);
                mtp_norm_ = synth_vec(H, 0.f, 0.1f);
            } else {
                mtp_fc_ = upload_lin({need(find, "mtp.fc")}, H, 2 * H);
                mtp_nh_ = upload_vec(need(find, "mtp.pre_fc_norm_hidden"), H);
                mtp_ne_ = upload_vec(need(find, "mtp.pre_fc_norm_embedding"), H);
                mtp_norm_ = upload_vec(need(find, "mtp.norm"), H);
            }
            const std::string mp = "mtp.layers[0].";
            if (nq > 0 && hd == 256 && (synthetic_ || find(mp + "attn.wq"))) {
                Layer& Ly = mtp_layer_;
                Ly.kind = RL_LAYER_ATTN;
                Ly.attn_norm = synthetic_ ? synth_vec(H, 0.f, 0.1f) : upload_vec(need(find, mp + "attn_norm"), H);
                Ly.ffn_norm = synthetic_ ? synth_vec(H, 0.f, 0.1f) : upload_vec(need(find, mp + "ffn_norm"), H);
                build_attn(Ly, mp, find);
                build_mlp(Ly, mp, find);
                max_width = std::max(max_width, Ly.qkv_width);
                // fp16 K / V of the draft positions, in the decode cache layout
                const size_t kv = static_cast<size_t>(nkv) * kMtpCtx * hd;
                mtp_kc_ = mem_.get_n<uint16_t>(2 * kv);
                mtp_vt_ = mtp_kc_ + kv;
                mtp_attn_ws_bytes_ = attn_workspace_bytes(nkv, kMtpCtx);
                mtp_attn_ws_ = mem_.get(mtp_attn_ws_bytes_);
                mtp_pos_ = mem_.get_n<int>(kMtpCtx);
                std::vector<int> iota(kMtpCtx);
                for (int i = 0; i < kMtpCtx; ++i) iota[i] = i;
                RL_HIP(hipMemcpyAsync(mtp_pos_, iota.data(), sizeof(int) * kMtpCtx, hipMemcpyHostToDevice, st_));
                RL_HIP(hipStreamSynchronize(st_));
                has_mtp_layer_ = true;
            }
        }

        // states (the recurrent state S is allocated below, once the kernel is chosen)
        s_slot_ = static_cast<size_t>(nv) * dv * dk;
        conv_slot_ = static_cast<size_t>(conv_dim) * c_.conv_k;
        conv_bstride_ = conv_slot_ * R_;  // a ring of R windows per layer and slot
        for (int l = 0; l < nd; ++l) conv_.push_back(mem_.get_n<float>(conv_bstride_ * mb_));
        RL_REQUIRE(static_cast<int>(kc_.size()) == na, RL_ERR_INTERNAL, "engine: attention layer count");

        // activations
        const int T = tcap_;  // rows: verify tokens or batch sequences
        max_in_ = std::max({H, zdim, nq * hd, I, 2 * H});
        scal_ = mem_.get_n<int>(static_cast<size_t>(kScalars) * mb_);  // one block per slot
        tok_ = mem_.get_n<int>(kMaxSlots);
        preds_ = mem_.get_n<int>(kMaxSlots);
        gen_ = mem_.get_n<int>(kGenCap);
        xres_[0] = mem_.get_n<float>(static_cast<size_t>(T) * H);
        xres_[1] = mem_.get_n<float>(static_cast<size_t>(T) * H);
        part_ = mem_.get_n<float>(static_cast<size_t>(kSplit) * T * H);
        xn_ = mem_.get_n<float>(static_cast<size_t>(T) * max_in_);
        frag_ = mem_.get(act_frag_bytes(max_in_, T));
        frag_h_ = mem_.get(act_frag_bytes(I, T));
        frag_x_ = mem_.get(act_frag_bytes(H, T));
        ss_ = mem_.get_n<float>(static_cast<size_t>(add_norm_groups(H)) * T);
        // RL_FOLD_NORM=0 keeps the separate RMSNorm kernels (for A/B measurement)
        const char* fold_env = std::getenv("RL_FOLD_NORM");
        fold_norm_ = can_fold_norm() && !(fold_env && fold_env[0] == '0');
        kq_fold_ = !fold_norm_ && can_fold_kquant() && !(fold_env && fold_env[0] == '0');
        if (kq_fold_) {
            kq_groups_ = kq_norm_groups(H);
            kq_ss_ = mem_.get_n<float>(static_cast<size_t>(kq_groups_) * T);
            xg_ = mem_.get_n<float>(static_cast<size_t>(T) * H);
            kq_abpart_ = mem_.get_n<float>(static_cast<size_t>(kAbSlices) * T * 2 * align16(nv));
        }
        // per-head gated norm (gamma of dv values, zdim >= 256: ops.cpp:129-156) in the
        // DeltaNet kernel, when one workgroup can hold a head
        {
            const int zd = c_.n_v_heads * c_.v_dim;
            bool per_head = gdn_fused_supported(c_.k_dim, c_.v_dim, c_.conv_k) && c_.v_dim == 128 && zd >= 256;
            for (const Layer& Ly : L_)
                if (Ly.kind == RL_LAYER_DELTA && Ly.gnorm_n != c_.v_dim) per_head = false;
            gdn_fused_norm_ = fold_norm_ && per_head;
            gdn_fused_ = gdn_fused_norm_ ||
                         (kq_fold_ && nd > 0 && gdn_fused_supported(c_.k_dim, c_.v_dim, c_.conv_k) && tmax_ <= 8);
            kq_gnorm_ = kq_fold_ && gdn_fused_ && per_head;
        }
        // one committed S per layer plus R banks of per-token records with the fused
        // kernel, a ring of R states with the unfused one
        // batch decode runs the folded-norm steps with B rows: FP8/BF16 linears
        // (step_batch) or K-quant linears (step_kq_folded, at most 16 rows), and with
        // DeltaNet layers the fused DeltaNet kernel over the slots' states
        RL_REQUIRE(mb_ == 1 || (fold_norm_ && (gdn_fused_norm_ || nd == 0)) ||
                       (kq_fold_ && tmax_ <= kKqGroupRows && (gdn_fused_ || nd == 0)),
                   RL_ERR_UNSUPPORTED,
                   "engine: batch decode needs folded norms: FP8/BF16 linears (v_dim 128 for DeltaNet), or "
                   "K-quant linears with max_T <= 8 and the fused DeltaNet kernel");
        s_bstride_ = s_slot_ * (gdn_fused_ ? 1 : R_);
        rec_bstride_ = static_cast<size_t>(R_) * tmax_ * nv * kGdnRecFloats;
        recn_bstride_ = R_ * nv;
        for (int l = 0; l < nd; ++l) {
            S_.push_back(mem_.get_n<float>(s_bstride_ * mb_));
            if (gdn_fused_) {
                rec_.push_back(mem_.get_n<float>(rec_bstride_ * mb_));
                rec_n_.push_back(mem_.get_n<int>(static_cast<size_t>(recn_bstride_) * mb_));
            }
        }
        gss_ = mem_.get_n<float>(static_cast<size_t>(nv) * tcap_ * 4);
        // in_proj = [qkv; z; a; b]: when the qkv and z rows fill whole rounds of two
        // workgroups per CU and the a/b block would run as a short round of its own,
        // the a/b rows are computed as K-slices by the first workgroups
        if (gdn_fused_norm_ && nd > 0) {
            const Layer* d0 = nullptr;
            for (const Layer& Ly : L_)
                if (Ly.kind == RL_LAYER_DELTA) d0 = &Ly;
            const int m_tiles = d0->in_parts[0].m / 16, n_kb = (H + 127) / 128;
            const int tile0 = d0->off_a / 16;
            const int rpw = gemm_store_rows_per_wg(), slots = 2 * device_cus();
            const int wg0 = tile0 / rpw;
            if (d0->in_parts[0].kind == RL_Q_FP8_E4M3_B128 && tile0 < m_tiles && d0->off_a % (16 * rpw) == 0 &&
                wg0 % slots == 0 && (m_tiles - tile0) * kAbSlices <= wg0 &&
                (n_kb + kAbSlices - 1) / kAbSlices <= gemm_store_waves() && d0->in_width == m_tiles * 16) {
                ab_tile0_ = tile0;
                ab_rows_ = (m_tiles - tile0) * 16;
                abpart_ = mem_.get_n<float>(static_cast<size_t>(kAbSlices) * tcap_ * ab_rows_);
            }
        }
        ybuf_ = mem_.get_n<float>(static_cast<size_t>(T) * std::max(max_width, 16));
        o_ = mem_.get_n<float>(static_cast<size_t>(T) * std::max(zdim, nq * hd));
        h_ = mem_.get_n<float>(static_cast<size_t>(T) * I);
        g_ = mem_.get_n<float>(static_cast<size_t>(T) * I);
        u_ = mem_.get_n<float>(static_cast<size_t>(T) * I);
        logits_ = mem_.get_n<float>(static_cast<size_t>(std::max(T, mb_)) * c_.vocab);
        if (mb_ > 1) eq_logits_ = mem_.get_n<float>(static_cast<size_t>(mb_) * c_.vocab);
        mtp_logits_ = mem_.get_n<float>(c_.vocab);
        mtp_e_ = mem_.get_n<float>(H);
        mtp_cat_ = mem_.get_n<float>(2 * static_cast<size_t>(H));
        mtp_hp_ = mem_.get_n<float>(H);
        mtp_x1_ = mem_.get_n<float>(H);
        h_last_ = mem_.get_n<float>(H);
        h_prev_ = mem_.get_n<float>(H);
        // one workspace per batch slot (batch decode runs all slots' attention at once)
        attn_ws_bytes_ = attn_workspace_bytes(std::max(nkv, 1), ctx_) * mb_;
        attn_ws_ = mem_.get(attn_ws_bytes_);
        arg_ws_ = mem_.get(argmax_workspace_bytes(T, c_.vocab));
        kq_ws_bytes_ = std::max<size_t>(kq_need_, 256);
        kq_ws_ = mem_.get(kq_ws_bytes_);
        RL_HIP(hipHostMalloc(reinterpret_cast<void**>(&host_rb_), kRbInts * sizeof(int), hipHostMallocDefault));
        RL_HIP(hipHostMalloc(reinterpret_cast<void**>(&host_in_), (static_cast<size_t>(ctx_capacity()) + 16) * sizeof(int),
                             hipHostMallocDefault));
        tok_all_ = mem_.get_n<int>(static_cast<size_t>(ctx_capacity()) + 16);
        RL_HIP(hipStreamSynchronize(st_));
        tab_.clear();
    }

    // Attention projections of a gated-attention layer: q|gate, k, v as one fused
    // linear, o_proj, the q / k head norms (weights under prefix p).
    template <class Find>
    void build_attn(Layer& Ly, const std::string& p, Find& find) {
        const int H = c_.hidden, nq = c_.n_q, nkv = c_.n_kv, hd = c_.head_dim;
        Ly.qkv_width = 2 * nq * hd + 2 * nkv * hd;
        const std::vector<std::string> names = {p + "attn.wq", p + "attn.wk", p + "attn.wv"};
        const std::vector<int> rows = {2 * nq * hd, nkv * hd, nkv * hd};
        const std::vector<int> offs = {0, 2 * nq * hd, 2 * nq * hd + nkv * hd};
        make_fused(find, names, rows, offs, H, Ly.qkv_parts, Ly.qkv_offs);
        Ly.o_proj = synthetic_ ? synth_layer_lin(H, nq * hd) : upload_lin({need(find, p + "attn.wo")}, H, nq * hd);
        Ly.q_norm = synthetic_ ? synth_vec(hd, 0.f, 0.1f) : upload_vec(need(find, p + "attn.q_norm"), hd);
        Ly.k_norm = synthetic_ ? synth_vec(hd, 0.f, 0.1f) : upload_vec(need(find, p + "attn.k_norm"), hd);
    }

    // MLP of a layer: gate/up in half tiles (FP8 / BF16) or as K-quant parts, down.
    template <class Find>
    void build_mlp(Layer& Ly, const std::string& p, Find& find) {
        const int H = c_.hidden;
        int I = c_.intermediate;
        if (synthetic_ && synth_quant_ != RL_Q_FP8_E4M3_B128) {
            Ly.gate = synth_kq(synth_quant_, 2 * I, H);
            Ly.gate_cat = true;
            Ly.down = synth_kq(synth_quant_, H, I);
        } else if (synthetic_) {
            Ly.gate_up = synth_gate_up(I, H);
            Ly.down = synth_lin(RL_Q_FP8_E4M3_B128, H, I);
        } else {
            const RlTensor* g = need(find, p + "mlp.gate");
            const RlTensor* u = need(find, p + "mlp.up");
            const RlTensor* d = need(find, p + "mlp.down");
            I = static_cast<int>(d->cols);
            RL_REQUIRE(I == c_.intermediate, RL_ERR_FORMAT, "mlp.down shape disagrees with intermediate");
            if (g->quant == u->quant && (g->quant == RL_Q_FP8_E4M3_B128 || g->quant == RL_Q_BF16)) {
                Ly.gate_up = upload_gate_up(g, u, I, H);
            } else if (g->quant == u->quant && (g->quant == RL_Q_Q4_K || g->quant == RL_Q_Q6_K) && I % 64 == 0) {
                // one K-quant launch for gate and up over half tiles (8 gate rows,
                // then the same 8 up rows), writing h = silu(gate) * up
                Ly.gate = upload_kq_cat(g, u, I, H);
                Ly.gate_cat = true;
            } else {
                Ly.gate = upload_lin({g}, I, H);
                Ly.up = upload_lin({u}, I, H);
            }
            Ly.down = upload_lin({d}, H, I);
        }
    }

    template <class Find>
    const RlTensor* need(Find& find, const std::string& name) {
        const RlTensor* t = find(name);
        if (!t) throw Error(RL_ERR_FORMAT, "missing weight " + name);
        return t;
    }

    uint64_t next_seed() { return synth_seed_ * 0x9E3779B97F4A7C15ull + (++synth_ctr_) * 0xD1B54A32D192ED03ull; }

    const float* upload_vec(const RlTensor* t, size_t n) {
        RL_REQUIRE(t->quant == RL_Q_F32, RL_ERR_UNSUPPORTED, std::string(t->name) + ": expected F32");
        RL_REQUIRE(static_cast<size_t>(t->rows * t->cols) == n, RL_ERR_FORMAT, std::string(t->name) + ": shape");
        float* d = mem_.get_n<float>(n);
        RL_HIP(hipMemcpyAsync(d, t->data, n * sizeof(float), hipMemcpyHostToDevice, st_));
        return d;
    }

    const float* synth_vec(size_t n, float mean, float stdv) {
        float* d = mem_.get_n<float>(n);
        fill_normal_f32(d, n, mean, stdv, next_seed(), st_);
        return d;
    }

    static size_t lin_bytes(int kind, int m_pad, int n) {
        const size_t nkb = (n + 127) / 128;
        if (kind == RL_Q_FP8_E4M3_B128) return static_cast<size_t>(m_pad) * nkb * 128;
        return static_cast<size_t>(m_pad) * nkb * 256;  // BF16
    }

    // Upload one (or several row-concatenated, 16-row aligned) FP8 / BF16 matrices.
    void place_dense(Lin& L, const RlTensor* t, int rows, int n, int rt_stride, int rt_offset) {
        RL_REQUIRE(t->rows == rows && t->cols == n, RL_ERR_FORMAT, std::string(t->name) + ": shape mismatch");
        if (L.kind == RL_Q_FP8_E4M3_B128) {
            RL_REQUIRE(t->scale != nullptr, RL_ERR_FORMAT, std::string(t->name) + ": FP8 weight without scale");
            const size_t wb = static_cast<size_t>(rows) * n;
            const size_t sb = static_cast<size_t>((rows + 127) / 128) * ((n + 127) / 128) * 4;
            uint8_t* tmp = nullptr;
            float* stmp = nullptr;
            RL_HIP(hipMalloc(&tmp, wb));
            RL_HIP(hipMalloc(&stmp, sb));
            RL_HIP(hipMemcpyAsync(tmp, t->data, wb, hipMemcpyHostToDevice, st_));
            RL_HIP(hipMemcpyAsync(stmp, t->scale, sb, hipMemcpyHostToDevice, st_));
            pack_fp8_rows(tmp, stmp, L.w, L.ts, rows, n, rt_stride, rt_offset, st_);
            RL_HIP(hipStreamSynchronize(st_));
            (void)hipFree(tmp);
            (void)hipFree(stmp);
        } else {
            const size_t wb = static_cast<size_t>(rows) * n * 2;
            uint16_t* tmp = nullptr;
            RL_HIP(hipMalloc(&tmp, wb));
            RL_HIP(hipMemcpyAsync(tmp, t->data, wb, hipMemcpyHostToDevice, st_));
            pack_bf16_rows(tmp, reinterpret_cast<uint16_t*>(L.w), rows, n, rt_stride, rt_offset, st_);
            RL_HIP(hipStreamSynchronize(st_));
            (void)hipFree(tmp);
        }
    }

    Lin alloc_dense(int kind, int m_pad, int n) {
        Lin L;
        L.kind = kind;
        L.m = m_pad;
        L.n = n;
        L.w = static_cast<uint8_t*>(mem_.get(lin_bytes(kind, m_pad, n)));
        if (kind == RL_Q_FP8_E4M3_B128) L.ts = mem_.get_n<float>(static_cast<size_t>(m_pad / 16) * ((n + 127) / 128));
        return L;
    }

    Lin upload_lin(std::vector<const RlTensor*> ts, int rows, int n) {
        const RlTensor* t = ts[0];
        if (t->quant == RL_Q_FP8_E4M3_B128 || t->quant == RL_Q_BF16) {
            Lin L = alloc_dense(t->quant, align16(rows), n);
            place_dense(L, t, rows, n, 1, 0);
            return L;
        }
        RL_REQUIRE(t->quant == RL_Q_Q4_K || t->quant == RL_Q_Q6_K, RL_ERR_UNSUPPORTED,
                   std::string(t->name) + ": linear must be FP8_E4M3_B128, BF16, Q4_K or Q6_K");
        RL_REQUIRE(t->rows == rows && t->cols == n && n % 256 == 0, RL_ERR_FORMAT, std::string(t->name) + ": shape");
        Lin L;
        L.kind = t->quant;
        L.m = rows;
        L.n = n;
        kq_need_ = std::max(kq_need_, kq_workspace_bytes(rows, n, kq_rows()));
        const size_t tb = rl_hip_kquant_tiled_bytes(t->quant, rows, n);
        L.w = static_cast<uint8_t*>(mem_.get(tb));
        const size_t bb = static_cast<size_t>(rows) * (n / 256) * (t->quant == RL_Q_Q4_K ? 144 : 210);
        uint8_t* tmp = nullptr;
        RL_HIP(hipMalloc(&tmp, bb));
        RL_HIP(hipMemcpyAsync(tmp, t->data, bb, hipMemcpyHostToDevice, st_));
        const int rc = rl_hip_pack_kquant(t->quant, tmp, L.w, rows, n, st_);
        RL_HIP(hipStreamSynchronize(st_));
        (void)hipFree(tmp);
        if (rc != RL_OK) throw Error(rc, rl_hip_last_error());
        return L;
    }

    // Fused linear over several weights sharing the input: one tiled matrix when
    // all parts are FP8 or all BF16 (parts start on 16-row boundaries = the output
    // column offsets), else one Lin per part.
    template <class Find>
    void make_fused(Find& find, const std::vector<std::string>& names, const std::vector<int>& rows,
                    const std::vector<int>& offs, int n, std::vector<Lin>& parts, std::vector<int>& out_offs) {
        const int total = offs.back() + align16(rows.back());
        // every part's tiles start at its output offset / 16, and a K-quant launch
        // writes align16(rows) outputs: offsets must sit on 16-row boundaries
        for (size_t k = 0; k < offs.size(); ++k)
            RL_REQUIRE(offs[k] % 16 == 0 && (k == 0 || offs[k] >= offs[k - 1] + align16(rows[k - 1])),
                       RL_ERR_INTERNAL, "engine: fused linear part offsets must be 16-row aligned");
        if (synthetic_ && synth_quant_ != RL_Q_FP8_E4M3_B128) {
            parts.clear();
            out_offs.clear();
            for (size_t k = 0; k < rows.size(); ++k) {
                // DeltaNet a / b rows (a few dozen) stay BF16, as in K-quant files,
                // and share one BF16 matrix (one launch)
                const bool small = rows[k] < 256;
                size_t e = k + 1;
                while (e < rows.size() && (rows[e] < 256) == small) ++e;
                const int total_k = offs[e - 1] - offs[k] + (small ? rows[e - 1] : align16(rows[e - 1]));
                parts.push_back(small ? synth_lin(RL_Q_BF16, total_k, n) : synth_kq(synth_quant_, total_k, n));
                out_offs.push_back(offs[k]);
                k = e - 1;
            }
            return;
        }
        if (synthetic_) {
            Lin L = alloc_dense(RL_Q_FP8_E4M3_B128, total, n);
            synth_fill_dense(L, total, n);
            parts = {L};
            out_offs = {0};
            return;
        }
        std::vector<const RlTensor*> ts;
        for (auto& nm : names) ts.push_back(need(find, nm));
        bool same = true;
        for (auto* t : ts) same = same && t->quant == ts[0]->quant;
        if (same && (ts[0]->quant == RL_Q_FP8_E4M3_B128 || ts[0]->quant == RL_Q_BF16)) {
            Lin L = alloc_dense(ts[0]->quant, total, n);
            for (size_t k = 0; k < ts.size(); ++k) place_dense(L, ts[k], rows[k], n, 1, offs[k] / 16);
            parts = {L};
            out_offs = {0};
            return;
        }
        // mixed formats: consecutive FP8 / BF16 parts of one format still share one
        // tiled matrix (e.g. the BF16 a / b rows beside K-quant q|k|v and z)
        parts.clear();
        out_offs.clear();
        for (size_t k = 0; k < ts.size();) {
            const int q = ts[k]->quant;
            size_t e = k + 1;
            while (e < ts.size() && ts[e]->quant == q) ++e;
            if (e - k > 1 && (q == RL_Q_Q4_K || q == RL_Q_Q6_K)) {
                // consecutive K-quant parts of one type: one tiled matrix, each part's
                // 16-row tiles at its (16-row aligned) output offset
                const int base = offs[k];
                Lin L;
                L.kind = q;
                L.m = offs[e - 1] - base + align16(rows[e - 1]);
                L.n = n;
                kq_need_ = std::max(kq_need_, kq_workspace_bytes(L.m, n, kq_rows()));
                L.w = static_cast<uint8_t*>(mem_.get(rl_hip_kquant_tiled_bytes(q, L.m, n)));
                const size_t tile_row_bytes = rl_hip_kquant_tiled_bytes(q, 16, n);
                for (size_t j = k; j < e; ++j) {
                    const RlTensor* t = ts[j];
                    RL_REQUIRE(t->rows == rows[j] && t->cols == n && n % 256 == 0, RL_ERR_FORMAT,
                               std::string(t->name) + ": shape");
                    const size_t bb = static_cast<size_t>(rows[j]) * (n / 256) * (q == RL_Q_Q4_K ? 144 : 210);
                    uint8_t* tmp = nullptr;
                    RL_HIP(hipMalloc(&tmp, bb));
                    RL_HIP(hipMemcpyAsync(tmp, t->data, bb, hipMemcpyHostToDevice, st_));
                    const int rc = rl_hip_pack_kquant(q, tmp, L.w + static_cast<size_t>((offs[j] - base) / 16) * tile_row_bytes,
                                                      rows[j], n, st_);
                    RL_HIP(hipStreamSynchronize(st_));
                    (void)hipFree(tmp);
                    if (rc != RL_OK) throw Error(rc, rl_hip_last_error());
                }
                parts.push_back(L);
            } else if (e - k > 1 && (q == RL_Q_FP8_E4M3_B128 || q == RL_Q_BF16)) {
                const int base = offs[k];
                Lin L = alloc_dense(q, offs[e - 1] - base + align16(rows[e - 1]), n);
                for (size_t j = k; j < e; ++j) place_dense(L, ts[j], rows[j], n, 1, (offs[j] - base) / 16);
                parts.push_back(L);
            } else {
                parts.push_back(upload_lin({ts[k]}, rows[k], n));
            }
            out_offs.push_back(offs[k]);
            k = e;
        }
    }

    // Gate and up in half tiles (tile k: gate rows 8k..8k+7, then up rows), each half
    // with its own block scale; whole-tile interleave when I is not a multiple of 8.
    Lin upload_gate_up(const RlTensor* g, const RlTensor* u, int I, int H) {
        if (I % 8 != 0) {
            const int tiles = (I + 15) / 16;
            Lin L = alloc_dense(g->quant, 2 * tiles * 16, H);
            place_dense(L, g, I, H, 2, 0);
            place_dense(L, u, I, H, 2, 1);
            return L;
        }
        for (const RlTensor* t : {g, u})
            RL_REQUIRE(t->rows == I && t->cols == H, RL_ERR_FORMAT, std::string(t->name) + ": shape mismatch");
        Lin L = alloc_guh(g->quant, I, H);
        const size_t wb = static_cast<size_t>(I) * H * (g->quant == RL_Q_FP8_E4M3_B128 ? 1 : 2);
        const size_t sb = static_cast<size_t>((I + 127) / 128) * ((H + 127) / 128) * 4;
        uint8_t *tg = nullptr, *tu = nullptr;
        float *sg = nullptr, *su = nullptr;
        RL_HIP(hipMalloc(&tg, wb));
        RL_HIP(hipMalloc(&tu, wb));
        RL_HIP(hipMemcpyAsync(tg, g->data, wb, hipMemcpyHostToDevice, st_));
        RL_HIP(hipMemcpyAsync(tu, u->data, wb, hipMemcpyHostToDevice, st_));
        if (g->quant == RL_Q_FP8_E4M3_B128) {
            RL_REQUIRE(g->scale && u->scale, RL_ERR_FORMAT, std::string(g->name) + ": FP8 weight without scale");
            RL_HIP(hipMalloc(&sg, sb));
            RL_HIP(hipMalloc(&su, sb));
            RL_HIP(hipMemcpyAsync(sg, g->scale, sb, hipMemcpyHostToDevice, st_));
            RL_HIP(hipMemcpyAsync(su, u->scale, sb, hipMemcpyHostToDevice, st_));
            pack_fp8_gate_up(tg, sg, tu, su, L.w, L.ts, I, H, st_);
        } else {
            pack_bf16_gate_up(reinterpret_cast<const uint16_t*>(tg), reinterpret_cast<const uint16_t*>(tu),
                              reinterpret_cast<uint16_t*>(L.w), I, H, st_);
        }
        RL_HIP(hipStreamSynchronize(st_));
        for (void* p : {static_cast<void*>(tg), static_cast<void*>(tu), static_cast<void*>(sg), static_cast<void*>(su)})
            if (p) (void)hipFree(p);
        return L;
    }

    Lin alloc_guh(int kind, int I, int n) {
        Lin L;
        L.kind = kind;
        L.m = 2 * I;
        L.n = n;
        L.guh = true;
        L.w = static_cast<uint8_t*>(mem_.get(lin_bytes(kind, 2 * I, n)));
        if (kind == RL_Q_FP8_E4M3_B128) L.ts = mem_.get_n<float>(rl_hip_fp8_gate_up_tile_scales(I, n));
        return L;
    }

    void synth_fill_dense(Lin& L, int rows, int n) {
        // random row-major source, then the same packing path as loaded weights
        if (L.kind == RL_Q_FP8_E4M3_B128) {
            const size_t wb = static_cast<size_t>(rows) * n;
            const size_t ns = static_cast<size_t>((rows + 127) / 128) * ((n + 127) / 128);
            uint8_t* tmp = nullptr;
            float* stmp = nullptr;
            RL_HIP(hipMalloc(&tmp, wb));
            RL_HIP(hipMalloc(&stmp, ns * 4));
            fill_fp8(tmp, wb, next_seed(), st_);
            fill_loguniform(stmp, ns, 1e-3f, 1e-1f, next_seed(), st_);
            pack_fp8_rows(tmp, stmp, L.w, L.ts, rows, n, 1, 0, st_);
            RL_HIP(hipStreamSynchronize(st_));
            (void)hipFree(tmp);
            (void)hipFree(stmp);
        } else {
            const size_t ne = static_cast<size_t>(rows) * n;
            uint16_t* tmp = nullptr;
            RL_HIP(hipMalloc(&tmp, ne * 2));
            fill_normal_bf16(tmp, ne, 0.02f, next_seed(), st_);
            pack_bf16_rows(tmp, reinterpret_cast<uint16_t*>(L.w), rows, n, 1, 0, st_);
            RL_HIP(hipStreamSynchronize(st_));
            (void)hipFree(tmp);
        }
    }

    Lin upload_kq_cat(const RlTensor* g, const RlTensor* u, int I, int H) {
        RL_REQUIRE(g->rows == I && u->rows == I && g->cols == H && u->cols == H && H % 256 == 0, RL_ERR_FORMAT,
                   std::string(g->name) + ": shape");
        Lin L;
        L.kind = g->quant;
        L.m = 2 * I;
        L.n = H;
        kq_need_ = std::max(kq_need_, kq_workspace_bytes(2 * I, H, kq_rows()));
        L.w = static_cast<uint8_t*>(mem_.get(rl_hip_kquant_tiled_bytes(g->quant, 2 * I, H)));
        const size_t bb = static_cast<size_t>(I) * (H / 256) * (g->quant == RL_Q_Q4_K ? 144 : 210);
        uint8_t* tmp = nullptr;
        RL_HIP(hipMalloc(&tmp, 2 * bb));
        RL_HIP(hipMemcpyAsync(tmp, g->data, bb, hipMemcpyHostToDevice, st_));
        RL_HIP(hipMemcpyAsync(tmp + bb, u->data, bb, hipMemcpyHostToDevice, st_));
        const int rc = rl_hip_pack_kquant_gate_up(g->quant, tmp, tmp + bb, L.w, I, H, st_);
        RL_HIP(hipStreamSynchronize(st_));
        if (rc != RL_OK) {
            (void)hipFree(tmp);
            throw Error(rc, rl_hip_last_error());
        }
        (void)hipFree(tmp);
        return L;
    }

    Lin synth_kq(int type, int rows, int n) {
        RL_REQUIRE(n % 256 == 0, RL_ERR_UNSUPPORTED, "synthetic K-quant: columns must be a multiple of 256");
        Lin L;
        L.kind = type;
        L.m = rows;
        L.n = n;
        kq_need_ = std::max(kq_need_, kq_workspace_bytes(rows, n, kq_rows()));
        L.w = static_cast<uint8_t*>(mem_.get(rl_hip_kquant_tiled_bytes(type, rows, n)));
        const size_t nb = static_cast<size_t>(rows) * (n / 256);
        uint8_t* tmp = nullptr;
        RL_HIP(hipMalloc(&tmp, nb * (type == RL_Q_Q4_K ? 144 : 210)));
        fill_kquant(tmp, type, nb, next_seed(), st_);
        const int rc = rl_hip_pack_kquant(type, tmp, L.w, rows, n, st_);
        RL_HIP(hipStreamSynchronize(st_));
        (void)hipFree(tmp);
        if (rc != RL_OK) throw Error(rc, rl_hip_last_error());
        return L;
    }

    Lin synth_layer_lin(int rows, int n) {
        return synth_quant_ == RL_Q_FP8_E4M3_B128 ? synth_lin(RL_Q_FP8_E4M3_B128, rows, n)
                                                  : synth_kq(synth_quant_, rows, n);
    }

    Lin synth_lin(int kind, int rows, int n) {
        Lin L = alloc_dense(kind, align16(rows), n);
        synth_fill_dense(L, rows, n);
        return L;
    }

    Lin synth_gate_up(int I, int H) {
        // gate and up each random like a loaded matrix, then packed into half tiles
        RL_REQUIRE(I % 8 == 0, RL_ERR_UNSUPPORTED, "synthetic model: intermediate must be a multiple of 8");
        Lin L = alloc_guh(RL_Q_FP8_E4M3_B128, I, H);
        const size_t wb = static_cast<size_t>(I) * H;
        const size_t ns = static_cast<size_t>((I + 127) / 128) * ((H + 127) / 128);
        uint8_t* tmp[2] = {};
        float* stmp[2] = {};
        for (int half = 0; half < 2; ++half) {
            RL_HIP(hipMalloc(&tmp[half], wb));
            RL_HIP(hipMalloc(&stmp[half], ns * 4));
            fill_fp8(tmp[half], wb, next_seed(), st_);
            fill_loguniform(stmp[half], ns, 1e-3f, 1e-1f, next_seed(), st_);
        }
        pack_fp8_gate_up(tmp[0], stmp[0], tmp[1], stmp[1], L.w, L.ts, I, H, st_);
        RL_HIP(hipStreamSynchronize(st_));
        for (int half = 0; half < 2; ++half) {
            (void)hipFree(tmp[half]);
            (void)hipFree(stmp[half]);
        }
        return L;
    }

    void check_ids(const int32_t* ids, int n) const {
        for (int i = 0; i < n; ++i)
            if (ids[i] < 0 || ids[i] >= c_.vocab) throw Error(RL_ERR_RANGE, "token id out of range");
    }

    // ---------------------------------------------------------------- step
    // Linear on the current activation: FP8 / BF16 read the packed fragments frag_,
    // K-quants read the fp32 rows x32 (the same values, written by the producer).
    void linear(const Lin& L, const float* x32, float* Y, int ldy, int m_valid, int T, int epi) {
        if (L.kind == RL_Q_FP8_E4M3_B128)
            gemm_fp8_frag(L.w, L.ts, frag_, Y, L.m, L.n, T, epi, ldy, m_valid, st_);
        else if (L.kind == RL_Q_BF16)
            gemm_bf16_frag(reinterpret_cast<const uint16_t*>(L.w), frag_, Y, L.m, L.n, T, epi, ldy, m_valid, st_);
        else
            kq_gemm(L.kind == RL_Q_Q4_K ? 4 : 6, L.w, x32, Y, kq_ws_, kq_ws_bytes_, L.m, L.n, T, epi == kEpiAdd, ldy,
                    st_);
    }

    // Residual-add linear [H rows]: writes partial sums into part_ and returns the
    // number of slices the next residual_rmsnorm_pack must add.
    int linear_residual(const Lin& L, const float* x32, int T, const void* frag_in = nullptr) {
        const int H = c_.hidden;
        const void* fr = frag_in ? frag_in : frag_;
        if (L.kind == RL_Q_FP8_E4M3_B128) {
            gemm_fp8_frag(L.w, L.ts, fr, part_, L.m, L.n, T, kEpiPartial, H, H, st_, kSplit);
            return kSplit;
        }
        if (L.kind == RL_Q_BF16) {
            gemm_bf16_frag(reinterpret_cast<const uint16_t*>(L.w), fr, part_, L.m, L.n, T, kEpiPartial, H, H, st_,
                           kSplit);
            return kSplit;
        }
        linear(L, x32, part_, H, H, T, kEpiStore);
        return 1;
    }

    // x <- x + pending partials (if any), then RMSNorm into xn_ / frag_.
    void norm_residual(int& cur, int& pending, const float* gamma, int T) {
        const int H = c_.hidden;
        if (pending > 0) {
            residual_rmsnorm_pack(xres_[cur], part_, pending, xres_[cur ^ 1], gamma, xn_, frag_, H, T, c_.rms_eps,
                                  st_);
            cur ^= 1;
            pending = 0;
        } else {
            rmsnorm_pack(xres_[cur], H, gamma, xn_, frag_, H, T, c_.rms_eps, st_);
        }
    }

    void linear_parts(const std::vector<Lin>& parts, const std::vector<int>& offs, const float* x32, float* Y,
                      int ldy, int T) {
        for (size_t k = 0; k < parts.size(); ++k) linear(parts[k], x32, Y + offs[k], ldy, parts[k].m, T, kEpiStore);
    }

    static bool frag_kind(const Lin& L) { return L.kind == RL_Q_FP8_E4M3_B128 || L.kind == RL_Q_BF16; }

    // The folded-norm step needs every linear that reads or writes the residual
    // stream on the fragment path, one fused input projection per layer, and an
    // interleaved gate/up; otherwise the step keeps the separate norm kernels.
    bool can_fold_norm() const {
        if (!frag_kind(lm_head_) || add_norm_groups(c_.hidden) > 256 || tmax_ > 8) return false;
        for (const Layer& Ly : L_) {
            const auto& in = Ly.kind == RL_LAYER_DELTA ? Ly.in_parts : Ly.qkv_parts;
            const Lin& res = Ly.kind == RL_LAYER_DELTA ? Ly.out_proj : Ly.o_proj;
            if (in.size() != 1 || !frag_kind(in[0]) || !frag_kind(res) || !frag_kind(Ly.down)) return false;
            if (Ly.gate_up.kind < 0 || !frag_kind(Ly.gate_up)) return false;
        }
        return true;
    }

    static bool is_kq(const Lin& L) { return L.kind == RL_Q_Q4_K || L.kind == RL_Q_Q6_K; }
    static bool known_kind(const Lin& L) { return is_kq(L) || frag_kind(L); }

    // K-quant folded norms: every residual linear a K-quant GEMV (one writer per row
    // of x), every other linear of a known kind, at most 512 row groups of x
    bool can_fold_kquant() const {
        if (tmax_ > 4 || !kq_fold_supported() || kq_norm_groups(c_.hidden) > 512 || !known_kind(lm_head_))
            return false;
        for (const Layer& Ly : L_) {
            const Lin& res = Ly.kind == RL_LAYER_DELTA ? Ly.out_proj : Ly.o_proj;
            if (!is_kq(res) || !is_kq(Ly.down) || res.m != c_.hidden || Ly.down.m != c_.hidden) return false;
            for (const Lin& L : Ly.kind == RL_LAYER_DELTA ? Ly.in_parts : Ly.qkv_parts)
                if (!known_kind(L)) return false;
            if (Ly.gate_up.kind >= 0 ? !frag_kind(Ly.gate_up) : (!is_kq(Ly.gate) || (!Ly.gate_cat && !is_kq(Ly.up))))
                return false;
        }
        return true;
    }

    // RL_AB_IN_KQ=0 keeps the K-quant models' BF16 a/b rows as a launch of their own
    // (A/B measurement)
    static bool ab_rows_in_kq_enabled() {
        static const bool on = [] {
            const char* v = std::getenv("RL_AB_IN_KQ");
            return !(v && v[0] == '0');
        }();
        return on;
    }

    // FP8 / BF16 GEMM on given input fragments.
    void gemm_on(const Lin& L, const void* fr, float* Y, int ldy, int m_valid, int T, int epi,
                 void* frag_out = nullptr, const NormIO* io = nullptr) {
        if (L.kind == RL_Q_FP8_E4M3_B128)
            gemm_fp8_frag(L.w, L.ts, fr, Y, L.m, L.n, T, epi, ldy, m_valid, st_, 1, frag_out, io);
        else
            gemm_bf16_frag(reinterpret_cast<const uint16_t*>(L.w), fr, Y, L.m, L.n, T, epi, ldy, m_valid, st_, 1,
                           frag_out, io);
    }

    // One step with the RMSNorms folded into the GEMMs (see fold_norm_): per layer
    // in_proj/qkv -> mixer -> out/o_proj (+= x) -> gate/up -> down (+= x).
    void step_folded(int T, int force_all, bool feed) {
        const int H = c_.hidden, nk = c_.n_k_heads, nv = c_.n_v_heads, dv = c_.v_dim;
        const int zdim = nv * dv, nq = c_.n_q, nkv = c_.n_kv, hd = c_.head_dim, I = c_.intermediate;
        const float eps = c_.rms_eps;
        float* x = xres_[0];
        const bool ends = only_layer_ < 0 || only_layer_ >= c_.n_layers;  // head and tail of the step
        if (ends) {
            if (feed) copy_int(sc() + kNextTok, tok_, st_);
            embed_rows(embed_, embed_kind_, tok_, x, H, c_.vocab, T, st_);
            rmsnorm_pack(x, H, L_[0].attn_norm, xn_, frag_x_, H, T, eps, st_);
        }
        NormIO in;
        in.ss_in = ss_;
        in.groups_in = add_norm_groups(H);
        in.n_norm = H;
        in.eps = eps;
        for (int i = 0; i < c_.n_layers; ++i) {
            if (only_layer_ >= 0 && i != only_layer_) continue;
            Layer& Ly = L_[i];
            const NormIO* io_in = i == 0 ? nullptr : &in;  // layer 0 reads normalised fragments
            NormIO out;
            out.gamma_out = Ly.ffn_norm;
            out.ss_out = ss_;
            if (Ly.kind == RL_LAYER_DELTA) {
                NormIO in_ab = io_in ? *io_in : NormIO{};
                if (abpart_) {
                    in_ab.xpart = abpart_;
                    in_ab.x_tile0 = ab_tile0_;
                    in_ab.x_slices = kAbSlices;
                    in_ab.x_rows = ab_rows_;
                }
                gemm_on(Ly.in_parts[0], frag_x_, ybuf_, Ly.in_width, Ly.in_parts[0].m, T, kEpiStore, nullptr,
                        abpart_ ? &in_ab : io_in);
                if (gdn_fused_norm_) {
                    // recurrent update + gated RMSNorm's elementwise part + out_proj
                    // packing in one kernel; out_proj applies the per-head 1/rms.  A step
                    // that consumes all its tokens commits S directly.
                    const GdnRecords rec{slot_rec(Ly.dslot), slot_recn(Ly.dslot), sc() + kNCons, tmax_,
                                         T > 1 && !force_all};
                    const float* a_in = abpart_ ? abpart_ : ybuf_ + Ly.off_a;
                    const float* b_in = abpart_ ? abpart_ + (Ly.off_b - Ly.off_a) : ybuf_ + Ly.off_b;
                    gdn_decode_fused(ybuf_, a_in, b_in, Ly.in_width, Ly.A_log, Ly.dt_bias, Ly.conv_w, slot_conv(Ly.dslot),
                                     nullptr, slot_S(Ly.dslot), slot_S(Ly.dslot), sc() + kSlot, conv_slot_, R_, &rec, nullptr,
                                     ybuf_ + Ly.off_z, Ly.gnorm, frag_, gss_, T, nk, nv, c_.k_dim, dv, c_.conv_k,
                                     c_.v_tiled, st_, abpart_ ? kAbSlices : 1, ab_rows_);
                    out.kss = gss_;
                    out.kss_n = dv;
                    out.kss_eps = 1e-6f;
                } else {
                    gdn_decode(ybuf_, ybuf_ + Ly.off_a, ybuf_ + Ly.off_b, Ly.in_width, Ly.A_log, Ly.dt_bias,
                               Ly.conv_w, slot_conv(Ly.dslot), nullptr, slot_S(Ly.dslot), nullptr, sc() + kSlot, conv_slot_,
                               s_slot_, R_, o_, T, nk, nv, c_.k_dim, dv, c_.conv_k, c_.v_tiled, st_);
                    gnorm_pack(o_, ybuf_ + Ly.off_z, Ly.in_width, Ly.gnorm, Ly.gnorm_n, xn_, frag_, zdim, T, 1e-6f,
                               st_);
                }
                gemm_on(Ly.out_proj, frag_, x, H, H, T, kEpiAddNorm, frag_x_, &out);
                out.kss = nullptr;
            } else {
                gemm_on(Ly.qkv_parts[0], frag_x_, ybuf_, Ly.qkv_width, Ly.qkv_parts[0].m, T, kEpiStore, nullptr,
                        io_in);
                attn_decode_layer(ybuf_, Ly.qkv_width, Ly.q_norm, Ly.k_norm, slot_kc(Ly.aslot), slot_vt(Ly.aslot), ctx_,
                                  sc() + kPos, T, nq, nkv, hd, c_.rotary_dim, c_.rope_theta, eps, attn_ws_,
                                  attn_ws_bytes_, xn_, frag_, st_);
                gemm_on(Ly.o_proj, frag_, x, H, H, T, kEpiAddNorm, frag_x_, &out);
            }
            gemm_on(Ly.gate_up, frag_x_, nullptr, I, I, T, Ly.gate_up.swiglu_epi(), frag_h_, &in);
            out.gamma_out = i + 1 < c_.n_layers ? L_[i + 1].attn_norm : final_norm_;
            gemm_on(Ly.down, frag_h_, x, H, H, T, kEpiAddNorm, frag_x_, &out);
        }
        if (!ends) return;
        x_ = x;  // hidden after the layers (pre final norm), for the MTP history
        gemm_on(lm_head_, frag_x_, logits_, c_.vocab, c_.vocab, T, kEpiStore, nullptr, &in);
        argmax_rows(logits_, T, c_.vocab, preds_, nullptr, arg_ws_, st_);
        accept(tok_, preds_, T, force_all, sc() + kPos, sc() + kSlot, R_, sc() + kNCons, sc() + kNextTok, gen_,
               sc() + kGenCount, kGenCap, x_, h_last_, h_prev_, H, st_);
    }

    // Linear on the current activation with the folded RMSNorm: K-quant from the fp32
    // x * (1 + gamma) rows x32 (KqNorm), FP8 / BF16 from frag_ (NormIO).
    void linear_folded(const Lin& L, const float* x32, float* Y, int ldy, int m_valid, int T, const KqNorm& kn,
                       const NormIO& io) {
        if (L.kind == RL_Q_FP8_E4M3_B128)
            gemm_fp8_frag(L.w, L.ts, frag_, Y, L.m, L.n, T, kEpiStore, ldy, m_valid, st_, 1, nullptr, &io);
        else if (L.kind == RL_Q_BF16)
            gemm_bf16_frag(reinterpret_cast<const uint16_t*>(L.w), frag_, Y, L.m, L.n, T, kEpiStore, ldy, m_valid, st_,
                           1, nullptr, &io);
        else
            kq_gemm(L.kind == RL_Q_Q4_K ? 4 : 6, L.w, x32, Y, kq_ws_, kq_ws_bytes_, L.m, L.n, T, 0, ldy, st_, &kn);
    }

    // One step of a K-quant model with the RMSNorms folded (see kq_fold_): layer 0's
    // first linears read the normalised rows; from then on the residual GEMVs add
    // into x in place and leave the sums of squares (and x * (1 + gamma) fragments)
    // for the next linears.
    // batch: the batch step (T == B rows, one token of each slot b at its own
    // position; the DeltaNet kernel and attention run over the B slots' states and
    // caches, and batch_advance replaces the acceptance)
    void step_kq_folded(int T, int force_all, bool feed, int B = 1, bool batch = false) {
        const int Ts = batch ? 1 : T;  // tokens per sequence
        const int H = c_.hidden, nk = c_.n_k_heads, nv = c_.n_v_heads, dv = c_.v_dim;
        const int zdim = nv * dv, nq = c_.n_q, nkv = c_.n_kv, hd = c_.head_dim, I = c_.intermediate;
        const float eps = c_.rms_eps;
        float* x = xres_[0];
        const bool ends = only_layer_ < 0 || only_layer_ >= c_.n_layers;  // head and tail of the step
        if (ends) {
            if (feed) copy_int(sc() + kNextTok, tok_, st_);
            embed_rows(embed_, embed_kind_, tok_ + gb_, x, H, c_.vocab, T, st_);
            rmsnorm_pack(x, H, L_[0].attn_norm, xn_, frag_, H, T, eps, st_);
        }
        KqNorm kin;
        kin.ss_in = kq_ss_;
        kin.groups_in = kq_groups_;
        kin.n_norm = H;
        kin.eps = eps;
        NormIO io;
        io.ss_in = kq_ss_;
        io.groups_in = kq_groups_;
        io.n_norm = H;
        io.eps = eps;
        bool normalised = only_layer_ <= 0;  // xn_ / frag_ hold the normalised rows (layer 0 only)
        auto consume = [&](const Lin& L, float* Y, int ldy, int m_valid) {
            if (normalised)
                linear(L, xn_, Y, ldy, m_valid, T, kEpiStore);
            else
                linear_folded(L, xg_, Y, ldy, m_valid, T, kin, io);
        };
        auto produce = [&](const Lin& L, const float* a32, const float* gamma_next, const float* bss = nullptr) {
            KqNorm kp;
            kp.bss = bss;
            kp.ss_out = kq_ss_;
            kp.gamma_out = gamma_next;
            kp.xg_out = xg_;
            kp.frag_out = frag_;
            kq_gemm(L.kind == RL_Q_Q4_K ? 4 : 6, L.w, a32, x, kq_ws_, kq_ws_bytes_, L.m, L.n, T, 1, H, st_, &kp);
            normalised = false;
        };
        for (int i = 0; i < c_.n_layers; ++i) {
            Layer& Ly = L_[i];
            if (Ly.kind == RL_LAYER_DELTA) {
                // the a/b rows (an FP8 / BF16 part of their own, a few tiles) as K-slice
                // partials that the fused DeltaNet kernel adds: one short launch over
                // many workgroups instead of a handful of long ones
                int ab_part = -1;
                for (size_t k = 0; k < Ly.in_parts.size(); ++k)
                    if (gdn_fused_ && Ly.in_offs[k] == Ly.off_a && frag_kind(Ly.in_parts[k]) &&
                        Ly.off_a + Ly.in_parts[k].m == Ly.in_width)
                        ab_part = static_cast<int>(k);
                // BF16 a/b rows beside K-quant parts: computed by extra workgroups of the
                // last K-quant launch (same x, same partial layout), no launch of their own
                int kq_host = -1;
                if (ab_part >= 0 && Ly.in_parts[ab_part].kind == RL_Q_BF16 && kq_fold_supported() &&
                    ab_rows_in_kq_enabled())
                    for (size_t k = 0; k < Ly.in_parts.size(); ++k)
                        if (static_cast<int>(k) != ab_part && is_kq(Ly.in_parts[k])) kq_host = static_cast<int>(k);
                for (size_t k = 0; k < Ly.in_parts.size(); ++k) {
                    const Lin& L = Ly.in_parts[k];
                    if (static_cast<int>(k) == kq_host) {
                        const Lin& A = Ly.in_parts[ab_part];
                        KqNorm kn = normalised ? KqNorm{} : kin;
                        kn.ab_w = reinterpret_cast<const uint16_t*>(A.w);
                        kn.ab_rows = A.m;
                        kn.ab_slices = kAbSlices;
                        kn.ab_out = kq_abpart_;
                        kn.ab_ld = A.m;
                        kq_gemm(L.kind == RL_Q_Q4_K ? 4 : 6, L.w, normalised ? xn_ : xg_, ybuf_ + Ly.in_offs[k], kq_ws_,
                                kq_ws_bytes_, L.m, L.n, T, 0, Ly.in_width, st_, &kn);
                        continue;
                    }
                    if (static_cast<int>(k) != ab_part) {
                        consume(L, ybuf_ + Ly.in_offs[k], Ly.in_width, L.m);
                        continue;
                    }
                    if (kq_host >= 0) continue;
                    const NormIO* iop = normalised ? nullptr : &io;
                    if (L.kind == RL_Q_FP8_E4M3_B128)
                        gemm_fp8_frag(L.w, L.ts, frag_, kq_abpart_, L.m, L.n, T, kEpiPartial, L.m, L.m, st_, kAbSlices,
                                      nullptr, iop);
                    else
                        gemm_bf16_frag(reinterpret_cast<const uint16_t*>(L.w), frag_, kq_abpart_, L.m, L.n, T,
                                       kEpiPartial, L.m, L.m, st_, kAbSlices, nullptr, iop);
                }
                if (gdn_fused_) {
                    const bool bat = batch;
                    const GdnRecords rec{bat ? b_rec(Ly.dslot) : slot_rec(Ly.dslot),
                                         bat ? b_recn(Ly.dslot) : slot_recn(Ly.dslot), bat ? b_scal() + kNCons : sc() + kNCons,
                                         tmax_, Ts > 1 && !force_all};
                    const GdnBatch bt{B, s_bstride_, conv_bstride_, rec_bstride_, recn_bstride_, kScalars};
                    const bool split = ab_part >= 0;
                    const int ab_rows = split ? Ly.in_parts[ab_part].m : 0;
                    gdn_decode_fused(ybuf_, split ? kq_abpart_ : ybuf_ + Ly.off_a,
                                     split ? kq_abpart_ + (Ly.off_b - Ly.off_a) : ybuf_ + Ly.off_b, Ly.in_width,
                                     Ly.A_log, Ly.dt_bias, Ly.conv_w, bat ? b_conv(Ly.dslot) : slot_conv(Ly.dslot), nullptr,
                                     bat ? b_S(Ly.dslot) : slot_S(Ly.dslot), bat ? b_S(Ly.dslot) : slot_S(Ly.dslot),
                                     bat ? b_scal() + kSlot : sc() + kSlot, conv_slot_, R_, &rec, kq_gnorm_ ? nullptr : o_,
                                     kq_gnorm_ ? ybuf_ + Ly.off_z : nullptr, kq_gnorm_ ? Ly.gnorm : nullptr, nullptr,
                                     kq_gnorm_ ? gss_ : nullptr, Ts, nk, nv, c_.k_dim, dv, c_.conv_k, c_.v_tiled, st_,
                                     split ? kAbSlices : 1, ab_rows, bat ? &bt : nullptr, 0, 0,
                                     kq_gnorm_ ? xn_ : nullptr);
                } else {
                    RL_REQUIRE(B == 1, RL_ERR_UNSUPPORTED, "engine: batch decode needs the fused DeltaNet kernel");
                    gdn_decode(ybuf_, ybuf_ + Ly.off_a, ybuf_ + Ly.off_b, Ly.in_width, Ly.A_log, Ly.dt_bias, Ly.conv_w,
                               slot_conv(Ly.dslot), nullptr, slot_S(Ly.dslot), nullptr, sc() + kSlot, conv_slot_, s_slot_,
                               R_, o_, T, nk, nv, c_.k_dim, dv, c_.conv_k, c_.v_tiled, st_);
                }
                if (kq_gnorm_) {
                    produce(Ly.out_proj, xn_, Ly.ffn_norm, gss_);
                } else {
                    gnorm_pack(o_, ybuf_ + Ly.off_z, Ly.in_width, Ly.gnorm, Ly.gnorm_n, xn_, frag_, zdim, T, 1e-6f,
                               st_);
                    produce(Ly.out_proj, xn_, Ly.ffn_norm);
                }
            } else {
                for (size_t k = 0; k < Ly.qkv_parts.size(); ++k)
                    consume(Ly.qkv_parts[k], ybuf_ + Ly.qkv_offs[k], Ly.qkv_width, Ly.qkv_parts[k].m);
                if (batch)
                    attn_decode_layer(ybuf_, Ly.qkv_width, Ly.q_norm, Ly.k_norm, b_kc(Ly.aslot), b_vt(Ly.aslot), ctx_,
                                      b_scal() + kPos, 1, nq, nkv, hd, c_.rotary_dim, c_.rope_theta, eps, attn_ws_,
                                      attn_ws_bytes_, xn_, frag_, st_, 0, B, B, kv_bstride_, kScalars);
                else
                    attn_decode_layer(ybuf_, Ly.qkv_width, Ly.q_norm, Ly.k_norm, slot_kc(Ly.aslot), slot_vt(Ly.aslot),
                                      ctx_, sc() + kPos, T, nq, nkv, hd, c_.rotary_dim, c_.rope_theta, eps, attn_ws_,
                                      attn_ws_bytes_, xn_, frag_, st_);
                produce(Ly.o_proj, xn_, Ly.ffn_norm);
            }
            if (Ly.gate_up.kind >= 0) {
                // fused FP8 / BF16 gate/up reading x * (1 + gamma) fragments; the K-quant
                // down reads fp32 h
                if (Ly.gate_up.kind == RL_Q_FP8_E4M3_B128)
                    gemm_fp8_frag(Ly.gate_up.w, Ly.gate_up.ts, frag_, h_, Ly.gate_up.m, Ly.gate_up.n, T,
                                  Ly.gate_up.swiglu_epi(), I, I, st_, 1, nullptr, &io);
                else
                    gemm_bf16_frag(reinterpret_cast<const uint16_t*>(Ly.gate_up.w), frag_, h_, Ly.gate_up.m,
                                   Ly.gate_up.n, T, Ly.gate_up.swiglu_epi(), I, I, st_, 1, nullptr, &io);
            } else if (Ly.gate_cat) {
                KqNorm ks = normalised ? KqNorm{} : kin;
                ks.swiglu = 1;
                kq_gemm(Ly.gate.kind == RL_Q_Q4_K ? 4 : 6, Ly.gate.w, normalised ? xn_ : xg_, h_, kq_ws_, kq_ws_bytes_,
                        Ly.gate.m, Ly.gate.n, T, 0, I, st_, &ks);
            } else {
                consume(Ly.gate, g_, I, I);
                consume(Ly.up, u_, I, I);
                swiglu(g_, I, u_, I, h_, I, T, st_);
            }
            produce(Ly.down, h_, i + 1 < c_.n_layers ? L_[i + 1].attn_norm : final_norm_);
        }
        if (!ends) return;
        consume(lm_head_, b_logits(), c_.vocab, c_.vocab);
        argmax_rows(b_logits(), T, c_.vocab, preds_ + gb_, nullptr, arg_ws_, st_);
        if (batch) {
            batch_advance(b_scal(), kScalars, B, R_, kPos, kSlot, kNCons, st_);
            return;
        }
        x_ = x;  // hidden after the layers (pre final norm), for the MTP history
        accept(tok_, preds_, T, force_all, sc() + kPos, sc() + kSlot, R_, sc() + kNCons, sc() + kNextTok, gen_,
               sc() + kGenCount, kGenCap, x_, h_last_, h_prev_, H, st_);
    }

    void step(int T, int force_all, bool feed) {
        if (fold_norm_) {
            step_folded(T, force_all, feed);
            return;
        }
        if (kq_fold_) {
            step_kq_folded(T, force_all, feed);
            return;
        }
        const int H = c_.hidden, nk = c_.n_k_heads, nv = c_.n_v_heads, dv = c_.v_dim;
        const int zdim = nv * dv, nq = c_.n_q, nkv = c_.n_kv, hd = c_.head_dim, I = c_.intermediate;
        const float eps = c_.rms_eps;
        int cur = 0, pending = 0;
        if (feed) copy_int(sc() + kNextTok, tok_, st_);
        embed_rows(embed_, embed_kind_, tok_, xres_[cur], H, c_.vocab, T, st_);
        for (int i = 0; i < c_.n_layers; ++i) {
            Layer& Ly = L_[i];
            norm_residual(cur, pending, Ly.attn_norm, T);
            if (Ly.kind == RL_LAYER_DELTA) {
                linear_parts(Ly.in_parts, Ly.in_offs, xn_, ybuf_, Ly.in_width, T);
                gdn_decode(ybuf_, ybuf_ + Ly.off_a, ybuf_ + Ly.off_b, Ly.in_width, Ly.A_log, Ly.dt_bias, Ly.conv_w,
                           slot_conv(Ly.dslot), nullptr, slot_S(Ly.dslot), nullptr, sc() + kSlot, conv_slot_, s_slot_, R_, o_,
                           T, nk, nv, c_.k_dim, dv, c_.conv_k, c_.v_tiled, st_);
                gnorm_pack(o_, ybuf_ + Ly.off_z, Ly.in_width, Ly.gnorm, Ly.gnorm_n, xn_, frag_, zdim, T, 1e-6f, st_);
                pending = linear_residual(Ly.out_proj, xn_, T);
            } else {
                linear_parts(Ly.qkv_parts, Ly.qkv_offs, xn_, ybuf_, Ly.qkv_width, T);
                attn_decode_layer(ybuf_, Ly.qkv_width, Ly.q_norm, Ly.k_norm, slot_kc(Ly.aslot), slot_vt(Ly.aslot), ctx_,
                                  sc() + kPos, T, nq, nkv, hd, c_.rotary_dim, c_.rope_theta, eps, attn_ws_,
                                  attn_ws_bytes_, xn_, frag_, st_);
                pending = linear_residual(Ly.o_proj, xn_, T);
            }
            norm_residual(cur, pending, Ly.ffn_norm, T);
            pending = mlp_unfolded(Ly, T);
        }
        norm_residual(cur, pending, final_norm_, T);
        x_ = xres_[cur];  // hidden after the layers (pre final norm), for the MTP history
        linear(lm_head_, xn_, logits_, c_.vocab, c_.vocab, T, kEpiStore);
        argmax_rows(logits_, T, c_.vocab, preds_, nullptr, arg_ws_, st_);
        accept(tok_, preds_, T, force_all, sc() + kPos, sc() + kSlot, R_, sc() + kNCons, sc() + kNextTok, gen_,
               sc() + kGenCount, kGenCap, x_, h_last_, h_prev_, H, st_);
    }

    // MLP of one layer on the normalised input (xn_ / frag_): gate/up (SwiGLU) then
    // down into the residual partials; returns the partial count for norm_residual.
    int mlp_unfolded(const Layer& Ly, int T) {
        const int I = c_.intermediate;
        const bool down_frag = Ly.down.kind == RL_Q_FP8_E4M3_B128 || Ly.down.kind == RL_Q_BF16;
        if (Ly.gate_up.kind >= 0) {
            // SwiGLU epilogue: fp32 h only when a K-quant down needs it
            if (Ly.gate_up.kind == RL_Q_FP8_E4M3_B128)
                gemm_fp8_frag(Ly.gate_up.w, Ly.gate_up.ts, frag_, down_frag ? nullptr : h_, Ly.gate_up.m,
                              Ly.gate_up.n, T, Ly.gate_up.swiglu_epi(), I, I, st_, 1, down_frag ? frag_h_ : nullptr);
            else
                gemm_bf16_frag(reinterpret_cast<const uint16_t*>(Ly.gate_up.w), frag_, down_frag ? nullptr : h_,
                               Ly.gate_up.m, Ly.gate_up.n, T, Ly.gate_up.swiglu_epi(), I, I, st_, 1,
                               down_frag ? frag_h_ : nullptr);
        } else {
            if (Ly.gate_cat) {
                KqNorm ks;
                ks.swiglu = 1;
                kq_gemm(Ly.gate.kind == RL_Q_Q4_K ? 4 : 6, Ly.gate.w, xn_, h_, kq_ws_, kq_ws_bytes_, Ly.gate.m,
                        Ly.gate.n, T, 0, I, st_, &ks);
            } else {
                linear(Ly.gate, xn_, g_, I, I, T, kEpiStore);
                linear(Ly.up, xn_, u_, I, I, T, kEpiStore);
                swiglu(g_, I, u_, I, h_, I, T, st_);
            }
            if (down_frag) pack_act(h_, frag_h_, I, T, st_);
        }
        return linear_residual(Ly.down, h_, T, down_frag ? frag_h_ : frag_);
    }

    // The MTP decoder layer on the draft's hidden h (in place), at draft position
    // `dpos` of its own cache (Session::mtp_layer_step, session.cpp:561-617: the
    // fused attention decode then the fused MLP decode with the mtp.layers[0]
    // weights, each adding into h).  Leaves norm_mtp(h) in xn_ / frag_ for the
    // lm_head, as the stem's final RMSNorm does.
    void mtp_layer_step(float* h, int dpos) {
        const int H = c_.hidden;
        const float eps = c_.rms_eps;
        const Layer& Ly = mtp_layer_;
        rmsnorm_pack(h, H, Ly.attn_norm, xn_, frag_, H, 1, eps, st_);
        linear_parts(Ly.qkv_parts, Ly.qkv_offs, xn_, ybuf_, Ly.qkv_width, 1);
        attn_decode_layer(ybuf_, Ly.qkv_width, Ly.q_norm, Ly.k_norm, mtp_kc_, mtp_vt_, kMtpCtx, mtp_pos_ + dpos, 1,
                          c_.n_q, c_.n_kv, c_.head_dim, c_.rotary_dim, c_.rope_theta, eps, mtp_attn_ws_,
                          mtp_attn_ws_bytes_, xn_, frag_, st_);
        int pending = linear_residual(Ly.o_proj, xn_, 1);
        residual_rmsnorm_pack(h, part_, pending, mtp_x1_, Ly.ffn_norm, xn_, frag_, H, 1, eps, st_);
        pending = mlp_unfolded(Ly, 1);
        residual_rmsnorm_pack(mtp_x1_, part_, pending, h, mtp_norm_, xn_, frag_, H, 1, eps, st_);
    }

    // MTP draft of n tokens: tok_[0] = next token, tok_[1..n] = drafts.  The stem
    // (Session::mtp_draft): h' = fc([norm_e(embed tok) ; norm_h(h)]), token =
    // argmax(lm_head(norm_mtp(h'))); with the decoder layer (mtp_mode_ ==
    // RL_MTP_LAYER) h' passes through mtp_layer_step at draft position i first.
    void mtp_body(int n) {
        const int H = c_.hidden;
        const float eps = c_.rms_eps;
        copy_int(sc() + kNextTok, tok_, st_);
        const size_t half_units = static_cast<size_t>(H / 128) * 16 * 2;  // fragment units of H columns, T = 1
        for (int i = 0; i < n; ++i) {
            embed_rows(embed_, embed_kind_, tok_ + i, mtp_e_, H, c_.vocab, 1, st_);
            // cat = [norm_e(embed(tok)) ; norm_h(h)]  (session.cpp:650-658)
            rmsnorm_pack(mtp_e_, H, mtp_ne_, xn_, frag_, H, 1, eps, st_);
            rmsnorm_pack(i == 0 ? h_last_ : h_prev_, H, mtp_nh_, xn_ + H, static_cast<i32x4*>(frag_) + half_units, H, 1,
                         eps, st_);
            linear(mtp_fc_, xn_, mtp_hp_, H, H, 1, kEpiStore);
            if (mtp_mode_ == RL_MTP_LAYER)
                mtp_layer_step(mtp_hp_, i);
            else
                rmsnorm_pack(mtp_hp_, H, mtp_norm_, xn_, frag_, H, 1, eps, st_);
            linear(lm_head_, xn_, mtp_logits_, c_.vocab, c_.vocab, 1, kEpiStore);
            argmax_rows(mtp_logits_, 1, c_.vocab, tok_ + i + 1, nullptr, arg_ws_, st_);
        }
    }

    // Replay (capturing on first use) the graph for a T-token step.  T = 1 feeds the
    // device's next token; T > 1 reads tok_ as written by the host or the MTP draft.
    void run_graph(int T, bool from_host = false) {
        (void)from_host;
        launch_captured(T, [&] { step(T, T == 1 ? 1 : 0, /*feed=*/T == 1); });
    }

    void run_mtp(int n) {
        launch_captured((mtp_mode_ == RL_MTP_LAYER ? kKeyMtpLayer : kKeyMtpStem) + n, [&] { mtp_body(n); });
    }

    // RL_HIP_GRAPHS=0 runs every step eagerly (same kernels, launched one by one):
    // for tools that cannot follow graph launches.
    static bool graphs_enabled() {
        static const bool on = [] {
            const char* v = std::getenv("RL_HIP_GRAPHS");
            return !(v && v[0] == '0');
        }();
        return on;
    }

    // Graph keys: the T-token step is T; each other recording has its own range
    static constexpr int kKeyMtpStem = 100, kKeyMtpLayer = 200, kKeyBatch = 300, kKeyLayer = 1000;

    template <class F>
    void launch_captured(int key, F body) {
        if (!graphs_enabled()) {
            body();
            return;
        }
        auto it = graphs_.find(key);
        if (it == graphs_.end()) {
            hipGraph_t g = nullptr;
            hipGraphExec_t ex = nullptr;
            RL_HIP(hipStreamBeginCapture(st_, hipStreamCaptureModeThreadLocal));
            try {
                body();
            } catch (...) {
                hipGraph_t dead = nullptr;
                (void)hipStreamEndCapture(st_, &dead);
                if (dead) (void)hipGraphDestroy(dead);
                throw;
            }
            RL_HIP(hipStreamEndCapture(st_, &g));
            RL_HIP(hipGraphInstantiate(&ex, g, nullptr, nullptr, 0));
            (void)hipGraphDestroy(g);
            it = graphs_.emplace(key, ex).first;
        }
        RL_HIP(hipGraphLaunch(it->second, st_));
    }

    void sync_graph_state() { RL_HIP(hipStreamSynchronize(st_)); }

    // Zero slot b's sequence state: scalars, DeltaNet state and the conv window the
    // ring starts from, record counts.
    void zero_slot_state(int b) {
        RL_HIP(hipMemsetAsync(scal_ + b * kScalars, 0, kScalars * sizeof(int), st_));
        for (size_t l = 0; l < S_.size(); ++l) {
            RL_HIP(hipMemsetAsync(S_[l] + b * s_bstride_, 0, s_slot_ * sizeof(float), st_));
            RL_HIP(hipMemsetAsync(conv_[l] + b * conv_bstride_, 0, conv_slot_ * sizeof(float), st_));
        }
        for (size_t l = 0; l < rec_n_.size(); ++l)
            RL_HIP(hipMemsetAsync(rec_n_[l] + b * recn_bstride_, 0, recn_bstride_ * sizeof(int), st_));
    }

    // Batch step: B sequences, one token each (tok_[b] at slot b's position); the
    // folded-norm linears with B rows, the DeltaNet kernel over the B slots, one
    // attention launch set over the slots (slot b writes column b of o_proj's
    // input).  K-quant models run the K-quant step with B rows.
    // One batch step over slots 0 .. B-1: groups of at most group_rows() slots, one
    // weight pass each (gb_ = the group's first slot while it is recorded).
    void batch_groups(int B) {
        struct Reset {
            int& g;
            ~Reset() { g = 0; }
        } reset{gb_};
        const int G = group_rows();
        for (int off = 0; off < B; off += G) {
            gb_ = off;
            step_batch(std::min(G, B - off));
        }
    }

    void step_batch(int B) {
        if (kq_fold_) {
            step_kq_folded(B, 0, false, B, true);
            return;
        }
        const int H = c_.hidden, nk = c_.n_k_heads, nv = c_.n_v_heads, dv = c_.v_dim;
        const int nq = c_.n_q, nkv = c_.n_kv, hd = c_.head_dim, I = c_.intermediate;
        const float eps = c_.rms_eps;
        float* x = xres_[0];
        embed_rows(embed_, embed_kind_, tok_ + gb_, x, H, c_.vocab, B, st_);
        rmsnorm_pack(x, H, L_[0].attn_norm, xn_, frag_x_, H, B, eps, st_);
        NormIO in;
        in.ss_in = ss_;
        in.groups_in = add_norm_groups(H);
        in.n_norm = H;
        in.eps = eps;
        const GdnBatch bt{B, s_bstride_, conv_bstride_, rec_bstride_, recn_bstride_, kScalars};
        for (int i = 0; i < c_.n_layers; ++i) {
            Layer& Ly = L_[i];
            const NormIO* io_in = i == 0 ? nullptr : &in;
            NormIO out;
            out.gamma_out = Ly.ffn_norm;
            out.ss_out = ss_;
            if (Ly.kind == RL_LAYER_DELTA) {
                // the a/b rows as K-slices of the first workgroups (one row tile per
                // workgroup) up to 8 rows; above that the in_proj takes four row tiles
                // per workgroup and the a/b rows with them
                float* abp = B <= 8 ? abpart_ : nullptr;
                NormIO in_ab = io_in ? *io_in : NormIO{};
                if (abp) {
                    in_ab.xpart = abp;
                    in_ab.x_tile0 = ab_tile0_;
                    in_ab.x_slices = kAbSlices;
                    in_ab.x_rows = ab_rows_;
                }
                gemm_on(Ly.in_parts[0], frag_x_, ybuf_, Ly.in_width, Ly.in_parts[0].m, B, kEpiStore, nullptr,
                        abp ? &in_ab : io_in);
                const GdnRecords rec{b_rec(Ly.dslot), b_recn(Ly.dslot), b_scal() + kNCons, tmax_, 0};
                const float* a_in = abp ? abp : ybuf_ + Ly.off_a;
                const float* b_in = abp ? abp + (Ly.off_b - Ly.off_a) : ybuf_ + Ly.off_b;
                gdn_decode_fused(ybuf_, a_in, b_in, Ly.in_width, Ly.A_log, Ly.dt_bias, Ly.conv_w, b_conv(Ly.dslot),
                                 nullptr, b_S(Ly.dslot), b_S(Ly.dslot), b_scal() + kSlot, conv_slot_, R_, &rec, nullptr,
                                 ybuf_ + Ly.off_z, Ly.gnorm, frag_, gss_, 1, nk, nv, c_.k_dim, dv, c_.conv_k,
                                 c_.v_tiled, st_, abp ? kAbSlices : 1, abp ? ab_rows_ : 0, &bt);
                out.kss = gss_;
                out.kss_n = dv;
                out.kss_eps = 1e-6f;
                gemm_on(Ly.out_proj, frag_, x, H, H, B, kEpiAddNorm, frag_x_, &out);
                out.kss = nullptr;
            } else {
                gemm_on(Ly.qkv_parts[0], frag_x_, ybuf_, Ly.qkv_width, Ly.qkv_parts[0].m, B, kEpiStore, nullptr,
                        io_in);
                // all slots in one launch set (slot b: its own cache, position and
                // workspace; output column b)
                attn_decode_layer(ybuf_, Ly.qkv_width, Ly.q_norm, Ly.k_norm, b_kc(Ly.aslot), b_vt(Ly.aslot), ctx_,
                                  b_scal() + kPos, 1, nq, nkv, hd, c_.rotary_dim, c_.rope_theta, eps, attn_ws_,
                                  attn_ws_bytes_, xn_, frag_, st_, 0, B, B, kv_bstride_, kScalars);
                gemm_on(Ly.o_proj, frag_, x, H, H, B, kEpiAddNorm, frag_x_, &out);
            }
            gemm_on(Ly.gate_up, frag_x_, nullptr, I, I, B, Ly.gate_up.swiglu_epi(), frag_h_, &in);
            out.gamma_out = i + 1 < c_.n_layers ? L_[i + 1].attn_norm : final_norm_;
            gemm_on(Ly.down, frag_h_, x, H, H, B, kEpiAddNorm, frag_x_, &out);
        }
        gemm_on(lm_head_, frag_x_, b_logits(), c_.vocab, c_.vocab, B, kEpiStore, nullptr, &in);
        argmax_rows(b_logits(), B, c_.vocab, preds_ + gb_, nullptr, arg_ws_, st_);
        batch_advance(b_scal(), kScalars, B, R_, kPos, kSlot, kNCons, st_);
    }

    void readback() {
        RL_HIP(hipMemcpyAsync(host_rb_, sc(), kScalars * sizeof(int), hipMemcpyDeviceToHost, st_));
        RL_HIP(hipMemcpyAsync(host_rb_ + kRbPreds, preds_, kMaxSlots * sizeof(int), hipMemcpyDeviceToHost, st_));
        RL_HIP(hipMemcpyAsync(host_rb_ + kRbToks, tok_, 8 * sizeof(int), hipMemcpyDeviceToHost, st_));
        RL_HIP(hipStreamSynchronize(st_));
        pos_ = host_rb_[kPos];
        n_last_ = host_rb_[kNCons];
        greedy_ = host_rb_[kNextTok];
    }
};

}  // namespace rl

struct RlEngine {
    std::unique_ptr<rl::Engine> e;
};

extern "C" {

RlEngine* rl_hip_engine_create(const RlModelConfig* cfg, const RlTensor* tensors, int n_tensors, int ctx, int max_T,
                               int* status) {
    RlEngine* out = nullptr;
    const int rc = guard([&] {
        RL_REQUIRE(cfg && tensors && n_tensors > 0, RL_ERR_RANGE, "engine_create: null config or weights");
        auto e = std::make_unique<rl::Engine>(*cfg, ctx, max_T);
        e->load(tensors, n_tensors);
        e->reset();
        out = new RlEngine{std::move(e)};
    });
    if (status) *status = rc;
    return out;
}

RlEngine* rl_hip_engine_create_synthetic(const RlModelConfig* cfg, uint64_t seed, int ctx, int max_T, int* status) {
    RlEngine* out = nullptr;
    const int rc = guard([&] {
        RL_REQUIRE(cfg != nullptr, RL_ERR_RANGE, "engine_create_synthetic: null config");
        auto e = std::make_unique<rl::Engine>(*cfg, ctx, max_T);
        e->load_synthetic(seed);
        e->reset();
        out = new RlEngine{std::move(e)};
    });
    if (status) *status = rc;
    return out;
}

RlEngine* rl_hip_engine_create_batch(const RlModelConfig* cfg, const RlTensor* tensors, int n_tensors, int ctx,
                                     int max_T, int max_batch, int* status) {
    RlEngine* out = nullptr;
    const int rc = guard([&] {
        RL_REQUIRE(cfg && tensors && n_tensors > 0, RL_ERR_RANGE, "engine_create: null config or weights");
        auto e = std::make_unique<rl::Engine>(*cfg, ctx, max_T, max_batch);
        e->load(tensors, n_tensors);
        e->zero_slots(max_batch);
        e->reset();
        out = new RlEngine{std::move(e)};
    });
    if (status) *status = rc;
    return out;
}

RlEngine* rl_hip_engine_create_synthetic_batch(const RlModelConfig* cfg, uint64_t seed, int ctx, int max_T,
                                               int max_batch, int* status) {
    RlEngine* out = nullptr;
    const int rc = guard([&] {
        RL_REQUIRE(cfg != nullptr, RL_ERR_RANGE, "engine_create_synthetic: null config");
        auto e = std::make_unique<rl::Engine>(*cfg, ctx, max_T, max_batch);
        e->load_synthetic(seed);
        e->zero_slots(max_batch);
        e->reset();
        out = new RlEngine{std::move(e)};
    });
    if (status) *status = rc;
    return out;
}

void rl_hip_engine_destroy(RlEngine* e) { delete e; }

#define RL_ENGINE(e) RL_REQUIRE((e) && (e)->e, RL_ERR_RANGE, "null engine")

int rl_hip_engine_reset(RlEngine* e) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->reset();
    });
}
int rl_hip_engine_prefill(RlEngine* e, const int32_t* ids, int n) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->prefill(ids, n);
    });
}
int rl_hip_engine_decode_token(RlEngine* e, int32_t token) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->decode_token(token);
    });
}
int rl_hip_engine_decode_steps(RlEngine* e, int n) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->decode_steps(n);
    });
}
int rl_hip_engine_copy_gen_tokens(RlEngine* e, int32_t* host, int n) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->copy_gen_tokens(host, n);
    });
}
int rl_hip_engine_copy_logits(RlEngine* e, float* host) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->copy_logits(host);
    });
}
int rl_hip_engine_copy_last_hidden(RlEngine* e, float* host) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->copy_last_hidden(host);
    });
}
int rl_hip_engine_mtp_draft(RlEngine* e, int32_t first, int n, int32_t* out, int* n_out) {
    return guard([&] {
        RL_ENGINE(e);
        const int k = e->e->mtp_draft(first, n, out);
        if (n_out) *n_out = k;
    });
}
int rl_hip_engine_spec_verify(RlEngine* e, const int32_t* toks, int T, int32_t* preds, int* n_consumed) {
    return guard([&] {
        RL_ENGINE(e);
        const int k = e->e->spec_verify(toks, T, preds);
        if (n_consumed) *n_consumed = k;
    });
}
int rl_hip_engine_set_mtp_mode(RlEngine* e, int mode) {
    return guard([&] {
        RL_REQUIRE(e, RL_ERR_RANGE, "null engine");
        e->e->set_mtp_mode(mode);
    });
}

int rl_hip_engine_mtp_mode(RlEngine* e, int* mode, int* layer_available) {
    return guard([&] {
        RL_REQUIRE(e && mode && layer_available, RL_ERR_RANGE, "null argument");
        *mode = e->e->mtp_mode();
        *layer_available = e->e->has_mtp_layer() ? 1 : 0;
    });
}

int rl_hip_engine_copy_mtp_hidden(RlEngine* e, float* out) {
    return guard([&] {
        RL_REQUIRE(e && out, RL_ERR_RANGE, "null argument");
        e->e->copy_mtp_hidden(out);
    });
}

int rl_hip_engine_mtp_spec(RlEngine* e, int32_t t0, int T, int32_t* toks_out, int32_t* preds, int* n_consumed) {
    return guard([&] {
        RL_ENGINE(e);
        const int k = e->e->mtp_spec(t0, T, toks_out, preds);
        if (n_consumed) *n_consumed = k;
    });
}
int rl_hip_engine_greedy(RlEngine* e, int32_t* tok) {
    return guard([&] {
        RL_ENGINE(e);
        *tok = e->e->greedy();
    });
}
int rl_hip_engine_pos(RlEngine* e, int* pos) {
    return guard([&] {
        RL_ENGINE(e);
        *pos = e->e->pos();
    });
}
int rl_hip_engine_set_pos(RlEngine* e, int pos) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->set_pos(pos);
    });
}
int rl_hip_engine_synthetic_context(RlEngine* e, int n, uint64_t seed) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->synthetic_context(n, seed);
    });
}
int rl_hip_engine_time_steps(RlEngine* e, int T, int iters, int mtp_drafts, float* ms) {
    return guard([&] {
        RL_ENGINE(e);
        *ms = e->e->time_steps(T, iters, mtp_drafts);
    });
}
int rl_hip_engine_info(RlEngine* e, int* vocab, int* hidden, int* ctx_capacity, size_t* device_bytes) {
    return guard([&] {
        RL_ENGINE(e);
        if (vocab) *vocab = e->e->vocab();
        if (hidden) *hidden = e->e->hidden();
        if (ctx_capacity) *ctx_capacity = e->e->ctx_capacity();
        if (device_bytes) *device_bytes = e->e->device_bytes();
    });
}
void* rl_hip_engine_stream(RlEngine* e) { return e && e->e ? e->e->stream() : nullptr; }

int rl_hip_engine_max_batch(RlEngine* e, int* max_batch) {
    return guard([&] {
        RL_ENGINE(e);
        RL_REQUIRE(max_batch, RL_ERR_RANGE, "max_batch: null output");
        *max_batch = e->e->max_batch();
    });
}
int rl_hip_engine_decode_tokens(RlEngine* e, const int32_t* tokens, const int* poss, int B) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->decode_tokens(tokens, poss, B);
    });
}
int rl_hip_engine_copy_logits_n(RlEngine* e, float* host, int B) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->copy_logits_n(host, B);
    });
}
int rl_hip_engine_copy_greedy_n(RlEngine* e, int32_t* host, int B) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->copy_greedy_n(host, B);
    });
}
int rl_hip_engine_replicate_slot0(RlEngine* e, int n_slots) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->replicate_slot0(n_slots);
    });
}
int rl_hip_engine_zero_slots(RlEngine* e, int n_slots) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->zero_slots(n_slots);
    });
}
int rl_hip_engine_prefill_slot(RlEngine* e, const int32_t* ids, int n, int slot) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->prefill_slot(ids, n, slot);
    });
}
int rl_hip_engine_prefill_eq_batch(RlEngine* e, const int32_t* ids, int T, int B) {
    return guard([&] {
        RL_ENGINE(e);
        e->e->prefill_eq_batch(ids, T, B);
    });
}
int rl_hip_engine_time_layer(RlEngine* e, int layer, int T, int iters, float* ms) {
    return guard([&] {
        RL_ENGINE(e);
        RL_REQUIRE(ms, RL_ERR_RANGE, "time_layer: bad arguments");
        *ms = e->e->time_layer(layer, T, iters);
    });
}
int rl_hip_engine_time_batch(RlEngine* e, int B, int iters, float* ms) {
    return guard([&] {
        RL_ENGINE(e);
        RL_REQUIRE(ms && iters >= 1, RL_ERR_RANGE, "time_batch: bad arguments");
        *ms = e->e->time_batch(B, iters);
    });
}

}  // extern "C"
