// hip_device.cpp -- rapidllm::Device (include/rapidllm/backend/device.h:49-60) for
// HIP, with launch(name, args, params) mapped onto the backend's kernel entry points.
//
// Kernel names and parameter structs are the reference's (params.h:5-22, the name
// table in docs/architecture.md:1040-1059); the argument order follows the matching
// ops:: function (include/rapidllm/kernels/ops.h) -- Session::dev_rms passes
// {x, gamma, y} with {n, eps} (src/runtime/session.cpp:96-118), and the others keep
// that convention:
//   rmsnorm          {x, gamma, y}                      RmsNormParams
//   gated_rmsnorm    {x, z, gamma, y}                   RmsNormParams (gamma_n = gamma's length)
//   gemv_fp8         {W u8 [m][n], scale f32, x, y}     GemvFp8Params (block 128)
//   gemv_q4k/q6k     {W blocks [m][n/256], x, y}        GemvKQuantParams
//   conv1d_update    {x_t, w, state, y}                 Conv1dParams (silu 1)
//   delta_recurrent  {S, q, k, v, beta, g_log, o}       DeltaRecurrentParams
//   attn_decode      {q, k_cache, v_cache, o} fp32      AttnDecodeParams (pos, kv_dtype F32)
// The linears read the device's tiled weight layouts: the first launch on a weight
// buffer packs it into a cache keyed by the buffer's serial number (unique for the
// process, never reused when an allocator hands out the same address again) and
// the view's offset and shape. Weights are immutable once uploaded, as
// WeightStore's are; forget() drops a buffer's entries after its contents change,
// and a destroyed buffer's entries are freed by the device's next call.
// Each Stream owns its activation-fragment buffer and its K-quant split-K
// workspace (tickets and partials), so launches on different streams never share
// them.
#include "hip_backend.h"

#include "rapidllm/backend/params.h"
#include "rapidllm_hip.h"

#include <atomic>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>

namespace rapidllm::hip_gen {
namespace {

void check(int st) {
    if (st != RL_OK) throw std::runtime_error(std::string("hip device: ") + rl_hip_last_error());
}

// DeviceKind's entry for HIP: the enumerator a HIP build appends after CUDA
// (device.h:12 lists CPU, Vulkan, CUDA).
constexpr DeviceKind kHipKind = static_cast<DeviceKind>(3);

// Serial numbers of destroyed buffers, handed from ~HipBuffer to the device that
// allocated them (which may already be gone: the buffer holds it weakly).
struct Graveyard {
    std::mutex mu;
    std::vector<uint64_t> ids;
};

uint64_t next_serial() {
    static std::atomic<uint64_t> n{0};
    return ++n;
}

class HipBuffer final : public Buffer {
public:
    HipBuffer(size_t n, bool host, std::weak_ptr<Graveyard> gy)
        : n_(n), host_(host), serial_(next_serial()), gy_(std::move(gy)) {
        check(host ? rl_hip_host_alloc(&p_, n) : rl_hip_malloc(&p_, n));
    }
    ~HipBuffer() override {
        if (auto g = gy_.lock()) {
            std::lock_guard<std::mutex> lk(g->mu);
            g->ids.push_back(serial_);
        }
        if (host_)
            rl_hip_host_free(p_);
        else
            rl_hip_free(p_);
    }
    uint64_t serial() const { return serial_; }
    // Host-visible buffers are pinned host memory (host and device use the same
    // address); device buffers have no host mapping.
    void* host_ptr() override { return host_ ? p_ : nullptr; }
    size_t bytes() const override { return n_; }
    void* device_ptr() const { return p_; }
    bool host() const { return host_; }

private:
    void* p_ = nullptr;
    size_t n_ = 0;
    bool host_ = false;
    uint64_t serial_ = 0;
    std::weak_ptr<Graveyard> gy_;
};

// grow a device scratch buffer to `need` bytes; true when (re)allocated
bool grow(void*& p, size_t& have, size_t need) {
    if (have >= need && p) return false;
    rl_hip_free(p);
    p = nullptr;
    check(rl_hip_malloc(&p, need));
    have = need;
    return true;
}

class HipStream final : public Stream {
public:
    HipStream() { check(rl_hip_stream_create(&s_)); }
    ~HipStream() override {
        if (frag_ || ws_) (void)rl_hip_stream_synchronize(s_);
        rl_hip_free(frag_);
        rl_hip_free(ws_);
        rl_hip_stream_destroy(s_);
    }
    void begin_step(const char*) override {}
    void end_step() override {}
    void synchronize() override { check(rl_hip_stream_synchronize(s_)); }
    void* handle() const { return s_; }
    // activation fragments of a GEMM's input (this stream's launches only)
    void* frag(size_t need) {
        grow(frag_, frag_bytes_, need);
        return frag_;
    }
    // split-K tickets and partials; tickets start at zero and the GEMV leaves them zero
    void* ws(size_t need, size_t* have) {
        if (grow(ws_, ws_bytes_, need)) check(rl_hip_memset(ws_, 0, ws_bytes_, s_));
        *have = ws_bytes_;
        return ws_;
    }

private:
    void* s_ = nullptr;
    void* frag_ = nullptr;
    size_t frag_bytes_ = 0;
    void* ws_ = nullptr;
    size_t ws_bytes_ = 0;
};

size_t dtype_bytes(DType d) {
    switch (d) {
    case DType::F32:
    case DType::I32: return 4;
    case DType::F16:
    case DType::BF16: return 2;
    case DType::F8_E4M3:
    case DType::I8: return 1;
    default: throw std::runtime_error("hip device: no element size for a block-quantised view");
    }
}

void* dptr(const TensorView& v) {
    const auto* b = dynamic_cast<const HipBuffer*>(v.buf);
    if (!b) throw std::runtime_error("hip device: tensor view is not on a HIP buffer");
    return static_cast<uint8_t*>(b->device_ptr()) + v.byte_offset;
}

size_t view_bytes(const TensorView& v) {
    if (v.ndim <= 0) return 0;
    size_t n = dtype_bytes(v.dtype);
    for (int k = 0; k < v.ndim; ++k) n *= static_cast<size_t>(v.shape[k]);
    return n;
}

template <class P>
const P& params_as(const void* params, size_t bytes, const char* name) {
    if (!params || bytes < sizeof(P)) throw std::runtime_error(std::string("hip device: bad params for ") + name);
    return *static_cast<const P*>(params);
}

void need_args(int nargs, int want, const char* name) {
    if (nargs < want) throw std::runtime_error(std::string("hip device: ") + name + " needs " + std::to_string(want) + " args");
}

class HipDevice final : public Device {
public:
    ~HipDevice() override {
        for (auto& [k, p] : fp8_) {
            rl_hip_free(p.w);
            rl_hip_free(p.ts);
        }
        for (auto& [k, w] : kq_) rl_hip_free(w);
    }
    DeviceKind kind() const override { return kHipKind; }
    const char* name() const override { return "hip"; }
    std::unique_ptr<Buffer> allocate(const BufferDesc& d) override {
        return std::make_unique<HipBuffer>(d.bytes, d.host_visible || d.usage == BufferDesc::Usage::HostStaging,
                                           graveyard_);
    }
    std::unique_ptr<Stream> create_stream() override { return std::make_unique<HipStream>(); }

    void memcpy(TensorView dst, TensorView src, Stream& s) override {
        const size_t n = view_bytes(src);
        if (view_bytes(dst) < n) throw std::runtime_error("hip device: memcpy destination too small");
        const auto* db = dynamic_cast<const HipBuffer*>(dst.buf);
        const auto* sb = dynamic_cast<const HipBuffer*>(src.buf);
        if (!db || !sb) throw std::runtime_error("hip device: memcpy between non-HIP buffers");
        void* st = stream_of(s);
        if (db->host() && sb->host()) {
            check(rl_hip_stream_synchronize(st));
            std::memcpy(dptr(dst), dptr(src), n);
        } else if (sb->host()) {
            check(rl_hip_memcpy_h2d(dptr(dst), dptr(src), n, st));
        } else if (db->host()) {
            check(rl_hip_memcpy_d2h(dptr(dst), dptr(src), n, st));
        } else {
            check(rl_hip_memcpy_d2d(dptr(dst), dptr(src), n, st));
        }
    }

    bool has_kernel(const char* k) const override {
        static const char* names[] = {"rmsnorm",       "gated_rmsnorm",   "gemv_fp8",   "gemv_q4k", "gemv_q6k",
                                      "conv1d_update", "delta_recurrent", "attn_decode"};
        for (const char* n : names)
            if (std::strcmp(n, k) == 0) return true;
        return false;
    }

    void launch(const char* k, const TensorView* a, int nargs, const void* params, size_t pbytes,
                Stream& s) override {
        HipStream& hs = hip_stream(s);
        void* st = hs.handle();
        bury();
        const std::string name(k);
        if (name == "rmsnorm") {
            need_args(nargs, 3, k);
            const auto& p = params_as<RmsNormParams>(params, pbytes, k);
            check(rl_hip_rmsnorm_pack(f(a[0]), p.n, f(a[1]), f(a[2]), nullptr, p.n, 1, p.eps, st));
        } else if (name == "gated_rmsnorm") {
            need_args(nargs, 4, k);
            const auto& p = params_as<RmsNormParams>(params, pbytes, k);
            const int gamma_n = a[2].ndim >= 1 ? static_cast<int>(a[2].shape[0]) : p.n;
            check(rl_hip_gated_rmsnorm_pack(f(a[0]), f(a[1]), p.n, f(a[2]), gamma_n, f(a[3]), nullptr, p.n, 1, p.eps, st));
        } else if (name == "gemv_fp8") {
            need_args(nargs, 4, k);
            const auto& p = params_as<GemvFp8Params>(params, pbytes, k);
            if (p.block != 128) throw std::runtime_error("hip device: gemv_fp8 needs 128x128 block scales");
            const Fp8Packed& w = fp8_packed(a[0], a[1], p.m, p.n, st);
            void* frag = hs.frag(rl_hip_act_frag_bytes(p.n, 1));
            check(rl_hip_gemm_fp8(w.w, w.ts, f(a[2]), f(a[3]), frag, p.m, p.n, 1, st));
        } else if (name == "gemv_q4k" || name == "gemv_q6k") {
            need_args(nargs, 3, k);
            const auto& p = params_as<GemvKQuantParams>(params, pbytes, k);
            const int type = name == "gemv_q4k" ? RL_Q_Q4_K : RL_Q_Q6_K;
            uint8_t* w = kq_packed(type, a[0], p.m, p.n, st);
            size_t ws_bytes = 0;
            void* ws = hs.ws(rl_hip_kquant_workspace_bytes(p.m, p.n, 1), &ws_bytes);
            check(rl_hip_gemm_kquant(type, w, f(a[1]), f(a[2]), ws, ws_bytes, p.m, p.n, 1, 0, st));
        } else if (name == "conv1d_update") {
            need_args(nargs, 4, k);
            const auto& p = params_as<Conv1dParams>(params, pbytes, k);
            if (!p.silu) throw std::runtime_error("hip device: conv1d_update without SiLU is not provided");
            check(rl_hip_conv1d_update(f(a[0]), f(a[1]), f(a[2]), f(a[3]), p.dim, p.k, st));
        } else if (name == "delta_recurrent") {
            need_args(nargs, 7, k);
            const auto& p = params_as<DeltaRecurrentParams>(params, pbytes, k);
            check(rl_hip_delta_recurrent(f(a[0]), f(a[1]), f(a[2]), f(a[3]), f(a[4]), f(a[5]), f(a[6]), p.n_v, p.dk,
                                         p.dv, p.eps_l2, st));
        } else if (name == "attn_decode") {
            need_args(nargs, 4, k);
            const auto& p = params_as<AttnDecodeParams>(params, pbytes, k);
            if (p.kv_dtype != static_cast<int>(DType::F32))
                throw std::runtime_error("hip device: attn_decode takes fp32 caches (the decode engine keeps fp16)");
            check(rl_hip_attn_decode_f32(f(a[0]), f(a[1]), f(a[2]), f(a[3]), p.pos, p.n_q, p.n_kv, p.head_dim, st));
        } else {
            throw std::runtime_error("hip device: no kernel named " + name);
        }
    }

    // Drop the packed copy of a weight buffer (after its contents change).
    void forget(const Buffer* b) {
        const auto* hb = dynamic_cast<const HipBuffer*>(b);
        if (hb) drop(hb->serial());
    }

private:
    // free the packed copies of one buffer (by serial number)
    void drop(uint64_t id) {
        for (auto it = fp8_.begin(); it != fp8_.end();) {
            if (std::get<0>(it->first) == id) {
                rl_hip_free(it->second.w);
                rl_hip_free(it->second.ts);
                it = fp8_.erase(it);
            } else {
                ++it;
            }
        }
        for (auto it = kq_.begin(); it != kq_.end();) {
            if (std::get<0>(it->first) == id) {
                rl_hip_free(it->second);
                it = kq_.erase(it);
            } else {
                ++it;
            }
        }
    }

    // free the packed copies of buffers destroyed since the last launch (hipFree
    // waits for the device's queued work, which may still read them)
    void bury() {
        std::vector<uint64_t> ids;
        {
            std::lock_guard<std::mutex> lk(graveyard_->mu);
            ids.swap(graveyard_->ids);
        }
        for (uint64_t id : ids) drop(id);
    }

    struct Fp8Packed {
        uint8_t* w = nullptr;
        float* ts = nullptr;
    };
    // (buffer serial, view byte offset [K-quant: x16 + type], rows, cols)
    using Key = std::tuple<uint64_t, uint64_t, int, int>;

    static float* f(const TensorView& v) { return static_cast<float*>(dptr(v)); }
    static HipStream& hip_stream(Stream& s) {
        auto* hs = dynamic_cast<HipStream*>(&s);
        if (!hs) throw std::runtime_error("hip device: stream is not a HIP stream");
        return *hs;
    }
    static void* stream_of(Stream& s) { return hip_stream(s).handle(); }
    static uint64_t serial_of(const TensorView& v) {
        const auto* b = dynamic_cast<const HipBuffer*>(v.buf);
        if (!b) throw std::runtime_error("hip device: tensor view is not on a HIP buffer");
        return b->serial();
    }

    const Fp8Packed& fp8_packed(const TensorView& w, const TensorView& scale, int m, int n, void* st) {
        const Key key{serial_of(w), w.byte_offset, m, n};
        auto it = fp8_.find(key);
        if (it != fp8_.end()) return it->second;
        Fp8Packed p;
        check(rl_hip_malloc(reinterpret_cast<void**>(&p.w), rl_hip_fp8_packed_bytes(m, n)));
        check(rl_hip_malloc(reinterpret_cast<void**>(&p.ts), rl_hip_fp8_tile_scales(m, n) * sizeof(float)));
        check(rl_hip_pack_fp8(static_cast<const uint8_t*>(dptr(w)), f(scale), p.w, p.ts, m, n, st));
        return fp8_.emplace(key, p).first->second;
    }

    uint8_t* kq_packed(int type, const TensorView& w, int m, int n, void* st) {
        const Key key{serial_of(w), w.byte_offset * 16 + static_cast<uint64_t>(type), m, n};
        auto it = kq_.find(key);
        if (it != kq_.end()) return it->second;
        void* p = nullptr;
        check(rl_hip_malloc(&p, rl_hip_kquant_tiled_bytes(type, m, n)));
        check(rl_hip_pack_kquant(type, static_cast<const uint8_t*>(dptr(w)), static_cast<uint8_t*>(p), m, n, st));
        return kq_.emplace(key, static_cast<uint8_t*>(p)).first->second;
    }

    std::map<Key, Fp8Packed> fp8_;
    std::map<Key, uint8_t*> kq_;
    std::shared_ptr<Graveyard> graveyard_ = std::make_shared<Graveyard>();
};

}  // namespace

std::unique_ptr<Device> create_device() { return std::make_unique<HipDevice>(); }

}  // namespace rapidllm::hip_gen
