// loader.cpp -- on-disk checkpoints -> the engine's weight table (host code only).
//
// Replaces the reference's frontend: make_loader / IWeightLoader::load /
// WeightStore::open (include/rapidllm/frontend/weight_store.h:55-72,
// src/frontend/weight_store.cpp:125-155), the HF safetensors loader
// (src/frontend/hf_loader.cpp:87-251), the GGUF loader (src/frontend/
// gguf_loader.cpp:128-397) and the name maps (src/frontend/name_map.cpp:115-226).
//
// Files are memory-mapped; a tensor the engine takes as stored points into the
// mapping (no host copy before the upload).  Tensors that need a conversion get an
// owned buffer:
//   - FP8 `weight_scale_inv` in F32 / BF16 / F16 -> fp32 block scales
//     (hf_loader.cpp:186-219);
//   - F16 / BF16 norm weights, A_log, dt_bias, conv1d and other 1-D tensors ->
//     F32 (weight_store.cpp:13-25, 86-102);
//   - GGUF: DeltaNet in_proj_a / in_proj_b stored as Q8_0 / Q4_K / Q5_K / Q6_K ->
//     F32 (gguf_loader.cpp:323-352); the raw Qwen RMSNorm scale (mean >= 0.5) ->
//     scale - 1 for the (1 + gamma) kernels (weight_store.cpp:27-50); llama.cpp's
//     ssm_a = -exp(A_log) -> A_log = log(max(-ssm_a, 1e-20)), which also marks
//     the file's V heads as tiled (weight_store.cpp:52-84, 144-153).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <filesystem>
#include <map>
#include <memory>
#include <regex>
#include <set>
#include <string>
#include <string_view>
#include <vector>

#include "common.h"

#pragma clang fp contract(off)

namespace fs = std::filesystem;

namespace rl {
namespace {

// ------------------------------------------------------------------ errors
[[noreturn]] void fail(int code, const std::string& m) { throw Error(code, m); }
[[noreturn]] void bad(const std::string& m) { fail(RL_ERR_FORMAT, m); }

// ------------------------------------------------------------------ JSON
// Enough JSON for config.json, model.safetensors.index.json and safetensors
// headers: objects, arrays, strings (with escapes), numbers, true / false / null.
struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json* get(std::string_view k) const {
        if (kind != Obj) return nullptr;
        for (auto& [key, v] : obj)
            if (key == k) return &v;
        return nullptr;
    }
};

class JsonParser {
public:
    explicit JsonParser(std::string_view s) : s_(s) {}
    Json parse() {
        Json v = value(0);
        ws();
        if (i_ != s_.size()) err("trailing characters");
        return v;
    }

private:
    std::string_view s_;
    size_t i_ = 0;

    [[noreturn]] void err(const char* what) { bad(std::string("JSON: ") + what + " at offset " + std::to_string(i_)); }
    void ws() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
    }
    char peek() {
        ws();
        if (i_ >= s_.size()) err("unexpected end");
        return s_[i_];
    }
    void expect(char c) {
        if (peek() != c) err("unexpected character");
        ++i_;
    }
    bool word(std::string_view w) {
        if (s_.substr(i_, w.size()) == w) {
            i_ += w.size();
            return true;
        }
        return false;
    }
    static void put_utf8(std::string& o, uint32_t cp) {
        if (cp < 0x80) {
            o += static_cast<char>(cp);
        } else if (cp < 0x800) {
            o += static_cast<char>(0xC0 | (cp >> 6));
            o += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            o += static_cast<char>(0xE0 | (cp >> 12));
            o += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            o += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            o += static_cast<char>(0xF0 | (cp >> 18));
            o += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            o += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            o += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }
    uint32_t hex4() {
        if (i_ + 4 > s_.size()) err("short \\u escape");
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = s_[i_++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else err("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        expect('"');
        std::string o;
        while (true) {
            if (i_ >= s_.size()) err("unterminated string");
            const char c = s_[i_++];
            if (c == '"') break;
            if (c != '\\') {
                o += c;
                continue;
            }
            if (i_ >= s_.size()) err("unterminated escape");
            const char e = s_[i_++];
            switch (e) {
            case '"': o += '"'; break;
            case '\\': o += '\\'; break;
            case '/': o += '/'; break;
            case 'b': o += '\b'; break;
            case 'f': o += '\f'; break;
            case 'n': o += '\n'; break;
            case 'r': o += '\r'; break;
            case 't': o += '\t'; break;
            case 'u': {
                uint32_t cp = hex4();
                if (cp >= 0xD800 && cp < 0xDC00 && s_.substr(i_, 2) == "\\u") {
                    i_ += 2;
                    const uint32_t lo = hex4();
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                put_utf8(o, cp);
                break;
            }
            default: err("bad escape");
            }
        }
        return o;
    }
    Json value(int depth) {
        if (depth > 64) err("nesting too deep");
        Json v;
        const char c = peek();
        if (c == '{') {
            ++i_;
            v.kind = Json::Obj;
            if (peek() == '}') {
                ++i_;
                return v;
            }
            while (true) {
                std::string k = string();
                expect(':');
                v.obj.emplace_back(std::move(k), value(depth + 1));
                const char d = peek();
                ++i_;
                if (d == '}') break;
                if (d != ',') err("expected , or }");
            }
        } else if (c == '[') {
            ++i_;
            v.kind = Json::Arr;
            if (peek() == ']') {
                ++i_;
                return v;
            }
            while (true) {
                v.arr.push_back(value(depth + 1));
                const char d = peek();
                ++i_;
                if (d == ']') break;
                if (d != ',') err("expected , or ]");
            }
        } else if (c == '"') {
            v.kind = Json::Str;
            v.str = string();
        } else if (word("true")) {
            v.kind = Json::Bool;
            v.b = true;
        } else if (word("false")) {
            v.kind = Json::Bool;
        } else if (word("null")) {
        } else {
            const size_t b = i_;
            while (i_ < s_.size() && s_[i_] != '\0' && std::strchr("+-0123456789.eE", s_[i_])) ++i_;
            if (b == i_) err("unexpected character");
            v.kind = Json::Num;
            v.num = std::strtod(std::string(s_.substr(b, i_ - b)).c_str(), nullptr);
        }
        return v;
    }
};

int64_t as_int(const Json& j, const char* what) {
    if (j.kind != Json::Num) bad(std::string(what) + ": expected a number");
    return static_cast<int64_t>(j.num);
}

// ------------------------------------------------------------------ mapped files
struct MappedFile {
    std::string path;
    const uint8_t* p = nullptr;
    size_t size = 0;

    explicit MappedFile(const fs::path& f) : path(f.string()) {
        const int fd = ::open(path.c_str(), O_RDONLY);
        if (fd < 0) fail(RL_ERR_IO, "cannot open " + path);
        struct stat st {};
        if (::fstat(fd, &st) != 0) {
            ::close(fd);
            fail(RL_ERR_IO, "cannot stat " + path);
        }
        size = static_cast<size_t>(st.st_size);
        if (size) {
            void* m = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
            if (m == MAP_FAILED) {
                ::close(fd);
                fail(RL_ERR_IO, "cannot map " + path);
            }
            p = static_cast<const uint8_t*>(m);
        }
        ::close(fd);
    }
    ~MappedFile() {
        if (p) ::munmap(const_cast<uint8_t*>(p), size);
    }
    MappedFile(const MappedFile&) = delete;
    MappedFile& operator=(const MappedFile&) = delete;
};

// ------------------------------------------------------------------ numbers
float f16_to_f32(uint16_t h) {
    const uint32_t s = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FFu;
    uint32_t u;
    if (e == 0) {
        if (m == 0) {
            u = s;
        } else {  // subnormal: m * 2^-24, exact in fp32
            const float v = static_cast<float>(m) * 0x1p-24f;
            std::memcpy(&u, &v, 4);
            u |= s;
        }
    } else if (e == 31) {
        u = s | 0x7F800000u | (m << 13);
    } else {
        u = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

float bf16_to_f32(uint16_t h) {
    const uint32_t u = static_cast<uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

uint16_t rd16(const uint8_t* p) {
    uint16_t v;
    std::memcpy(&v, p, 2);
    return v;
}

// GGML block formats (public llama.cpp layouts).  Each value is rounded as the
// reference's scalar dequantisers round it: the block scale product first, then
// the quant multiply, then the min subtraction (src/kernels/ops.cpp:199-210,
// 255-282, 307-337, 357-385); this file is compiled without FMA contraction.
void q4k_sm(const uint8_t* sc, int j, int& s, int& m) {
    if (j < 4) {
        s = sc[j] & 63;
        m = sc[j + 4] & 63;
    } else {
        s = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4);
        m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}

void deq_q8_0(const uint8_t* p, float* y, int64_t n) {
    for (int64_t b = 0; b < n / 32; ++b, p += 34) {
        const float d = f16_to_f32(rd16(p));
        for (int i = 0; i < 32; ++i) y[b * 32 + i] = d * static_cast<float>(static_cast<int8_t>(p[2 + i]));
    }
}

void deq_q4_k(const uint8_t* p, float* y, int64_t n) {
    for (int64_t b = 0; b < n / 256; ++b, p += 144) {
        const float d = f16_to_f32(rd16(p)), dmin = f16_to_f32(rd16(p + 2));
        const uint8_t* q = p + 16;
        float* o = y + b * 256;
        for (int c = 0; c < 4; ++c) {
            int s0, m0, s1, m1;
            q4k_sm(p + 4, 2 * c, s0, m0);
            q4k_sm(p + 4, 2 * c + 1, s1, m1);
            const float a0 = d * static_cast<float>(s0), b0 = dmin * static_cast<float>(m0);
            const float a1 = d * static_cast<float>(s1), b1 = dmin * static_cast<float>(m1);
            for (int l = 0; l < 32; ++l) {
                o[64 * c + l] = a0 * static_cast<float>(q[32 * c + l] & 0xF) - b0;
                o[64 * c + 32 + l] = a1 * static_cast<float>(q[32 * c + l] >> 4) - b1;
            }
        }
    }
}

void deq_q5_k(const uint8_t* p, float* y, int64_t n) {
    for (int64_t b = 0; b < n / 256; ++b, p += 176) {
        const float d = f16_to_f32(rd16(p)), dmin = f16_to_f32(rd16(p + 2));
        const uint8_t* qh = p + 16;
        const uint8_t* ql = p + 48;
        float* o = y + b * 256;
        for (int c = 0; c < 4; ++c) {
            int s0, m0, s1, m1;
            q4k_sm(p + 4, 2 * c, s0, m0);
            q4k_sm(p + 4, 2 * c + 1, s1, m1);
            const float a0 = d * static_cast<float>(s0), b0 = dmin * static_cast<float>(m0);
            const float a1 = d * static_cast<float>(s1), b1 = dmin * static_cast<float>(m1);
            for (int l = 0; l < 32; ++l) {
                const int lo = (ql[32 * c + l] & 0xF) + (((qh[l] >> (2 * c)) & 1) << 4);
                const int hi = (ql[32 * c + l] >> 4) + (((qh[l] >> (2 * c + 1)) & 1) << 4);
                o[64 * c + l] = a0 * static_cast<float>(lo) - b0;
                o[64 * c + 32 + l] = a1 * static_cast<float>(hi) - b1;
            }
        }
    }
}

void deq_q6_k(const uint8_t* p, float* y, int64_t n) {
    for (int64_t b = 0; b < n / 256; ++b, p += 210) {
        const float d = f16_to_f32(rd16(p + 208));
        float* o = y + b * 256;
        for (int h = 0; h < 2; ++h) {
            const uint8_t* ql = p + 64 * h;
            const uint8_t* qh = p + 128 + 32 * h;
            const int8_t* sc = reinterpret_cast<const int8_t*>(p + 192 + 8 * h);
            for (int l = 0; l < 32; ++l) {
                const int q[4] = {((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32,
                                  ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32,
                                  ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32,
                                  ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32};
                for (int r = 0; r < 4; ++r)
                    o[128 * h + 32 * r + l] = d * static_cast<float>(sc[l / 16 + 2 * r]) * static_cast<float>(q[r]);
            }
        }
    }
}

// ------------------------------------------------------------------ name maps
// Source tensor names -> the IR names the engine takes (the reference's
// name_map.cpp tables; "" = not a language-model tensor this path uses).
bool starts(std::string_view s, std::string_view p) { return s.substr(0, p.size()) == p; }
bool ends(std::string_view s, std::string_view p) { return s.size() >= p.size() && s.substr(s.size() - p.size()) == p; }
bool has(std::string_view s, std::string_view p) { return s.find(p) != std::string_view::npos; }

bool is_visual(std::string_view n) {  // name_map.cpp:12-16
    return has(n, "visual") || has(n, "vision");
}

std::string layer_ir(const std::string& idx, const char* rest) { return "layers[" + idx + "]." + rest; }

// per-layer tails shared by the MTP block and the main stack (HF and GGUF spellings)
const char* common_tail(const std::string& t) {
    static const std::map<std::string, const char*> m = {
        {"input_layernorm.weight", "attn_norm"},      {"attn_norm.weight", "attn_norm"},
        {"post_attention_layernorm.weight", "ffn_norm"}, {"ffn_norm.weight", "ffn_norm"},
        {"self_attn.q_proj.weight", "attn.wq"},       {"attn_q.weight", "attn.wq"},
        {"self_attn.k_proj.weight", "attn.wk"},       {"attn_k.weight", "attn.wk"},
        {"self_attn.v_proj.weight", "attn.wv"},       {"attn_v.weight", "attn.wv"},
        {"self_attn.o_proj.weight", "attn.wo"},       {"attn_output.weight", "attn.wo"},
        {"self_attn.q_norm.weight", "attn.q_norm"},   {"attn_q_norm.weight", "attn.q_norm"},
        {"self_attn.k_norm.weight", "attn.k_norm"},   {"attn_k_norm.weight", "attn.k_norm"},
        {"mlp.gate_proj.weight", "mlp.gate"},         {"ffn_gate.weight", "mlp.gate"},
        {"mlp.up_proj.weight", "mlp.up"},             {"ffn_up.weight", "mlp.up"},
        {"mlp.down_proj.weight", "mlp.down"},         {"ffn_down.weight", "mlp.down"},
    };
    auto it = m.find(t);
    return it == m.end() ? nullptr : it->second;
}

// "mtp." / "nextn." tails (name_map.cpp:20-54)
std::string map_mtp(const std::string& rest) {
    if (rest == "fc.weight") return "mtp.fc";
    if (rest == "norm.weight") return "mtp.norm";
    if (rest == "pre_fc_norm_hidden.weight") return "mtp.pre_fc_norm_hidden";
    if (rest == "pre_fc_norm_embedding.weight") return "mtp.pre_fc_norm_embedding";
    static const std::regex re(R"((?:layers\.|blk\.)?(\d+)\.(.+))");
    std::smatch m;
    if (!std::regex_match(rest, m, re)) return {};
    const char* t = common_tail(m[2].str());
    return t ? "mtp.layers[" + m[1].str() + "]." + t : std::string();
}

std::string map_hf(const std::string& src) {  // name_map.cpp:115-164
    if (is_visual(src)) return {};
    std::string s = src;
    if (starts(s, "model.language_model.")) s = s.substr(21);
    else if (starts(s, "model.") && !has(s, "language_model")) s = s.substr(6);
    if (starts(src, "mtp.")) return map_mtp(src.substr(4));
    if (starts(s, "mtp.")) return map_mtp(s.substr(4));
    if (s == "embed_tokens.weight") return "embed";
    if (s == "lm_head.weight" || src == "lm_head.weight") return "lm_head";
    if (s == "norm.weight" || s == "language_model.norm.weight") return "final_norm";
    static const std::regex re(R"(layers\.(\d+)\.(.+))");
    std::smatch m;
    if (!std::regex_match(s, m, re)) return {};
    const std::string i = std::to_string(std::stoi(m[1].str())), rest = m[2].str();
    if (const char* t = common_tail(rest)) return layer_ir(i, t);
    static const std::map<std::string, const char*> delta = {
        {"linear_attn.in_proj_qkv.weight", "delta.gemm.in_proj_qkv"},
        {"linear_attn.in_proj_qkvz.weight", "delta.gemm.in_proj_qkv"},
        {"linear_attn.in_proj_z.weight", "delta.gemm.in_proj_z"},
        {"linear_attn.out_proj.weight", "delta.gemm.out_proj"},
        {"linear_attn.in_proj_a.weight", "delta.leftover.in_proj_a"},
        {"linear_attn.in_proj_b.weight", "delta.leftover.in_proj_b"},
        {"linear_attn.in_proj_ba.weight", "delta.leftover.in_proj_ba"},
        {"linear_attn.A_log", "delta.leftover.a_log"},
        {"linear_attn.dt_bias", "delta.leftover.dt_bias"},
        {"linear_attn.conv1d.weight", "delta.leftover.conv1d"},
        {"linear_attn.norm.weight", "delta.leftover.norm"},
    };
    auto it = delta.find(rest);
    return it == delta.end() ? std::string() : layer_ir(i, it->second);
}

std::string map_gguf(const std::string& s) {  // name_map.cpp:166-226
    if (starts(s, "nextn.") || starts(s, "mtp.")) {
        std::string ir = map_mtp(s.substr(s.find('.') + 1));
        if (!ir.empty()) return ir;
    }
    static const std::regex re_nextn(R"(blk\.(\d+)\.nextn\.(.+))");
    std::smatch m;
    if (std::regex_match(s, m, re_nextn)) {
        std::string t = m[2].str();
        if (ends(t, ".weight")) t.resize(t.size() - 7);
        if (t == "eh_proj") return "mtp.fc";
        if (t == "enorm") return "mtp.pre_fc_norm_embedding";
        if (t == "hnorm") return "mtp.pre_fc_norm_hidden";
        if (t == "shared_head_norm") return "mtp.norm";
        std::string ir = map_mtp("0." + m[2].str());
        if (!ir.empty()) return ir;
    }
    if (s == "token_embd.weight") return "embed";
    if (s == "output.weight") return "lm_head";
    if (s == "output_norm.weight") return "final_norm";
    static const std::regex re(R"(blk\.(\d+)\.(.+))");
    if (!std::regex_match(s, m, re)) return {};
    const std::string i = std::to_string(std::stoi(m[1].str())), rest = m[2].str();
    static const std::map<std::string, const char*> delta = {
        {"attn_norm.weight", "attn_norm"},             {"ffn_norm.weight", "ffn_norm"},
        {"post_attention_norm.weight", "ffn_norm"},    {"attn_q.weight", "attn.wq"},
        {"attn_k.weight", "attn.wk"},                  {"attn_v.weight", "attn.wv"},
        {"attn_output.weight", "attn.wo"},             {"attn_o.weight", "attn.wo"},
        {"attn_q_norm.weight", "attn.q_norm"},         {"attn_k_norm.weight", "attn.k_norm"},
        {"ffn_gate.weight", "mlp.gate"},               {"ffn_up.weight", "mlp.up"},
        {"ffn_down.weight", "mlp.down"},
        {"ssm_in.weight", "delta.gemm.in_proj_qkv"},   {"in_proj_qkv.weight", "delta.gemm.in_proj_qkv"},
        {"attn_qkv.weight", "delta.gemm.in_proj_qkv"}, {"ssm_z.weight", "delta.gemm.in_proj_z"},
        {"in_proj_z.weight", "delta.gemm.in_proj_z"},  {"attn_gate.weight", "delta.gemm.in_proj_z"},
        {"ssm_out.weight", "delta.gemm.out_proj"},     {"ssm_a.weight", "delta.leftover.in_proj_a"},
        {"in_proj_a.weight", "delta.leftover.in_proj_a"}, {"ssm_alpha.weight", "delta.leftover.in_proj_a"},
        {"ssm_beta.weight", "delta.leftover.in_proj_b"}, {"in_proj_b.weight", "delta.leftover.in_proj_b"},
        {"ssm_a_log", "delta.leftover.a_log"},         {"A_log", "delta.leftover.a_log"},
        {"ssm_a", "delta.leftover.a_log"},             {"ssm_dt", "delta.leftover.dt_bias"},
        {"dt_bias", "delta.leftover.dt_bias"},         {"ssm_dt.bias", "delta.leftover.dt_bias"},
        {"ssm_conv1d.weight", "delta.leftover.conv1d"}, {"shortconv.weight", "delta.leftover.conv1d"},
        {"ssm_conv1d", "delta.leftover.conv1d"},       {"ssm_norm.weight", "delta.leftover.norm"},
        {"ssm_norm", "delta.leftover.norm"},
    };
    auto it = delta.find(rest);
    return it == delta.end() ? std::string() : layer_ir(i, it->second);
}

// DeltaNet leftovers and norms: never block-quantised on the engine side
// (name_map.cpp:56-66)
bool is_leftover(std::string_view n) {
    for (const char* k : {"A_log", "a_log", "dt_bias", "ssm_dt", "conv1d", "ssm_conv", "shortconv", "q_norm",
                          "k_norm", "input_layernorm", "post_attention_layernorm", "attn_norm", "ffn_norm",
                          "output_norm", ".norm.weight", "ssm_norm", "in_proj_a", "in_proj_b", "ssm_a",
                          "ssm_beta"})
        if (has(n, k)) return true;
    return false;
}

// ------------------------------------------------------------------ the table
struct Tensor {
    std::string ir, src;
    int quant = RL_Q_F32;
    int ndim = 0;
    int64_t shape[4] = {0, 0, 0, 0};
    int gguf_type = -1;
    const uint8_t* data = nullptr;  // into a mapping or into `own`
    size_t nbytes = 0;
    std::vector<uint8_t> own;
    std::vector<float> scale;

    int64_t numel() const {
        int64_t n = 1;
        for (int d = 0; d < ndim; ++d) n *= shape[d];
        return n;
    }
    void take(std::vector<uint8_t>&& v) {
        own = std::move(v);
        data = own.data();
        nbytes = own.size();
    }
    void set_f32(const std::vector<float>& f) {
        std::vector<uint8_t> b(f.size() * 4);
        std::memcpy(b.data(), f.data(), b.size());
        take(std::move(b));
        quant = RL_Q_F32;
    }
    float* f32() { return reinterpret_cast<float*>(own.data()); }
};

}  // namespace
}  // namespace rl

struct RlWeights {
    int source = 0;  // 0 HF safetensors directory, 1 GGUF file
    RlModelConfig cfg{};
    bool tie_embed = false;
    std::vector<std::unique_ptr<rl::MappedFile>> files;
    std::vector<rl::Tensor> tensors;
    std::vector<RlTensor> view;

    rl::Tensor* find(const std::string& ir) {
        for (auto& t : tensors)
            if (t.ir == ir) return &t;
        return nullptr;
    }
};

namespace rl {
namespace {

// Defaults: the 27B hybrid (model_desc.h:115-133) with layer kinds D D D A.
void default_27b(RlModelConfig& c) {
    c = RlModelConfig{};
    c.vocab = 248320;
    c.hidden = 5120;
    c.n_layers = 64;
    c.intermediate = 17408;
    c.n_k_heads = 16;
    c.n_v_heads = 48;
    c.k_dim = 128;
    c.v_dim = 128;
    c.conv_k = 4;
    c.n_q = 24;
    c.n_kv = 4;
    c.head_dim = 256;
    c.rotary_dim = 64;
    c.rope_theta = 1e7f;
    c.rms_eps = 1e-6f;
    for (int i = 0; i < 64; ++i) c.layer_kind[i] = (i % 4) == 3 ? RL_LAYER_ATTN : RL_LAYER_DELTA;
}

// The 8-layer test hybrid (src/ir/model_desc.cpp:77-110).
void default_tiny(RlModelConfig& c) {
    default_27b(c);
    c.vocab = 48;
    c.hidden = 32;
    c.n_layers = 8;
    c.intermediate = 64;
    c.n_k_heads = 2;
    c.n_v_heads = 6;
    c.k_dim = 8;
    c.v_dim = 8;
    c.n_q = 4;
    c.n_kv = 2;
    c.head_dim = 8;
    c.rotary_dim = 2;
    c.rope_theta = 10000.f;
}

void finish_tensor_shape(Tensor& t, const std::vector<int64_t>& shape) {
    if (shape.size() > 4) bad(t.src + ": more than 4 dimensions");
    t.ndim = static_cast<int>(shape.size());
    for (int d = 0; d < t.ndim; ++d) t.shape[d] = shape[d];
}

// ---- HF safetensors directory (hf_loader.cpp:87-251)
struct StEntry {
    std::string dtype;
    std::vector<int64_t> shape;
    const uint8_t* p;
    size_t bytes;
};

void read_safetensors(RlWeights& W, const fs::path& f, std::map<std::string, StEntry>& all) {
    W.files.push_back(std::make_unique<MappedFile>(f));
    const MappedFile& mf = *W.files.back();
    if (mf.size < 8) bad("safetensors: truncated header size in " + mf.path);
    uint64_t hlen;
    std::memcpy(&hlen, mf.p, 8);
    if (hlen > 64ull << 20 || 8 + hlen > mf.size) bad("safetensors: bad header length in " + mf.path);
    const Json h = JsonParser(std::string_view(reinterpret_cast<const char*>(mf.p) + 8, hlen)).parse();
    if (h.kind != Json::Obj) bad("safetensors: header is not an object in " + mf.path);
    const uint64_t base = 8 + hlen;
    for (auto& [name, meta] : h.obj) {
        if (name == "__metadata__" || meta.kind != Json::Obj) continue;
        const Json *dt = meta.get("dtype"), *sh = meta.get("shape"), *off = meta.get("data_offsets");
        if (!dt || dt->kind != Json::Str || !sh || sh->kind != Json::Arr || !off || off->kind != Json::Arr ||
            off->arr.size() != 2)
            bad("safetensors: bad entry " + name);
        StEntry e;
        e.dtype = dt->str;
        for (auto& d : sh->arr) e.shape.push_back(as_int(d, "shape"));
        const uint64_t b = static_cast<uint64_t>(as_int(off->arr[0], "offset")),
                       en = static_cast<uint64_t>(as_int(off->arr[1], "offset"));
        if (en < b || base + en > mf.size) bad("safetensors: data past EOF for " + name);
        e.p = mf.p + base + b;
        e.bytes = en - b;
        all[name] = std::move(e);
    }
}

void load_hf(RlWeights& W, const fs::path& dir, int max_layers) {
    const fs::path cfgp = dir / "config.json";
    MappedFile cf(cfgp);
    const Json root = JsonParser(std::string_view(reinterpret_cast<const char*>(cf.p), cf.size)).parse();
    const Json* tc = root.get("text_config");
    if (!tc) tc = &root;
    RlModelConfig& c = W.cfg;
    default_27b(c);
    auto geti = [&](const char* k, int& dst) {
        if (const Json* v = tc->get(k)) dst = static_cast<int>(as_int(*v, k));
    };
    geti("hidden_size", c.hidden);
    geti("intermediate_size", c.intermediate);
    geti("vocab_size", c.vocab);
    geti("linear_num_key_heads", c.n_k_heads);
    geti("linear_num_value_heads", c.n_v_heads);
    geti("linear_key_head_dim", c.k_dim);
    geti("linear_value_head_dim", c.v_dim);
    geti("linear_conv_kernel_dim", c.conv_k);
    geti("num_attention_heads", c.n_q);
    geti("num_key_value_heads", c.n_kv);
    geti("head_dim", c.head_dim);
    if (const Json* v = tc->get("rms_norm_eps")) c.rms_eps = static_cast<float>(v->num);
    if (const Json* v = tc->get("tie_word_embeddings")) W.tie_embed = v->kind == Json::Bool && v->b;
    float theta = c.rope_theta, partial = 0.25f;
    if (const Json* v = tc->get("rope_theta")) theta = static_cast<float>(v->num);
    if (const Json* rp = tc->get("rope_parameters"); rp && rp->kind == Json::Obj) {
        if (const Json* v = rp->get("rope_theta")) theta = static_cast<float>(v->num);
        if (const Json* v = rp->get("partial_rotary_factor")) partial = static_cast<float>(v->num);
    }
    if (const Json* v = tc->get("partial_rotary_factor")) partial = static_cast<float>(v->num);
    c.rope_theta = theta;
    c.rotary_dim = static_cast<int>(static_cast<float>(c.head_dim) * partial);
    const Json* lt = tc->get("layer_types");
    if (!lt || lt->kind != Json::Arr) bad("HF config missing text_config.layer_types");
    if (lt->arr.size() > RL_MAX_LAYERS) fail(RL_ERR_UNSUPPORTED, "HF config: too many layers");
    c.n_layers = static_cast<int>(lt->arr.size());
    int n_delta = 0;
    for (int i = 0; i < c.n_layers; ++i) {
        const std::string& t = lt->arr[i].str;
        if (t == "linear_attention") c.layer_kind[i] = RL_LAYER_DELTA, ++n_delta;
        else if (t == "full_attention") c.layer_kind[i] = RL_LAYER_ATTN;
        else fail(RL_ERR_UNSUPPORTED, "unknown layer_types entry: " + t);
    }
    if (max_layers > 0 && max_layers < c.n_layers) c.n_layers = max_layers;
    if (n_delta == 0) bad("HF hybrid missing DeltaNet layers");

    // shards: index.json weight_map, else model.safetensors, else every *.safetensors
    std::vector<fs::path> shards;
    if (fs::exists(dir / "model.safetensors.index.json")) {
        MappedFile ix(dir / "model.safetensors.index.json");
        const Json idx = JsonParser(std::string_view(reinterpret_cast<const char*>(ix.p), ix.size)).parse();
        const Json* wm = idx.get("weight_map");
        if (!wm || wm->kind != Json::Obj) bad("bad weight_map");
        std::set<std::string> seen;
        for (auto& [_, f] : wm->obj)
            if (seen.insert(f.str).second) shards.push_back(dir / f.str);
    } else if (fs::exists(dir / "model.safetensors")) {
        shards.push_back(dir / "model.safetensors");
    } else {
        for (auto& e : fs::directory_iterator(dir))
            if (e.path().extension() == ".safetensors") shards.push_back(e.path());
        if (shards.empty()) fail(RL_ERR_IO, "no safetensors in " + dir.string());
        std::sort(shards.begin(), shards.end());
    }
    std::map<std::string, StEntry> all;
    for (auto& s : shards) read_safetensors(W, s, all);

    for (auto& [name, e] : all) {
        const std::string ir = map_hf(name);
        if (ir.empty()) continue;
        if (max_layers > 0 && starts(ir, "layers[") && std::stoi(ir.substr(7)) >= max_layers) continue;
        Tensor t;
        t.ir = ir;
        t.src = name;
        finish_tensor_shape(t, e.shape);
        t.data = e.p;
        t.nbytes = e.bytes;
        if (e.dtype == "F32") t.quant = RL_Q_F32;
        else if (e.dtype == "F16") t.quant = RL_Q_F16;
        else if (e.dtype == "BF16") t.quant = RL_Q_BF16;
        else if (e.dtype == "F8_E4M3") t.quant = RL_Q_FP8_E4M3_B128;
        else fail(RL_ERR_UNSUPPORTED, name + ": unsupported safetensors dtype " + e.dtype);
        const size_t esz = t.quant == RL_Q_F32 ? 4 : t.quant == RL_Q_FP8_E4M3_B128 ? 1 : 2;
        if (t.nbytes != static_cast<size_t>(t.numel()) * esz) bad(name + ": byte size disagrees with its shape");
        if (t.quant == RL_Q_FP8_E4M3_B128) {
            std::string sname = name;
            const size_t w = sname.rfind(".weight");
            if (w != std::string::npos) sname.replace(w, 7, ".weight_scale_inv");
            auto it = all.find(sname);
            if (it == all.end()) it = all.find(name + ".weight_scale_inv");
            if (it == all.end()) bad("FP8 tensor missing weight_scale_inv: " + name);
            const StEntry& s = it->second;
            const int64_t rows = t.ndim >= 2 ? t.numel() / t.shape[t.ndim - 1] : t.numel();
            const int64_t cols = t.ndim >= 2 ? t.shape[t.ndim - 1] : 1;
            const size_t ns = static_cast<size_t>((rows + 127) / 128) * ((cols + 127) / 128);
            const size_t ssz = s.dtype == "F32" ? 4 : 2;
            if (s.dtype != "F32" && s.dtype != "BF16" && s.dtype != "F16")
                fail(RL_ERR_UNSUPPORTED, it->first + ": scale dtype " + s.dtype);
            if (s.bytes != ns * ssz) bad(it->first + ": expected " + std::to_string(ns) + " block scales");
            t.scale.resize(ns);
            for (size_t k = 0; k < ns; ++k) {
                if (ssz == 4) std::memcpy(&t.scale[k], s.p + 4 * k, 4);
                else t.scale[k] = s.dtype == "BF16" ? bf16_to_f32(rd16(s.p + 2 * k)) : f16_to_f32(rd16(s.p + 2 * k));
            }
        }
        W.tensors.push_back(std::move(t));
    }
}

// ---- GGUF file (gguf_loader.cpp:128-397)
class Cursor {
public:
    Cursor(const MappedFile& f) : f_(f) {}
    template <class T>
    T rd() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, f_.p + at, sizeof(T));
        at += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = rd<uint64_t>();
        if (n > (16u << 20)) bad("GGUF string too long");
        need(n);
        std::string s(reinterpret_cast<const char*>(f_.p + at), n);
        at += n;
        return s;
    }
    void need(uint64_t n) {
        if (at + n > f_.size) bad("GGUF truncated");
    }
    uint64_t at = 0;

private:
    const MappedFile& f_;
};

enum { G_U8, G_I8, G_U16, G_I16, G_U32, G_I32, G_F32, G_BOOL, G_STR, G_ARR, G_U64, G_I64, G_F64 };

// one metadata value: numbers widened to double, strings kept, arrays skipped
struct GVal {
    bool is_num = false, is_str = false;
    double num = 0;
    std::string str;
};

GVal read_value(Cursor& c, uint32_t t, int depth = 0) {
    GVal v;
    switch (t) {
    case G_U8: v.num = c.rd<uint8_t>(), v.is_num = true; break;
    case G_I8: v.num = c.rd<int8_t>(), v.is_num = true; break;
    case G_BOOL: v.num = c.rd<uint8_t>(), v.is_num = true; break;
    case G_U16: v.num = c.rd<uint16_t>(), v.is_num = true; break;
    case G_I16: v.num = c.rd<int16_t>(), v.is_num = true; break;
    case G_U32: v.num = c.rd<uint32_t>(), v.is_num = true; break;
    case G_I32: v.num = c.rd<int32_t>(), v.is_num = true; break;
    case G_F32: v.num = c.rd<float>(), v.is_num = true; break;
    case G_U64: v.num = static_cast<double>(c.rd<uint64_t>()), v.is_num = true; break;
    case G_I64: v.num = static_cast<double>(c.rd<int64_t>()), v.is_num = true; break;
    case G_F64: v.num = c.rd<double>(), v.is_num = true; break;
    case G_STR: v.str = c.str(), v.is_str = true; break;
    case G_ARR: {
        if (depth > 4) bad("GGUF arrays nested too deep");
        const uint32_t at = c.rd<uint32_t>();
        const uint64_t n = c.rd<uint64_t>();
        static const int fixed[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
        if (at < 13 && fixed[at]) {
            c.need(n * fixed[at]);
            c.at += n * fixed[at];
        } else {
            for (uint64_t i = 0; i < n; ++i) read_value(c, at, depth + 1);
        }
        break;
    }
    default: bad("GGUF unknown value type");
    }
    return v;
}

enum { GGML_F32 = 0, GGML_F16 = 1, GGML_Q8_0 = 8, GGML_Q4_K = 12, GGML_Q5_K = 13, GGML_Q6_K = 14, GGML_BF16 = 30 };

void load_gguf(RlWeights& W, const fs::path& path, int max_layers) {
    W.files.push_back(std::make_unique<MappedFile>(path));
    const MappedFile& mf = *W.files.back();
    if (mf.size < 4 || std::memcmp(mf.p, "GGUF", 4) != 0) bad("not a GGUF file");
    Cursor c(mf);
    c.at = 4;
    const uint32_t version = c.rd<uint32_t>();
    if (version < 2 || version > 3) fail(RL_ERR_UNSUPPORTED, "unsupported GGUF version");
    const uint64_t n_tensors = c.rd<uint64_t>(), n_kv = c.rd<uint64_t>();
    std::map<std::string, GVal> kv;
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string k = c.str();
        const uint32_t t = c.rd<uint32_t>();
        GVal v = read_value(c, t);
        if (v.is_num || v.is_str) kv[k] = std::move(v);
    }
    const std::string arch = kv.count("general.architecture") ? kv["general.architecture"].str : "";
    auto meta = [&](const std::string& key, double& out) {
        auto it = kv.find(arch + "." + key);
        if (it == kv.end() || !it->second.is_num) return false;
        out = it->second.num;
        return true;
    };
    uint64_t alignment = 32;
    if (auto it = kv.find("general.alignment"); it != kv.end() && it->second.is_num && it->second.num >= 1)
        alignment = static_cast<uint64_t>(it->second.num);

    struct Meta {
        std::string name;
        std::vector<int64_t> shape;  // slowest dimension first
        uint32_t type;
        uint64_t offset;
    };
    std::vector<Meta> metas(n_tensors);
    for (auto& m : metas) {
        m.name = c.str();
        const uint32_t nd = c.rd<uint32_t>();
        if (nd == 0 || nd > 4) bad("GGUF tensor " + m.name + ": bad rank");
        m.shape.resize(nd);
        for (uint32_t d = 0; d < nd; ++d) m.shape[nd - 1 - d] = static_cast<int64_t>(c.rd<uint64_t>());
        m.type = c.rd<uint32_t>();
        m.offset = c.rd<uint64_t>();
    }
    const uint64_t data0 = (c.at + alignment - 1) / alignment * alignment;

    // layer kinds from the tensor names; the last block holding nextn.* tensors is
    // the MTP block (gguf_loader.cpp:202-235)
    int max_blk = -1, mtp_blk = -1;
    std::vector<int> kind(RL_MAX_LAYERS + 1, -1);
    static const std::regex re_blk(R"(blk\.(\d+)\..*)");
    for (auto& m : metas) {
        if (is_visual(m.name)) continue;
        std::smatch sm;
        if (!std::regex_match(m.name, sm, re_blk)) continue;
        const int b = std::stoi(sm[1].str());
        if (b > RL_MAX_LAYERS) fail(RL_ERR_UNSUPPORTED, "GGUF: too many blocks");
        max_blk = std::max(max_blk, b);
        if (has(m.name, ".nextn.")) mtp_blk = std::max(mtp_blk, b);
        if (has(m.name, "ssm_") || has(m.name, "linear_attn") || has(m.name, "A_log") || has(m.name, "attn_qkv"))
            kind[b] = RL_LAYER_DELTA;
        if (has(m.name, "attn_q.weight") || has(m.name, "attn_q_norm")) kind[b] = RL_LAYER_ATTN;
    }
    if (max_blk < 0) bad("GGUF has no blk.* tensors; architecture=" + arch);
    double nextn = 0;
    if (mtp_blk < 0 && meta("nextn_predict_layers", nextn) && nextn > 0) mtp_blk = max_blk;
    int n_layers = max_blk + 1;
    if (mtp_blk >= 0 && mtp_blk == max_blk) n_layers = mtp_blk;
    int n_delta = 0;
    for (int i = 0; i < n_layers; ++i) n_delta += kind[i] == RL_LAYER_DELTA;
    if (n_delta == 0) bad("GGUF missing DeltaNet tensors (A_log/ssm_*); architecture=" + arch);

    // model description: the 27B hybrid or the 8-layer test hybrid
    // (gguf_loader.cpp:237-267), then the file's own dimensions where it has them
    int64_t emb_v = -1, emb_h = -1;
    for (auto& m : metas)
        if (m.name == "token_embd.weight" && m.shape.size() >= 2) emb_v = m.shape[0], emb_h = m.shape[1];
    double v = 0;
    int hidden = meta("embedding_length", v) ? static_cast<int>(v) : static_cast<int>(emb_h);
    int vocab = meta("vocab_size", v) ? static_cast<int>(v) : static_cast<int>(emb_v);
    const bool fam27 = has(arch, "qwen35") || has(arch, "qwen3_5") || has(arch, "qwen36") || has(arch, "qwen38") ||
                       has(arch, "qwen3_8") || has(arch, "qwen3.8");
    RlModelConfig& cfg = W.cfg;
    if ((n_layers >= 32 && (hidden == 5120 || emb_h == 5120)) || (fam27 && n_layers >= 32)) default_27b(cfg);
    else default_tiny(cfg);
    if (hidden > 0) cfg.hidden = hidden;
    if (vocab > 0) cfg.vocab = vocab;
    double blocks = 0;
    if (meta("block_count", blocks) && blocks != n_layers && blocks != n_layers + (mtp_blk == max_blk ? 1 : 0))
        bad("GGUF block_count mismatch");
    cfg.n_layers = n_layers;
    for (int i = 0; i < n_layers; ++i) cfg.layer_kind[i] = kind[i] == RL_LAYER_ATTN ? RL_LAYER_ATTN : RL_LAYER_DELTA;
    // llama.cpp qwen35 hyper-parameters (absent in the test hybrid's files)
    if (meta("feed_forward_length", v)) cfg.intermediate = static_cast<int>(v);
    if (meta("attention.head_count", v)) cfg.n_q = static_cast<int>(v);
    if (meta("attention.head_count_kv", v)) cfg.n_kv = static_cast<int>(v);
    if (meta("attention.key_length", v)) cfg.head_dim = static_cast<int>(v);
    if (meta("attention.layer_norm_rms_epsilon", v)) cfg.rms_eps = static_cast<float>(v);
    if (meta("rope.freq_base", v)) cfg.rope_theta = static_cast<float>(v);
    if (meta("rope.dimension_count", v)) cfg.rotary_dim = static_cast<int>(v);
    if (meta("ssm.conv_kernel", v)) cfg.conv_k = static_cast<int>(v);
    if (meta("ssm.state_size", v)) cfg.k_dim = static_cast<int>(v);
    if (meta("ssm.group_count", v)) cfg.n_k_heads = static_cast<int>(v);
    if (meta("ssm.time_step_rank", v)) cfg.n_v_heads = static_cast<int>(v);
    if (meta("ssm.inner_size", v) && cfg.n_v_heads > 0) cfg.v_dim = static_cast<int>(v) / cfg.n_v_heads;

    for (auto& m : metas) {
        if (is_visual(m.name)) continue;
        const std::string ir = map_gguf(m.name);
        if (ir.empty()) continue;
        if (max_layers > 0 && starts(ir, "layers[") && std::stoi(ir.substr(7)) >= max_layers) continue;
        Tensor t;
        t.ir = ir;
        t.src = m.name;
        t.gguf_type = static_cast<int>(m.type);
        finish_tensor_shape(t, m.shape);
        const int64_t ne = t.numel();
        const int64_t inner = m.shape.back();
        size_t nbytes;
        switch (m.type) {
        case GGML_F32: t.quant = RL_Q_F32, nbytes = ne * 4; break;
        case GGML_F16: t.quant = RL_Q_F16, nbytes = ne * 2; break;
        case GGML_BF16: t.quant = RL_Q_BF16, nbytes = ne * 2; break;
        case GGML_Q8_0: t.quant = RL_Q_Q8_0, nbytes = ne / 32 * 34; break;
        case GGML_Q4_K: t.quant = RL_Q_Q4_K, nbytes = ne / 256 * 144; break;
        case GGML_Q5_K: t.quant = RL_Q_Q5_K, nbytes = ne / 256 * 176; break;
        case GGML_Q6_K: t.quant = RL_Q_Q6_K, nbytes = ne / 256 * 210; break;
        default: fail(RL_ERR_UNSUPPORTED, "unsupported ggml_type " + std::to_string(m.type) + " on " + m.name);
        }
        if ((m.type == GGML_Q8_0 && inner % 32) ||
            ((m.type == GGML_Q4_K || m.type == GGML_Q5_K || m.type == GGML_Q6_K) && inner % 256))
            bad(m.name + ": row length not a whole number of blocks");
        if (data0 + m.offset + nbytes > mf.size) bad("GGUF truncated tensor " + m.name);
        t.data = mf.p + data0 + m.offset;
        t.nbytes = nbytes;
        if (is_leftover(ir) && (t.quant == RL_Q_Q8_0 || t.quant == RL_Q_Q4_K || t.quant == RL_Q_Q5_K ||
                                t.quant == RL_Q_Q6_K)) {
            // quantised in_proj_a / in_proj_b are dequantised; other leftovers must
            // be stored uncompressed (gguf_loader.cpp:323-352)
            const bool lin = has(ir, "in_proj_a") || has(ir, "in_proj_b") || has(ir, "in_proj_ba");
            if (!lin || ne <= 0 || ne > (64ll << 20)) bad("leftover over-quantized: " + m.name);
            std::vector<float> f(ne);
            if (t.quant == RL_Q_Q8_0) deq_q8_0(t.data, f.data(), ne);
            else if (t.quant == RL_Q_Q4_K) deq_q4_k(t.data, f.data(), ne);
            else if (t.quant == RL_Q_Q5_K) deq_q5_k(t.data, f.data(), ne);
            else deq_q6_k(t.data, f.data(), ne);
            t.set_f32(f);
        }
        W.tensors.push_back(std::move(t));
    }
    if (!W.find("embed")) bad("GGUF missing embed architecture=" + arch);
    if (max_layers > 0 && max_layers < cfg.n_layers) cfg.n_layers = max_layers;
    if (mtp_blk >= 0) {  // peel the NextN block off the main stack
        const std::string pre = "layers[" + std::to_string(mtp_blk) + "].";
        for (auto& t : W.tensors)
            if (starts(t.ir, pre)) t.ir = "mtp.layers[0]." + t.ir.substr(pre.size());
    }
    for (int i = 0; i < cfg.n_layers; ++i) {
        if (cfg.layer_kind[i] != RL_LAYER_DELTA) continue;
        const std::string p = "layers[" + std::to_string(i) + "].delta.leftover.";
        if (!W.find(p + "a_log") && !W.find(p + "conv1d"))
            bad("GGUF missing DeltaNet leftovers on blk." + std::to_string(i) + " architecture=" + arch);
    }
}

// ---- WeightStore::open post-processing (weight_store.cpp:13-50, 86-102, 137-155)
bool materialize_f32(const Tensor& t) {
    if (t.quant != RL_Q_F16 && t.quant != RL_Q_BF16) return false;
    const std::string& n = t.ir;
    if (has(n, "in_proj") || has(n, "gemm") || has(n, "mlp.") || has(n, "attn.w") || n == "embed" || n == "lm_head")
        return false;
    if (has(n, "norm") || has(n, "a_log") || has(n, "dt_bias") || has(n, "conv")) return true;
    return t.ndim == 1;
}

bool qwen_rms_gamma(const std::string& n) {
    if (has(n, "leftover.norm")) return false;
    return has(n, "attn_norm") || has(n, "ffn_norm") || n == "final_norm" || n == "mtp.norm" || has(n, "pre_fc_norm") ||
           has(n, "q_norm") || has(n, "k_norm");
}

bool llama_ssm_a(const std::string& src) {
    return ends(src, "ssm_a") && !ends(src, "ssm_a_log") && !ends(src, "ssm_a.weight");
}

void post_process(RlWeights& W) {
    for (auto& t : W.tensors) {
        if (!materialize_f32(t)) continue;
        const int64_t n = t.numel();
        std::vector<float> f(n);
        for (int64_t i = 0; i < n; ++i) {
            const uint16_t h = rd16(t.data + 2 * i);
            f[i] = t.quant == RL_Q_F16 ? f16_to_f32(h) : bf16_to_f32(h);
        }
        t.set_f32(f);
    }
    if (W.source != 1) return;
    for (auto& t : W.tensors) {
        if (t.quant != RL_Q_F32 || t.nbytes < 4) continue;
        const int64_t n = t.nbytes / 4;
        if (qwen_rms_gamma(t.ir)) {
            // raw GGUF Qwen RMSNorm scale (~1) -> the (1 + gamma) convention; files
            // already in that convention (mean < 0.5) stay as they are
            double mean = 0;
            for (int64_t i = 0; i < n; ++i) {
                float x;
                std::memcpy(&x, t.data + 4 * i, 4);
                mean += x;
            }
            if (mean / static_cast<double>(n) < 0.5) continue;
            std::vector<float> f(n);
            std::memcpy(f.data(), t.data, n * 4);
            for (auto& x : f) x -= 1.f;
            t.set_f32(f);
        } else if (has(t.ir, "a_log") && llama_ssm_a(t.src)) {
            std::vector<float> f(n);
            std::memcpy(f.data(), t.data, n * 4);
            for (auto& x : f) x = std::log(std::fmax(-x, 1e-20f));
            t.set_f32(f);
            W.cfg.v_tiled = 1;
        }
    }
}

void finish(RlWeights& W) {
    if (!W.find("lm_head")) {  // tied head (hf_loader.cpp:234-241)
        if (!W.tie_embed || !W.find("embed")) bad("HF missing required tensor lm_head");
        Tensor lh = *W.find("embed");
        lh.ir = "lm_head";
        lh.src = "tied:" + lh.src;
        if (!lh.own.empty()) lh.data = lh.own.data();
        W.tensors.push_back(std::move(lh));
    }
    if (W.source == 0) {
        for (const char* n : {"embed", "final_norm"})
            if (!W.find(n)) bad(std::string("HF missing required tensor ") + n);
        for (int i = 0; i < W.cfg.n_layers; ++i) {
            if (W.cfg.layer_kind[i] != RL_LAYER_DELTA) continue;
            for (const char* k : {"a_log", "conv1d"}) {
                const std::string n = "layers[" + std::to_string(i) + "].delta.leftover." + k;
                if (!W.find(n)) bad("HF missing required tensor " + n);
            }
        }
    }
    W.cfg.has_mtp = W.find("mtp.fc") && W.find("mtp.norm");
    // own buffers moved with their tensors: re-point data at them
    for (auto& t : W.tensors)
        if (!t.own.empty()) t.data = t.own.data();
    W.view.resize(W.tensors.size());
    for (size_t i = 0; i < W.tensors.size(); ++i) {
        const Tensor& t = W.tensors[i];
        RlTensor& r = W.view[i];
        r.name = t.ir.c_str();
        r.quant = t.quant;
        r.cols = t.ndim >= 2 ? t.shape[t.ndim - 1] : 1;
        r.rows = t.ndim >= 2 ? t.numel() / r.cols : t.numel();
        r.data = t.data;
        r.scale = t.scale.empty() ? nullptr : t.scale.data();
    }
}

}  // namespace

void dequant_host(int quant, const uint8_t* blocks, float* out, int64_t n) {
    switch (quant) {
    case RL_Q_Q8_0: deq_q8_0(blocks, out, n); break;
    case RL_Q_Q4_K: deq_q4_k(blocks, out, n); break;
    case RL_Q_Q5_K: deq_q5_k(blocks, out, n); break;
    case RL_Q_Q6_K: deq_q6_k(blocks, out, n); break;
    default: fail(RL_ERR_UNSUPPORTED, "dequant_host: not a block format");
    }
}

}  // namespace rl

extern "C" {

RlWeights* rl_hip_weights_open(const char* path, int max_layers, int* status) {
    RlWeights* out = nullptr;
    const int rc = rl::guard([&] {
        RL_REQUIRE(path != nullptr, RL_ERR_RANGE, "weights_open: null path");
        auto W = std::make_unique<RlWeights>();
        const fs::path p(path);
        std::string ext = p.extension().string();
        std::transform(ext.begin(), ext.end(), ext.begin(), [](unsigned char ch) { return std::tolower(ch); });
        if (fs::is_directory(p)) {
            if (!fs::exists(p / "config.json"))
                throw rl::Error(RL_ERR_IO, "directory is not an HF model (missing config.json): " + p.string());
            W->source = 0;
            rl::load_hf(*W, p, max_layers);
        } else if (ext == ".gguf") {
            W->source = 1;
            rl::load_gguf(*W, p, max_layers);
        } else {
            throw rl::Error(RL_ERR_IO, "unknown model path (need HF dir or *.gguf): " + p.string());
        }
        rl::post_process(*W);
        rl::finish(*W);
        out = W.release();
    });
    if (status) *status = rc;
    return out;
}

void rl_hip_weights_close(RlWeights* w) { delete w; }

int rl_hip_weights_config(const RlWeights* w, RlModelConfig* cfg, int* source) {
    return rl::guard([&] {
        RL_REQUIRE(w && cfg, RL_ERR_RANGE, "weights_config: null argument");
        *cfg = w->cfg;
        if (source) *source = w->source;
    });
}

int rl_hip_weights_table(const RlWeights* w, const RlTensor** tensors, int* n) {
    return rl::guard([&] {
        RL_REQUIRE(w && tensors && n, RL_ERR_RANGE, "weights_table: null argument");
        *tensors = w->view.data();
        *n = static_cast<int>(w->view.size());
    });
}

int rl_hip_weights_info(const RlWeights* w, int i, const char** src_name, int* ndim, int64_t* shape4, int* gguf_type,
                        uint64_t* nbytes, int* n_scale) {
    return rl::guard([&] {
        RL_REQUIRE(w && i >= 0 && i < static_cast<int>(w->tensors.size()), RL_ERR_RANGE, "weights_info: bad index");
        const rl::Tensor& t = w->tensors[i];
        if (src_name) *src_name = t.src.c_str();
        if (ndim) *ndim = t.ndim;
        if (shape4)
            for (int d = 0; d < 4; ++d) shape4[d] = t.shape[d];
        if (gguf_type) *gguf_type = t.gguf_type;
        if (nbytes) *nbytes = t.nbytes;
        if (n_scale) *n_scale = static_cast<int>(t.scale.size());
    });
}

int rl_hip_map_name(int gguf, const char* src, char* out, int cap) {
    return rl::guard([&] {
        RL_REQUIRE(src && out && cap > 0, RL_ERR_RANGE, "map_name: null argument");
        const std::string ir = gguf ? rl::map_gguf(src) : rl::map_hf(src);
        RL_REQUIRE(static_cast<int>(ir.size()) < cap, RL_ERR_RANGE, "map_name: buffer too small");
        std::memcpy(out, ir.c_str(), ir.size() + 1);
    });
}

}  // extern "C"
