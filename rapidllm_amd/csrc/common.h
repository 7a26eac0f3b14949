// common.h -- shared device/host helpers for the gfx950 decode backend.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>

#include "../../include/rapidllm_hip.h"
#include "../../include/rapidllm_hip_bench.h"

namespace rl {

// Status codes: identical values to RapidStatus (include/rapidllm/api.h:11-25 of the
// reference), so the C API layer can pass them through unchanged.
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void set_last_error(const char* msg);

#define RL_HIP(expr)                                                                                 \
    do {                                                                                             \
        hipError_t e_ = (expr);                                                                      \
        if (e_ != hipSuccess)                                                                        \
            throw ::rl::Error(RL_ERR_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_));     \
    } while (0)

#define RL_REQUIRE(cond, code, msg)                                   \
    do {                                                              \
        if (!(cond)) throw ::rl::Error((code), std::string(msg));     \
    } while (0)

// Run `body` and translate exceptions into a status code + thread-local message.
// No exception ever crosses the C ABI (mirrors rapidllm_c.cpp:46-50, 246-251).
template <class F>
int guard(F&& body) {
    try {
        body();
        return RL_OK;
    } catch (const Error& e) {
        set_last_error(e.what());
        return e.code;
    } catch (const std::bad_alloc&) {
        set_last_error("out of memory");
        return RL_ERR_NOMEM;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return RL_ERR_INTERNAL;
    }
}

inline hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

// After an async launch: surface launch-configuration errors immediately.
inline void check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw Error(RL_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

constexpr int kWave = 64;

}  // namespace rl

// ------------------------------------------------------------------ device side
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

// Wave-wide sum / max through cross-lane moves (DPP/permute lowered by the compiler).

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Sum over aligned groups of 8 (or 16) consecutive lanes with DPP lane moves
// (no LDS round trip).  Butterfly pairing as xor 1, 2, 4 (, 8): every lane of a
// group ends with the bitwise same sum.
template <int kCtrl>
__device__ inline float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}
__device__ inline float group8_sum(float v) {
    v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]: xor 1
    v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]: xor 2
    v += dpp_move<0x141>(v);  // row_half_mirror: the other quad of the 8-lane half row
    return v;
}
__device__ inline float group16_sum(float v) {
    v = group8_sum(v);
    v += dpp_move<0x140>(v);  // row_mirror: the other half of the 16-lane row
    return v;
}

// Whole-wave sums (all 64 lanes active): the 16-lane row sums by DPP, then the four
// rows combined as (row0 + row1) + (row2 + row3) from lanes 0, 16, 32, 48; every
// lane returns the same value.
__device__ inline float wave_sum(float v) {
    v = group16_sum(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (a + b) + (c + d);
}

template <int kCtrl>
__device__ inline double dpp_move_d(double v) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(v));
    const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(u & 0xffffffffu), kCtrl, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(u >> 32), kCtrl, 0xF, 0xF, false);
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(static_cast<unsigned>(hi)) << 32) |
                                                       static_cast<unsigned>(lo)));
}
__device__ inline double readlane_d(double v, int lane) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(v));
    const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(u & 0xffffffffu), lane));
    const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), lane));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}
// 16-lane row sum of doubles (every lane of the row gets the same value)
__device__ inline double group16_sum_d(double v) {
    v += dpp_move_d<0xB1>(v);
    v += dpp_move_d<0x4E>(v);
    v += dpp_move_d<0x141>(v);
    v += dpp_move_d<0x140>(v);
    return v;
}
__device__ inline double wave_sum_d(double v) {
    v = group16_sum_d(v);
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}

// Split an fp32 value into two bf16 terms whose sum carries 16 significant bits:
// hi = x truncated to bf16, mid = (x - hi) truncated to bf16.  x - hi is exact in
// fp32; the remainder lost is < 2^-16 |x|.  bf16 keeps fp32's exponent range, so
// no activation can overflow the split.
__device__ inline void split_bf16(float x, uint16_t& hi, uint16_t& mid) {
    const uint32_t xb = __float_as_uint(x);
    hi = static_cast<uint16_t>(xb >> 16);
    const float r = x - __uint_as_float(xb & 0xffff0000u);
    mid = static_cast<uint16_t>(__float_as_uint(r) >> 16);
}

// Fragment unit (16 B = 8 bf16) holding columns [8u, 8u+8) of token t, hi part.
// The mid part sits T units later.  Layout of the GEMM input
// fragments (pack_act_kernel, gemm.hip): [kb][i][g][2T][8 bf16].
__device__ inline size_t frag_unit(int col8, int t, int T) {
    const int kb = col8 >> 4;           // 16 units per 128-column block
    const int jb = (col8 & 15) * 8;     // first column within the block
    const int g = jb >> 5, i = (jb >> 3) & 3;
    return ((static_cast<size_t>(kb) * 4 + i) * 4 + g) * (2 * T) + t;
}

__device__ inline void write_frag8(i32x4* frag, int col8, int t, int T, const float (&v)[8]) {
    union {
        uint16_t h[8];
        i32x4 q;
    } hi, mid;
#pragma unroll
    for (int e = 0; e < 8; ++e) split_bf16(v[e], hi.h[e], mid.h[e]);
    const size_t u = frag_unit(col8, t, T);
    frag[u] = hi.q;
    frag[u + T] = mid.q;
}

