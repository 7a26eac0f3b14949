// runtime.hip -- C ABI for device memory, streams and events.
//
// Stands in for the reference's rapidllm::Device allocate / create_stream / memcpy
// and Stream::synchronize (include/rapidllm/backend/device.h:41-60) on HIP.
#include <cstring>
#include <string>

#include "common.h"

namespace rl {

static thread_local std::string g_last_error;

void set_last_error(const char* msg) { g_last_error = msg ? msg : ""; }

}  // namespace rl

using namespace rl;

extern "C" {

int rl_hip_abi_version(void) { return RL_HIP_ABI_VERSION; }

const char* rl_hip_last_error(void) { return rl::g_last_error.c_str(); }

int rl_hip_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, 0) != hipSuccess) return 0;
    return std::strncmp(p.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int rl_hip_device_info(char* arch, int cap, int* n_cu, size_t* hbm_bytes) {
    return guard([&] {
        hipDeviceProp_t p;
        RL_HIP(hipGetDeviceProperties(&p, 0));
        if (arch && cap > 0) {
            std::strncpy(arch, p.gcnArchName, cap - 1);
            arch[cap - 1] = 0;
        }
        if (n_cu) *n_cu = p.multiProcessorCount;
        if (hbm_bytes) *hbm_bytes = p.totalGlobalMem;
    });
}

int rl_hip_malloc(void** ptr, size_t bytes) {
    return guard([&] {
        RL_REQUIRE(ptr != nullptr, RL_ERR_RANGE, "rl_hip_malloc: null out pointer");
        *ptr = nullptr;
        hipError_t e = hipMalloc(ptr, bytes ? bytes : 256);
        if (e == hipErrorOutOfMemory) throw Error(RL_ERR_NOMEM, "hipMalloc: out of device memory");
        RL_HIP(e);
    });
}

int rl_hip_free(void* ptr) {
    return guard([&] {
        if (ptr) RL_HIP(hipFree(ptr));
    });
}

int rl_hip_host_alloc(void** ptr, size_t bytes) {
    return guard([&] {
        RL_REQUIRE(ptr != nullptr, RL_ERR_RANGE, "rl_hip_host_alloc: null out pointer");
        *ptr = nullptr;
        hipError_t e = hipHostMalloc(ptr, bytes ? bytes : 256, hipHostMallocDefault);
        if (e == hipErrorOutOfMemory) throw Error(RL_ERR_NOMEM, "hipHostMalloc: out of pinned host memory");
        RL_HIP(e);
    });
}

int rl_hip_host_free(void* ptr) {
    return guard([&] {
        if (ptr) RL_HIP(hipHostFree(ptr));
    });
}

int rl_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    return guard([&] { RL_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, S(stream))); });
}

int rl_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    return guard([&] {
        RL_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, S(stream)));
        RL_HIP(hipStreamSynchronize(S(stream)));
    });
}

int rl_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    return guard([&] { RL_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, S(stream))); });
}

int rl_hip_memset(void* ptr, int value, size_t bytes, void* stream) {
    return guard([&] { RL_HIP(hipMemsetAsync(ptr, value, bytes, S(stream))); });
}

int rl_hip_stream_create(void** stream) {
    return guard([&] {
        hipStream_t s;
        RL_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
        *stream = s;
    });
}

int rl_hip_stream_destroy(void* stream) {
    return guard([&] {
        if (stream) RL_HIP(hipStreamDestroy(S(stream)));
    });
}

int rl_hip_stream_synchronize(void* stream) {
    return guard([&] { RL_HIP(hipStreamSynchronize(S(stream))); });
}

int rl_hip_device_synchronize(void) {
    return guard([&] { RL_HIP(hipDeviceSynchronize()); });
}

int rl_hip_event_create(void** ev) {
    return guard([&] {
        hipEvent_t e;
        RL_HIP(hipEventCreate(&e));
        *ev = e;
    });
}

int rl_hip_event_destroy(void* ev) {
    return guard([&] {
        if (ev) RL_HIP(hipEventDestroy(static_cast<hipEvent_t>(ev)));
    });
}

int rl_hip_event_record(void* ev, void* stream) {
    return guard([&] { RL_HIP(hipEventRecord(static_cast<hipEvent_t>(ev), S(stream))); });
}

int rl_hip_event_elapsed_ms(void* start, void* stop, float* ms) {
    return guard([&] {
        RL_HIP(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
        RL_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
    });
}

}  // extern "C"
