// hip_backend.h -- reference-side adapters over the HIP decode backend's C ABI.
//
// These translation units are compiled inside a RapidLLM tree (they include the
// reference's own headers, include/rapidllm/...) and link librapidllm_hip.so.
//   hip_gen::HipEngine  implements cuda_gen::Engine
//                       (include/rapidllm/runtime/cuda_engine.h:13-83) over
//                       rl_hip_engine_*;
//   hip_gen::HipDevice  implements rapidllm::Device
//                       (include/rapidllm/backend/device.h:49-60) with
//                       launch(name, ...) mapped onto the kernel entry points.
#pragma once

#include "rapidllm/backend/device.h"
#include "rapidllm/runtime/cuda_engine.h"

#include <memory>

namespace rapidllm::hip_gen {

// A gfx950 device is visible (the analogue of cuda_gen::available(), cuda_engine.h:11).
bool available();

// The Session's engine factory (cuda_gen::Engine::create(store, ctx)).  Continuous
// batch slots come from RAPIDLLM_MAX_BATCH as in the reference engine.
std::unique_ptr<cuda_gen::Engine> create(WeightStore& store, int ctx);
// Same, from a tensor table (what create(store) passes on).
std::unique_ptr<cuda_gen::Engine> create_from_table(const TensorTable& table, int ctx, int max_batch);

// The kernel-name device (rapidllm::create_device(DeviceKind::HIP) once the enum
// has the HIP entry).
std::unique_ptr<Device> create_device();

}  // namespace rapidllm::hip_gen
