// hip_backend.hpp — factory of the MI355X (gfx950) accelerator backend.
//
// Replaces make_cuda_backend() (reference cpp/src/cuda_backend.cpp:475-477),
// which callers declare under SOLIDATTENTION_ENABLE_CUDA and pick with
// --backend (reference cpp/src/attention_main.cpp:23-30, 101-116).  Errors
// are std::runtime_error("operation: message"), as in the reference's
// cuda_check (cuda_backend.cpp:16-21).  There is no token limit: the device
// kernel is the paged sparse decode attention kernel over a contiguous
// buffer.
#pragma once

#include <memory>

#include "solidattention/backend.hpp"

namespace solidattention {

std::unique_ptr<AcceleratorBackend> make_hip_backend();

}  // namespace solidattention
