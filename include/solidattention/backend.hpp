// backend.hpp — the accelerator contract of the decode engine's native core.
//
// Same type names, members and virtual interface as the reference's
// cpp/include/solidattention/backend.hpp:10-58, so code written against the
// CUDA backend (make_cuda_backend(), cpp/src/cuda_backend.cpp:475-477) drops
// onto make_hip_backend() (solidattention/hip_backend.hpp) unchanged.
//
// AttentionProblem: borrowed host pointers.  interleaved_kv holds `tokens`
// tokens of [K: kv_heads x head_dim][V: kv_heads x head_dim] FP16 bits;
// query is [query_heads][head_dim] fp32.  Timings are milliseconds.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace solidattention {

struct TransferResult {
  double read_ms{};
  double h2d_ms{};
  double kernel_ms{};
  double d2h_ms{};
  std::uint64_t checksum{};
};

struct AttentionProblem {
  const std::uint16_t* interleaved_kv{};
  const float* query{};
  std::size_t tokens{};
  std::size_t query_heads{};
  std::size_t kv_heads{};
  std::size_t head_dim{};
  float scale{};

  std::size_t kv_elements() const { return tokens * 2 * kv_heads * head_dim; }
  std::size_t query_elements() const { return query_heads * head_dim; }
};

struct AttentionResult {
  double h2d_ms{};
  double kernel_ms{};
  double consumer_ms{};
  double d2h_ms{};
  std::vector<float> output;
};

class AcceleratorBackend {
 public:
  virtual ~AcceleratorBackend() = default;
  virtual std::string name() const = 0;
  // Pinned host memory owned by the caller (registered with io_uring by it).
  virtual void* allocate_host(std::size_t bytes) = 0;
  virtual void free_host(void* pointer) = 0;
  // H2D, out[i] = in[i] ^ mask on the device, D2H, byte checksum.
  virtual TransferResult execute(void* pinned_input, std::size_t bytes, std::uint8_t mask) = 0;
  // H2D of KV and query, GQA attention, D2H of the output.
  virtual AttentionResult attention(const AttentionProblem& problem) = 0;
  virtual AttentionResult attention_optimized(const AttentionProblem& problem) = 0;
  // As attention_optimized with persistent device buffers and events.
  virtual AttentionResult attention_persistent(const AttentionProblem& problem) = 0;
  // Output stays on the device unless audit_output.
  virtual AttentionResult attention_resident(const AttentionProblem& problem, bool audit_output) = 0;
  // A device consumer reduces the output to one checksum, copied back when
  // audit_checksum.
  virtual AttentionResult attention_consumed(const AttentionProblem& problem, bool audit_checksum) = 0;
};

}  // namespace solidattention
