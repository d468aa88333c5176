// hip_backend.hip — AcceleratorBackend on MI355X (gfx950): make_hip_backend().
//
// The drop-in for the reference's CudaBackend (cpp/src/cuda_backend.cpp
// :171-471): one non-blocking stream, device buffers grown on demand and
// reused, persistent events for the "persistent/resident/consumed"
// variants, fresh events per call for "attention/optimized", and the same
// timing fields (H2D, kernel, consumer, D2H in ms).  The device kernel of
// every attention variant is the library's sparse decode attention kernel in
// contiguous-buffer mode, so none of the reference's 128/256-token limits
// apply (cuda_backend.cpp:288-290, 329-332).
#include "solidattention/backend.hpp"
#include "solidattention/hip_backend.hpp"

#include "sa_hip.h"
#include "sa_internal.hpp"

#include <hip/hip_runtime.h>

#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace solidattention {
namespace {

void hip_check(hipError_t result, const char* operation) {
  if (result != hipSuccess) throw std::runtime_error(std::string(operation) + ": " + hipGetErrorString(result));
}

void sa_check(int rc, const char* operation) {
  if (rc != SA_HIP_OK) throw std::runtime_error(std::string(operation) + ": " + sa_hip_last_error());
}

// A device allocation that only grows.
struct GrowBuffer {
  void* ptr{};
  std::size_t bytes{};
  void ensure(std::size_t need, const char* what) {
    if (need <= bytes) return;
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
    hip_check(hipMalloc(&ptr, need), what);
    bytes = need;
  }
  ~GrowBuffer() {
    if (ptr) (void)hipFree(ptr);
  }
};

struct Events {
  hipEvent_t start{}, h2d_end{}, kernel_end{}, consumer_end{}, d2h_end{};
  void create() {
    hip_check(hipEventCreate(&start), "hipEventCreate");
    hip_check(hipEventCreate(&h2d_end), "hipEventCreate");
    hip_check(hipEventCreate(&kernel_end), "hipEventCreate");
    hip_check(hipEventCreate(&consumer_end), "hipEventCreate");
    hip_check(hipEventCreate(&d2h_end), "hipEventCreate");
  }
  void destroy() {
    for (hipEvent_t* e : {&start, &h2d_end, &kernel_end, &consumer_end, &d2h_end})
      if (*e) (void)hipEventDestroy(*e), *e = nullptr;
  }
};

class HipBackend final : public AcceleratorBackend {
 public:
  HipBackend() {
    hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
    persistent_.create();
  }

  ~HipBackend() override {
    persistent_.destroy();
    if (stream_) (void)hipStreamDestroy(stream_);
  }

  std::string name() const override { return "hip-gfx950"; }

  void* allocate_host(std::size_t bytes) override {
    void* pointer = nullptr;
    hip_check(hipHostMalloc(&pointer, bytes, hipHostMallocDefault), "hipHostMalloc");
    return pointer;
  }

  void free_host(void* pointer) override { hip_check(hipHostFree(pointer), "hipHostFree"); }

  TransferResult execute(void* pinned_input, std::size_t bytes, std::uint8_t mask) override {
    input_.ensure(bytes, "hipMalloc input");
    output_.ensure(bytes, "hipMalloc output");
    Events ev;
    ev.create();
    std::vector<std::uint8_t> out(bytes);
    hip_check(hipEventRecord(ev.start, stream_), "hipEventRecord");
    hip_check(hipMemcpyAsync(input_.ptr, pinned_input, bytes, hipMemcpyHostToDevice, stream_), "hipMemcpyAsync H2D");
    hip_check(hipEventRecord(ev.h2d_end, stream_), "hipEventRecord");
    hip_check(sa::launch_xor_bytes(static_cast<const std::uint8_t*>(input_.ptr), static_cast<std::uint8_t*>(output_.ptr),
                                   bytes, mask, stream_),
              "xor launch");
    hip_check(hipEventRecord(ev.kernel_end, stream_), "hipEventRecord");
    hip_check(hipMemcpyAsync(out.data(), output_.ptr, bytes, hipMemcpyDeviceToHost, stream_), "hipMemcpyAsync D2H");
    hip_check(hipEventRecord(ev.d2h_end, stream_), "hipEventRecord");
    hip_check(hipEventSynchronize(ev.d2h_end), "hipEventSynchronize");
    float h2d = 0, kernel = 0, d2h = 0;
    (void)hipEventElapsedTime(&h2d, ev.start, ev.h2d_end);
    (void)hipEventElapsedTime(&kernel, ev.h2d_end, ev.kernel_end);
    (void)hipEventElapsedTime(&d2h, ev.kernel_end, ev.d2h_end);
    std::uint64_t checksum = 0;
    for (const auto value : out) checksum += value;
    ev.destroy();
    TransferResult r;
    r.h2d_ms = h2d;
    r.kernel_ms = kernel;
    r.d2h_ms = d2h;
    r.checksum = checksum;
    return r;
  }

  AttentionResult attention(const AttentionProblem& problem) override {
    return run(problem, false, true, false);
  }
  AttentionResult attention_optimized(const AttentionProblem& problem) override {
    return run(problem, false, true, false);
  }
  AttentionResult attention_persistent(const AttentionProblem& problem) override {
    return run(problem, true, true, false);
  }
  AttentionResult attention_resident(const AttentionProblem& problem, bool audit_output) override {
    return run(problem, true, audit_output, false);
  }
  AttentionResult attention_consumed(const AttentionProblem& problem, bool audit_checksum) override {
    return run(problem, true, audit_checksum, true);
  }

 private:
  AttentionResult run(const AttentionProblem& problem, bool reuse_events, bool copy_output, bool consume_output) {
    if (problem.tokens == 0 || problem.kv_heads == 0 || problem.query_heads % problem.kv_heads != 0 ||
        !problem.interleaved_kv || !problem.query)
      throw std::runtime_error("unsupported HIP attention dimensions");
    const std::size_t kv_bytes = problem.kv_elements() * sizeof(std::uint16_t);
    const std::size_t query_bytes = problem.query_elements() * sizeof(float);
    const int32_t hq = static_cast<int32_t>(problem.query_heads);
    const int32_t hkv = static_cast<int32_t>(problem.kv_heads);
    const int32_t hd = static_cast<int32_t>(problem.head_dim);
    const int64_t tokens = static_cast<int64_t>(problem.tokens);
    const std::size_t ws_bytes = sa_hip_contiguous_workspace_bytes(tokens, hq, hkv, hd);
    kv_.ensure(kv_bytes, "hipMalloc attention KV");
    query_.ensure(query_bytes, "hipMalloc attention query");
    out_.ensure(query_bytes, "hipMalloc attention output");
    checksum_.ensure(sizeof(float), "hipMalloc consumer checksum");
    workspace_.ensure(ws_bytes ? ws_bytes : 16, "hipMalloc attention workspace");

    Events local;
    if (!reuse_events) local.create();
    const Events& ev = reuse_events ? persistent_ : local;
    AttentionResult result;
    if (copy_output) result.output.resize(consume_output ? 1 : problem.query_elements());
    try {
      hip_check(hipEventRecord(ev.start, stream_), "hipEventRecord");
      hip_check(hipMemcpyAsync(kv_.ptr, problem.interleaved_kv, kv_bytes, hipMemcpyHostToDevice, stream_),
                "attention KV H2D");
      hip_check(hipMemcpyAsync(query_.ptr, problem.query, query_bytes, hipMemcpyHostToDevice, stream_),
                "attention query H2D");
      hip_check(hipEventRecord(ev.h2d_end, stream_), "hipEventRecord");
      sa_check(sa_hip_attention_contiguous(static_cast<const std::uint16_t*>(kv_.ptr),
                                           static_cast<const float*>(query_.ptr), tokens, hq, hkv, hd, problem.scale,
                                           static_cast<float*>(out_.ptr), workspace_.ptr, ws_bytes, stream_),
               "attention launch");
      hip_check(hipEventRecord(ev.kernel_end, stream_), "hipEventRecord");
      if (consume_output)
        sa_check(sa_hip_consume_checksum(static_cast<const float*>(out_.ptr),
                                         static_cast<int32_t>(problem.query_elements()),
                                         static_cast<float*>(checksum_.ptr), stream_),
                 "consume launch");
      hip_check(hipEventRecord(ev.consumer_end, stream_), "hipEventRecord");
      if (copy_output) {
        const void* source = consume_output ? checksum_.ptr : out_.ptr;
        const std::size_t bytes = consume_output ? sizeof(float) : query_bytes;
        hip_check(hipMemcpyAsync(result.output.data(), source, bytes, hipMemcpyDeviceToHost, stream_),
                  "attention output D2H");
      }
      hip_check(hipEventRecord(ev.d2h_end, stream_), "hipEventRecord");
      hip_check(hipEventSynchronize(ev.d2h_end), "attention synchronize");
      float h2d = 0, kernel = 0, consumer = 0, d2h = 0;
      (void)hipEventElapsedTime(&h2d, ev.start, ev.h2d_end);
      (void)hipEventElapsedTime(&kernel, ev.h2d_end, ev.kernel_end);
      (void)hipEventElapsedTime(&consumer, ev.kernel_end, ev.consumer_end);
      (void)hipEventElapsedTime(&d2h, ev.consumer_end, ev.d2h_end);
      result.h2d_ms = h2d;
      result.kernel_ms = kernel;
      result.consumer_ms = consumer;
      result.d2h_ms = d2h;
    } catch (...) {
      local.destroy();
      throw;
    }
    local.destroy();
    return result;
  }

  hipStream_t stream_{};
  Events persistent_;
  GrowBuffer input_, output_, kv_, query_, out_, checksum_, workspace_;
};

}  // namespace

std::unique_ptr<AcceleratorBackend> make_hip_backend() { return std::make_unique<HipBackend>(); }

}  // namespace solidattention
