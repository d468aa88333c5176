// hip_kv.hpp — C++ API of the MI355X KV-cache decode hot path, over the
// C-ABI of sa_hip.h (header-only; link libsa_hip.so).
//
// New next to the reference's contract (the reference has no paged pool, no
// GPU selection, no GPU seal and no device gather; README.md:68-70 of the
// reference).  The semantics it carries are the reference's:
//   PagedKvPool::append_seal   decode append + seal (qwen_layer_main.cpp
//                              :270-281, kv_lifecycle_main.cpp:31-45,92-113)
//   SparseDecoder::select      select_shared_blocks per selection group
//                              (selection.hpp:24-29, selection.cpp:96-147)
//   SparseDecoder::attend      attention_reference over the selected blocks
//                              and the tail (attention_reference.cpp:55-96)
//   SparseDecoder::select_attend  select then attend (one launch where the
//                              fused kernel applies)
//   SparseDecoder::decode_step append + seal, select, attend: one layer's
//                              decode step (qwen_chain_main.cpp:390-395 with
//                              selection on the GPU), one launch where the
//                              fused kernel applies
//   SparseDecoder::decode_step_qkv  the same fed by the q/k/v projections,
//                              head RMS norm and RoPE (qwen_chain_main.cpp:
//                              365-395): two launches where the one-launch
//                              step takes the producer's epilogue
//   MissCorrector              CudaPipeline::correct_and_wait without the
//                              host barrier (pipeline_main.cpp:305-331)
//   SplitAttention             attention of the resident blocks while the
//                              misses are copied, then of the misses, merged
//                              (the overlap of pipeline_main.cpp:811-848)
//   compare_prediction         pipeline_main.cpp:686-717
// Errors are std::runtime_error("operation: message"), as the reference's
// cuda_check does (cuda_backend.cpp:16-21).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "sa_hip.h"

namespace solidattention::hip {

inline void check(int rc, const char* operation) {
  if (rc != SA_HIP_OK) throw std::runtime_error(std::string(operation) + ": " + sa_hip_last_error());
}

inline void hip_check(hipError_t e, const char* operation) {
  if (e != hipSuccess) throw std::runtime_error(std::string(operation) + ": " + hipGetErrorString(e));
}

// Owning device allocation (zero-filled).
template <class T>
class DeviceArray {
 public:
  DeviceArray() = default;
  explicit DeviceArray(std::size_t n) : n_(n) {
    if (n_) {
      hip_check(hipMalloc(reinterpret_cast<void**>(&p_), n_ * sizeof(T)), "hipMalloc");
      hip_check(hipMemset(p_, 0, n_ * sizeof(T)), "hipMemset");
    }
  }
  ~DeviceArray() {
    if (p_) (void)hipFree(p_);
  }
  DeviceArray(const DeviceArray&) = delete;
  DeviceArray& operator=(const DeviceArray&) = delete;
  DeviceArray(DeviceArray&& o) noexcept : p_(std::exchange(o.p_, nullptr)), n_(std::exchange(o.n_, 0)) {}
  DeviceArray& operator=(DeviceArray&& o) noexcept {
    if (this != &o) {
      if (p_) (void)hipFree(p_);
      p_ = std::exchange(o.p_, nullptr);
      n_ = std::exchange(o.n_, 0);
    }
    return *this;
  }
  T* get() const { return p_; }
  std::size_t size() const { return n_; }
  void upload(const std::vector<T>& v) {
    if (v.size() != n_) throw std::runtime_error("upload: host vector size differs from the device array's");
    hip_check(hipMemcpy(p_, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy H2D");
  }
  std::vector<T> download() const {
    std::vector<T> v(n_);
    if (n_) hip_check(hipMemcpy(v.data(), p_, n_ * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return v;
  }

 private:
  T* p_{};
  std::size_t n_{};
};

// One layer's paged FP16 KV slot pool in HBM with its block tables,
// lengths and block representatives.  The default representative row stride
// is a multiple of 32 floats: every [rep head][d] row starts on a 128-byte
// line, so the scoring kernels' streaming loads fetch no line twice.
class PagedKvPool {
 public:
  PagedKvPool(std::size_t batch, std::size_t query_heads, std::size_t kv_heads, std::size_t table_stride,
              std::size_t num_pages, std::size_t rep_heads = 0, std::size_t rep_stride = 0,
              std::size_t head_dim = 128)
      : batch_(batch), query_heads_(query_heads), kv_heads_(kv_heads), head_dim_(head_dim),
        table_stride_(table_stride), num_pages_(num_pages), rep_heads_(rep_heads ? rep_heads : kv_heads),
        rep_stride_(rep_stride ? rep_stride : (table_stride + 31) / 32 * 32),
        pool_(num_pages * page_elems()), table_(batch * table_stride), seq_len_(batch), sealed_(batch),
        generation_(batch), reps_(batch * rep_heads_ * head_dim * rep_stride_) {}

  std::size_t page_elems() const { return SA_HIP_PAGE_TOKENS * 2 * kv_heads_ * head_dim_; }
  std::size_t page_bytes() const { return page_elems() * sizeof(std::uint16_t); }
  std::size_t batch() const { return batch_; }
  std::size_t query_heads() const { return query_heads_; }
  std::size_t kv_heads() const { return kv_heads_; }
  std::size_t head_dim() const { return head_dim_; }
  std::size_t table_stride() const { return table_stride_; }
  std::size_t rep_heads() const { return rep_heads_; }
  std::size_t rep_stride() const { return rep_stride_; }

  sa_paged_kv view() const {
    sa_paged_kv v{};
    v.pool = pool_.get();
    v.block_table = table_.get();
    v.seq_len = seq_len_.get();
    v.sealed = sealed_.get();
    v.generation = generation_.get();
    v.reps = reps_.get();
    v.num_pages = static_cast<int64_t>(num_pages_);
    v.batch = static_cast<int32_t>(batch_);
    v.table_stride = static_cast<int32_t>(table_stride_);
    v.rep_heads = static_cast<int32_t>(rep_heads_);
    v.rep_stride = static_cast<int32_t>(rep_stride_);
    v.query_heads = static_cast<int32_t>(query_heads_);
    v.kv_heads = static_cast<int32_t>(kv_heads_);
    v.head_dim = static_cast<int32_t>(head_dim_);
    return v;
  }

  DeviceArray<std::uint16_t>& pool() { return pool_; }
  DeviceArray<int32_t>& block_table() { return table_; }
  DeviceArray<int32_t>& seq_len() { return seq_len_; }
  DeviceArray<int32_t>& sealed() { return sealed_; }
  DeviceArray<int32_t>& generation() { return generation_; }
  DeviceArray<float>& reps() { return reps_; }

  // Append one token per sequence (fp32 K/V [batch][kv_heads][head_dim] on
  // the device) and seal full blocks beyond local_tokens of tail.
  void append_seal(const float* k, const float* v, int local_tokens, hipStream_t stream = nullptr,
                   int32_t* status = nullptr) {
    const sa_paged_kv kv = view();
    check(sa_hip_append_seal(&kv, k, v, local_tokens, status, stream), "append_seal");
  }
  void append_seal_f16(const std::uint16_t* k, const std::uint16_t* v, int local_tokens,
                       hipStream_t stream = nullptr, int32_t* status = nullptr) {
    const sa_paged_kv kv = view();
    check(sa_hip_append_seal_f16(&kv, k, v, local_tokens, status, stream), "append_seal_f16");
  }
  // Seal every complete block beyond local_tokens of tail (after a prefill).
  void seal(int local_tokens, hipStream_t stream = nullptr, int32_t* status = nullptr) {
    const sa_paged_kv kv = view();
    check(sa_hip_seal(&kv, local_tokens, status, stream), "seal");
  }

 private:
  std::size_t batch_, query_heads_, kv_heads_, head_dim_, table_stride_, num_pages_, rep_heads_, rep_stride_;
  DeviceArray<std::uint16_t> pool_;
  DeviceArray<int32_t> table_, seq_len_, sealed_, generation_;
  DeviceArray<float> reps_;
};

// Budgeted selection + sparse decode attention with the scratch they need.
class SparseDecoder {
 public:
  // chunk_pages: page-list chunk of attend_chunked() (lists of very
  // different lengths: mixed contexts and per-sequence budgets)
  SparseDecoder(const PagedKvPool& pool, sa_select_params params, int splits = 0, int chunk_pages = 128)
      : params_(params),
        splits_(splits > 0 ? splits
                           : sa_hip_attention_splits_for(static_cast<int32_t>(pool.batch()),
                                                         static_cast<int32_t>(pool.query_heads()),
                                                         static_cast<int32_t>(pool.kv_heads()),
                                                         params.budget_blocks + 2)),
        selected_(pool.batch() * params.select_groups * params.sel_stride),
        counts_(pool.batch() * params.select_groups),
        workspace_bytes_(sa_hip_attention_workspace_bytes(static_cast<int32_t>(pool.batch()),
                                                          static_cast<int32_t>(pool.query_heads()),
                                                          static_cast<int32_t>(pool.kv_heads()),
                                                          static_cast<int32_t>(pool.head_dim()), splits_)),
        workspace_((workspace_bytes_ + 3) / 4),
        step_splits_(fused_splits(pool, params, splits)),
        step_workspace_bytes_(step_bytes(pool, step_splits_)),
        step_workspace_((step_workspace_bytes_ + 3) / 4),
        chunk_pages_(chunk_pages),
        max_chunks_(chunks_for(params.sel_stride, chunk_pages)),
        // the partial records and the longest-list-first schedule
        chunk_workspace_bytes_(sa_hip_attention_chunked_workspace_bytes(static_cast<int32_t>(pool.batch()),
                                                                        static_cast<int32_t>(pool.query_heads()),
                                                                        static_cast<int32_t>(pool.kv_heads()),
                                                                        static_cast<int32_t>(pool.head_dim()),
                                                                        max_chunks_)),
        chunk_workspace_((chunk_workspace_bytes_ + 3) / 4),
        // at a head_dim other than 128 the scoring hands its scores to the
        // selection through this buffer
        scores_(pool.head_dim() == 128 ? 0 : pool.batch() * params.select_groups * pool.rep_stride()) {}

  // Score every sealed block against the query [batch][query_heads][head_dim]
  // (device) and select per group; ids stay on the device.
  void select(const PagedKvPool& pool, const float* query, hipStream_t stream = nullptr,
              float* scores = nullptr, int32_t* status = nullptr) {
    const sa_paged_kv kv = pool.view();
    if (!scores && scores_.size()) scores = scores_.get();
    check(sa_hip_score_select(&kv, query, &params_, selected_.get(), counts_.get(), scores, status, stream),
          "score_select");
  }
  // out [batch][query_heads][head_dim] fp32 (device).
  void attend(const PagedKvPool& pool, const float* query, float scale, float* out,
              hipStream_t stream = nullptr, int32_t* status = nullptr) {
    const sa_paged_kv kv = pool.view();
    check(sa_hip_sparse_decode_attention(&kv, query, selected_.get(), counts_.get(), params_.select_groups,
                                         params_.sel_stride, scale, out, workspace_.get(), workspace_bytes_,
                                         splits_, status, stream),
          "sparse_decode_attention");
  }

  // attend() with every page list cut into chunk_pages-page chunks, one
  // workgroup each: for batches whose lists differ widely in length.
  void attend_chunked(const PagedKvPool& pool, const float* query, float scale, float* out,
                      hipStream_t stream = nullptr, int32_t* status = nullptr) {
    const sa_paged_kv kv = pool.view();
    check(sa_hip_sparse_decode_attention_chunked(&kv, query, selected_.get(), counts_.get(), params_.select_groups,
                                                 params_.sel_stride, scale, out, chunk_workspace_.get(),
                                                 chunk_workspace_bytes_, chunk_pages_, max_chunks_, status, stream),
          "sparse_decode_attention_chunked");
  }

  // select() then attend(): one launch when fused() is true.
  void select_attend(const PagedKvPool& pool, const float* query, float scale, float* out,
                     hipStream_t stream = nullptr, int32_t* status = nullptr) {
    const sa_paged_kv kv = pool.view();
    // the split records of the non-fused path sit after the arrival counters
    const std::size_t skip = arrive_bytes(pool.batch());
    check(sa_hip_select_attend(&kv, query, &params_, scale, selected_.get(), counts_.get(), out,
                               step_workspace_.get() + skip / 4, step_workspace_bytes_ - skip, step_splits_, status,
                               stream),
          "select_attend");
  }
  // One layer's decode step: pool.append_seal(k, v, local_tokens) then
  // select_attend(); one launch when fused() is true.  k, v: fp32
  // [batch][kv_heads][head_dim] on the device.  (select_attend() is built
  // for head_dim 128; decode_step() takes any multiple of 8 up to 512.)
  void decode_step(const PagedKvPool& pool, const float* k, const float* v, int local_tokens, const float* query,
                   float scale, float* out, hipStream_t stream = nullptr, int32_t* status = nullptr) {
    const sa_paged_kv kv = pool.view();
    check(sa_hip_decode_step(&kv, k, v, local_tokens, query, &params_, scale, selected_.get(), counts_.get(), out,
                             step_workspace_.get(), step_workspace_bytes_, step_splits_, status, stream),
          "decode_step");
  }
  // decode_step() fed by its q/k/v producer (sa_hip_decode_step_qkv): the
  // projection of producer.hidden_rows into producer.q/k/v, then the step on
  // them; two launches where the one launch applies with 1 or 2 query heads
  // per KV head.  head_dim 128.
  void decode_step_qkv(const PagedKvPool& pool, const sa_qkv_producer& producer, int local_tokens, float scale,
                       float* out, hipStream_t stream = nullptr, int32_t* status = nullptr) {
    const sa_paged_kv kv = pool.view();
    check(sa_hip_decode_step_qkv(&kv, &producer, local_tokens, &params_, scale, selected_.get(), counts_.get(), out,
                                 step_workspace_.get(), step_workspace_bytes_, step_splits_, status, stream),
          "decode_step_qkv");
  }
  bool fused(const PagedKvPool& pool) const {
    const sa_paged_kv kv = pool.view();
    return sa_hip_select_attend_fused(&kv, &params_, step_splits_) != 0;
  }

  const DeviceArray<int32_t>& selected() const { return selected_; }
  const DeviceArray<int32_t>& counts() const { return counts_; }
  DeviceArray<int32_t>& selected() { return selected_; }
  DeviceArray<int32_t>& counts() { return counts_; }
  int splits() const { return splits_; }

 private:
  sa_select_params params_;
  int splits_;
  DeviceArray<int32_t> selected_, counts_;
  std::size_t workspace_bytes_;
  DeviceArray<float> workspace_;
  // select_attend / decode_step: the fused launch where it applies and
  // fills the device (unless the caller fixed the splits), with a workspace
  // of arrival counters (zeroed here; every step leaves them zero) and split
  // records
  int step_splits_;
  std::size_t step_workspace_bytes_;
  DeviceArray<int32_t> step_workspace_;

  // attend_chunked(): chunks enough for a list of every selectable block
  // plus two tail pages (a longer list's last chunk takes the rest)
  int chunk_pages_;
  int max_chunks_;
  std::size_t chunk_workspace_bytes_;
  DeviceArray<float> chunk_workspace_;
  DeviceArray<float> scores_;

  static int chunks_for(int sel_stride, int chunk_pages) {
    if (chunk_pages < 1) throw std::runtime_error("SparseDecoder: chunk_pages must be positive");
    const int n = (sel_stride + 2 + chunk_pages - 1) / chunk_pages;
    return n < 2 ? 2 : (n > 65535 ? 65535 : n);
  }
  static int fused_splits(const PagedKvPool& pool, const sa_select_params& params, int splits) {
    if (splits > 0) return splits;
    const sa_paged_kv kv = pool.view();
    return sa_hip_select_attend_default_splits(&kv, &params);
  }
  static std::size_t step_bytes(const PagedKvPool& pool, int splits) {
    const sa_paged_kv kv = pool.view();
    return sa_hip_decode_step_workspace_bytes(&kv, splits);
  }
  // the decode-step workspace starts with one int32 arrival counter per
  // sequence, padded to 256 bytes (sa_hip_decode_step_workspace_bytes)
  static std::size_t arrive_bytes(std::size_t batch) { return (batch * 4 + 255) / 256 * 256; }
};

struct Correction {
  std::size_t hits{};
  std::vector<int32_t> misses;
  std::vector<int32_t> replacement_slots;
};

// Host set logic of a history prediction versus the selection.
inline Correction compare_prediction(const std::vector<int32_t>& predicted, const std::vector<int32_t>& oracle) {
  if (predicted.size() != oracle.size())
    throw std::runtime_error("prediction correction cardinality mismatch");
  Correction c;
  c.misses.resize(predicted.size());
  c.replacement_slots.resize(predicted.size());
  int32_t hits = 0, misses = 0;
  check(sa_hip_compare_prediction(predicted.data(), oracle.data(), static_cast<int32_t>(predicted.size()), &hits,
                                  c.misses.data(), c.replacement_slots.data(), &misses),
        "compare_prediction");
  c.hits = static_cast<std::size_t>(hits);
  c.misses.resize(static_cast<std::size_t>(misses));
  c.replacement_slots.resize(static_cast<std::size_t>(misses));
  return c;
}

// Copy stream + completion event for miss-correction slot fills from pinned
// host memory; the compute stream orders itself after the fills on the
// device (hipStreamWaitEvent), not with a host barrier.
class MissCorrector {
 public:
  MissCorrector() {
    hip_check(hipStreamCreateWithFlags(&copy_, hipStreamNonBlocking), "hipStreamCreate copy");
    hip_check(hipEventCreateWithFlags(&done_, hipEventDisableTiming), "hipEventCreate");
  }
  ~MissCorrector() {
    if (after_) (void)hipEventDestroy(after_);
    if (done_) (void)hipEventDestroy(done_);
    if (copy_) (void)hipStreamDestroy(copy_);
  }
  MissCorrector(const MissCorrector&) = delete;
  MissCorrector& operator=(const MissCorrector&) = delete;

  void fill(std::uint16_t* pool, std::size_t page_bytes, const std::vector<int32_t>& dst_pages,
            const void* pinned_src, const std::vector<int64_t>& src_blocks) {
    if (dst_pages.size() != src_blocks.size()) throw std::runtime_error("fill: page/block count mismatch");
    check(sa_hip_fill_pages_async(pool, static_cast<int64_t>(page_bytes), dst_pages.data(), pinned_src,
                                  src_blocks.data(), static_cast<int32_t>(dst_pages.size()), copy_, done_),
          "fill_pages_async");
  }
  // The same fills as one kernel on the copy stream reading the pinned
  // store through its device mapping (pinned_src from hipHostMalloc, holding
  // src_total pages); dst_pages_dev / src_blocks_dev are device arrays,
  // e.g. uploaded on copy_stream() just before.
  void fill_gather(std::uint16_t* pool, std::size_t page_bytes, int64_t num_pages, const int32_t* dst_pages_dev,
                   const void* pinned_src, int64_t src_total, const int64_t* src_blocks_dev, int32_t count,
                   int32_t* status = nullptr) {
    check(sa_hip_fill_pages_gather_async(pool, static_cast<int64_t>(page_bytes), num_pages, dst_pages_dev,
                                         pinned_src, src_total, src_blocks_dev, count, status, copy_, done_),
          "fill_pages_gather_async");
  }
  // Make `compute` wait (on the device) for the last fill.
  void order(hipStream_t compute) { check(sa_hip_stream_wait_event(compute, done_), "stream_wait_event"); }
  // Host barrier on the fills (the reference's correct_and_wait,
  // pipeline_main.cpp:322-323).
  void wait() { hip_check(hipStreamSynchronize(copy_), "hipStreamSynchronize copy"); }
  // Make the next fills wait for the work queued so far on `s` (earlier
  // writers or readers of the destination pages, e.g. a prefetch the compute
  // stream was ordered after).
  void after(hipStream_t s) {
    if (!after_) hip_check(hipEventCreateWithFlags(&after_, hipEventDisableTiming), "hipEventCreate");
    hip_check(hipEventRecord(after_, s), "hipEventRecord");
    check(sa_hip_stream_wait_event(copy_, after_), "stream_wait_event");
  }
  hipStream_t copy_stream() const { return copy_; }

 private:
  hipStream_t copy_{};
  hipEvent_t done_{};
  hipEvent_t after_{};
};

// Split-phase attention over several id lists of one step (for example the
// blocks already resident, then the blocks a copy stream fills meanwhile),
// merged with log-sum-exp into one output: the same result as one
// SparseDecoder::attend over the union, within fp32 rounding.  Each partial
// call writes `splits` records from split_base of total_splits; the tail is
// included by exactly one call.  Calls sharing the object must not run
// concurrently.
class SplitAttention {
 public:
  SplitAttention(const PagedKvPool& pool, int total_splits)
      : total_(total_splits),
        bytes_(sa_hip_attention_workspace_bytes(static_cast<int32_t>(pool.batch()),
                                                static_cast<int32_t>(pool.query_heads()),
                                                static_cast<int32_t>(pool.kv_heads()),
                                                static_cast<int32_t>(pool.head_dim()), total_splits)),
        workspace_((bytes_ + 3) / 4) {
    if (total_splits < 2) throw std::runtime_error("SplitAttention: total_splits must be >= 2");
  }
  void partial(const PagedKvPool& pool, const float* query, const int32_t* ids, const int32_t* counts,
               int select_groups, int sel_stride, float scale, bool include_tail, int split_base, int splits,
               hipStream_t stream = nullptr, int32_t* status = nullptr) {
    const sa_paged_kv kv = pool.view();
    check(sa_hip_sparse_decode_attention_partial(&kv, query, ids, counts, select_groups, sel_stride, scale,
                                                 include_tail ? 1 : 0, workspace_.get(), bytes_, split_base, splits,
                                                 total_, status, stream),
          "sparse_decode_attention_partial");
  }
  // out [batch][query_heads][head_dim] fp32 (device).
  void merge(const PagedKvPool& pool, float* out, hipStream_t stream = nullptr) {
    const sa_paged_kv kv = pool.view();
    check(sa_hip_attention_merge(&kv, workspace_.get(), bytes_, total_, out, stream), "attention_merge");
  }

 private:
  int total_;
  std::size_t bytes_;
  DeviceArray<float> workspace_;
};

}  // namespace solidattention::hip
