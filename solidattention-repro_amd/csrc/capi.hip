// capi.hip — the extern "C" boundary (include/sa_hip.h): argument
// validation, error strings, launch dispatch.  Hot entry points allocate
// nothing; scratch comes in through workspace arguments, or for
// sa_hip_decode_step_noalloc from the static `scratch` array below.
#include "qkv_epilogue.hpp"
#include "sa_hip.h"
#include "sa_internal.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return SA_HIP_OK;
  return fail(SA_HIP_ERUNTIME, "%s: %s", what, hipGetErrorString(e));
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// any_head_dim: the entry point also takes a head_dim other than 128 (any
// multiple of 8 up to 512), which its general kernels serve.
int check_geometry(const sa_paged_kv* kv, const char* op, bool any_head_dim = false) {
  if (!kv) return fail(SA_HIP_EINVAL, "%s: null sa_paged_kv", op);
  if (kv->head_dim != sa::kHeadDim) {
    if (!any_head_dim)
      return fail(SA_HIP_EINVAL, "%s: head_dim %d unsupported (this entry point is built for %d)", op,
                  kv->head_dim, sa::kHeadDim);
    if (kv->head_dim <= 0 || kv->head_dim % 8 != 0 || kv->head_dim > sa::kAnyMaxHeadDim)
      return fail(SA_HIP_EINVAL, "%s: head_dim %d unsupported (128, or a multiple of 8 up to %d)", op,
                  kv->head_dim, sa::kAnyMaxHeadDim);
  }
  if (kv->kv_heads <= 0 || kv->query_heads <= 0 || kv->query_heads % kv->kv_heads != 0)
    return fail(SA_HIP_EINVAL, "%s: invalid GQA dimensions %d/%d", op, kv->query_heads, kv->kv_heads);
  const int group = kv->query_heads / kv->kv_heads;
  if (group != 1 && group != 2 && group != 4 && group != 8)
    return fail(SA_HIP_EINVAL, "%s: query heads per KV head must be 1, 2, 4 or 8 (got %d)", op, group);
  if (kv->batch <= 0 || kv->batch > 65535) return fail(SA_HIP_EINVAL, "%s: batch %d out of range", op, kv->batch);
  if (kv->table_stride <= 0) return fail(SA_HIP_EINVAL, "%s: table_stride must be positive", op);
  if (kv->num_pages <= 0) return fail(SA_HIP_EINVAL, "%s: num_pages must be positive", op);
  if (!kv->pool || !kv->block_table || !kv->seq_len || !kv->sealed)
    return fail(SA_HIP_EINVAL, "%s: null pool/table/seq_len/sealed", op);
  if (!aligned16(kv->pool)) return fail(SA_HIP_EINVAL, "%s: pool must be 16-byte aligned", op);
  return SA_HIP_OK;
}

int check_reps(const sa_paged_kv* kv, const char* op) {
  if (!kv->reps) return fail(SA_HIP_EINVAL, "%s: null reps", op);
  if (kv->rep_heads != kv->kv_heads && kv->rep_heads != kv->query_heads)
    return fail(SA_HIP_EINVAL, "%s: rep_heads must equal kv_heads or query_heads", op);
  if (kv->rep_stride <= 0) return fail(SA_HIP_EINVAL, "%s: rep_stride must be positive", op);
  return SA_HIP_OK;
}

}  // namespace

namespace sa {
// Error reporting for the host-only parts of the library (store.cpp).
int report_error(int code, const char* message) {
  g_last_error = message;
  return code;
}
}  // namespace sa

// ---- scratch of the allocation-free decode step (sa_hip_decode_step_noalloc) ----
// One array per GPU, held until the process ends: kNoallocCounterBytes of
// arrival counters (65535 sequences, the batch limit) at the front, split
// records of the unfused launches after them.  In host code `scratch` is a
// host-side stand-in, never a device address: the device address comes from
// hipGetSymbolAddress, once per device, and only that address is passed on.
static constexpr size_t kNoallocScratchBytes = SA_HIP_NOALLOC_SCRATCH_BYTES;
static constexpr size_t kNoallocCounterBytes = SA_HIP_NOALLOC_COUNTER_BYTES;
static_assert(kNoallocCounterBytes >= 65535 * sizeof(int32_t), "a counter for every sequence of a batch");
static_assert(kNoallocScratchBytes > kNoallocCounterBytes, "room for split records");
static __device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

// Zeroes the arrival counters with vector stores (a kernel, not
// hipMemsetAsync, so that a captured graph holds no memset node).
__global__ void clear_counters_kernel(int32_t* counters, int32_t n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) counters[i] = 0;
}

namespace {

constexpr int kNoallocMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kNoallocMaxDevices];  // device address of `scratch` per device

// The device address of the current device's `scratch`, looked up on the
// first call on that device (with the device current) and kept for the life
// of the process: a device reset (hipDeviceReset) unloads the module and
// leaves the kept address dangling, so resetting a device the library has
// run on is not supported.  The lookup is not a stream operation and may
// load the module, so the first call on a device must not run under graph
// capture: a first call on a capturing stream is refused.
int noalloc_scratch(void** out, const char* op, hipStream_t stream) {
  int dev = -1;
  if (int e = check_hip(hipGetDevice(&dev), "decode_step_noalloc: hipGetDevice")) return e;
  if (dev < 0 || dev >= kNoallocMaxDevices)
    return fail(SA_HIP_EINVAL, "%s: device %d beyond the %d devices the scratch table holds", op, dev,
                kNoallocMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone)
      return fail(SA_HIP_EINVAL, "%s: the first call on device %d must run outside graph capture (it looks up "
                  "the static scratch); call it once eagerly before capturing", op, dev);
    void* p = nullptr;
    if (int e = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "decode_step_noalloc: hipGetSymbolAddress"))
      return e;
    if (!p) return fail(SA_HIP_ERUNTIME, "%s: no device address for the scratch array", op);
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return SA_HIP_OK;
}

}  // namespace

extern "C" {

const char* sa_hip_last_error(void) { return g_last_error.c_str(); }

int sa_hip_abi_version(void) { return 1; }

int sa_hip_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

// ---- attention ---------------------------------------------------------------

size_t sa_hip_attention_workspace_bytes(int32_t batch, int32_t query_heads, int32_t kv_heads,
                                        int32_t head_dim, int32_t splits) {
  if (batch <= 0 || kv_heads <= 0 || query_heads <= 0 || splits <= 1) return 0;
  const size_t group = static_cast<size_t>(query_heads / kv_heads);
  return static_cast<size_t>(batch) * kv_heads * splits * group * sa::part_stride(head_dim) * sizeof(float);
}

size_t sa_hip_attention_chunked_workspace_bytes(int32_t batch, int32_t query_heads, int32_t kv_heads,
                                                int32_t head_dim, int32_t max_chunks) {
  const size_t records = sa_hip_attention_workspace_bytes(batch, query_heads, kv_heads, head_dim, max_chunks);
  if (!records) return 0;
  return records + 2 * static_cast<size_t>(batch) * kv_heads * max_chunks * sizeof(int32_t);
}

int32_t sa_hip_attention_splits_for(int32_t batch, int32_t query_heads, int32_t kv_heads,
                                    int32_t pages_per_group_hint) {
  // Workgroups per (sequence, KV head) so that every CU holds as many as can
  // be resident: two 8-wave workgroups per CU for 1-2 query heads per KV
  // head (registers), one for 4 (its eight 16 KiB LDS page slots) and one
  // 4-wave workgroup for 8 (registers).  Measured at B=64, 8 KV heads, G=2:
  // splits of 2-4 plus the merge kernel ran 3-7% slower than 1; at B=32,
  // G=4: one workgroup per list without the merge ran 52 us against 63 us
  // for splits of 2.  Smaller batches split the page list until every
  // resident slot is used, keeping at least ~4 pages per wave.
  const int group = kv_heads > 0 && query_heads >= kv_heads ? query_heads / kv_heads : 1;
  const int per_cu = group <= 2 ? 2 : 1;
  const int waves = group >= 8 ? 4 : 8;
  const int64_t target = static_cast<int64_t>(per_cu) * sa::compute_units();
  const int64_t pages = std::max<int32_t>(pages_per_group_hint, 1);
  const int64_t groups = static_cast<int64_t>(std::max(batch, 1)) * std::max(kv_heads, 1);
  int64_t splits = 1;
  while (groups * splits < target && (splits * 2) * waves * 4 <= pages) splits *= 2;
  return static_cast<int32_t>(std::min<int64_t>(splits, 64));
}

int32_t sa_hip_attention_default_splits(int32_t batch, int32_t kv_heads, int32_t pages_per_group_hint) {
  return sa_hip_attention_splits_for(batch, 2 * std::max(kv_heads, 1), kv_heads, pages_per_group_hint);
}

static int attention_common(const sa_paged_kv* kv, const float* query, const int32_t* selected,
                            const int32_t* counts, int32_t select_groups, int32_t sel_stride, float scale,
                            float* out, void* workspace, size_t workspace_bytes, int32_t splits,
                            int32_t* status, void* stream, int64_t contig_tokens, int32_t chunk_pages = 0,
                            int32_t* sched = nullptr) {
  sa::AttnLaunch a{};
  a.pool = kv->pool;
  a.table = kv->block_table;
  a.seq_len = kv->seq_len;
  a.sealed = kv->sealed;
  a.selected = selected;
  a.counts = counts;
  a.query = query;
  a.out = out;
  a.part = static_cast<float*>(workspace);
  a.status = status;
  a.num_pages = kv->num_pages;
  a.contig_tokens = contig_tokens;
  a.batch = kv->batch;
  a.table_stride = kv->table_stride;
  a.sel_stride = sel_stride;
  a.select_groups = select_groups;
  a.query_heads = kv->query_heads;
  a.kv_heads = kv->kv_heads;
  a.splits = splits;
  a.scale = scale;
  a.chunk_pages = chunk_pages;
  a.sched = sched;
  a.head_dim = kv->head_dim;
  const size_t need =
      sa_hip_attention_workspace_bytes(kv->batch, kv->query_heads, kv->kv_heads, kv->head_dim, splits);
  if (workspace_bytes < need || (need && !workspace))
    return fail(SA_HIP_EINVAL, "attention: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  if (sa::general_head_dim(a.head_dim))
    return check_hip(sa::launch_paged_attention_any(a, as_stream(stream)), "attention launch");
  return check_hip(sa::launch_sparse_decode_attention(a, as_stream(stream)), "attention launch");
}

int sa_hip_sparse_decode_attention(const sa_paged_kv* kv, const float* query, const int32_t* selected,
                                   const int32_t* counts, int32_t select_groups, int32_t sel_stride,
                                   float scale, float* out, void* workspace, size_t workspace_bytes,
                                   int32_t splits, int32_t* status, void* stream) {
  if (int e = check_geometry(kv, "sparse_decode_attention", true)) return e;
  if (!query || !out || !selected || !counts)
    return fail(SA_HIP_EINVAL, "sparse_decode_attention: null query/out/selected/counts");
  if (!aligned16(query)) return fail(SA_HIP_EINVAL, "sparse_decode_attention: query must be 16-byte aligned");
  if (select_groups <= 0 || kv->kv_heads % select_groups != 0)
    return fail(SA_HIP_EINVAL, "sparse_decode_attention: select_groups must divide kv_heads");
  if (sel_stride <= 0) return fail(SA_HIP_EINVAL, "sparse_decode_attention: sel_stride must be positive");
  if (splits < 1 || splits > 1024) return fail(SA_HIP_EINVAL, "sparse_decode_attention: splits out of range");
  return attention_common(kv, query, selected, counts, select_groups, sel_stride, scale, out, workspace,
                          workspace_bytes, splits, status, stream, 0);
}

int sa_hip_sparse_decode_attention_chunked(const sa_paged_kv* kv, const float* query, const int32_t* selected,
                                           const int32_t* counts, int32_t select_groups, int32_t sel_stride,
                                           float scale, float* out, void* workspace, size_t workspace_bytes,
                                           int32_t chunk_pages, int32_t max_chunks, int32_t* status,
                                           void* stream) {
  if (int e = check_geometry(kv, "attention_chunked")) return e;
  if (!query || !out || !selected || !counts)
    return fail(SA_HIP_EINVAL, "attention_chunked: null query/out/selected/counts");
  if (!aligned16(query)) return fail(SA_HIP_EINVAL, "attention_chunked: query must be 16-byte aligned");
  if (select_groups <= 0 || kv->kv_heads % select_groups != 0)
    return fail(SA_HIP_EINVAL, "attention_chunked: select_groups must divide kv_heads");
  if (sel_stride <= 0) return fail(SA_HIP_EINVAL, "attention_chunked: sel_stride must be positive");
  if (chunk_pages < 1) return fail(SA_HIP_EINVAL, "attention_chunked: chunk_pages must be positive");
  if (max_chunks < 2 || max_chunks > 65535)
    return fail(SA_HIP_EINVAL, "attention_chunked: max_chunks must lie in [2, 65535]");
  // with room for it after the records, the chunks run longest list first
  const size_t records =
      sa_hip_attention_workspace_bytes(kv->batch, kv->query_heads, kv->kv_heads, kv->head_dim, max_chunks);
  int32_t* sched = nullptr;
  if (workspace && workspace_bytes >= sa_hip_attention_chunked_workspace_bytes(kv->batch, kv->query_heads,
                                                                                 kv->kv_heads, kv->head_dim,
                                                                                 max_chunks))
    sched = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(workspace) + records);
  return attention_common(kv, query, selected, counts, select_groups, sel_stride, scale, out, workspace,
                          workspace_bytes, max_chunks, status, stream, 0, chunk_pages, sched);
}

int sa_hip_sparse_decode_attention_partial(const sa_paged_kv* kv, const float* query, const int32_t* selected,
                                           const int32_t* counts, int32_t select_groups, int32_t sel_stride,
                                           float scale, int32_t include_tail, void* workspace,
                                           size_t workspace_bytes, int32_t split_base, int32_t splits,
                                           int32_t total_splits, int32_t* status, void* stream) {
  if (int e = check_geometry(kv, "attention_partial")) return e;
  if (!query || !selected || !counts || !workspace)
    return fail(SA_HIP_EINVAL, "attention_partial: null query/selected/counts/workspace");
  if (!aligned16(query)) return fail(SA_HIP_EINVAL, "attention_partial: query must be 16-byte aligned");
  if (select_groups <= 0 || kv->kv_heads % select_groups != 0)
    return fail(SA_HIP_EINVAL, "attention_partial: select_groups must divide kv_heads");
  if (sel_stride <= 0) return fail(SA_HIP_EINVAL, "attention_partial: sel_stride must be positive");
  if (total_splits < 2 || splits < 1 || split_base < 0 || split_base + splits > total_splits)
    return fail(SA_HIP_EINVAL, "attention_partial: splits [%d, %d) outside [0, %d) (total_splits >= 2)", split_base,
                split_base + splits, total_splits);
  const size_t need =
      sa_hip_attention_workspace_bytes(kv->batch, kv->query_heads, kv->kv_heads, kv->head_dim, total_splits);
  if (workspace_bytes < need)
    return fail(SA_HIP_EINVAL, "attention_partial: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  sa::AttnLaunch a{};
  a.pool = kv->pool;
  a.table = kv->block_table;
  a.seq_len = kv->seq_len;
  a.sealed = kv->sealed;
  a.selected = selected;
  a.counts = counts;
  a.query = query;
  a.part = static_cast<float*>(workspace);
  a.status = status;
  a.num_pages = kv->num_pages;
  a.batch = kv->batch;
  a.table_stride = kv->table_stride;
  a.sel_stride = sel_stride;
  a.select_groups = select_groups;
  a.query_heads = kv->query_heads;
  a.kv_heads = kv->kv_heads;
  a.splits = splits;
  a.scale = scale;
  a.mode = 1;
  a.part_base = split_base;
  a.part_total = total_splits;
  a.include_tail = include_tail ? 1 : 0;
  return check_hip(sa::launch_sparse_decode_attention(a, as_stream(stream)), "attention_partial launch");
}

int sa_hip_attention_merge(const sa_paged_kv* kv, const void* workspace, size_t workspace_bytes,
                           int32_t total_splits, float* out, void* stream) {
  if (int e = check_geometry(kv, "attention_merge")) return e;
  if (!workspace || !out) return fail(SA_HIP_EINVAL, "attention_merge: null workspace/out");
  if (total_splits < 2) return fail(SA_HIP_EINVAL, "attention_merge: total_splits must be >= 2");
  const size_t need =
      sa_hip_attention_workspace_bytes(kv->batch, kv->query_heads, kv->kv_heads, kv->head_dim, total_splits);
  if (workspace_bytes < need)
    return fail(SA_HIP_EINVAL, "attention_merge: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  sa::AttnLaunch a{};
  a.out = out;
  a.part = static_cast<float*>(const_cast<void*>(workspace));
  a.batch = kv->batch;
  a.query_heads = kv->query_heads;
  a.kv_heads = kv->kv_heads;
  a.select_groups = 1;
  a.splits = total_splits;
  a.mode = 2;
  a.part_total = total_splits;
  return check_hip(sa::launch_sparse_decode_attention(a, as_stream(stream)), "attention_merge launch");
}

static int32_t contiguous_splits(int64_t tokens, int32_t query_heads, int32_t kv_heads) {
  const int64_t pages = (tokens + SA_HIP_PAGE_TOKENS - 1) / SA_HIP_PAGE_TOKENS;
  return sa_hip_attention_splits_for(1, query_heads, kv_heads,
                                     static_cast<int32_t>(std::min<int64_t>(pages, 1 << 30)));
}

size_t sa_hip_contiguous_workspace_bytes(int64_t tokens, int32_t query_heads, int32_t kv_heads,
                                         int32_t head_dim) {
  if (tokens <= 0 || kv_heads <= 0) return 0;
  if (head_dim != sa::kHeadDim) return sa::attention_any_workspace_bytes(tokens, query_heads, kv_heads, head_dim);
  return sa_hip_attention_workspace_bytes(1, query_heads, kv_heads, head_dim,
                                          contiguous_splits(tokens, query_heads, kv_heads));
}

int sa_hip_attention_contiguous(const uint16_t* kv, const float* query, int64_t tokens, int32_t query_heads,
                                int32_t kv_heads, int32_t head_dim, float scale, float* out, void* workspace,
                                size_t workspace_bytes, void* stream) {
  if (!kv || !query || !out) return fail(SA_HIP_EINVAL, "attention_contiguous: null pointer");
  if (tokens <= 0) return fail(SA_HIP_EINVAL, "attention_contiguous: tokens must be positive");
  if (!aligned16(kv) || !aligned16(query))
    return fail(SA_HIP_EINVAL, "attention_contiguous: kv and query must be 16-byte aligned");
  if (head_dim != sa::kHeadDim) {
    if (!sa::attention_any_supported(query_heads, kv_heads, head_dim))
      return fail(SA_HIP_EINVAL,
                  "attention_contiguous: head_dim %d with %d/%d heads unsupported (head_dim a multiple of 8 up "
                  "to %d; 1, 2, 4 or 8 query heads per KV head)",
                  head_dim, query_heads, kv_heads, sa::kAnyMaxHeadDim);
    const size_t need = sa::attention_any_workspace_bytes(tokens, query_heads, kv_heads, head_dim);
    if (workspace_bytes < need || (need && !workspace))
      return fail(SA_HIP_EINVAL, "attention_contiguous: workspace of %zu bytes needed, %zu given", need,
                  workspace_bytes);
    return check_hip(sa::launch_attention_any(kv, query, tokens, query_heads, kv_heads, head_dim, scale, out,
                                              workspace, as_stream(stream)),
                     "attention_contiguous launch");
  }
  sa_paged_kv view{};
  view.pool = const_cast<uint16_t*>(kv);
  view.block_table = reinterpret_cast<int32_t*>(1);  // unused in contiguous mode
  view.seq_len = reinterpret_cast<int32_t*>(1);
  view.sealed = reinterpret_cast<int32_t*>(1);
  view.num_pages = (tokens + SA_HIP_PAGE_TOKENS - 1) / SA_HIP_PAGE_TOKENS;
  view.batch = 1;
  view.table_stride = 1;
  view.query_heads = query_heads;
  view.kv_heads = kv_heads;
  view.head_dim = head_dim;
  if (int e = check_geometry(&view, "attention_contiguous")) return e;
  return attention_common(&view, query, nullptr, nullptr, 1, 1, scale, out, workspace, workspace_bytes,
                          contiguous_splits(tokens, query_heads, kv_heads), nullptr, stream, tokens);
}

int sa_hip_consume_checksum(const float* input, int32_t elements, float* checksum, void* stream) {
  if (!input || !checksum || elements < 0) return fail(SA_HIP_EINVAL, "consume_checksum: bad arguments");
  return check_hip(sa::launch_consume_checksum(input, elements, checksum, as_stream(stream)), "consume launch");
}

// ---- selection ---------------------------------------------------------------

static int lifecycle_common(const sa_paged_kv* kv, const float* k, const float* v, const uint16_t* k16,
                            const uint16_t* v16, int32_t local_tokens, int append, int32_t* status,
                            void* stream, const char* op, const float* query = nullptr,
                            const sa_online_seal* seal = nullptr);

// The InfLLM online seal's arguments: a query ring that holds every token of
// the tail (local + 32), a window >= 1, top-k within a block, one
// representative per query head, and this step's queries.
static int online_check(const sa_paged_kv* kv, const sa_online_seal* seal, const float* query,
                        int32_t local_tokens, const char* op) {
  if (!seal || !seal->query_ring) return fail(SA_HIP_EINVAL, "%s: null online seal / query ring", op);
  if (!query) return fail(SA_HIP_EINVAL, "%s: null query", op);
  if (local_tokens < 0 || static_cast<int64_t>(seal->ring_tokens) < static_cast<int64_t>(local_tokens) + 32)
    return fail(SA_HIP_EINVAL, "%s: ring_tokens %d must hold the tail (local_tokens %d + 32)", op,
                seal->ring_tokens, local_tokens);
  if (seal->local_window < 1) return fail(SA_HIP_EINVAL, "%s: local_window must be >= 1", op);
  if (seal->topk < 1 || seal->topk > SA_HIP_PAGE_TOKENS)
    return fail(SA_HIP_EINVAL, "%s: topk %d outside [1, 32]", op, seal->topk);
  if (kv->rep_heads != kv->query_heads)
    return fail(SA_HIP_EINVAL, "%s: the online seal writes one representative per query head "
                "(rep_heads must equal query_heads)", op);
  return SA_HIP_OK;
}

static int select_launch(const sa_paged_kv* kv, const float* query, const sa_select_params* params,
                         int32_t* selected, int32_t* counts, float* scores, int32_t* status, const char* op,
                         sa::SelectLaunch* l) {
  if (int e = check_geometry(kv, op, true)) return e;
  if (int e = check_reps(kv, op)) return e;
  if (!params || !query || !selected || !counts)
    return fail(SA_HIP_EINVAL, "%s: null params/query/selected/counts", op);
  const sa_select_params& s = *params;
  if (s.select_groups <= 0 || kv->kv_heads % s.select_groups != 0)
    return fail(SA_HIP_EINVAL, "%s: select_groups must divide kv_heads", op);
  const int heads_per_sel = kv->query_heads / s.select_groups;
  if (heads_per_sel > sa::kMaxSelectHeads)
    return fail(SA_HIP_EINVAL, "%s: %d query heads per selection group exceeds %d", op, heads_per_sel,
                sa::kMaxSelectHeads);
  if (sa::general_head_dim(kv->head_dim) && heads_per_sel * kv->head_dim > sa::kMaxAnySelectQuery)
    return fail(SA_HIP_EINVAL, "%s: %d query heads x head_dim %d per selection group exceed %d floats", op,
                heads_per_sel, kv->head_dim, sa::kMaxAnySelectQuery);
  if (s.budget_blocks <= 0 || s.init_blocks < 0 || s.local_blocks < 0 ||
      s.init_blocks + s.local_blocks > s.budget_blocks)
    return fail(SA_HIP_EINVAL, "%s: invalid representative selection dimensions "
                               "(budget %d, init %d, local %d)", op, s.budget_blocks, s.init_blocks, s.local_blocks);
  if (s.sel_stride < s.budget_blocks)
    return fail(SA_HIP_EINVAL, "%s: sel_stride %d < budget %d", op, s.sel_stride, s.budget_blocks);
  *l = sa::SelectLaunch{};
  l->query = query;
  l->reps = kv->reps;
  l->sealed = kv->sealed;
  l->selected = selected;
  l->counts = counts;
  l->scores = scores;
  l->status = status;
  l->batch = kv->batch;
  l->query_heads = kv->query_heads;
  l->kv_heads = kv->kv_heads;
  l->rep_heads = kv->rep_heads;
  l->rep_stride = kv->rep_stride;
  l->select_groups = s.select_groups;
  l->budget = s.budget_blocks;
  l->budgets = s.budgets;
  l->init_blocks = s.init_blocks;
  l->local_blocks = s.local_blocks;
  l->sel_stride = s.sel_stride;
  l->head_dim = kv->head_dim;
  return SA_HIP_OK;
}

int sa_hip_score_select(const sa_paged_kv* kv, const float* query, const sa_select_params* params,
                        int32_t* selected, int32_t* counts, float* scores, int32_t* status, void* stream) {
  sa::SelectLaunch l;
  if (int e = select_launch(kv, query, params, selected, counts, scores, status, "score_select", &l)) return e;
  if (sa::general_head_dim(l.head_dim)) {
    // the general scoring hands its scores to the selection launch
    if (!scores)
      return fail(SA_HIP_EINVAL, "score_select: head_dim %d needs the scores buffer", kv->head_dim);
    return check_hip(sa::launch_score_select_split(l, as_stream(stream)), "score_select launch");
  }
  return check_hip(sa::launch_score_select(l, as_stream(stream)), "score_select launch");
}

int sa_hip_score_select_split(const sa_paged_kv* kv, const float* query, const sa_select_params* params,
                              int32_t* selected, int32_t* counts, float* scores, int32_t* status, void* stream) {
  sa::SelectLaunch l;
  if (int e = select_launch(kv, query, params, selected, counts, scores, status, "score_select_split", &l)) return e;
  if (!scores) return fail(SA_HIP_EINVAL, "score_select_split: the scores buffer is required");
  return check_hip(sa::launch_score_select_split(l, as_stream(stream)), "score_select_split launch");
}

size_t sa_hip_score_select_chunked_workspace_bytes(const sa_paged_kv* kv, const sa_select_params* params) {
  if (!kv || !params || kv->batch <= 0 || params->select_groups <= 0 || kv->rep_stride <= 0) return 0;
  return sa::score_select_chunked_workspace_bytes(kv->batch, params->select_groups, kv->rep_stride);
}

int sa_hip_score_select_chunked(const sa_paged_kv* kv, const float* query, const sa_select_params* params,
                                int32_t* selected, int32_t* counts, void* workspace, size_t workspace_bytes,
                                int32_t* status, void* stream) {
  sa::SelectLaunch l;
  if (int e = select_launch(kv, query, params, selected, counts, nullptr, status, "score_select_chunked", &l))
    return e;
  if (sa::general_head_dim(l.head_dim))
    return fail(SA_HIP_EINVAL, "score_select_chunked: head_dim %d unsupported (128 only; sa_hip_score_select_split "
                "takes any)", kv->head_dim);
  if (!sa::score_select_chunked_supported(l))
    return fail(SA_HIP_EINVAL, "score_select_chunked: representatives must be 16-byte aligned with rep_stride a "
                               "multiple of 4");
  const size_t need = sa::score_select_chunked_workspace_bytes(kv->batch, params->select_groups, kv->rep_stride);
  if (!workspace || workspace_bytes < need)
    return fail(SA_HIP_EINVAL, "score_select_chunked: workspace of %zu bytes needed, %zu given", need,
                workspace_bytes);
  return check_hip(sa::launch_score_select_chunked(l, workspace, as_stream(stream)), "score_select_chunked launch");
}

int sa_hip_score_select_split_preferred(const sa_paged_kv* kv, const sa_select_params* params) {
  if (!kv || !params || params->select_groups <= 0) return 0;
  // measured on MI355X: spreading the scoring pays while the lists alone
  // leave compute units idle (8 lists of 4096 blocks: 424 -> 95 us; 64 lists:
  // 75 -> 41 us) and costs ~10% once every CU has a list (256 lists of 1024
  // blocks: 32 -> 35 us; 1024 lists of 2048 blocks: 204 -> 220 us)
  const int64_t lists = static_cast<int64_t>(kv->batch) * params->select_groups;
  return lists < static_cast<int64_t>(sa::compute_units()) ? 1 : 0;
}

int32_t sa_hip_select_attend_default_splits(const sa_paged_kv* kv, const sa_select_params* params) {
  if (!kv || !params) return 1;
  if (sa::general_head_dim(kv->head_dim)) {
    const int64_t lists = static_cast<int64_t>(kv->batch) * kv->kv_heads;
    // the one-launch step once its workgroups (two per CU) fill the device
    if (sa::select_attend_rows_supported(kv->query_heads, kv->kv_heads, kv->rep_heads, params->select_groups,
                                         kv->head_dim) &&
        lists >= 2LL * sa::compute_units())
      return 1;
    // the token-row attention (4-wave workgroups, several per CU): about four
    // workgroups per CU with at least 4 pages per wave (measured at B=64, 8
    // KV heads, head_dim 64: splits 2 81 us against 85 us for 1 and 88 us for 4)
    const int64_t pages = std::max<int32_t>(params->budget_blocks + 2, 1);
    int64_t splits = 1;
    while (lists * splits < 4LL * sa::compute_units() && (splits * 2) * 4 * 4 <= pages) splits *= 2;
    return static_cast<int32_t>(std::min<int64_t>(splits, 64));
  }
  // the fused kernel (two workgroups per CU, one at 4 query heads per KV
  // head) is the better choice once it fills the device
  if (sa::select_attend_supported(kv->query_heads, kv->kv_heads, params->select_groups, params->sel_stride,
                                  kv->reps, kv->rep_stride) &&
      static_cast<int64_t>(kv->batch) * kv->kv_heads >=
          sa::select_attend_per_cu(kv->query_heads, kv->kv_heads) * static_cast<int64_t>(sa::compute_units()))
    return 1;
  // the shared selection's one launch (short lists, few sequences) against
  // its three or four split launches
  if (sa::select_attend_shared_supported(kv->batch, kv->query_heads, kv->kv_heads, kv->rep_heads,
                                         params->select_groups, kv->rep_stride))
    return 1;
  return sa_hip_attention_splits_for(kv->batch, kv->query_heads, kv->kv_heads, params->budget_blocks + 2);
}

int sa_hip_select_attend_fused(const sa_paged_kv* kv, const sa_select_params* params, int32_t splits) {
  if (!kv || !params || splits != 1) return 0;
  if (sa::general_head_dim(kv->head_dim))  // the decode step only
    return sa::select_attend_rows_supported(kv->query_heads, kv->kv_heads, kv->rep_heads, params->select_groups,
                                            kv->head_dim)
               ? 1
               : 0;
  return sa::select_attend_supported(kv->query_heads, kv->kv_heads, params->select_groups, params->sel_stride,
                                     kv->reps, kv->rep_stride) ||
                 sa::select_attend_shared_supported(kv->batch, kv->query_heads, kv->kv_heads, kv->rep_heads,
                                                    params->select_groups, kv->rep_stride)
             ? 1
             : 0;
}

static sa::SelectAttendLaunch fused_launch(const sa_paged_kv* kv, const sa::SelectLaunch& l, float scale,
                                           float* out) {
  sa::SelectAttendLaunch f{};
  f.pool = kv->pool;
  f.table = kv->block_table;
  f.seq_len = kv->seq_len;
  f.sealed = kv->sealed;
  f.generation = kv->generation;
  f.reps = kv->reps;
  f.query = l.query;
  f.selected = l.selected;
  f.counts = l.counts;
  f.out = out;
  f.status = l.status;
  f.num_pages = kv->num_pages;
  f.batch = kv->batch;
  f.table_stride = kv->table_stride;
  f.query_heads = kv->query_heads;
  f.kv_heads = kv->kv_heads;
  f.rep_heads = kv->rep_heads;
  f.rep_stride = kv->rep_stride;
  f.budget = l.budget;
  f.budgets = l.budgets;
  f.init_blocks = l.init_blocks;
  f.local_blocks = l.local_blocks;
  f.sel_stride = l.sel_stride;
  f.select_groups = l.select_groups;
  f.head_dim = kv->head_dim;
  f.scale = scale;
  return f;
}

int sa_hip_select_attend(const sa_paged_kv* kv, const float* query, const sa_select_params* params, float scale,
                         int32_t* selected, int32_t* counts, float* out, void* workspace, size_t workspace_bytes,
                         int32_t splits, int32_t* status, void* stream) {
  sa::SelectLaunch l;
  if (int e = select_launch(kv, query, params, selected, counts, nullptr, status, "select_attend", &l)) return e;
  if (sa::general_head_dim(l.head_dim))
    return fail(SA_HIP_EINVAL, "select_attend: head_dim %d unsupported (128 only; sa_hip_decode_step, or "
                "sa_hip_score_select_split then sa_hip_sparse_decode_attention, take any)", kv->head_dim);
  if (!out) return fail(SA_HIP_EINVAL, "select_attend: null out");
  if (!aligned16(query)) return fail(SA_HIP_EINVAL, "select_attend: query must be 16-byte aligned");
  if (splits < 1 || splits > 1024) return fail(SA_HIP_EINVAL, "select_attend: splits out of range");
  if (!sa_hip_select_attend_fused(kv, params, splits)) {
    if (int e = check_hip(sa::launch_score_select(l, as_stream(stream)), "select_attend: score_select launch"))
      return e;
    return attention_common(kv, query, selected, counts, params->select_groups, params->sel_stride, scale, out,
                            workspace, workspace_bytes, splits, status, stream, 0);
  }
  const sa::SelectAttendLaunch f = fused_launch(kv, l, scale, out);
  return check_hip(sa::launch_select_attend(f, as_stream(stream)), "select_attend launch");
}

// Decode-step workspace: [batch] int32 arrival counters (padded to 256 B),
// then the attention's split records when the step is not fused.
static size_t arrive_bytes(int32_t batch) { return (static_cast<size_t>(batch) * 4 + 255) / 256 * 256; }

// When the step runs as separate launches its split selection (the only
// scoring at a head_dim other than 128; at 128 the shared selection's, for
// few lists) keeps the scores after the records: [batch][query_heads]
// [rep_stride] floats (enough for any select_groups).
static size_t split_records_bytes(const sa_paged_kv* kv, int32_t splits) {
  return (sa_hip_attention_workspace_bytes(kv->batch, kv->query_heads, kv->kv_heads, kv->head_dim, splits) + 255) /
         256 * 256;
}

static size_t split_scores_bytes(const sa_paged_kv* kv, int32_t select_groups) {
  return static_cast<size_t>(kv->batch) * select_groups * (kv->rep_stride > 0 ? kv->rep_stride : 0) * sizeof(float);
}

size_t sa_hip_decode_step_workspace_bytes(const sa_paged_kv* kv, int32_t splits) {
  if (!kv || kv->batch <= 0) return 0;
  return arrive_bytes(kv->batch) + split_records_bytes(kv, splits) + split_scores_bytes(kv, kv->query_heads);
}

// The decode step on explicit scratch: `arrive` holds kv->batch arrival
// counters, zero on entry to the fused launch, which leaves them at zero
// (clear_arrive: zeroed here first, whatever they hold); `records` the
// attention's split records of the unfused launches (records_bytes of them).
// With a producer (validated by the caller; k, v and query are its q/k/v
// outputs), its partial launch precedes the one-launch step that runs its
// epilogue (decode_step_qkv_supported()), else its whole projection runs
// before the step's launches.
static int decode_step_run(const sa_paged_kv* kv, const float* k, const float* v, const uint16_t* k16,
                           const uint16_t* v16, int32_t local_tokens, const float* query,
                           const sa_select_params* params, float scale, int32_t* selected, int32_t* counts,
                           float* out, int32_t* arrive, bool clear_arrive, void* records, size_t records_bytes,
                           int32_t splits, int32_t* status, void* stream, const char* op,
                           const sa_online_seal* seal = nullptr, const sa::QkvLaunch* producer = nullptr) {
  sa::SelectLaunch l;
  if (int e = select_launch(kv, query, params, selected, counts, nullptr, status, op, &l)) return e;
  if (!out) return fail(SA_HIP_EINVAL, "%s: null out", op);
  if (!aligned16(query)) return fail(SA_HIP_EINVAL, "%s: query must be 16-byte aligned", op);
  if (local_tokens < 0) return fail(SA_HIP_EINVAL, "%s: local_tokens must be >= 0", op);
  if (splits < 1 || splits > 1024) return fail(SA_HIP_EINVAL, "%s: splits out of range", op);
  const void* ka = k16 ? static_cast<const void*>(k16) : static_cast<const void*>(k);
  const void* va = v16 ? static_cast<const void*>(v16) : static_cast<const void*>(v);
  if (!ka || !va) return fail(SA_HIP_EINVAL, "%s: null k/v", op);
  if (!aligned16(ka) || !aligned16(va)) return fail(SA_HIP_EINVAL, "%s: k/v must be 16-byte aligned", op);
  if (seal)
    if (int e = online_check(kv, seal, query, local_tokens, op)) return e;
  if (producer && (seal || k16 || sa::general_head_dim(kv->head_dim)))
    return fail(SA_HIP_EINVAL, "%s: the q/k/v producer feeds head_dim %d and fp32 tokens, without the online seal",
                op, sa::kHeadDim);
  if (sa::general_head_dim(kv->head_dim) && (seal || !sa_hip_select_attend_fused(kv, params, splits))) {
    // the general kernels in sequence (where the one-launch step does not
    // apply): append + seal, scoring into the workspace's scores, selection,
    // attention
    if (seal) return fail(SA_HIP_EINVAL, "%s: the online seal is built for head_dim %d", op, sa::kHeadDim);
    const size_t rb = split_records_bytes(kv, splits);
    const size_t sb = split_scores_bytes(kv, params->select_groups);
    if (records_bytes < rb + sb)
      return fail(SA_HIP_EINVAL, "%s: workspace too small for the records and scores", op);
    l.scores = reinterpret_cast<float*>(static_cast<uint8_t*>(records) + rb);
    if (int e = lifecycle_common(kv, k, v, k16, v16, local_tokens, 1, status, stream, op, query, nullptr)) return e;
    if (int e = check_hip(sa::launch_score_select_split(l, as_stream(stream)), "decode_step: score_select launch"))
      return e;
    return attention_common(kv, query, selected, counts, params->select_groups, params->sel_stride, scale, out,
                            records, rb, splits, status, stream, 0);
  }
  // (the online seal's one launch selects per KV group)
  const bool fused =
      sa_hip_select_attend_fused(kv, params, splits) && !(seal && params->select_groups != kv->kv_heads);
  if (producer && !(fused && sa::decode_step_qkv_supported(kv->query_heads, kv->kv_heads, params->select_groups,
                                                           kv->head_dim)))
    if (int e = check_hip(sa::launch_qkv_project(*producer, as_stream(stream)), "decode_step: q/k/v producer launch"))
      return e;
  if (!fused) {
    if (int e = lifecycle_common(kv, k, v, k16, v16, local_tokens, 1, status, stream, op, query, seal)) return e;
    // few lists: the split selection (scoring spread over the device, the
    // scores after the records) where the scratch holds the scores; the same
    // ids as the one-workgroup-per-list selection
    const size_t rb = split_records_bytes(kv, splits);
    if (sa_hip_score_select_split_preferred(kv, params) &&
        records_bytes >= rb + split_scores_bytes(kv, params->select_groups)) {
      l.scores = reinterpret_cast<float*>(static_cast<uint8_t*>(records) + rb);
      if (int e = check_hip(sa::launch_score_select_split(l, as_stream(stream)), "decode_step: score_select launch"))
        return e;
    } else if (int e = check_hip(sa::launch_score_select(l, as_stream(stream)), "decode_step: score_select launch")) {
      return e;
    }
    return attention_common(kv, query, selected, counts, params->select_groups, params->sel_stride, scale, out,
                            records, records_bytes, splits, status, stream, 0);
  }
  sa::SelectAttendLaunch f = fused_launch(kv, l, scale, out);
  f.append = 1;
  f.local_tokens = local_tokens;
  f.k = k;
  f.v = v;
  f.k16 = k16;
  f.v16 = v16;
  f.arrive = arrive;
  if (seal) {
    f.ring = seal->query_ring;
    f.ring_tokens = seal->ring_tokens;
    f.window = seal->local_window;
    f.topk = seal->topk;
    f.seal_scale = 1.0f / sqrtf(static_cast<float>(kv->head_dim));
  }
  if (clear_arrive) {
    hipLaunchKernelGGL(clear_counters_kernel, dim3((kv->batch + 255) / 256), dim3(256), 0, as_stream(stream),
                       arrive, kv->batch);
    if (int e = check_hip(hipGetLastError(), "decode_step: counter clear launch")) return e;
  }
  if (producer && sa::decode_step_qkv_supported(kv->query_heads, kv->kv_heads, params->select_groups,
                                                kv->head_dim)) {
    // the producer's partial launch, then the step running its epilogue
    sa::qkv::ReduceParams r;
    if (int e = check_hip(sa::launch_qkv_partials(*producer, &r, as_stream(stream)),
                          "decode_step: q/k/v partials launch"))
      return e;
    return check_hip(sa::launch_decode_step_qkv(f, r, as_stream(stream)), "decode_step launch");
  }
  return check_hip(sa::launch_select_attend(f, as_stream(stream)), "decode_step launch");
}

static int decode_step_common(const sa_paged_kv* kv, const float* k, const float* v, const uint16_t* k16,
                              const uint16_t* v16, int32_t local_tokens, const float* query,
                              const sa_select_params* params, float scale, int32_t* selected, int32_t* counts,
                              float* out, void* workspace, size_t workspace_bytes, int32_t splits, int32_t* status,
                              void* stream, const char* op, const sa::QkvLaunch* producer = nullptr) {
  if (!kv || kv->batch <= 0) return fail(SA_HIP_EINVAL, "%s: null sa_paged_kv or empty batch", op);
  const size_t need = sa_hip_decode_step_workspace_bytes(kv, splits);
  if (!workspace || workspace_bytes < need)
    return fail(SA_HIP_EINVAL, "%s: workspace of %zu bytes needed, %zu given", op, need, workspace_bytes);
  if (!aligned16(workspace)) return fail(SA_HIP_EINVAL, "%s: workspace must be 16-byte aligned", op);
  const size_t ab = arrive_bytes(kv->batch);
  return decode_step_run(kv, k, v, k16, v16, local_tokens, query, params, scale, selected, counts, out,
                         static_cast<int32_t*>(workspace), false, static_cast<uint8_t*>(workspace) + ab,
                         workspace_bytes - ab, splits, status, stream, op, nullptr, producer);
}

int sa_hip_decode_step(const sa_paged_kv* kv, const float* k, const float* v, int32_t local_tokens,
                       const float* query, const sa_select_params* params, float scale, int32_t* selected,
                       int32_t* counts, float* out, void* workspace, size_t workspace_bytes, int32_t splits,
                       int32_t* status, void* stream) {
  return decode_step_common(kv, k, v, nullptr, nullptr, local_tokens, query, params, scale, selected, counts, out,
                            workspace, workspace_bytes, splits, status, stream, "decode_step");
}

int sa_hip_decode_step_f16(const sa_paged_kv* kv, const uint16_t* k, const uint16_t* v, int32_t local_tokens,
                           const float* query, const sa_select_params* params, float scale, int32_t* selected,
                           int32_t* counts, float* out, void* workspace, size_t workspace_bytes, int32_t splits,
                           int32_t* status, void* stream) {
  if (!k || !v) return fail(SA_HIP_EINVAL, "decode_step_f16: null k/v");
  return decode_step_common(kv, nullptr, nullptr, k, v, local_tokens, query, params, scale, selected, counts, out,
                            workspace, workspace_bytes, splits, status, stream, "decode_step_f16");
}

int sa_hip_decode_step_online(const sa_paged_kv* kv, const float* k, const float* v, int32_t local_tokens,
                              const float* query, const sa_online_seal* seal, const sa_select_params* params,
                              float scale, int32_t* selected, int32_t* counts, float* out, void* workspace,
                              size_t workspace_bytes, int32_t splits, int32_t* status, void* stream) {
  const char* op = "decode_step_online";
  if (!seal) return fail(SA_HIP_EINVAL, "%s: null online seal", op);
  if (!kv || kv->batch <= 0) return fail(SA_HIP_EINVAL, "%s: null sa_paged_kv or empty batch", op);
  const size_t need = sa_hip_decode_step_workspace_bytes(kv, splits);
  if (!workspace || workspace_bytes < need)
    return fail(SA_HIP_EINVAL, "%s: workspace of %zu bytes needed, %zu given", op, need, workspace_bytes);
  if (!aligned16(workspace)) return fail(SA_HIP_EINVAL, "%s: workspace must be 16-byte aligned", op);
  const size_t ab = arrive_bytes(kv->batch);
  return decode_step_run(kv, k, v, nullptr, nullptr, local_tokens, query, params, scale, selected, counts, out,
                         static_cast<int32_t*>(workspace), false, static_cast<uint8_t*>(workspace) + ab,
                         workspace_bytes - ab, splits, status, stream, op, seal);
}

int sa_hip_decode_step_noalloc(const sa_paged_kv* kv, const float* k, const float* v, int32_t local_tokens,
                               const float* query, const sa_select_params* params, float scale, int32_t* selected,
                               int32_t* counts, float* out, int32_t splits, int32_t* status, void* stream) {
  const char* op = "decode_step_noalloc";
  if (!kv || kv->batch <= 0) return fail(SA_HIP_EINVAL, "%s: null sa_paged_kv or empty batch", op);
  if (kv->head_dim != sa::kHeadDim)
    return fail(SA_HIP_EINVAL, "%s: head_dim %d unsupported (built for %d)", op, kv->head_dim, sa::kHeadDim);
  if (kv->batch > 65535) return fail(SA_HIP_EINVAL, "%s: batch %d out of range", op, kv->batch);
  if (splits < 1 || splits > 1024) return fail(SA_HIP_EINVAL, "%s: splits out of range", op);
  // the fused launch needs only the counters; the unfused ones need records
  // (and keep the split selection's scores after them where they fit)
  const size_t records =
      sa_hip_attention_workspace_bytes(kv->batch, kv->query_heads, kv->kv_heads, kv->head_dim, splits);
  if (records > kNoallocScratchBytes - kNoallocCounterBytes)
    return fail(SA_HIP_EINVAL, "%s: %zu bytes of split records exceed the %zu-byte static scratch (fewer splits "
                "or a smaller batch, or sa_hip_decode_step with a workspace)", op, records,
                kNoallocScratchBytes - kNoallocCounterBytes);
  void* base = nullptr;
  if (int e = noalloc_scratch(&base, op, as_stream(stream))) return e;
  // the counters are cleared before the fused launch, whatever an earlier
  // call on this GPU left in them
  return decode_step_run(kv, k, v, nullptr, nullptr, local_tokens, query, params, scale, selected, counts, out,
                         static_cast<int32_t*>(base), true, static_cast<uint8_t*>(base) + kNoallocCounterBytes,
                         kNoallocScratchBytes - kNoallocCounterBytes, splits, status, stream, op);
}

// ---- InfLLM local-causal representatives (prefill) -----------------------------

// A window of at least `tokens` keys starts every query's window at token 0,
// exactly as a window of `tokens` keys does; the probability rows are sized
// by the smaller one.
static int32_t effective_window(int64_t tokens, int32_t local_window) {
  return local_window > tokens ? static_cast<int32_t>(tokens) : local_window;
}

size_t sa_hip_local_causal_workspace_bytes(int64_t tokens, int32_t query_heads, int32_t local_window) {
  if (tokens <= 0 || query_heads <= 0 || local_window <= 0) return 0;
  return sa::local_causal_workspace_bytes(tokens, query_heads, effective_window(tokens, local_window));
}

int sa_hip_local_causal_representatives(const float* prompt_queries, const uint16_t* kv, int64_t tokens,
                                        int32_t query_heads, int32_t kv_heads, int32_t head_dim,
                                        int32_t block_tokens, int32_t local_window, int32_t topk, float* values,
                                        int32_t* offsets, float* reps, int32_t rep_stride, float* received,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  // the reference's argument checks (selection.cpp:18-23), then the library's limits
  if (!prompt_queries || !kv || tokens <= 0 || kv_heads <= 0 || query_heads % kv_heads != 0 ||
      block_tokens <= 0 || tokens % block_tokens != 0 || local_window <= 0 || topk <= 0 || topk > block_tokens)
    return fail(SA_HIP_EINVAL, "local_causal_representatives: invalid local-causal representative dimensions");
  if (head_dim <= 0) return fail(SA_HIP_EINVAL, "local_causal_representatives: head_dim must be positive");
  if (topk > sa::kMaxGeneralTopk)
    return fail(SA_HIP_EINVAL, "local_causal_representatives: topk %d above %d", topk, sa::kMaxGeneralTopk);
  if (tokens > (int64_t{1} << 31) / query_heads)
    return fail(SA_HIP_EINVAL, "local_causal_representatives: tokens x query_heads too large");
  if (!values && !reps && !offsets)
    return fail(SA_HIP_EINVAL, "local_causal_representatives: no output given");
  if (reps && rep_stride < tokens / block_tokens)
    return fail(SA_HIP_EINVAL, "local_causal_representatives: rep_stride %d below the block count", rep_stride);
  if (kv_heads > 65536) return fail(SA_HIP_EINVAL, "local_causal_representatives: kv_heads %d above 65536", kv_heads);
  if (!aligned16(kv) || !aligned16(prompt_queries))
    return fail(SA_HIP_EINVAL, "local_causal_representatives: prompt_queries and kv must be 16-byte aligned");
  const size_t need = sa_hip_local_causal_workspace_bytes(tokens, query_heads, local_window);
  if (need == 0) return fail(SA_HIP_EINVAL, "local_causal_representatives: workspace size overflows");
  if (!workspace || workspace_bytes < need)
    return fail(SA_HIP_EINVAL, "local_causal_representatives: workspace of %zu bytes needed, %zu given", need,
                workspace_bytes);
  sa::RepresentativeLaunch r{};
  r.prompt_queries = prompt_queries;
  r.kv = kv;
  r.workspace = static_cast<float*>(workspace);
  r.received = received;
  r.values = values;
  r.reps = reps;
  r.offsets = offsets;
  r.tokens = tokens;
  r.query_heads = query_heads;
  r.kv_heads = kv_heads;
  r.head_dim = head_dim;
  r.block_tokens = block_tokens;
  r.window = effective_window(tokens, local_window);
  r.topk = topk;
  r.rep_stride = rep_stride;
  // the reference's scale: 1.0f / std::sqrt(static_cast<float>(head_dim)) (selection.cpp:26)
  r.scale = 1.0f / std::sqrt(static_cast<float>(head_dim));
  return check_hip(sa::launch_local_causal_representatives(r, as_stream(stream)), "local_causal launch");
}

// ---- append / seal -------------------------------------------------------------

static int lifecycle_common(const sa_paged_kv* kv, const float* k, const float* v, const uint16_t* k16,
                            const uint16_t* v16, int32_t local_tokens, int append, int32_t* status,
                            void* stream, const char* op, const float* query, const sa_online_seal* seal) {
  if (int e = check_geometry(kv, op, !seal)) return e;
  if (int e = check_reps(kv, op)) return e;
  if (local_tokens < 0) return fail(SA_HIP_EINVAL, "%s: local_tokens must be >= 0", op);
  if (append) {
    const void* a = k16 ? static_cast<const void*>(k16) : static_cast<const void*>(k);
    const void* b = v16 ? static_cast<const void*>(v16) : static_cast<const void*>(v);
    if (!a || !b) return fail(SA_HIP_EINVAL, "%s: null k/v", op);
    if (!aligned16(a) || !aligned16(b)) return fail(SA_HIP_EINVAL, "%s: k/v must be 16-byte aligned", op);
  }
  sa::LifecycleLaunch l{};
  l.pool = kv->pool;
  l.table = kv->block_table;
  l.seq_len = kv->seq_len;
  l.sealed = kv->sealed;
  l.generation = kv->generation;
  l.reps = kv->reps;
  l.status = status;
  l.k = k;
  l.v = v;
  l.k16 = k16;
  l.v16 = v16;
  l.num_pages = kv->num_pages;
  l.batch = kv->batch;
  l.table_stride = kv->table_stride;
  l.rep_heads = kv->rep_heads;
  l.rep_stride = kv->rep_stride;
  l.query_heads = kv->query_heads;
  l.kv_heads = kv->kv_heads;
  l.head_dim = kv->head_dim;
  l.local_tokens = local_tokens;
  l.append = append;
  if (seal) {
    if (!append || k16) return fail(SA_HIP_EINVAL, "%s: the online seal needs an fp32 append", op);
    if (int e = online_check(kv, seal, query, local_tokens, op)) return e;
    l.query = query;
    l.ring = seal->query_ring;
    l.ring_tokens = seal->ring_tokens;
    l.window = seal->local_window;
    l.topk = seal->topk;
    l.seal_scale = 1.0f / sqrtf(static_cast<float>(kv->head_dim));
  }
  return check_hip(sa::launch_append_seal(l, as_stream(stream)), op);
}

int sa_hip_append_seal_online(const sa_paged_kv* kv, const float* k, const float* v, int32_t local_tokens,
                              const float* query, const sa_online_seal* seal, int32_t* status, void* stream) {
  if (!seal) return fail(SA_HIP_EINVAL, "append_seal_online: null online seal");
  return lifecycle_common(kv, k, v, nullptr, nullptr, local_tokens, 1, status, stream, "append_seal_online", query,
                          seal);
}

int sa_hip_append_seal(const sa_paged_kv* kv, const float* k, const float* v, int32_t local_tokens,
                       int32_t* status, void* stream) {
  return lifecycle_common(kv, k, v, nullptr, nullptr, local_tokens, 1, status, stream, "append_seal");
}

int sa_hip_append_seal_f16(const sa_paged_kv* kv, const uint16_t* k, const uint16_t* v, int32_t local_tokens,
                           int32_t* status, void* stream) {
  if (!k || !v) return fail(SA_HIP_EINVAL, "append_seal_f16: null k/v");
  return lifecycle_common(kv, nullptr, nullptr, k, v, local_tokens, 1, status, stream, "append_seal_f16");
}

int sa_hip_seal(const sa_paged_kv* kv, int32_t local_tokens, int32_t* status, void* stream) {
  return lifecycle_common(kv, nullptr, nullptr, nullptr, nullptr, local_tokens, 0, status, stream, "seal");
}

// ---- read reference ------------------------------------------------------------

int sa_hip_read_step_bytes(const sa_paged_kv* kv, const int32_t* selected, const int32_t* counts,
                           int32_t select_groups, int32_t sel_stride, uint32_t* out, int32_t* status,
                           void* stream) {
  if (int e = check_geometry(kv, "read_step_bytes")) return e;
  if (int e = check_reps(kv, "read_step_bytes")) return e;
  if (!selected || !counts || !out) return fail(SA_HIP_EINVAL, "read_step_bytes: null selected/counts/out");
  if (!aligned16(kv->reps) || kv->rep_stride % 4 != 0)
    return fail(SA_HIP_EINVAL, "read_step_bytes: reps must be 16-byte aligned with rep_stride a multiple of 4");
  if (select_groups <= 0 || kv->kv_heads % select_groups != 0)
    return fail(SA_HIP_EINVAL, "read_step_bytes: select_groups must divide kv_heads");
  if (sel_stride <= 0) return fail(SA_HIP_EINVAL, "read_step_bytes: sel_stride must be positive");
  sa::ReadStepLaunch l{};
  l.pool = kv->pool;
  l.table = kv->block_table;
  l.seq_len = kv->seq_len;
  l.sealed = kv->sealed;
  l.reps = kv->reps;
  l.selected = selected;
  l.counts = counts;
  l.out = out;
  l.status = status;
  l.num_pages = kv->num_pages;
  l.batch = kv->batch;
  l.table_stride = kv->table_stride;
  l.kv_heads = kv->kv_heads;
  l.rep_heads = kv->rep_heads;
  l.rep_stride = kv->rep_stride;
  l.select_groups = select_groups;
  l.sel_stride = sel_stride;
  return check_hip(sa::launch_read_step_bytes(l, as_stream(stream)), "read_step_bytes launch");
}

// ---- gather --------------------------------------------------------------------

int sa_hip_gather_pages(const uint16_t* pool, int64_t page_bytes, int64_t num_pages, const int32_t* pages,
                        int32_t count, uint16_t* out, int32_t* status, void* stream) {
  if (!pool || !pages || !out) return fail(SA_HIP_EINVAL, "gather_pages: null pointer");
  if (page_bytes <= 0 || page_bytes % 16 != 0)
    return fail(SA_HIP_EINVAL, "gather_pages: page_bytes must be a positive multiple of 16");
  if (!aligned16(pool) || !aligned16(out)) return fail(SA_HIP_EINVAL, "gather_pages: pool/out must be 16-byte aligned");
  if (count < 0 || count > 65535) return fail(SA_HIP_EINVAL, "gather_pages: count out of range");
  return check_hip(sa::launch_gather_pages(pool, page_bytes, num_pages, pages, count, out, status,
                                           as_stream(stream)),
                   "gather launch");
}

// ---- history prediction and correction -------------------------------------

int sa_hip_compare_prediction(const int32_t* predicted, const int32_t* oracle, int32_t n, int32_t* hits,
                              int32_t* misses, int32_t* replacement_slots, int32_t* miss_count) {
  if (n < 0 || (n > 0 && (!predicted || !oracle || !misses || !replacement_slots)) || !hits || !miss_count)
    return fail(SA_HIP_EINVAL, "compare_prediction: bad arguments");
  int32_t evicted = 0, missing = 0, h = 0;
  const int32_t* oe = oracle + n;
  const int32_t* pe = predicted + n;
  for (int32_t slot = 0; slot < n; ++slot) {
    if (std::find(oracle, oe, predicted[slot]) != oe) ++h;
    else replacement_slots[evicted++] = slot;
  }
  for (int32_t i = 0; i < n; ++i)
    if (std::find(predicted, pe, oracle[i]) == pe) misses[missing++] = oracle[i];
  *hits = h;
  *miss_count = missing;
  if (missing != evicted) return fail(SA_HIP_EINVAL, "prediction correction cardinality mismatch");
  return SA_HIP_OK;
}

static int fill_args_ok(uint16_t* pool, int64_t page_bytes, const int32_t* dst_pages, const void* src_base,
                        const int64_t* src_blocks, int32_t count, const char* op) {
  if (count < 0 || (count > 0 && (!pool || !dst_pages || !src_base || !src_blocks)) || page_bytes <= 0 ||
      page_bytes % 16 != 0)
    return fail(SA_HIP_EINVAL, "%s: bad arguments", op);
  for (int32_t i = 0; i < count; ++i)
    if (dst_pages[i] < 0 || src_blocks[i] < 0)
      return fail(SA_HIP_EINVAL, "%s: negative page/block index at %d", op, i);
  return SA_HIP_OK;
}

// ---- query producer / output consumer ----------------------------------------

int sa_hip_rms_norm(const float* x, const float* w, float* out, int32_t rows, int32_t width, float eps,
                    void* stream) {
  if (!x || !w || !out || rows <= 0 || rows > 2147483647 / 2 || width <= 0 || width % 4 != 0)
    return fail(SA_HIP_EINVAL, "rms_norm: bad arguments (width must be a positive multiple of 4)");
  if (!aligned16(x) || !aligned16(w) || !aligned16(out))
    return fail(SA_HIP_EINVAL, "rms_norm: x, w and out must be 16-byte aligned");
  return check_hip(sa::launch_rms_norm(x, w, out, rows, width, eps, as_stream(stream)), "rms_norm launch");
}

static int linear_shape_ok(int32_t rows, int32_t in, int32_t out, const char* op) {
  if (rows <= 0 || rows > 65535 * 64 || in <= 0 || in % 256 != 0 || out <= 0 || out % 64 != 0 ||
      out > 65535 * 16)
    return fail(SA_HIP_EINVAL, "%s: rows %d, in %d, out %d unsupported (in a multiple of 256, out of 64)", op,
                rows, in, out);
  return SA_HIP_OK;
}

size_t sa_hip_linear_workspace_bytes(int32_t rows, int32_t in, int32_t out) {
  if (rows <= 0 || in <= 0 || out <= 0) return 0;
  return sa::split_part_bytes(rows, in, out, false);
}

int sa_hip_linear(const float* x, const float* w, const float* residual, float* y, int32_t rows, int32_t in,
                  int32_t out, void* workspace, size_t workspace_bytes, void* stream) {
  if (int e = linear_shape_ok(rows, in, out, "linear")) return e;
  if (!x || !w || !y || !workspace) return fail(SA_HIP_EINVAL, "linear: null x/w/y/workspace");
  if (!aligned16(x) || !aligned16(w) || !aligned16(y) || (residual && !aligned16(residual)))
    return fail(SA_HIP_EINVAL, "linear: x, w, residual and y must be 16-byte aligned");
  if (workspace_bytes < sa_hip_linear_workspace_bytes(rows, in, out))
    return fail(SA_HIP_EINVAL, "linear: workspace of %zu bytes < %zu", workspace_bytes,
                sa_hip_linear_workspace_bytes(rows, in, out));
  if (!aligned16(workspace)) return fail(SA_HIP_EINVAL, "linear: workspace must be 16-byte aligned");
  sa::LinearLaunch l{x, w, residual, y, static_cast<float*>(workspace), rows, in, out};
  return check_hip(sa::launch_linear(l, as_stream(stream)), "linear launch");
}

size_t sa_hip_qkv_workspace_bytes(int32_t rows, int32_t hidden, int32_t q_heads, int32_t kv_heads) {
  if (rows <= 0 || hidden <= 0 || q_heads <= 0 || kv_heads <= 0) return 0;
  const int64_t out = static_cast<int64_t>(q_heads + 2 * kv_heads) * sa::kHeadDim;
  return sa::split_part_bytes(rows, hidden, out, true);
}

static int qkv_prepare(const float* x, const float* gain, float in_eps, const float* wq, const float* wk,
                       const float* wv, const float* q_norm, const float* k_norm, const int32_t* positions,
                       int32_t rows, int32_t hidden, int32_t q_heads, int32_t kv_heads, float theta, float eps,
                       float* q, float* k, float* v, void* workspace, size_t workspace_bytes,
                       sa::QkvLaunch* out, const char* op) {
  if (q_heads <= 0 || kv_heads <= 0 || q_heads > 256 || kv_heads > 256)
    return fail(SA_HIP_EINVAL, "%s: bad head counts %d/%d", op, q_heads, kv_heads);
  if (int e = linear_shape_ok(rows, hidden, (q_heads + 2 * kv_heads) * sa::kHeadDim, op)) return e;
  if (!x || !wq || !wk || !wv || !q_norm || !k_norm || !positions || !q || !k || !v || !workspace)
    return fail(SA_HIP_EINVAL, "%s: null argument", op);
  if (!aligned16(x) || !aligned16(wq) || !aligned16(wk) || !aligned16(wv) || (gain && !aligned16(gain)) ||
      !aligned16(q_norm) || !aligned16(k_norm) || !aligned16(q) || !aligned16(k) || !aligned16(v) ||
      !aligned16(workspace))
    return fail(SA_HIP_EINVAL, "%s: x, the weights, the norms, q/k/v and the workspace must be 16-byte aligned",
                op);
  if (!(theta > 1.0f)) return fail(SA_HIP_EINVAL, "%s: rope theta must exceed 1", op);
  if (workspace_bytes < sa_hip_qkv_workspace_bytes(rows, hidden, q_heads, kv_heads))
    return fail(SA_HIP_EINVAL, "%s: workspace of %zu bytes < %zu", op, workspace_bytes,
                sa_hip_qkv_workspace_bytes(rows, hidden, q_heads, kv_heads));
  sa::QkvLaunch& l = *out;
  l = sa::QkvLaunch{};
  l.x = x;
  l.gain = gain;
  l.in_eps = in_eps;
  l.wq = wq;
  l.wk = wk;
  l.wv = wv;
  l.q_norm = q_norm;
  l.k_norm = k_norm;
  l.positions = positions;
  l.q = q;
  l.k = k;
  l.v = v;
  l.workspace = static_cast<float*>(workspace);
  l.rows = rows;
  l.hidden = hidden;
  l.q_heads = q_heads;
  l.kv_heads = kv_heads;
  l.eps = eps;
  // theta^(-2i/128), correctly rounded (the reference's powf is within 2 ulp)
  for (int i = 0; i < 64; ++i)
    l.inv_freq[i] = static_cast<float>(std::pow(static_cast<double>(theta), -2.0 * i / sa::kHeadDim));
  return 0;
}

static int qkv_common(const float* x, const float* gain, float in_eps, const float* wq, const float* wk,
                      const float* wv, const float* q_norm, const float* k_norm, const int32_t* positions,
                      int32_t rows, int32_t hidden, int32_t q_heads, int32_t kv_heads, float theta, float eps,
                      float* q, float* k, float* v, void* workspace, size_t workspace_bytes, void* stream,
                      const char* op) {
  sa::QkvLaunch l;
  if (int e = qkv_prepare(x, gain, in_eps, wq, wk, wv, q_norm, k_norm, positions, rows, hidden, q_heads, kv_heads,
                          theta, eps, q, k, v, workspace, workspace_bytes, &l, op))
    return e;
  return check_hip(sa::launch_qkv_project(l, as_stream(stream)), op);
}

int sa_hip_qkv_project(const float* x, const float* wq, const float* wk, const float* wv, const float* q_norm,
                       const float* k_norm, const int32_t* positions, int32_t rows, int32_t hidden,
                       int32_t q_heads, int32_t kv_heads, float theta, float eps, float* q, float* k, float* v,
                       void* workspace, size_t workspace_bytes, void* stream) {
  return qkv_common(x, nullptr, 0.0f, wq, wk, wv, q_norm, k_norm, positions, rows, hidden, q_heads, kv_heads, theta,
                    eps, q, k, v, workspace, workspace_bytes, stream, "qkv_project");
}

int sa_hip_qkv_project_rms(const float* hidden_rows, const float* input_norm, float input_eps, const float* wq,
                           const float* wk, const float* wv, const float* q_norm, const float* k_norm,
                           const int32_t* positions, int32_t rows, int32_t hidden, int32_t q_heads,
                           int32_t kv_heads, float theta, float eps, float* q, float* k, float* v, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (!input_norm) return fail(SA_HIP_EINVAL, "qkv_project_rms: null input_norm");
  return qkv_common(hidden_rows, input_norm, input_eps, wq, wk, wv, q_norm, k_norm, positions, rows, hidden, q_heads,
                    kv_heads, theta, eps, q, k, v, workspace, workspace_bytes, stream, "qkv_project_rms");
}

int sa_hip_decode_step_qkv(const sa_paged_kv* kv, const sa_qkv_producer* producer, int32_t local_tokens,
                           const sa_select_params* params, float scale, int32_t* selected, int32_t* counts,
                           float* out, void* workspace, size_t workspace_bytes, int32_t splits, int32_t* status,
                           void* stream) {
  const char* op = "decode_step_qkv";
  if (!kv || kv->batch <= 0) return fail(SA_HIP_EINVAL, "%s: null sa_paged_kv or empty batch", op);
  if (!producer) return fail(SA_HIP_EINVAL, "%s: null producer", op);
  const sa_qkv_producer& pr = *producer;
  sa::QkvLaunch l;
  if (int e = qkv_prepare(pr.hidden_rows, pr.input_norm, pr.input_eps, pr.wq, pr.wk, pr.wv, pr.q_norm, pr.k_norm,
                          pr.positions, kv->batch, pr.hidden, kv->query_heads, kv->kv_heads, pr.theta, pr.eps, pr.q,
                          pr.k, pr.v, pr.workspace, pr.workspace_bytes, &l, op))
    return e;
  return decode_step_common(kv, pr.k, pr.v, nullptr, nullptr, local_tokens, pr.q, params, scale, selected, counts,
                            out, workspace, workspace_bytes, splits, status, stream, op, &l);
}

int sa_hip_pages_to_host_async(const uint16_t* pool, int64_t page_bytes, int64_t num_pages, const int32_t* pages,
                               int32_t count, void* dst, void* copy_stream, void* after_event, void* done_event) {
  if (count < 0 || (count > 0 && (!pool || !pages || !dst)) || page_bytes <= 0 || page_bytes % 16 != 0)
    return fail(SA_HIP_EINVAL, "pages_to_host_async: bad arguments");
  for (int32_t i = 0; i < count; ++i)
    if (pages[i] < 0 || pages[i] >= num_pages)
      return fail(SA_HIP_EINVAL, "pages_to_host_async: page %d outside [0, %lld) at %d", pages[i],
                  static_cast<long long>(num_pages), i);
  hipStream_t cs = as_stream(copy_stream);
  if (after_event)
    if (int e = check_hip(hipStreamWaitEvent(cs, reinterpret_cast<hipEvent_t>(after_event), 0),
                          "pages_to_host_async: hipStreamWaitEvent"))
      return e;
  // pinned host memory the device can address: one kernel launch per 256
  // pages writing through the mapping; anything else: one copy per page
  hipPointerAttribute_t attr{};
  const bool mapped = count > 0 && hipPointerGetAttributes(&attr, dst) == hipSuccess &&
                      attr.type == hipMemoryTypeHost && attr.devicePointer == dst;
  (void)hipGetLastError();  // a pageable pointer leaves an error behind
  if (mapped) {
    if (int e = check_hip(sa::launch_pages_to_host(pool, page_bytes, pages, count, dst, cs),
                          "pages_to_host_async: launch"))
      return e;
  } else {
    const auto* src = reinterpret_cast<const uint8_t*>(pool);
    auto* out = static_cast<uint8_t*>(dst);
    for (int32_t i = 0; i < count; ++i)
      if (int e = check_hip(hipMemcpyAsync(out + static_cast<int64_t>(i) * page_bytes,
                                           src + static_cast<int64_t>(pages[i]) * page_bytes,
                                           static_cast<size_t>(page_bytes), hipMemcpyDeviceToHost, cs),
                            "pages_to_host_async: hipMemcpyAsync"))
        return e;
  }
  if (done_event)
    return check_hip(hipEventRecord(reinterpret_cast<hipEvent_t>(done_event), cs), "pages_to_host_async: record");
  return SA_HIP_OK;
}

int sa_hip_fill_pages_async(uint16_t* pool, int64_t page_bytes, const int32_t* dst_pages, const void* src_base,
                            const int64_t* src_blocks, int32_t count, void* copy_stream, void* done_event) {
  if (int e = fill_args_ok(pool, page_bytes, dst_pages, src_base, src_blocks, count, "fill_pages_async")) return e;
  auto* dst = reinterpret_cast<uint8_t*>(pool);
  const auto* src = static_cast<const uint8_t*>(src_base);
  for (int32_t i = 0; i < count; ++i) {
    if (int e = check_hip(hipMemcpyAsync(dst + static_cast<int64_t>(dst_pages[i]) * page_bytes,
                                         src + src_blocks[i] * page_bytes, static_cast<size_t>(page_bytes),
                                         hipMemcpyHostToDevice, as_stream(copy_stream)),
                          "fill_pages_async: hipMemcpyAsync"))
      return e;
  }
  if (done_event)
    return check_hip(hipEventRecord(reinterpret_cast<hipEvent_t>(done_event), as_stream(copy_stream)),
                     "fill_pages_async: hipEventRecord");
  return SA_HIP_OK;
}

int sa_hip_fill_pages_gather_async(uint16_t* pool, int64_t page_bytes, int64_t num_pages,
                                   const int32_t* dst_pages_dev, const void* src_base, int64_t src_blocks_total,
                                   const int64_t* src_blocks_dev, int32_t count, int32_t* status, void* copy_stream,
                                   void* done_event) {
  if (count < 0 || (count > 0 && (!pool || !dst_pages_dev || !src_base || !src_blocks_dev)) || page_bytes <= 0 ||
      page_bytes % 16 != 0)
    return fail(SA_HIP_EINVAL, "fill_pages_gather_async: bad arguments");
  void* src_dev = nullptr;
  if (count > 0) {
    if (int e = check_hip(hipHostGetDevicePointer(&src_dev, const_cast<void*>(src_base), 0),
                          "fill_pages_gather_async: hipHostGetDevicePointer (source must be pinned host memory)"))
      return e;
    if (int e = check_hip(sa::launch_fill_from_host(pool, page_bytes, num_pages, dst_pages_dev,
                                                    static_cast<const uint8_t*>(src_dev), src_blocks_total,
                                                    src_blocks_dev, count, status, as_stream(copy_stream)),
                          "fill_pages_gather_async launch"))
      return e;
  }
  if (done_event)
    return check_hip(hipEventRecord(reinterpret_cast<hipEvent_t>(done_event), as_stream(copy_stream)),
                     "fill_pages_gather_async: hipEventRecord");
  return SA_HIP_OK;
}

int sa_hip_stream_wait_event(void* stream, void* event) {
  if (!event) return fail(SA_HIP_EINVAL, "stream_wait_event: null event");
  return check_hip(hipStreamWaitEvent(as_stream(stream), reinterpret_cast<hipEvent_t>(event), 0),
                   "hipStreamWaitEvent");
}

// ---- synthetic data --------------------------------------------------------------

int sa_hip_fill_synthetic_f16(uint16_t* dst, int64_t count, uint64_t seed, uint64_t first_index, void* stream) {
  if (!dst || count < 0) return fail(SA_HIP_EINVAL, "fill_synthetic_f16: bad arguments");
  return check_hip(sa::launch_fill_synthetic_f16(dst, count, seed, first_index, as_stream(stream)),
                   "fill_synthetic_f16 launch");
}

int sa_hip_fill_synthetic_f32(float* dst, int64_t count, uint64_t seed, uint64_t first_index, void* stream) {
  if (!dst || count < 0) return fail(SA_HIP_EINVAL, "fill_synthetic_f32: bad arguments");
  return check_hip(sa::launch_fill_synthetic_f32(dst, count, seed, first_index, as_stream(stream)),
                   "fill_synthetic_f32 launch");
}

}  // extern "C"
