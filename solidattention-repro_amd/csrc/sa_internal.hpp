// sa_internal.hpp — host-side launch interface between the C-ABI layer
// (capi.hip) and the kernel files.  Not installed; not part of the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace sa {

constexpr int kHeadDim = 128;      // head_dim the tuned kernels are built for
constexpr int kPartPad = 4;        // floats before the accumulator in a partial record
constexpr int kMaxSelectBlocks = 8192;
constexpr int kMaxSelectHeads = 32;
constexpr int kMaxStagedSelected = 2048;  // selected ids per list the fused kernel at 4 heads per KV head holds
// Longest shared list (one block set over every query head) the one-launch
// decode step takes: each of its workgroups scores the whole shared set, 64
// blocks per pass, so longer lists run faster as separate launches (measured
// at 250 blocks: 48.6 us one launch against 37.0 us separate, at 64 blocks
// 24.2 against 33.8 us).
constexpr int kMaxSharedFusedBlocks = 128;

// Partial-result record of one (sequence, KV head, split, query head):
// [0] running max (log2 domain), [1] denominator, [kPartPad, kPartPad + D)
// accumulator.
constexpr int part_stride(int head_dim) { return head_dim + kPartPad; }


struct AttnLaunch {
  const uint16_t* pool;
  const int32_t* table;
  const int32_t* seq_len;
  const int32_t* sealed;
  const int32_t* selected;
  const int32_t* counts;
  const float* query;
  float* out;
  float* part;             // split partial records
  int32_t* status;
  int64_t num_pages;
  int64_t contig_tokens;   // > 0: contiguous token buffer mode (batch 1, no table)
  int32_t batch;
  int32_t table_stride;
  int32_t sel_stride;
  int32_t select_groups;
  int32_t query_heads;
  int32_t kv_heads;
  int32_t splits;
  float scale;
  // 0: full attention (+ merge when splits > 1); 1: partial records
  // [part_base, part_base + splits) of part_total only; 2: merge of
  // part_total records only.
  int32_t mode;
  int32_t part_base;
  int32_t part_total;
  int32_t include_tail;
  int32_t chunk_pages;     // > 0 (mode 0): split by chunks of pages, `splits` chunks
  int32_t* sched;          // chunked: 2 x batch x kv_heads x splits int32 for the longest-first order, or null
  int32_t head_dim;        // 0 or kHeadDim: the paged kernels; another multiple of 8 up to
                           // kAnyMaxHeadDim: the general kernel (mode 0, no chunks)
};

hipError_t launch_sparse_decode_attention(const AttnLaunch& a, hipStream_t stream);

struct SelectLaunch {
  const float* query;
  const float* reps;
  const int32_t* sealed;
  int32_t* selected;
  int32_t* counts;
  float* scores;
  int32_t* status;
  int32_t batch;
  int32_t query_heads;
  int32_t kv_heads;
  int32_t rep_heads;
  int32_t rep_stride;
  int32_t select_groups;
  int32_t budget;
  const int32_t* budgets;
  int32_t init_blocks;
  int32_t local_blocks;
  int32_t sel_stride;
  int32_t head_dim;  // 0 or kHeadDim; another head_dim scores with the general kernel (split form only)
};

hipError_t launch_score_select(const SelectLaunch& s, hipStream_t stream);
// scoring over chunks of 256 blocks into s.scores, then selection from them
hipError_t launch_score_select_split(const SelectLaunch& s, hipStream_t stream);
// lists split into chunks of 512 blocks, one launch: workspace of
// score_select_chunked_workspace_bytes(), its arrival counters zeroed once
// (each launch leaves them at zero); needs 16-byte representative loads
size_t score_select_chunked_workspace_bytes(int64_t batch, int32_t select_groups, int32_t rep_stride);
bool score_select_chunked_supported(const SelectLaunch& s);
hipError_t launch_score_select_chunked(const SelectLaunch& s, void* workspace, hipStream_t stream);

// ---- query producer / output consumer (producer.hip) -----------------------
struct LinearLaunch {
  const float* x;         // [rows][in]
  const float* w;         // [out][in]
  const float* residual;  // [rows][out] or null
  float* y;               // [rows][out]
  float* workspace;       // split_part_bytes(rows, in, out, false): the slices' partial tiles
  int32_t rows, in, out;
};
struct QkvLaunch {
  const float* x;         // hidden [rows][hidden]: normalised, or raw with gain
  const float* gain;      // optional input RMSNorm weight [hidden] (folded into the projection)
  float in_eps;
  const float* wq;        // [q_heads*128][hidden]
  const float* wk;        // [kv_heads*128][hidden]
  const float* wv;
  const float* q_norm;    // [128]
  const float* k_norm;
  const int32_t* positions;  // [rows]
  float* q;               // [rows][q_heads][128]
  float* k;               // [rows][kv_heads][128]
  float* v;
  float* workspace;
  int32_t rows, hidden, q_heads, kv_heads;
  float eps;
  float inv_freq[64];
};
// Split-K projections: columns per workgroup and K slices; the workspace is
// the slices' partial tiles (plus per-slice sums of squares of x for q/k/v).
struct SplitShape {
  int32_t cols;
  int32_t slices;
  int32_t ks;  // k per slice: 256, or 128 for two 64-column workgroups per compute unit
};
SplitShape split_shape(int64_t rows, int64_t in, int64_t out);
size_t split_part_bytes(int64_t rows, int64_t in, int64_t out, bool with_ss);
hipError_t launch_rms_norm(const float* x, const float* w, float* out, int rows, int width, float eps,
                           hipStream_t stream);
hipError_t launch_linear(const LinearLaunch& l, hipStream_t stream);
hipError_t launch_qkv_project(const QkvLaunch& q, hipStream_t stream);
// The q/k/v projection's partial launch only; *r receives the parameters of
// its epilogue (qkv_epilogue.hpp), which the caller runs.
namespace qkv {
struct ReduceParams;
}
hipError_t launch_qkv_partials(const QkvLaunch& q, qkv::ReduceParams* r, hipStream_t stream);

// Compute units of the current device (cached per device; 256 if unknown).
int compute_units();

// Fused (append + seal +) score + select + attend, one workgroup per
// (sequence, KV head); select_groups is kv_heads, or 1 (the shared selection,
// select_attend_shared_supported()).
struct SelectAttendLaunch {
  const uint16_t* pool;
  const int32_t* table;
  int32_t* seq_len;
  int32_t* sealed;
  int32_t* generation;
  float* reps;
  const float* query;
  int32_t* selected;
  int32_t* counts;
  float* out;
  int32_t* status;
  int64_t num_pages;
  int32_t batch;
  int32_t table_stride;
  int32_t query_heads;
  int32_t kv_heads;
  int32_t rep_heads;
  int32_t rep_stride;
  int32_t budget;
  const int32_t* budgets;
  int32_t init_blocks;
  int32_t local_blocks;
  int32_t sel_stride;
  int32_t select_groups;  // kv_heads (a block set per KV group), or 1 (shared)
  int32_t head_dim;       // 0 or kHeadDim; another (decode step only): select_attend_rows_supported()
  float scale;
  // decode step: append one token per sequence (fp32 k/v or FP16 k16/v16),
  // seal, then select + attend; arrive = [batch] zeroed arrival counters
  int32_t append;
  int32_t local_tokens;
  const float* k;
  const float* v;
  const uint16_t* k16;
  const uint16_t* v16;
  int32_t* arrive;
  // InfLLM online seal (decode step; ring non-null, rep_heads == query_heads)
  float* ring;
  int32_t ring_tokens;
  int32_t window;
  int32_t topk;
  float seal_scale;
};

// The fused kernels: 1-2 query heads per KV head (registers), or 4 (LDS-staged
// pages; sel_stride <= kMaxStagedSelected, reps 8-byte aligned, rep_stride
// even).  Resident workgroups per CU: 2, or 1 for 4 query heads per KV head.
bool select_attend_supported(int32_t query_heads, int32_t kv_heads, int32_t select_groups, int32_t sel_stride,
                             const float* reps, int32_t rep_stride);
int select_attend_per_cu(int32_t query_heads, int32_t kv_heads);
// The one-launch form of the shared selection (select_groups 1 over several
// KV heads): 1, 2 or 4 query heads per KV head, representatives per KV head,
// rep_stride <= kMaxSharedFusedBlocks, and the representatives read once per
// KV head (every workgroup scores the whole set) within a small byte budget.
bool select_attend_shared_supported(int32_t batch, int32_t query_heads, int32_t kv_heads, int32_t rep_heads,
                                    int32_t select_groups, int32_t rep_stride);
// The one-launch decode step at a head_dim other than 128: a multiple of 8
// up to 256, 1, 2 or 4 query heads per KV head, selection per KV group,
// representatives per KV head.
bool select_attend_rows_supported(int32_t query_heads, int32_t kv_heads, int32_t rep_heads, int32_t select_groups,
                                  int32_t head_dim);
hipError_t launch_select_attend(const SelectAttendLaunch& s, hipStream_t stream);
// The decode step (append, with k, v and query the producer's outputs) fed
// by the q/k/v projection's partials: the producer's epilogue runs inside the
// one-launch step.  head_dim 128, selection per KV group, 1 or 2 query heads
// per KV head, fp32 token, no online seal; r from launch_qkv_partials() with
// rows == batch and r.q == s.query.
bool decode_step_qkv_supported(int32_t query_heads, int32_t kv_heads, int32_t select_groups, int32_t head_dim);
hipError_t launch_decode_step_qkv(const SelectAttendLaunch& s, const qkv::ReduceParams& r, hipStream_t stream);

// InfLLM local-causal block representatives of a prefill (contiguous KV).
struct RepresentativeLaunch {
  const float* prompt_queries;  // [query_heads][tokens][head_dim]
  const uint16_t* kv;           // [tokens][2][kv_heads][head_dim]
  float* workspace;             // local_causal_workspace_bytes()
  float* received;              // [query_heads][tokens] or null (kept in the workspace)
  float* values;                // [query_heads][blocks][head_dim] or null
  float* reps;                  // [query_heads][head_dim][rep_stride] or null
  int32_t* offsets;             // [query_heads][blocks][topk] or null
  int64_t tokens;
  int32_t query_heads;
  int32_t kv_heads;
  int32_t head_dim;
  int32_t block_tokens;
  int32_t window;
  int32_t topk;
  int32_t rep_stride;
  float scale;
};

// The tiled builder kernels take head_dim 128, 32-token blocks and windows
// up to 256; other shapes run the general kernels, whose one limit is topk
// (the chosen offsets of a block are ranked in LDS).
constexpr int kMaxTiledLocalWindow = 256;
constexpr int kMaxGeneralTopk = 16384;
size_t local_causal_workspace_bytes(int64_t tokens, int32_t query_heads, int32_t window);
hipError_t launch_local_causal_representatives(const RepresentativeLaunch& r, hipStream_t stream);

struct LifecycleLaunch {
  uint16_t* pool;
  const int32_t* table;
  int32_t* seq_len;
  int32_t* sealed;
  int32_t* generation;
  float* reps;
  int32_t* status;
  const float* k;
  const float* v;
  const uint16_t* k16;
  const uint16_t* v16;
  int64_t num_pages;
  int32_t batch;
  int32_t table_stride;
  int32_t rep_heads;
  int32_t rep_stride;
  int32_t query_heads;
  int32_t kv_heads;
  int32_t head_dim; // 0 or kHeadDim; another head_dim appends and seals one workgroup per sequence
  int32_t local_tokens;
  int32_t append;   // 0: seal only
  // InfLLM online seal (ring non-null; rep_heads == query_heads): the
  // decode queries [batch][query_heads][D] of this step are kept in
  // ring[batch][query_heads][ring_tokens][D] and a sealed block's
  // representative is the local-causal builder over the block
  const float* query;
  float* ring;
  int32_t ring_tokens;
  int32_t window;
  int32_t topk;
  float seal_scale;
};

hipError_t launch_append_seal(const LifecycleLaunch& l, hipStream_t stream);

// Contiguous attention for head dimensions other than 128 (attention_any.hip):
// multiples of 8 up to kAnyMaxHeadDim, 1/2/4/8 query heads per KV head.
constexpr int kAnyMaxHeadDim = 512;
// The paged path at a head_dim other than kHeadDim (any multiple of 8 up to
// kAnyMaxHeadDim): attention over the selected blocks and the tail
// (AttnLaunch mode 0, no chunks), with a merge of the splits in split order.
hipError_t launch_paged_attention_any(const AttnLaunch& a, hipStream_t stream);
inline bool general_head_dim(int32_t head_dim) { return head_dim != 0 && head_dim != kHeadDim; }
// The general scoring keeps a selection group's query rows in LDS.
constexpr int kMaxAnySelectQuery = 16384;  // heads_per_sel x head_dim floats (64 KiB)
bool attention_any_supported(int32_t query_heads, int32_t kv_heads, int32_t head_dim);
size_t attention_any_workspace_bytes(int64_t tokens, int32_t query_heads, int32_t kv_heads, int32_t head_dim);
hipError_t launch_attention_any(const uint16_t* kv, const float* query, int64_t tokens, int32_t query_heads,
                                int32_t kv_heads, int32_t head_dim, float scale, float* out, void* workspace,
                                hipStream_t stream);

// The decode step's bytes for each (sequence, KV head) read with no
// arithmetic: representatives of the sealed blocks, the selected pages' K/V
// slices and the tail; out[b * kv_heads + h] is the XOR of the 32-bit words.
struct ReadStepLaunch {
  const uint16_t* pool;
  const int32_t* table;
  const int32_t* seq_len;
  const int32_t* sealed;
  const float* reps;
  const int32_t* selected;
  const int32_t* counts;
  uint32_t* out;
  int32_t* status;
  int64_t num_pages;
  int32_t batch;
  int32_t table_stride;
  int32_t kv_heads;
  int32_t rep_heads;
  int32_t rep_stride;
  int32_t select_groups;
  int32_t sel_stride;
};
hipError_t launch_read_step_bytes(const ReadStepLaunch& l, hipStream_t stream);

hipError_t launch_gather_pages(const uint16_t* pool, int64_t page_bytes, int64_t num_pages,
                               const int32_t* pages, int32_t count, uint16_t* out,
                               int32_t* status, hipStream_t stream);

// Pool pages to (pinned, device-mapped) host memory, ids checked by the
// caller; one launch per kPagesPerHostCopy pages, ids in the arguments.
constexpr int kPagesPerHostCopy = 256;
hipError_t launch_pages_to_host(const uint16_t* pool, int64_t page_bytes, const int32_t* pages, int32_t count,
                                void* out, hipStream_t stream);
hipError_t launch_fill_synthetic_f16(uint16_t* dst, int64_t count, uint64_t seed,
                                     uint64_t first_index, hipStream_t stream);
hipError_t launch_fill_synthetic_f32(float* dst, int64_t count, uint64_t seed,
                                     uint64_t first_index, hipStream_t stream);
hipError_t launch_consume_checksum(const float* input, int32_t elements, float* checksum,
                                   hipStream_t stream);
hipError_t launch_fill_from_host(uint16_t* pool, int64_t page_bytes, int64_t num_pages, const int32_t* dst_pages,
                                 const uint8_t* src_dev, int64_t src_total, const int64_t* src_blocks, int32_t count,
                                 int32_t* status, hipStream_t stream);
hipError_t launch_xor_bytes(const uint8_t* input, uint8_t* output, uint64_t bytes, uint8_t mask,
                            hipStream_t stream);

}  // namespace sa
