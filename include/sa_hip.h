/*
 * sa_hip.h — C-ABI of the MI355X (gfx950) KV-cache decode hot path.
 *
 * Plain pointers and sizes only.  Device pointers are HIP device memory;
 * `stream` arguments are hipStream_t passed as void* (NULL = the null
 * stream).  Every entry point returns 0 on success or a negative SA_HIP_E*
 * code; sa_hip_last_error() returns the message of the last failure on the
 * calling thread.  Hot entry points allocate nothing: scratch memory comes
 * in through explicit workspace arguments sized by the *_workspace_bytes
 * queries (sa_hip_decode_step_noalloc: a static device array instead).
 * Launches are asynchronous on `stream`.
 *
 * Each entry point names the reference interface it replaces (paths are
 * relative to the reference checkout).  The C++ contract above this layer
 * is include/solidattention/backend.hpp (AcceleratorBackend, kept with the
 * reference's names and meaning) plus include/solidattention/hip_kv.hpp.
 */
#ifndef SA_HIP_H
#define SA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SA_HIP_OK 0
#define SA_HIP_EINVAL (-1)   /* invalid argument / unsupported shape */
#define SA_HIP_ERUNTIME (-2) /* HIP runtime error */
#define SA_HIP_EIO (-3)      /* file I/O error (sa_store.h) */

/* Tokens per page (and per selectable block).  Fixed: the reference's
 * 32-token blocks (selection_main.cpp:97, kv_lifecycle_main.cpp:21). */
#define SA_HIP_PAGE_TOKENS 32

/* Paged KV view.  All arrays are device memory.
 *   pool        [num_pages][32][2][kv_heads][head_dim] FP16 bits: a page is
 *               32 tokens in the reference token format
 *               [K: kv_heads x head_dim][V: kv_heads x head_dim]
 *               (backend.hpp:18-31, attention_reference.cpp:67-69,84-87).
 *   block_table [batch][table_stride] page id of each logical block.
 *   seq_len     [batch] tokens held by each sequence.
 *   sealed      [batch] sealed (selectable) blocks; tokens
 *               [sealed*32, seq_len) form the unsealed tail.
 *   generation  [batch] seal counter (may be NULL).
 *   reps        [batch][rep_heads][head_dim][rep_stride] fp32 block
 *               representatives, head_dim-major so that lanes reading
 *               consecutive blocks are coalesced.  rep_heads is kv_heads
 *               (one representative per KV head, shared by its query heads)
 *               or query_heads (one per query head).
 * head_dim: 128 everywhere; the reference's selection and attention take
 * any head_dim, and so do sa_hip_append_seal(_f16), sa_hip_seal,
 * sa_hip_score_select (given the scores buffer), sa_hip_score_select_split,
 * sa_hip_sparse_decode_attention and sa_hip_decode_step(_f16): at any other
 * multiple of 8 up to 512 they run general kernels (append + seal one
 * workgroup per sequence, the bulk seal spread over blocks and KV heads;
 * scoring one lane per block; attention over the page list in token rows up
 * to 256; the decode step as one launch up to 256 with selection per KV
 * group and representatives per KV head, else those launches in sequence),
 * with the same results (bit-exact selection and state, attention within
 * fp32 rounding).
 * The other entry points (chunked and split-phase attention, the chunked
 * selection, select-attend, the online seal, the allocation-free step)
 * refuse a head_dim other than 128 with SA_HIP_EINVAL. */
typedef struct sa_paged_kv {
  uint16_t* pool;
  int32_t* block_table;
  int32_t* seq_len;
  int32_t* sealed;
  int32_t* generation;
  float* reps;
  int64_t num_pages;
  int32_t batch;
  int32_t table_stride;
  int32_t rep_heads;
  int32_t rep_stride;
  int32_t query_heads;
  int32_t kv_heads;
  int32_t head_dim;
  int32_t reserved;
} sa_paged_kv;

/* Budgeted selection parameters.
 *   select_groups  kv_heads: each KV group (its G query heads) selects its own
 *                  blocks; 1: one block set shared by all query heads (the
 *                  reference's C2 call, selection_main.cpp:178-181).
 *   budget_blocks  blocks per selection (init + local + dynamic); when a
 *                  sequence has no more sealed blocks than this, all are
 *                  selected (the clamp of selection.py:120).
 *   init_blocks    always-selected leading blocks [0, init).
 *   local_blocks   always-selected trailing sealed blocks [n-local, n).
 *   sel_stride     row stride of the selected[] output (>= budget_blocks).
 *   budgets        optional device array [batch] of per-sequence budgets
 *                  (mixed-budget serving); each must lie in
 *                  [init + local, sel_stride], otherwise that sequence selects
 *                  nothing and status bit 16 is set.  NULL: budget_blocks. */
typedef struct sa_select_params {
  int32_t select_groups;
  int32_t budget_blocks;
  int32_t init_blocks;
  int32_t local_blocks;
  int32_t sel_stride;
  int32_t reserved;
  const int32_t* budgets;
} sa_select_params;

/* ---- library ------------------------------------------------------------ */

const char* sa_hip_last_error(void);
int sa_hip_abi_version(void);
/* Number of visible devices (0 when none); does not create a context. */
int sa_hip_device_count(void);

/* ---- R6: sparse GQA decode attention ------------------------------------ */

/* Workspace for sa_hip_sparse_decode_attention with `splits` partial
 * results per (sequence, KV head) (0 when splits == 1).  Launches that share
 * a workspace must not run concurrently. */
size_t sa_hip_attention_workspace_bytes(int32_t batch, int32_t query_heads,
                                        int32_t kv_heads, int32_t head_dim,
                                        int32_t splits);

/* Split count the library picks for a launch (>= 1): workgroups per
 * (sequence, KV head) until every CU holds as many as can be resident for
 * this many query heads per KV head (two for 1-2, one for 4 and 8), keeping
 * at least ~4 pages per wave.  No counterpart in the reference (its
 * attention is one CPU loop per head); the split is this library's launch
 * shape. */
int32_t sa_hip_attention_splits_for(int32_t batch, int32_t query_heads, int32_t kv_heads,
                                    int32_t pages_per_group_hint);

/* sa_hip_attention_splits_for with 2 query heads per KV head. */
int32_t sa_hip_attention_default_splits(int32_t batch, int32_t kv_heads,
                                        int32_t pages_per_group_hint);

/* out[b][h][:] = softmax(scale * q[b][h] . K) V over the tokens of the
 * selected sealed blocks of h's KV group followed by every tail token of
 * sequence b; fp32 stable softmax (online, split over `splits` partial
 * results merged with log-sum-exp).  selected: [batch][select_groups]
 * [sel_stride] logical block ids; counts: [batch][select_groups].
 * query, out: [batch][query_heads][head_dim] fp32.  status (optional,
 * device int32) receives SA status bits for invalid pages/blocks.
 * Replaces the device side of AcceleratorBackend::attention*
 * (backend.hpp:50-57; cuda_backend.cpp:109-158, 323-415) and the
 * tail-inclusive sparse_fp16_attention (qwen_layer_main.cpp:224-268);
 * semantics of attention_reference (attention_reference.cpp:55-96). */
int sa_hip_sparse_decode_attention(const sa_paged_kv* kv, const float* query,
                                   const int32_t* selected,
                                   const int32_t* counts,
                                   int32_t select_groups, int32_t sel_stride,
                                   float scale, float* out, void* workspace,
                                   size_t workspace_bytes, int32_t splits,
                                   int32_t* status, void* stream);

/* The same attention for lists of very different lengths (mixed contexts
 * and per-sequence budgets): each (sequence, KV head) page list is cut into
 * chunks of chunk_pages pages, one workgroup each; workgroups past a short
 * list's end contribute nothing and the last chunk takes any remainder
 * beyond max_chunks * chunk_pages.  The partial records (max_chunks per
 * (sequence, KV head), workspace as sa_hip_attention_workspace_bytes(...,
 * max_chunks)) are merged with log-sum-exp.  Same result as
 * sa_hip_sparse_decode_attention within fp32 rounding.  With a workspace of
 * sa_hip_attention_chunked_workspace_bytes (batch x kv_heads <= 4096) the
 * workgroups first run longest list first (below). */
int sa_hip_sparse_decode_attention_chunked(
    const sa_paged_kv* kv, const float* query, const int32_t* selected,
    const int32_t* counts, int32_t select_groups, int32_t sel_stride,
    float scale, float* out, void* workspace, size_t workspace_bytes,
    int32_t chunk_pages, int32_t max_chunks, int32_t* status, void* stream);
/* Workspace that also holds the chunk schedule: with at least this many
 * bytes (and batch x kv_heads <= 4096), sa_hip_sparse_decode_attention_chunked
 * first orders its workgroups by list length, longest first with each list's
 * chunks consecutive (one extra single-workgroup launch), so that short lists
 * fill the end of the launch; the results equal those of the grid order.  No
 * reference counterpart: a scheduling aid for mixed-length batches. */
size_t sa_hip_attention_chunked_workspace_bytes(int32_t batch, int32_t query_heads, int32_t kv_heads,
                                                int32_t head_dim, int32_t max_chunks);

/* Split-phase attention, for schedules that attend the blocks already
 * resident while missing blocks are still being copied in (the overlap the
 * reference gets from its copy stream, pipeline_main.cpp:811-848).  Each
 * call attends its own id list (plus the tail when include_tail) with
 * `splits` workgroups per (sequence, KV head) and writes their partial
 * records to [split_base, split_base + splits) of a workspace sized by
 * sa_hip_attention_workspace_bytes(..., total_splits) (total_splits >= 2);
 * once calls have written all total_splits records, sa_hip_attention_merge
 * forms `out` exactly as a single call over the union would (within fp32
 * rounding).  The tail must be included by exactly one call. */
int sa_hip_sparse_decode_attention_partial(
    const sa_paged_kv* kv, const float* query, const int32_t* selected,
    const int32_t* counts, int32_t select_groups, int32_t sel_stride,
    float scale, int32_t include_tail, void* workspace,
    size_t workspace_bytes, int32_t split_base, int32_t splits,
    int32_t total_splits, int32_t* status, void* stream);
int sa_hip_attention_merge(const sa_paged_kv* kv, const void* workspace,
                           size_t workspace_bytes, int32_t total_splits,
                           float* out, void* stream);

/* Attention over a contiguous token-major K/V-interleaved buffer of
 * `tokens` tokens (the AttentionProblem layout, backend.hpp:18-31); the
 * device kernel of AcceleratorBackend::attention (cuda_backend.cpp:70-158)
 * without its 128/256-token limits.  head_dim: 128 (the paged attention
 * kernel) or any other multiple of 8 up to 512 (attention_reference.cpp
 * :55-96 takes any head_dim), with 1, 2, 4 or 8 query heads per KV head;
 * the workspace size depends on head_dim. */
size_t sa_hip_contiguous_workspace_bytes(int64_t tokens, int32_t query_heads,
                                         int32_t kv_heads, int32_t head_dim);
int sa_hip_attention_contiguous(const uint16_t* kv, const float* query,
                                int64_t tokens, int32_t query_heads,
                                int32_t kv_heads, int32_t head_dim,
                                float scale, float* out, void* workspace,
                                size_t workspace_bytes, void* stream);

/* Weighted checksum of an output vector, out[0] = sum_i x[i] * (1 + (i%17) *
 * 0.001); the C1.4 device consumer (cuda_backend.cpp:160-168). */
int sa_hip_consume_checksum(const float* input, int32_t elements,
                            float* checksum, void* stream);

/* ---- R3: scoring + budgeted top-k selection ----------------------------- */

/* Per (sequence, selection group): score[b] = sum over the group's query
 * heads h, in head order, of (sequential fp32 dot(q_h, rep_b) / heads) with
 * no fused multiply-add, then init/local/dynamic selection with ties broken
 * towards the lower block id; ids ascending.  Bit-exact with
 * select_shared_blocks (selection.hpp:24-29, selection.cpp:96-147) applied
 * to the group.  scores (optional): [batch][select_groups][rep_stride].
 * Limit: sealed[b] <= 8192 blocks. */
int sa_hip_score_select(const sa_paged_kv* kv, const float* query,
                        const sa_select_params* params, int32_t* selected,
                        int32_t* counts, float* scores, int32_t* status,
                        void* stream);

/* The same selection with the scoring spread over workgroups of 256 blocks
 * each (two launches: scores, then selection from them), for batches with
 * few (sequence, group) lists or long ones, where one workgroup per list
 * leaves the device idle.  scores is required ([batch][select_groups]
 * [rep_stride] fp32, the same values sa_hip_score_select writes); ids,
 * counts and scores are bit-identical to sa_hip_score_select's. */
int sa_hip_score_select_split(const sa_paged_kv* kv, const float* query,
                              const sa_select_params* params, int32_t* selected,
                              int32_t* counts, float* scores, int32_t* status,
                              void* stream);

/* The same selection as one launch that spreads long lists over the device:
 * a workgroup scores at most 1024 consecutive blocks of a (sequence, group)
 * list (2048 once the lists outnumber the compute units); a list of one
 * such chunk selects on the spot, the chunks of a longer
 * list hand their keys to the last of them to finish, which selects.  For
 * batches of mixed lengths, where one workgroup per list leaves the compute
 * units that drew short lists idle while others walk long ones.  A budget
 * that takes every block skips the scoring.  workspace: at least
 * sa_hip_score_select_chunked_workspace_bytes(kv, params) bytes, zeroed
 * once when allocated; every call leaves its arrival counters at zero, and
 * calls that share a workspace must not run concurrently.  Needs 16-byte
 * aligned representatives and rep_stride % 4 == 0.  ids and counts are bit-
 * identical to sa_hip_score_select's (selection.cpp:96-147 per group). */
size_t sa_hip_score_select_chunked_workspace_bytes(const sa_paged_kv* kv,
                                                   const sa_select_params* params);
int sa_hip_score_select_chunked(const sa_paged_kv* kv, const float* query,
                                const sa_select_params* params, int32_t* selected,
                                int32_t* counts, void* workspace, size_t workspace_bytes,
                                int32_t* status, void* stream);

/* 1 when sa_hip_score_select_split is expected to be the faster form for
 * this geometry (fewer (sequence, group) lists than compute units), else 0. */
int sa_hip_score_select_split_preferred(const sa_paged_kv* kv,
                                        const sa_select_params* params);

/* ---- R3 + R6 fused: one layer's select-then-attend ----------------------- */

/* sa_hip_score_select(kv, query, params, selected, counts, NULL, status)
 * followed by sa_hip_sparse_decode_attention(kv, query, selected, counts,
 * params->select_groups, params->sel_stride, scale, out, workspace,
 * workspace_bytes, splits, status): the same selected ids and counts (bit-
 * exact) and the same attention output (within fp32 rounding).  When
 * sa_hip_select_attend_fused() is 1 it runs as ONE launch, one workgroup per
 * (sequence, KV head) that scores, selects, keeps the ids on chip and
 * attends; otherwise as the two launches.  Fused: splits == 1 and either
 * select_groups == kv_heads with 1, 2 or 4 query heads per KV head (4: also
 * sel_stride <= 2048 and an even rep_stride with 8-byte aligned
 * representatives), or the shared selection (select_groups 1) with 1, 2 or
 * 4 query heads per KV head, representatives per KV head, rep_stride <= 128
 * and batch x kv_heads x (kv_heads - 1) x rep_stride x 512 bytes <= 32 MiB
 * (every workgroup of a sequence scores the whole shared set, so the
 * representatives are read once per KV head).  At a head_dim other than 128
 * it answers for sa_hip_decode_step only (select_attend refuses that
 * head_dim): one launch up to 256 with select_groups == kv_heads, 1, 2 or 4
 * query heads per KV head and representatives per KV head.  splits >= 1;
 * workspace as for
 * sa_hip_sparse_decode_attention.  Replaces the reference's per-layer
 * select -> pack -> attention sequence (selection_main.cpp:178-230;
 * pipeline_main.cpp:803-876) with selection on the GPU. */
int sa_hip_select_attend_fused(const sa_paged_kv* kv,
                               const sa_select_params* params, int32_t splits);
/* The split count to pass to sa_hip_select_attend / sa_hip_decode_step: 1
 * (the fused launch) when the fused kernel applies and its workgroups fill
 * the device (batch x kv_heads >= 2 x CUs), or for the shared selection's
 * one launch whenever it applies; at a head_dim other than 128, 1 where the
 * one-launch step applies and fills the device, else splits that give about
 * four attention workgroups per CU with at least 4 pages per wave;
 * otherwise
 * sa_hip_attention_splits_for(batch, query_heads, kv_heads, budget_blocks + 2) for the
 * separate launches. */
int32_t sa_hip_select_attend_default_splits(const sa_paged_kv* kv,
                                            const sa_select_params* params);
int sa_hip_select_attend(const sa_paged_kv* kv, const float* query,
                         const sa_select_params* params, float scale,
                         int32_t* selected, int32_t* counts, float* out,
                         void* workspace, size_t workspace_bytes,
                         int32_t splits, int32_t* status, void* stream);

/* ---- R8/R9/R4 + R3 + R6 fused: one layer's whole decode step ------------- */

/* Workspace of sa_hip_decode_step: `batch` int32 arrival counters (padded
 * to 256 bytes) followed by the attention's split records (padded to 256
 * bytes) and the split selection's scores (batch x query_heads x rep_stride
 * floats; used when the step runs as separate launches with few lists, and
 * at every head_dim other than 128).  The caller
 * zeroes it ONCE before the first call; every call leaves the counters at
 * zero again.  Calls sharing a workspace must not run concurrently. */
size_t sa_hip_decode_step_workspace_bytes(const sa_paged_kv* kv,
                                          int32_t splits);

/* sa_hip_append_seal(kv, k, v, local_tokens) followed by
 * sa_hip_select_attend(kv, query, params, scale, selected, counts, out, ...):
 * the same page bytes, representatives, seq_len/sealed/generation, selected
 * ids (bit-exact) and attention output (within fp32 rounding).  When
 * sa_hip_select_attend_fused() is 1 it is ONE launch: each (sequence, KV
 * head) workgroup appends and seals its own head (with the shared selection:
 * seals every KV head's representative, identical values in every
 * workgroup), then scores, selects and attends; the last workgroup of a
 * sequence to arrive writes its counters.  The online seal (the _online
 * variant) runs as one launch only with select_groups == kv_heads.
 * Otherwise it runs the three launches.  The _f16 variant takes raw FP16
 * K/V bits like sa_hip_append_seal_f16.  Replaces the reference's per-layer
 * decode sequence of append_fp16_kv (qwen_layer_main.cpp:270-281 via
 * qwen_chain_main.cpp:390-391), the tail seal (kv_lifecycle_main.cpp:92-113),
 * select_shared_blocks and the sparse attention (qwen_chain_main.cpp:393-395). */
int sa_hip_decode_step(const sa_paged_kv* kv, const float* k, const float* v,
                       int32_t local_tokens, const float* query,
                       const sa_select_params* params, float scale,
                       int32_t* selected, int32_t* counts, float* out,
                       void* workspace, size_t workspace_bytes,
                       int32_t splits, int32_t* status, void* stream);
int sa_hip_decode_step_f16(const sa_paged_kv* kv, const uint16_t* k,
                           const uint16_t* v, int32_t local_tokens,
                           const float* query, const sa_select_params* params,
                           float scale, int32_t* selected, int32_t* counts,
                           float* out, void* workspace,
                           size_t workspace_bytes, int32_t splits,
                           int32_t* status, void* stream);

/* ---- R4/R9 InfLLM online seal -------------------------------------------- */

/* The InfLLM online seal of the reference's P1.3c.4 (online_seal_main.cpp
 * :41-44): when a decode step seals a 32-token block, the representative of
 * each query head h is build_local_causal_representatives (selection.hpp
 * :19-22, selection.cpp:12-94) applied to that block alone: its 32 keys (KV
 * head h / G), the 32 decode queries of head h issued with those tokens,
 * block_tokens 32, local_window and topk (the reference: 32 and 4); the
 * reference's arithmetic bit for bit (its std::exp restated, see
 * sa_hip_local_causal_representatives).  Representatives are per query head:
 * kv->rep_heads must equal kv->query_heads.
 *   query_ring   [batch][query_heads][ring_tokens][head_dim] fp32 device
 *                memory: the decode query issued with the token at position
 *                p is kept at slot p % ring_tokens, written by the call that
 *                appends the token.  A caller that starts decoding after a
 *                prefill copies the prefill queries of the unsealed tail
 *                positions into their slots first.
 *   ring_tokens  >= local_tokens + 32 (the whole tail). */
typedef struct sa_online_seal {
  float* query_ring;
  int32_t ring_tokens;
  int32_t local_window;
  int32_t topk;
  int32_t reserved;
} sa_online_seal;

/* sa_hip_append_seal (fp32 K/V) that also keeps the step's queries
 * ([batch][query_heads][head_dim]) in the ring and seals with the online
 * representative instead of the mean key. */
int sa_hip_append_seal_online(const sa_paged_kv* kv, const float* k,
                              const float* v, int32_t local_tokens,
                              const float* query, const sa_online_seal* seal,
                              int32_t* status, void* stream);

/* sa_hip_decode_step (fp32 K/V) with the online seal: one launch where
 * sa_hip_select_attend_fused() is 1, else sa_hip_append_seal_online, the
 * selection and the attention.  Same workspace as sa_hip_decode_step. */
int sa_hip_decode_step_online(const sa_paged_kv* kv, const float* k,
                              const float* v, int32_t local_tokens,
                              const float* query, const sa_online_seal* seal,
                              const sa_select_params* params, float scale,
                              int32_t* selected, int32_t* counts, float* out,
                              void* workspace, size_t workspace_bytes,
                              int32_t splits, int32_t* status, void* stream);

/* Static scratch of sa_hip_decode_step_noalloc, per GPU: the first
 * SA_HIP_NOALLOC_COUNTER_BYTES hold the arrival counters (one per sequence,
 * any batch up to 65535), the rest the attention's split records. */
#define SA_HIP_NOALLOC_SCRATCH_BYTES (4u << 20)
#define SA_HIP_NOALLOC_COUNTER_BYTES (256u << 10)

/* sa_hip_decode_step (fp32 k/v) without a workspace argument, allocating
 * nothing: no hipMalloc, hipFree or allocating library call on any call.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Its scratch is a static device array of
 * SA_HIP_NOALLOC_SCRATCH_BYTES on each GPU the library runs on, held until
 * the process ends; its device address is looked up on the first call on a
 * device.  The arrival counters are cleared by a small kernel on `stream`
 * before every fused launch.  Limit: launches whose split records
 * (sa_hip_attention_workspace_bytes(batch, query_heads, kv_heads, head_dim,
 * splits)) exceed SA_HIP_NOALLOC_SCRATCH_BYTES - SA_HIP_NOALLOC_COUNTER_BYTES
 * are refused with SA_HIP_EINVAL (the fused launch, splits == 1, needs no
 * records); the split selection keeps its scores after the records only
 * where the array holds them (else the one-workgroup-per-list selection:
 * the same ids).
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (unordered streams, or host threads) race and give wrong results; order
 * them on one stream.  Results equal sa_hip_decode_step's.
 * Graph capture: the first call on each device looks the array's address up
 * (hipGetSymbolAddress) and must run outside capture; a first call on a
 * capturing stream returns SA_HIP_EINVAL.  Later calls may be captured.  The
 * address is kept until the process ends: resetting the device
 * (hipDeviceReset) after a call is not supported. */
int sa_hip_decode_step_noalloc(const sa_paged_kv* kv, const float* k,
                               const float* v, int32_t local_tokens,
                               const float* query,
                               const sa_select_params* params, float scale,
                               int32_t* selected, int32_t* counts, float* out,
                               int32_t splits, int32_t* status, void* stream);

/* ---- R8/R9/R4: decode append, seal, representative ---------------------- */

/* Append one token per sequence at position seq_len[b] (fp32 K/V converted
 * round-to-nearest-even, or raw FP16 bits for the _f16 variant), advance
 * seq_len, then seal while the tail holds >= local_tokens + 32 tokens: the
 * oldest tail block becomes selectable, its mean-key representative
 * (sum of its 32 keys in token order / 32, per KV head) is written to reps
 * and sealed/generation advance.  k, v: [batch][kv_heads][head_dim].
 * Replaces append_fp16_kv (qwen_layer_main.cpp:270-281) and the tail seal
 * of kv_lifecycle_main.cpp:31-45, 92-113 (bit-exact bytes and
 * representatives). */
int sa_hip_append_seal(const sa_paged_kv* kv, const float* k, const float* v,
                       int32_t local_tokens, int32_t* status, void* stream);
int sa_hip_append_seal_f16(const sa_paged_kv* kv, const uint16_t* k,
                           const uint16_t* v, int32_t local_tokens,
                           int32_t* status, void* stream);
/* Seal only (e.g. after a prefill wrote whole pages and set seq_len). */
int sa_hip_seal(const sa_paged_kv* kv, int32_t local_tokens, int32_t* status,
                void* stream);

/* ---- R4 (InfLLM, prefill): local-causal block representatives ------------ */

/* Workspace for sa_hip_local_causal_representatives: the window
 * probabilities and the received mass, tokens x query_heads x
 * (min(local_window, tokens) + 1) floats (0 when that overflows). */
size_t sa_hip_local_causal_workspace_bytes(int64_t tokens, int32_t query_heads,
                                           int32_t local_window);

/* The reference's build_local_causal_representatives (selection.hpp:19-22,
 * selection.cpp:12-94) on the GPU: every query position attends its local
 * causal window of `local_window` keys (fp32 softmax over sequential fp32
 * dots, scale 1/sqrt(head_dim)); each key's received mass is summed over the
 * queries in order; per block of block_tokens tokens the `topk` keys with
 * the most mass (stable: ties keep token order) are averaged in rank order.
 *   prompt_queries  [query_heads][tokens][head_dim] fp32 (device)
 *   kv              [tokens][2][kv_heads][head_dim] FP16 bits (device, the
 *                   reference's interleaved token format)
 * Outputs (device, each optional, at least one given): values
 * [query_heads][blocks][head_dim] (the reference's layout), offsets
 * [query_heads][blocks][topk] int32 (the reference's chosen_token_offsets),
 * reps [query_heads][head_dim][rep_stride] (one sequence's slice of
 * sa_paged_kv.reps with rep_heads = query_heads), received
 * [query_heads][tokens].  The exponential restates glibc's expf (the
 * reference's std::exp(float)): the same table, polynomial and fused
 * multiply-adds in double, equal to it on every float, so the chosen tokens,
 * representatives and received masses are the reference's bit for bit.
 * Any head_dim, block_tokens and local_window, as in the reference: head_dim
 * 128 with 32-token blocks and windows up to 256 run tiled kernels (LDS-
 * staged queries and keys, several keys per lane), other shapes a wave per
 * query and a wave per block; the results are the same bits either way.
 * Limits: topk <= 16384, tokens x query_heads <= 2^31, kv_heads <= 65536;
 * prompt_queries and kv 16-byte aligned. */
int sa_hip_local_causal_representatives(
    const float* prompt_queries, const uint16_t* kv, int64_t tokens,
    int32_t query_heads, int32_t kv_heads, int32_t head_dim,
    int32_t block_tokens, int32_t local_window, int32_t topk, float* values,
    int32_t* offsets, float* reps, int32_t rep_stride, float* received,
    void* workspace, size_t workspace_bytes, void* stream);

/* ---- R5: gather / pack --------------------------------------------------- */

/* out + i * page_bytes <- pool + pages[i] * page_bytes for i < count (device
 * arrays), the placement of UringReader::read_blocks_fixed
 * (uring_reader.cpp:87-95) for pool-resident blocks.  page_bytes must be a
 * multiple of 16; pages outside [0, num_pages) are skipped and flagged in
 * status (optional). */
int sa_hip_gather_pages(const uint16_t* pool, int64_t page_bytes,
                        int64_t num_pages, const int32_t* pages,
                        int32_t count, uint16_t* out, int32_t* status,
                        void* stream);

/* ---- measurement: the decode step's bytes, read with no arithmetic ------ */

/* No counterpart in the reference: a measurement aid for the attention
 * kernels.  For every (sequence b, KV head h) it reads exactly the bytes a
 * decode step reads for that pair: the fp32 representative rows of the
 * sealed blocks (rep heads h, h + kv_heads, ...), the K/V slices of head h in
 * the pages of list b * select_groups + h / (kv_heads / select_groups) of
 * `selected` (first counts[...] entries, at most sel_stride), and the K/V of
 * the unsealed tail [32 * sealed, seq_len).  out[b * kv_heads + h] is the XOR
 * of every 32-bit word read (device, batch * kv_heads).  Needs 16-byte
 * aligned reps with rep_stride a multiple of 4; ids outside the sealed range
 * and pages outside [0, num_pages) are skipped and flagged in status
 * (optional). */
int sa_hip_read_step_bytes(const sa_paged_kv* kv, const int32_t* selected,
                           const int32_t* counts, int32_t select_groups,
                           int32_t sel_stride, uint32_t* out, int32_t* status,
                           void* stream);

/* ---- R10: history prediction and miss correction ------------------------ */

/* Host-only set logic of compare_prediction (pipeline_main.cpp:686-717):
 * hits, misses (oracle blocks absent from the prediction, oracle order) and
 * replacement slots (prediction slots whose block left, slot order).
 * Returns SA_HIP_EINVAL on a cardinality mismatch. */
int sa_hip_compare_prediction(const int32_t* predicted, const int32_t* oracle,
                              int32_t n, int32_t* hits, int32_t* misses,
                              int32_t* replacement_slots, int32_t* miss_count);

/* Seal writeback staging: on copy_stream, after after_event (a hipEvent_t
 * recorded on the compute stream behind the step that sealed the pages;
 * NULL: no wait), hipMemcpyAsync of pool pages pages[0..count) (host array,
 * each in [0, num_pages)) into dst + i * page_bytes (pinned host memory),
 * then record done_event (optional).  The store write of the staged pages
 * (sa_store_submit_writes) starts once done_event has completed; the
 * reference copies the sealed block out of its host tail before its
 * O_DIRECT pwrite (kv_lifecycle_main.cpp:104-108).  When dst is pinned
 * host memory the device maps (hipHostMalloc), one kernel per 256 pages
 * writes it through the mapping (dst must then hold count * page_bytes
 * bytes); other memory gets one hipMemcpyAsync per page. */
int sa_hip_pages_to_host_async(const uint16_t* pool, int64_t page_bytes,
                               int64_t num_pages, const int32_t* pages,
                               int32_t count, void* dst, void* copy_stream,
                               void* after_event, void* done_event);

/* Copy-stream slot fills: for i < count, hipMemcpyAsync of page_bytes from
 * pinned host memory src_base + src_blocks[i] * page_bytes into pool page
 * dst_pages[i] on copy_stream, then record done_event (hipEvent_t) on it.
 * dst_pages and src_blocks are host arrays.  The compute stream orders
 * itself after the fills with sa_hip_stream_wait_event instead of a host
 * barrier.  Replaces CudaPipeline::correct_and_wait
 * (pipeline_main.cpp:305-331). */
int sa_hip_fill_pages_async(uint16_t* pool, int64_t page_bytes,
                            const int32_t* dst_pages,
                            const void* src_base, const int64_t* src_blocks,
                            int32_t count, void* copy_stream,
                            void* done_event);
/* The same fills as one kernel on copy_stream that reads the pinned host
 * memory (src_base must come from hipHostMalloc / pinned allocation, holding
 * src_blocks_total pages) through its device mapping; dst_pages_dev and
 * src_blocks_dev are device arrays.  Entries outside [0, num_pages) or
 * [0, src_blocks_total) are skipped and flagged in status. */
int sa_hip_fill_pages_gather_async(uint16_t* pool, int64_t page_bytes,
                                   int64_t num_pages,
                                   const int32_t* dst_pages_dev,
                                   const void* src_base,
                                   int64_t src_blocks_total,
                                   const int64_t* src_blocks_dev,
                                   int32_t count, int32_t* status,
                                   void* copy_stream, void* done_event);
int sa_hip_stream_wait_event(void* stream, void* event);

/* ---- query producer / output consumer around the attention -------------- */
/* The reference computes these per decode token with its own kernels and
 * cuBLAS (qwen_layer_main.cpp:125-172 rms_norm, head_rms, rope; :576-584 and
 * :640-645 the projections and the residual add; qwen_chain_main.cpp
 * :365-399 the decode step).  Here they run for a batch of rows (one per
 * sequence), fp32 throughout. */

/* out = x * (1 / sqrt(mean(x^2) + eps)) * w per row; width % 4 == 0. */
int sa_hip_rms_norm(const float* x, const float* w, float* out, int32_t rows, int32_t width, float eps,
                    void* stream);
/* y[r][o] = sum_i x[r][i] * w[o][i] (+ residual[r][o] when non-null): the
 * reference's cublasSgemm(CUBLAS_OP_T) on its row-major [out][in] weights,
 * two launches on `stream` (K-slice partial tiles, then their sum in slice
 * order: deterministic).  in a multiple of 256, out of 64; x, w, residual, y
 * and the workspace 16-byte aligned; workspace of
 * sa_hip_linear_workspace_bytes(rows, in, out) bytes holding the partial
 * tiles (no initialisation needed).  Calls sharing a workspace must not run
 * concurrently. */
size_t sa_hip_linear_workspace_bytes(int32_t rows, int32_t in, int32_t out);
int sa_hip_linear(const float* x, const float* w, const float* residual, float* y, int32_t rows, int32_t in,
                  int32_t out, void* workspace, size_t workspace_bytes, void* stream);
/* The query producer of one layer for a batch of decode tokens, two launches:
 * from the normalised hidden x [rows][hidden], q = head_rms(x wq^T) then
 * RoPE, k = head_rms(x wk^T) then RoPE, v = x wv^T, with head_dim 128, the
 * rotation at positions[rows] (device int32), frequencies theta^(-2i/128)
 * correctly rounded to fp32 and the reference's NeoX pairing (d, d + 64).
 * Outputs [rows][heads][128] fp32, ready for sa_hip_decode_step (q) and its
 * k/v.  hidden % 256 == 0; x, the weights, the norms, q/k/v and the
 * workspace 16-byte aligned; workspace of sa_hip_qkv_workspace_bytes bytes
 * (the K-slice partial tiles; no initialisation needed). */
size_t sa_hip_qkv_workspace_bytes(int32_t rows, int32_t hidden, int32_t q_heads, int32_t kv_heads);
int sa_hip_qkv_project(const float* x, const float* wq, const float* wk, const float* wv, const float* q_norm,
                       const float* k_norm, const int32_t* positions, int32_t rows, int32_t hidden,
                       int32_t q_heads, int32_t kv_heads, float theta, float eps, float* q, float* k, float* v,
                       void* workspace, size_t workspace_bytes, void* stream);
/* sa_hip_rms_norm(hidden_rows, input_norm, input_eps) followed by
 * sa_hip_qkv_project, in the same two launches: the RMS scale of each row is applied to
 * its projected sums (x * w_norm is projected, then scaled by
 * 1 / sqrt(mean(x^2) + eps)), equal to the two calls within fp32 rounding.
 * Replaces the reference's rms_norm + q/k/v projections
 * (qwen_layer_main.cpp:125-145, :576-584). */
int sa_hip_qkv_project_rms(const float* hidden_rows, const float* input_norm, float input_eps, const float* wq,
                           const float* wk, const float* wv, const float* q_norm, const float* k_norm,
                           const int32_t* positions, int32_t rows, int32_t hidden, int32_t q_heads,
                           int32_t kv_heads, float theta, float eps, float* q, float* k, float* v, void* workspace,
                           size_t workspace_bytes, void* stream);

/* The arguments of sa_hip_qkv_project_rms (input_norm NULL:
 * sa_hip_qkv_project's) for a decode step's batch: rows = kv->batch,
 * q_heads = kv->query_heads, kv_heads = kv->kv_heads. */
typedef struct sa_qkv_producer {
  const float* hidden_rows; /* [batch][hidden] */
  const float* input_norm;  /* [hidden] or NULL */
  float input_eps;
  const float* wq;
  const float* wk;
  const float* wv;
  const float* q_norm;
  const float* k_norm;
  const int32_t* positions; /* [batch] device int32 (may be kv->seq_len) */
  int32_t hidden;
  float theta;
  float eps;
  float* q; /* [batch][query_heads][128]: written */
  float* k; /* [batch][kv_heads][128]: written */
  float* v;
  void* workspace; /* sa_hip_qkv_workspace_bytes(batch, hidden, query_heads, kv_heads) */
  size_t workspace_bytes;
} sa_qkv_producer;

/* The decode step fed by its q/k/v producer: sa_hip_qkv_project_rms (or
 * sa_hip_qkv_project) with producer's arguments, then
 * sa_hip_decode_step(kv, producer->k, producer->v, local_tokens,
 * producer->q, ...).  The same q/k/v bits, page bytes, representatives,
 * counters and selected ids, and the same attention output bits.  Where the
 * step's one launch applies (sa_hip_select_attend_fused() is 1) with 1 or 2
 * query heads per KV head and select_groups == kv_heads, it is TWO launches:
 * the producer's K-slice partials, then the step, whose workgroups run the
 * producer's epilogue (slice sums, RMSNorm scale, head RMS norm, RoPE) for
 * their own heads at entry; otherwise the two calls.  head_dim 128 only; the
 * positions are read before the step advances seq_len, so they may be
 * kv->seq_len.  Replaces the reference layer's rms -> Q/K/V projections ->
 * head_norm -> apply_rope -> pack_kv -> sparse_attention sequence
 * (qwen_chain_main.cpp:365-395) with the paged step. */
int sa_hip_decode_step_qkv(const sa_paged_kv* kv, const sa_qkv_producer* producer, int32_t local_tokens,
                           const sa_select_params* params, float scale, int32_t* selected, int32_t* counts,
                           float* out, void* workspace, size_t workspace_bytes, int32_t splits, int32_t* status,
                           void* stream);

/* ---- synthetic data ------------------------------------------------------ */

/* dst[i] = fp16_rne(normal(seed, first_index + i)), the generator of the
 * CPU oracle (bit-identical). */
int sa_hip_fill_synthetic_f16(uint16_t* dst, int64_t count, uint64_t seed,
                              uint64_t first_index, void* stream);
int sa_hip_fill_synthetic_f32(float* dst, int64_t count, uint64_t seed,
                              uint64_t first_index, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SA_HIP_H */
