/*
 * sa_oracle.h — CPU oracle for the KV-cache decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker: a plain-C restatement of
 * the reference's CPU path (C1 attention, C2 representative scoring and
 * budgeted selection, the decode-tail lifecycle and the history-correction
 * bookkeeping).  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.  The product library never links it and never
 * falls back to it.
 *
 * Every function cites the reference file:line it follows (paths relative to
 * the reference checkout).  Floating-point code is compiled with
 * -ffp-contract=off and no fast-math so that fp32 operations happen in the
 * same order and with the same rounding as the reference objects built by
 * g++ (which contain no FMA).
 *
 * Pinning: each function is checked in tests/ against the reference's
 * published golden values, against the reference sources compiled into
 * oracle/_ref/ (differential, many seeds) and against closed forms.  The
 * functions and their pins are listed in the table at the end of this file.
 */
#ifndef SA_ORACLE_H
#define SA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: 0 ok, negative = invalid arguments (the reference throws). */
#define SAO_OK 0
#define SAO_EINVAL (-1)

/* ---- FP16 codec -------------------------------------------------------- */

/* Fixture encoder of the reference: ties round away from zero and the
 * mantissa carry is OR-ed into the exponent field.
 * Follows cpp/src/attention_reference.cpp:11-28. */
uint16_t sao_float_to_half(float value);

/* Exact FP16 -> fp32 decode.  Follows cpp/src/attention_reference.cpp:30-53. */
float sao_half_to_float(uint16_t value);

/* IEEE round-to-nearest-even fp32 -> FP16, the conversion the reference's
 * decode-token append performs on the device (cvt.rn.f16.f32,
 * cpp/src/qwen_layer_main.cpp:277-278) and audits with a host _Float16 cast
 * (cpp/src/qwen_chain_main.cpp:474-481). */
uint16_t sao_float_to_half_rne(float value);

/* ---- C1: GQA attention over token-major K/V-interleaved FP16 ----------- */

/* out[Hq*D] = softmax(scale * q_h . K_g) V_g, two-pass stable softmax in fp32.
 * kv layout: token t = [K: Hkv x D][V: Hkv x D].
 * Follows cpp/src/attention_reference.cpp:55-96. */
int sao_attention_reference(const uint16_t* kv, const float* query,
                            size_t tokens, size_t query_heads, size_t kv_heads,
                            size_t head_dim, float scale, float* out);

/* ---- C2: representatives and selection --------------------------------- */

/* InfLLM local-causal representatives: received attention mass inside a
 * causal local window, per-block stable top-k by mass, mean of the chosen
 * keys.  values: [Hq][blocks][D]; offsets: [Hq][blocks][topk].
 * Follows cpp/src/selection.cpp:12-94. */
int sao_build_local_causal_representatives(
    const float* prompt_queries, const uint16_t* kv, size_t tokens,
    size_t query_heads, size_t kv_heads, size_t head_dim, size_t block_tokens,
    size_t local_window, size_t topk, float* values, size_t* offsets);

/* Mean-key representative of every block, [Hkv][blocks][D]:
 * (sum over the block's tokens in natural order of the exact key) / tokens.
 * Equal to sao_build_local_causal_representatives(window=1,
 * topk=block_tokens) for every query head of the group (all received masses
 * are exactly 1, so the stable order is the natural order). */
/* The same builder with sao_expf_glibc in place of libm's expf (the GPU
 * builder's arithmetic, bit for bit); received (optional): [Hq][tokens]
 * attention mass each key received. */
int sao_build_local_causal_representatives_restated(
    const float* prompt_queries, const uint16_t* kv, size_t tokens,
    size_t query_heads, size_t kv_heads, size_t head_dim, size_t block_tokens,
    size_t local_window, size_t topk, float* values, size_t* offsets,
    float* received);

/* glibc 2.35's expf restated (32-entry 2^(i/32) table, degree-3 polynomial
 * in double, the fused multiply-adds of its x86-64 FMA build); the GPU
 * builder runs the same operations.  _table copies the 32 table entries;
 * _mismatches counts the floats with bit patterns first, first + stride, ...
 * <= last where it differs from libm's expf. */
float sao_expf_glibc(float x);
void sao_expf_glibc_table(uint64_t* out);
long long sao_expf_glibc_mismatches(uint32_t first_bits, uint32_t last_bits, uint32_t stride);

int sao_mean_key_representatives(const uint16_t* kv, size_t tokens,
                                 size_t kv_heads, size_t head_dim,
                                 size_t block_tokens, float* values);

/* Head-mean block score and init/local/dynamic budgeted selection.
 * ids receives the chosen block ids ascending (count = budget);
 * scores (optional, may be NULL) receives the mean head scores [blocks].
 * Follows cpp/src/selection.cpp:96-147. */
int sao_select_shared_blocks(const float* query, const float* representatives,
                             size_t query_heads, size_t blocks,
                             size_t head_dim, size_t budget_blocks,
                             size_t init_blocks, size_t local_blocks,
                             size_t* ids, size_t* count, float* scores);

/* ---- Batched paged decode (the MI355X path's own contract) ------------- */

/* Paged KV pool: page p holds page_tokens tokens in the reference token
 * format, i.e. page p starts at pool + p * page_tokens * 2 * Hkv * D.
 * block_table[seq * table_stride + logical_block] = page id.
 * Representatives are stored d-major per sequence:
 *   reps[((seq * rep_heads + rh) * D + d) * rep_stride + block]
 * with rep_heads == Hkv (one per KV head, shared by its query heads) or
 * rep_heads == Hq (one per query head).
 *
 * Scoring + selection for one decode step.  Selection groups:
 * select_groups == Hkv (each KV group selects for itself: the reference's
 * select_shared_blocks applied to the group's G query heads) or
 * select_groups == 1 (one set shared by all heads, the reference's C2 call).
 * Candidates are the sealed blocks [0, sealed[seq]).  When the budget is not
 * smaller than the candidate count every sealed block is selected (the
 * Python reference clamps, src/solidattention_lab/selection.py:120; the C++
 * one throws, cpp/src/selection.cpp:101-105).
 * selected: [B][select_groups][sel_stride] ids ascending; counts:
 * [B][select_groups]; scores (optional): [B][select_groups][rep_stride]. */
int sao_paged_score_select(const float* query, const float* reps,
                           const int32_t* sealed, size_t batch,
                           size_t query_heads, size_t kv_heads,
                           size_t head_dim, size_t rep_heads,
                           size_t rep_stride, size_t select_groups,
                           size_t budget, size_t init_blocks,
                           size_t local_blocks, int32_t* selected,
                           int32_t* counts, size_t sel_stride, float* scores);

/* Sparse GQA decode attention: for every (seq, KV head g) the tokens of the
 * selected sealed blocks (ascending) followed by every tail token
 * [sealed * page_tokens, seq_len) are gathered and
 * sao_attention_reference's arithmetic is applied to each query head of the
 * group.  out: [B][Hq][D]. */
int sao_paged_sparse_attention(const uint16_t* pool, size_t page_tokens,
                               const int32_t* block_table,
                               size_t table_stride, const int32_t* seq_len,
                               const int32_t* sealed, const int32_t* selected,
                               const int32_t* counts, size_t sel_stride,
                               size_t select_groups, const float* query,
                               size_t batch, size_t query_heads,
                               size_t kv_heads, size_t head_dim, float scale,
                               float* out);

/* Decode-token append into the paged pool: token seq_len[s] of sequence s
 * receives K,V (fp32 converted with round-to-nearest-even, or raw FP16 bits
 * when k16/v16 are given), then seq_len[s] += 1.  k, v: [B][Hkv][D].
 * Follows cpp/src/qwen_layer_main.cpp:270-281 and
 * cpp/src/kv_lifecycle_main.cpp:31-39. */
int sao_paged_append(uint16_t* pool, size_t page_tokens,
                     const int32_t* block_table, size_t table_stride,
                     int32_t* seq_len, const float* k, const float* v,
                     const uint16_t* k16, const uint16_t* v16, size_t batch,
                     size_t kv_heads, size_t head_dim);

/* Seal: while seq_len - sealed*page_tokens >= local_tokens + page_tokens the
 * oldest tail block becomes selectable: its mean-key representative is
 * written (for each rep head) and sealed/generation advance.
 * Follows cpp/src/kv_lifecycle_main.cpp:92-113 (condition, erase,
 * generation) with the mean-key representative. */
int sao_paged_seal(const uint16_t* pool, size_t page_tokens,
                   const int32_t* block_table, size_t table_stride,
                   const int32_t* seq_len, int32_t* sealed,
                   int32_t* generation, float* reps, size_t rep_heads,
                   size_t rep_stride, size_t batch, size_t query_heads,
                   size_t kv_heads, size_t head_dim, size_t local_tokens);

/* Pack: copy the listed pages contiguously, in list order.
 * Follows the placement of cpp/src/uring_reader.cpp:87-95 (block i of the
 * request lands at buffer offset i * block_bytes). */
void sao_pack_blocks(const uint16_t* pool, size_t page_elems,
                     const int32_t* pages, size_t count, uint16_t* out);

/* ---- Decode-tail lifecycle (reference synthetic driver) ---------------- */

/* Runs the reference's synthetic native lifecycle: local_tokens initial
 * appends per layer, then decode_tokens steps x layers appends, each
 * followed by the seal loop with the per-head top-4 argmax audit.
 * Follows cpp/src/kv_lifecycle_main.cpp:25-45 and 83-115.
 * sealed_blocks_out: per layer; the sealed block bytes are checked against
 * the closed form of kv_lifecycle_main.cpp:127-134 inside (returns 1 on a
 * mismatch). */
typedef struct {
  size_t sealed_blocks;
  size_t representative_head_audits;
  size_t resident_tail_tokens;   /* layer 0 */
  size_t generation;             /* layer 0 */
  size_t store_bytes;
  uint64_t sealed_bytes_fnv;     /* FNV-1a of all sealed blocks, layer-major */
} sao_lifecycle_result;

int sao_run_synthetic_lifecycle(size_t layers, size_t decode_tokens,
                                sao_lifecycle_result* result);

/* Top-k argmax-first audit over a score vector: rank r picks the first
 * maximum among the tokens not yet picked.  Follows
 * cpp/src/kv_lifecycle_main.cpp:93-102. */
void sao_topk_argmax(const float* scores, size_t n, size_t k, size_t* top);

/* ---- History prediction and miss correction --------------------------- */

/* compare_prediction: hits, misses (oracle blocks absent from the
 * prediction, in oracle order) and replacement slots (prediction slots whose
 * block is absent from the oracle, in slot order); the corrected set must
 * equal the oracle.  Returns SAO_EINVAL on a cardinality mismatch and 2 when
 * the corrected set differs from the oracle.
 * Follows cpp/src/pipeline_main.cpp:686-717. */
int sao_compare_prediction(const size_t* predicted, const size_t* oracle,
                           size_t n, size_t* hits, size_t* misses,
                           size_t* replacement_slots, size_t* miss_count);

/* Closed-form 4-block oracle set for (step, layer).
 * Follows cpp/src/pipeline_main.cpp:439-447. */
void sao_oracle_blocks(size_t step, size_t layer, size_t out[4]);

/* Generation ticket check.  Follows cpp/src/pipeline_main.cpp:432-437. */
int sao_valid_ticket(size_t ticket_token, size_t ticket_layer,
                     size_t ticket_generation, const size_t ticket_blocks[4],
                     size_t token, size_t layer, size_t generation,
                     const size_t blocks[4]);

/* ---- Reference fixtures ------------------------------------------------ */

/* C1 128-token sin fixture (cpp/src/attention_main.cpp:131-156):
 * kv [tokens][2][Hkv][D] FP16 bits, query [Hq][D]. */
void sao_fixture_c1(size_t tokens, size_t query_heads, size_t kv_heads,
                    size_t head_dim, uint16_t* kv, float* query);

/* C2/P1 InfLLM sin/cos fixture (cpp/src/selection_main.cpp:113-147,
 * identical to cpp/src/pipeline_main.cpp:581-623):
 * kv [tokens][2][Hkv][D], prompt_queries [Hq][tokens][D]. */
void sao_fixture_c2(size_t tokens, size_t query_heads, size_t kv_heads,
                    size_t head_dim, uint16_t* kv, float* prompt_queries);

/* P1 history pipeline query position for (step, layer)
 * (cpp/src/pipeline_main.cpp:469-470). */
size_t sao_p1_query_position(size_t tokens, size_t step, size_t layer);

/* P1 dense audit: mean selected attention mass and mean recall of the
 * selected 4-block sets against the dense attention-mass oracle.
 * Follows cpp/src/pipeline_main.cpp:502-574. */
int sao_p1_dense_audit(const uint16_t* kv, const float* prompt_queries,
                       const float* representatives, size_t steps,
                       size_t layers, double* mass, double* recall);

/* ---- Synthetic data shared with the device generator ------------------- */

/* Query producer / output consumer (qwen_layer_main.cpp:125-183):
 * rms_norm, the [out][in] projections with an optional residual, and the
 * per-head RMS norm + rotary embedding (NeoX halves). */
int sao_rms_norm(const float* x, const float* w, float* out, size_t rows, size_t width, float eps);
int sao_linear(const float* x, const float* w, const float* residual, float* y, size_t rows, size_t in,
               size_t out);
void sao_rope_inv_freq(float theta, size_t head_dim, float* inv_freq);
int sao_qk_norm_rope(float* x, const float* w, const int32_t* positions, size_t rows, size_t heads,
                     size_t head_dim, float theta, float eps);

/* Counter-based generator.  sao_synth_normal(seed, index) is an
 * Irwin-Hall(4) approximation of N(0,1) computed with integer arithmetic and
 * one fp32 multiply, so the device generator produces the same bits. */
uint64_t sao_mix64(uint64_t x);
float sao_synth_normal(uint64_t seed, uint64_t index);
void sao_synth_fill_half(uint64_t seed, uint64_t first_index, size_t count,
                         uint16_t* out);
void sao_synth_fill_float(uint64_t seed, uint64_t first_index, size_t count,
                          float* out);

/*
 * Pins (tests/ file that holds each check):
 *   sao_float_to_half / sao_half_to_float  — all 65536 halves round trip;
 *       differential vs oracle/_ref on random floats (test_oracle_ref.py)
 *   sao_float_to_half_rne                  — numpy float16 cast, all
 *       classes (test_oracle_codec.py)
 *   sao_attention_reference                — oracle/_ref bit-exact; full
 *       budget == dense; one-token closed form (test_oracle_ref.py)
 *   sao_build_local_causal_representatives — C2.1 offset hash
 *       7873450381430813043 and oracle/_ref bit-exact (test_oracle_golden.py)
 *   sao_mean_key_representatives           — == local-causal(window 1,
 *       topk 32) via oracle/_ref (test_oracle_ref.py)
 *   sao_select_shared_blocks               — C2.1 ids [0,8,13,15],
 *       P1.1 recall/mass, oracle/_ref bit-exact incl. ties (golden, ref)
 *   sao_paged_*                            — reduce to the functions above
 *       on identity tables (test_oracle_paged.py)
 *   sao_run_synthetic_lifecycle            — P1.3b.0 metrics
 *       (448, 7168, 32, 16, 121110528) (test_oracle_golden.py)
 *   sao_compare_prediction                 — P1.0 346 misses / 0.80692,
 *       P1.1 742 / 0.585938 (test_oracle_golden.py)
 */

#ifdef __cplusplus
}
#endif

#endif /* SA_ORACLE_H */
