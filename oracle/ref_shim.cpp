// ref_shim.cpp — C-ABI wrappers so tests can call the reference's own CPU
// functions (compiled from the reference sources by oracle/Makefile into
// oracle/_ref/libsa_ref.so).  TEST INFRASTRUCTURE ONLY: a second checker for
// the oracle restatement, never part of the product.
#include "solidattention/attention_reference.hpp"
#include "solidattention/selection.hpp"

#include <cstring>
#include <exception>

namespace sa = solidattention;

extern "C" {

std::uint16_t saref_float_to_half(float value) { return sa::float_to_half(value); }
float saref_half_to_float(std::uint16_t value) { return sa::half_to_float(value); }

int saref_attention_reference(const std::uint16_t* kv, const float* query,
                              std::size_t tokens, std::size_t query_heads,
                              std::size_t kv_heads, std::size_t head_dim,
                              float scale, float* out) {
  try {
    sa::AttentionProblem problem{kv, query, tokens, query_heads, kv_heads,
                                 head_dim, scale};
    const auto result = sa::attention_reference(problem);
    std::memcpy(out, result.data(), result.size() * sizeof(float));
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

int saref_build_local_causal_representatives(
    const float* prompt_queries, const std::uint16_t* kv, std::size_t tokens,
    std::size_t query_heads, std::size_t kv_heads, std::size_t head_dim,
    std::size_t block_tokens, std::size_t local_window, std::size_t topk,
    float* values, std::size_t* offsets) {
  try {
    const auto result = sa::build_local_causal_representatives(
        prompt_queries, kv, tokens, query_heads, kv_heads, head_dim,
        block_tokens, local_window, topk);
    std::memcpy(values, result.values.data(),
                result.values.size() * sizeof(float));
    std::memcpy(offsets, result.chosen_token_offsets.data(),
                result.chosen_token_offsets.size() * sizeof(std::size_t));
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

int saref_select_shared_blocks(const float* query, const float* reps,
                               std::size_t query_heads, std::size_t blocks,
                               std::size_t head_dim, std::size_t budget,
                               std::size_t init_blocks,
                               std::size_t local_blocks, std::size_t* ids,
                               std::size_t* count, float* scores) {
  try {
    const auto result = sa::select_shared_blocks(
        query, reps, query_heads, blocks, head_dim, budget, init_blocks,
        local_blocks);
    std::memcpy(ids, result.block_ids.data(),
                result.block_ids.size() * sizeof(std::size_t));
    *count = result.block_ids.size();
    if (scores)
      std::memcpy(scores, result.mean_head_scores.data(),
                  result.mean_head_scores.size() * sizeof(float));
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

}  // extern "C"
