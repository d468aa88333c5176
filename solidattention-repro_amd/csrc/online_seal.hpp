// online_seal.hpp — the InfLLM online seal on the device (the reference's
// P1.3c.4, cpp/src/online_seal_main.cpp:41-44): when a decode step seals a
// 32-token block, the representative of query head h is
// build_local_causal_representatives (cpp/src/selection.cpp:12-94) applied to
// that block alone, with the block's 32 keys (KV head h / G) and the 32
// decode queries of head h issued with those tokens, block_tokens 32, a local
// window and a top-k: the mean of the top-k keys ranked by the softmax mass
// they received from the block's queries.  Same arithmetic as the reference,
// bit for bit: sequential fp32 dots (no fused multiply-add; the including
// file is compiled with -ffp-contract=off), logits scaled, the row maximum,
// glibc's expf (expf_glibc.hpp), the denominator summed in key order,
// probabilities divided, each key's mass summed in query order, a stable
// descending rank (ties keep token order) and the chosen keys summed in rank
// order, divided by top-k.
//
// The decode queries live in a ring in HBM: the query of head h issued with
// the token at position p is kept at slot p % ring_tokens of
// ring[b][h][slot][128], written by the decode step that appends the token.
#pragma once

#include "expf_glibc.hpp"
#include "sa_device.hpp"
#include "sa_internal.hpp"

namespace sa {
namespace online {

constexpr int kT = kPageTokens;           // tokens of a sealed block
constexpr int kDim = kHeadDim;
constexpr int kQStride = kDim + 1;        // padded query rows (floats): no bank conflicts
constexpr int kKStride = kDim / 2 + 1;    // padded key rows (dwords of two FP16 values)
constexpr int kLStride = kT + 1;          // padded logit rows
// LDS floats the seal of one (sequence, query head, block) borrows
constexpr int kSmemFloats = kT * kQStride + kT * kKStride + kT * kLStride + 3 * kT;

struct Args {
  float* ring;          // [batch][query_heads][ring_tokens][128] decode queries
  int32_t ring_tokens;
  int32_t window;       // local causal window of the builder (>= 1)
  int32_t topk;         // keys averaged per representative (1..32)
  int32_t query_heads;
  float scale;          // 1 / sqrt(128), as the reference computes it
};

// Keep the decode query rows of heads [h0, h0 + heads) of sequence b for the
// token at position pos (ring slot pos % ring_tokens).  Any thread layout.
__device__ inline void store_queries(const Args& a, const float* query, int b, int h0, int heads, int64_t pos,
                                     int tid, int threads) {
  const int64_t slot = pos % a.ring_tokens;
  for (int e = tid; e < heads * kDim; e += threads) {
    const int h = h0 + e / kDim;
    const int d = e % kDim;
    a.ring[((static_cast<int64_t>(b) * a.query_heads + h) * a.ring_tokens + slot) * kDim + d] =
        query[(static_cast<int64_t>(b) * a.query_heads + h) * kDim + d];
  }
}

// Representative of one sealed block for query head h.  keys: the block's
// key row of its KV head for token 0 (token t at keys + t * token_elems);
// first_pos: the position of the block's token 0; rep: the representative's
// value of d = 0 (d at rep + d * rep_stride).  Every thread of the workgroup
// calls it (workgroup barriers inside); smem: kSmemFloats floats of LDS.
template <int kThreads>
__device__ inline void seal_head(const Args& a, int b, int h, const uint16_t* keys, int64_t token_elems,
                                 int64_t first_pos, float* rep, int64_t rep_stride, float* smem) {
  const int tid = threadIdx.x;
  float* qs = smem;                                                     // [32][129]
  uint32_t* ks = reinterpret_cast<uint32_t*>(smem + kT * kQStride);     // [32][65]
  float* ls = smem + kT * kQStride + kT * kKStride;                     // [32][33]
  float* received = ls + kT * kLStride;                                 // [32]
  float* row = received + kT;                                           // [32] max, then denominator
  int* order = reinterpret_cast<int*>(row + kT);                        // [32]

  const float* ring_h = a.ring + (static_cast<int64_t>(b) * a.query_heads + h) * a.ring_tokens * kDim;
  for (int e = tid; e < kT * kDim; e += kThreads) {
    const int t = e / kDim;
    const int d = e % kDim;
    qs[t * kQStride + d] = ring_h[((first_pos + t) % a.ring_tokens) * kDim + d];
  }
  for (int e = tid; e < kT * kDim / 2; e += kThreads) {
    const int t = e / (kDim / 2);
    const int w = e % (kDim / 2);
    ks[t * kKStride + w] = *reinterpret_cast<const uint32_t*>(keys + t * token_elems + 2 * w);
  }
  __syncthreads();

  // logits of query i over keys j in [i + 1 - window, i] (selection.cpp:36-48)
  for (int e = tid; e < kT * kT; e += kThreads) {
    const int i = e / kT;
    const int j = e % kT;
    if (j > i || i - j >= a.window) continue;
    const float* q = qs + i * kQStride;
    const uint32_t* k = ks + j * kKStride;
    float dot = 0.0f;
#pragma unroll 8
    for (int w = 0; w < kDim / 2; ++w) {
      const uint32_t kw = k[w];
      dot = dot + q[2 * w] * lo_h2f(kw);
      dot = dot + q[2 * w + 1] * hi_h2f(kw);
    }
    ls[i * kLStride + j] = dot * a.scale;
  }
  __syncthreads();
  if (tid < kT) {
    const int i = tid;
    const int start = i + 1 > a.window ? i + 1 - a.window : 0;
    float maximum = -__builtin_huge_valf();
    for (int j = start; j <= i; ++j) maximum = fmaxf(maximum, ls[i * kLStride + j]);
    row[i] = maximum;
  }
  __syncthreads();
  // exponentials (selection.cpp:51-52)
  for (int e = tid; e < kT * kT; e += kThreads) {
    const int i = e / kT;
    const int j = e % kT;
    if (j > i || i - j >= a.window) continue;
    ls[i * kLStride + j] = expf_glibc(ls[i * kLStride + j] - row[i]);
  }
  __syncthreads();
  if (tid < kT) {  // denominators in key order (selection.cpp:53)
    const int i = tid;
    const int start = i + 1 > a.window ? i + 1 - a.window : 0;
    float denominator = 0.0f;
    for (int j = start; j <= i; ++j) denominator = denominator + ls[i * kLStride + j];
    row[i] = denominator;
  }
  __syncthreads();
  for (int e = tid; e < kT * kT; e += kThreads) {
    const int i = e / kT;
    const int j = e % kT;
    if (j > i || i - j >= a.window) continue;
    ls[i * kLStride + j] = ls[i * kLStride + j] / row[i];
  }
  __syncthreads();
  if (tid < kT) {  // the mass key j received, in query order (selection.cpp:55-58)
    const int j = tid;
    const int last = j + a.window - 1 < kT - 1 ? j + a.window - 1 : kT - 1;
    float r = 0.0f;
    for (int i = j; i <= last; ++i) r = r + ls[i * kLStride + j];
    received[j] = r;
  }
  __syncthreads();
  if (tid < kT) {  // stable descending rank (selection.cpp:71-76)
    const int j = tid;
    const float rj = received[j];
    int rank = 0;
    for (int k = 0; k < kT; ++k) {
      const float rk = received[k];
      rank += (mass_before(rk, rj) || (k < j && mass_tied(rk, rj))) ? 1 : 0;
    }
    order[rank] = j;
  }
  __syncthreads();
  for (int d = tid; d < kDim; d += kThreads) {  // top-k keys in rank order (selection.cpp:80-89)
    float value = 0.0f;
    for (int r = 0; r < a.topk; ++r) {
      const uint32_t kw = ks[order[r] * kKStride + d / 2];
      value = value + ((d & 1) ? hi_h2f(kw) : lo_h2f(kw));
    }
    rep[d * rep_stride] = value / static_cast<float>(a.topk);
  }
  __syncthreads();  // the LDS is free again
}

}  // namespace online
}  // namespace sa
