// qkv_epilogue.hpp — the q/k/v producer's epilogue for one (row, head):
// the K-slice partial sums added in slice order, the row's input RMSNorm
// scale, then for q and k heads the head RMS norm and RoPE (NeoX pairs d,
// d + 64).  Shared by the producer's reduce launch (producer.hip) and the
// decode step that takes the partials directly (select_attend.hip), so the
// two give the same bits.  Semantics of the reference's rms_norm, head_rms
// and rope (cpp/src/qwen_layer_main.cpp:125-172, :576-584).
#pragma once

#include "sa_device.hpp"
#include "sa_internal.hpp"

namespace sa {
namespace qkv {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct ReduceParams {
  const float* part;       // [slices][rows_pad][out]
  const float* ss;         // [slices][rows_pad] or null (no input RMSNorm)
  int32_t slices;
  int32_t rows;
  int32_t rows_pad;
  int32_t in;
  int32_t out;
  float in_eps;
  const float* q_norm;
  const float* k_norm;
  const int32_t* positions;
  float* q;
  float* k;
  float* v;
  int32_t q_heads;
  int32_t kv_heads;
  float eps;
  alignas(16) float inv_freq[64];  // 16-byte aligned: a lane reads its 4 frequencies in one load
};

// The K-slice partials at offset off of each slice (slice_stride floats
// apart), added in slice order to v0, together with the same slices' scalars
// (sum of squares) at soff of each ss_stride-float slice added to tot0 (in
// tot); each batch of 8 slices' loads is issued before its adds.
__device__ inline f32x4_t sum_slices4_ss(const float* part, int slices, int64_t slice_stride, int64_t off,
                                         const float* ss, int64_t ss_stride, int64_t soff, float& tot, f32x4_t v0,
                                         float tot0) {
  constexpr int kBatch = 8;
  f32x4_t v = v0;
  tot = tot0;
  for (int z0 = 0; z0 < slices; z0 += kBatch) {
    f32x4_t s[kBatch];
    float q[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int z = z0 + i < slices ? z0 + i : slices - 1;
      s[i] = *reinterpret_cast<const f32x4_t*>(part + z * slice_stride + off);
      q[i] = ss[z * ss_stride + soff];
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      if (z0 + i < slices) {
        v += s[i];
        tot += q[i];
      }
    }
  }
  return v;
}

// Dimensions 4 j .. 4 j + 3 of head hh (q heads, then k, then v: [0,
// q_heads + 2 kv_heads)) of row rr.  The 32 lanes j = 0..31 of the head must
// be the lanes of one half of a wave (the head's sums and RoPE pairs are
// exchanged within it); the two halves may hold different heads.  Every load
// of the row is issued first; the RoPE angles' sines and cosines, which need
// only the position, are computed while the slices are in flight.
__device__ inline f32x4_t head_value(const ReduceParams& p, int hh, int rr, int j) {
  constexpr int kBatch = 8;  // the first batch (a 1024-wide hidden has 8 slices of 128 k); the rest 8 at a time
  const int64_t col = static_cast<int64_t>(hh) * kHeadDim + 4 * j;
  const bool is_v = hh >= p.q_heads + p.kv_heads;
  const bool is_q = hh < p.q_heads;
  // the position, the head norm weights, the RoPE frequencies of d and d + 64
  // (the same 4), the first batch of slices and their sums of squares
  // (without an input RMSNorm those are read from the partials instead,
  // unconditionally, and not used)
  const float pos = static_cast<float>(p.positions[rr]);
  const f32x4_t n4 = *reinterpret_cast<const f32x4_t*>((is_q ? p.q_norm : p.k_norm) + 4 * j);
  const f32x4_t fr = *reinterpret_cast<const f32x4_t*>(p.inv_freq + 4 * (j % 16));
  const int64_t slice_stride = static_cast<int64_t>(p.rows_pad) * p.out;
  const int64_t off = static_cast<int64_t>(rr) * p.out + col;
  const float* ss = p.ss ? p.ss : p.part;
  f32x4_t s[kBatch];
  float q[kBatch];
#pragma unroll
  for (int i = 0; i < kBatch; ++i) {
    const int z = i < p.slices ? i : p.slices - 1;
    s[i] = *reinterpret_cast<const f32x4_t*>(p.part + z * slice_stride + off);
    q[i] = ss[static_cast<int64_t>(z) * p.rows_pad + rr];
  }
  float sn[4], cs[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) sincosf(pos * fr[e], &sn[e], &cs[e]);
  // the slices added in slice order from zero (with their sums of squares);
  // later batches are loaded before their adds
  f32x4_t v = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < kBatch; ++i) {
    if (i < p.slices) {
      v += s[i];
      tot += q[i];
    }
  }
  if (p.slices > kBatch) {
    float t2;
    const f32x4_t rest = sum_slices4_ss(p.part + kBatch * slice_stride, p.slices - kBatch, slice_stride, off,
                                        ss + static_cast<int64_t>(kBatch) * p.rows_pad, p.rows_pad, rr, t2, v, tot);
    v = rest;
    tot = t2;
  }
  if (p.ss) v *= 1.0f / __builtin_sqrtf(tot / static_cast<float>(p.in) + p.in_eps);
  // q and k heads: head RMS norm, then RoPE (v heads take v as it is; every
  // lane computes both, so the exchanges below run on full waves)
  float sq = v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) sq += __shfl_xor(sq, o, kWave);
  const float inv = 1.0f / __builtin_sqrtf(sq / static_cast<float>(kHeadDim) + p.eps);
  f32x4_t x, y, o;
#pragma unroll
  for (int e = 0; e < 4; ++e) x[e] = v[e] * inv * n4[e];
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = __shfl_xor(x[e], 16, kWave);  // the pair partner, d +- 64
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = j < 16 ? x[e] * cs[e] - y[e] * sn[e] : x[e] * cs[e] + y[e] * sn[e];
  return is_v ? v : o;
}

// Where head hh of row `row` goes in q, k or v ([row][heads][128]).
__device__ inline float* head_dst(const ReduceParams& p, int hh, int row) {
  if (hh >= p.q_heads + p.kv_heads)
    return p.v + (static_cast<int64_t>(row) * p.kv_heads + (hh - p.q_heads - p.kv_heads)) * kHeadDim;
  if (hh < p.q_heads) return p.q + (static_cast<int64_t>(row) * p.q_heads + hh) * kHeadDim;
  return p.k + (static_cast<int64_t>(row) * p.kv_heads + (hh - p.q_heads)) * kHeadDim;
}

}  // namespace qkv
}  // namespace sa
