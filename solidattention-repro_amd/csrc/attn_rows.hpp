// attn_rows.hpp — the token-row attention walk at head dimensions other than
// 128 (gfx950), shared by the separate attention (attention_any.hip) and the
// one-launch decode step (select_attend.hip).
//
// The lane layout of the head_dim-128 kernels (attn_core.hpp) at any head_dim
// up to 256: one KV head's K (or V) row of a token is read by LPR lanes, 16
// bytes (8 dimensions) each, LPR the power of two at or above head_dim / 8 and
// at least 8 (lanes past head_dim idle), so one load of a wave covers 64 / LPR
// whole rows and a page is 32 LPR / 64 loads of K and as many of V, issued
// together (a unit of at most 8 row groups; two units per page at LPR 32, and
// 4-row-group units at 8 query heads per KV head, whose state takes the
// registers).  A row's dot is summed across its lanes, the online softmax
// (log2 domain) runs per wave over the unit's rows, and P.V accumulates each
// lane's 8 dimensions over its rows; finish() adds the rows.  Semantics of
// the reference's attention_reference (cpp/src/attention_reference.cpp:55-96)
// over the tokens walked.
#pragma once

#include "sa_device.hpp"

namespace sa {
namespace rows {

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxHeadDim = 256;  // 32 lanes x 8 dimensions

// Lanes per token row at a head_dim (<= kMaxHeadDim).
__host__ __device__ constexpr int lanes_per_row(int head_dim) {
  return head_dim <= 64 ? 8 : (head_dim <= 128 ? 16 : 32);
}

// Sum over the LPR lanes of a token row (every lane of the row gets it).
template <int LPR>
__device__ inline float lane_row_sum(float v) {
  if constexpr (LPR == 8) {
    v += dpp_f<kDppQuadXor1>(v);
    v += dpp_f<kDppQuadXor2>(v);
    v += dpp_f<kDppRowHalfMirror>(v);  // the quads are uniform: exchanges the two quads of 8 lanes
    return v;
  } else if constexpr (LPR == 16) {
    return row16_sum(v);
  } else {
    static_assert(LPR == 32, "8, 16 or 32 lanes per row");
    v = row16_sum(v);
    return v + shfl_xor_f(v, 16);
  }
}

// Sum / max over the token rows of a wave (the lanes of one column).
template <int LPR>
__device__ inline float across_rows_sum(float v) {
#pragma unroll
  for (int o = LPR; o < kWave; o <<= 1) v += shfl_xor_f(v, o);
  return v;
}

template <int LPR>
__device__ inline float across_rows_max(float v) {
#pragma unroll
  for (int o = LPR; o < kWave; o <<= 1) v = fmaxf(v, shfl_xor_f(v, o));
  return v;
}

// Online-softmax state of one wave for the G query heads of a KV head.
template <int G, int LPR>
struct RowsState {
  static constexpr int kR = kWave / LPR;                  // token rows per load
  static constexpr int kI = kPageTokens / kR;             // loads per page (K or V)
  static constexpr int kMaxUnit = G == 8 ? 4 : 8;         // row groups held in registers
  static constexpr int NIT = kI < kMaxUnit ? kI : kMaxUnit;  // row groups per unit
  static constexpr int kParts = kI / NIT;                 // units per page

  int row;
  int col;
  bool dims;  // this lane's 8 dimensions exist
  float qf[G][8];
  float m[G];
  float l[G];
  float acc[G][8];

  // q: the G heads' rows of D floats (16-byte aligned); sl2 = scale * log2(e)
  __device__ inline void init(const float* q, int D, float sl2, int lane) {
    row = lane / LPR;
    col = lane % LPR;
    dims = col * 8 < D;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), c = a;
      if (dims) {
        a = *reinterpret_cast<const float4*>(q + h * D + col * 8);
        c = *reinterpret_cast<const float4*>(q + h * D + col * 8 + 4);
      }
      qf[h][0] = a.x * sl2;
      qf[h][1] = a.y * sl2;
      qf[h][2] = a.z * sl2;
      qf[h][3] = a.w * sl2;
      qf[h][4] = c.x * sl2;
      qf[h][5] = c.y * sl2;
      qf[h][6] = c.z * sl2;
      qf[h][7] = c.w * sl2;
      m[h] = kNegInf;
      l[h] = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[h][j] = 0.0f;
    }
  }

  // This lane's element offset within a page: its row's K row of KV head g.
  __device__ inline int64_t lane_offset(int64_t tok_elems, int g, int D) const {
    return static_cast<int64_t>(row) * tok_elems + static_cast<int64_t>(g) * D + col * 8;
  }

  // Unit `part` of a page (rows (part NIT + it) kR + row) with `valid`
  // tokens; base = the page's start plus lane_offset(); V is v_off elements
  // after K.
  __device__ inline void attend_unit(const uint16_t* base, int64_t tok_elems, int64_t v_off, int valid, int part) {
    uint4 kr[NIT], vr[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int rg = part * NIT + it;  // row group of the page
      if (dims && rg * kR + row < valid) {
        kr[it] = load_stream16(base + static_cast<int64_t>(rg) * kR * tok_elems);
        vr[it] = load_stream16(base + static_cast<int64_t>(rg) * kR * tok_elems + v_off);
      } else {
        kr[it] = make_uint4(0, 0, 0, 0);
        vr[it] = make_uint4(0, 0, 0, 0);
      }
    }
    // logits of this lane's rows for every head
    float sc[G][NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const uint32_t w[4] = {kr[it].x, kr[it].y, kr[it].z, kr[it].w};
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float kj = (j & 1) ? hi_h2f(w[j >> 1]) : lo_h2f(w[j >> 1]);
          a = __builtin_fmaf(qf[h][j], kj, a);
        }
        sc[h][it] = lane_row_sum<LPR>(a);
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float pmax = kNegInf;
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        if ((part * NIT + it) * kR + row >= valid) sc[h][it] = kNegInf;
        pmax = fmaxf(pmax, sc[h][it]);
      }
      pmax = across_rows_max<LPR>(pmax);
      const float mn = fmaxf(m[h], pmax);
      // mn == -inf only if nothing finite was seen: the state stays empty
      const float corr = (m[h] == mn) ? 1.0f : __builtin_amdgcn_exp2f(m[h] - mn);
      const float base_m = (mn == kNegInf) ? 0.0f : mn;
      m[h] = mn;
      float lsum = l[h] * corr;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[h][j] *= corr;
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        sc[h][it] = __builtin_amdgcn_exp2f(sc[h][it] - base_m);
        lsum += sc[h][it];
      }
      l[h] = lsum;
    }
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const uint32_t w[4] = {vr[it].x, vr[it].y, vr[it].z, vr[it].w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float vj = (j & 1) ? hi_h2f(w[j >> 1]) : lo_h2f(w[j >> 1]);
#pragma unroll
        for (int h = 0; h < G; ++h) acc[h][j] = __builtin_fmaf(sc[h][it], vj, acc[h][j]);
      }
    }
  }

  __device__ inline void attend_page(const uint16_t* base, int64_t tok_elems, int64_t v_off, int valid) {
#pragma unroll
    for (int part = 0; part < kParts; ++part) {
      if (part * NIT * kR >= valid) break;
      attend_unit(base, tok_elems, v_off, valid, part);
    }
  }

  // The wave's rows added: every lane holds its column's l and acc; m is
  // uniform over the wave.
  __device__ inline void finish() {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      l[h] = across_rows_sum<LPR>(l[h]);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[h][j] = across_rows_sum<LPR>(acc[h][j]);
    }
  }
};

}  // namespace rows
}  // namespace sa
