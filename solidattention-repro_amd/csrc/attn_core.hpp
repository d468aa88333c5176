// attn_core.hpp — device building blocks of the GQA sparse decode attention
// over paged FP16 KV (gfx950), shared by the attention kernel and the fused
// select + attend kernel.
//
// Semantics: attention_reference (reference cpp/src/attention_reference.cpp
// :55-96) applied, per (sequence, KV head g), to the tokens of the selected
// sealed blocks followed by the unsealed tail, for each of the G query heads
// of g.  Softmax is computed online in the log2 domain; fp32 arithmetic on
// exact FP16 decodes.  The reference's two-pass order is not reproduced
// (tolerance-checked, not bit-exact).
//
// Lane mapping (head_dim 128): one wave64 walks whole 32-token pages.  A
// 16-byte load per lane covers 4 rows of 256 B (16 lanes per K or V row of
// one KV head), so a page's K and V tiles for head g are 8 + 8 dwordx4 loads
// per lane.  Lane (row r, column c) owns dims [8c, 8c+8) of tokens
// {r, r+4, ...}.  q.k partial dots are reduced across the 16 lanes of a row
// with DPP; the G query heads of the group reuse every K/V register
// (v_fma_mix_f32 consumes the FP16 halves directly), so KV bytes are read
// from HBM once per group.  No MFMA: decode attention is a matrix-vector
// product (about 2 flop per KV byte at G=2).
#pragma once

#include "sa_device.hpp"
#include "sa_internal.hpp"

namespace sa {
namespace attn {

constexpr int D = kHeadDim;
constexpr int kLanesPerRow = D / 8;               // 16 lanes x 8 halves = one 256 B row
constexpr int kRows = kWave / kLanesPerRow;       // 4 rows per wave-wide load
constexpr int kIters = kPageTokens / kRows;       // 8 tokens per lane per page
constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;

__device__ inline void unpack8(const uint4& w, float (&f)[8]) {
  f[0] = lo_h2f(w.x);
  f[1] = hi_h2f(w.x);
  f[2] = lo_h2f(w.y);
  f[3] = hi_h2f(w.y);
  f[4] = lo_h2f(w.z);
  f[5] = hi_h2f(w.z);
  f[6] = lo_h2f(w.w);
  f[7] = hi_h2f(w.w);
}

// Where the K/V pages of one (sequence, KV head) live.
struct PoolView {
  const uint16_t* pool;
  const int32_t* table;     // [batch][table_stride]; unused when contig_tokens > 0
  int32_t* status;
  int64_t num_pages;
  int64_t contig_tokens;    // > 0: one contiguous token buffer, no table
  int64_t page_elems;
  int32_t token_elems;
  int32_t table_stride;
  int32_t kv_heads;
};

// Page `i` of the (sequence, KV head) list: selected sealed blocks first,
// then the tail pages.  valid = number of tokens to read (0 = skip).
struct PageRef {
  int64_t page;
  int valid;
};

struct PageList {
  const int32_t* sel;  // selected logical block ids (global or LDS)
  int64_t len;         // tokens held by the sequence
  int sealed;          // sealed blocks
  int n_sel;           // selected blocks
  int total;           // n_sel + tail pages
};

__device__ inline PageRef resolve_page(const PoolView& v, int b, int i, const PageList& L) {
  PageRef r{0, 0};
  if (i >= L.total) return r;
  int64_t logical;
  if (i < L.n_sel) {
    logical = L.sel[i];
    if (logical < 0 || logical >= L.sealed) {
      flag_status(v.status, kStatusBadBlock);
      return r;
    }
    r.valid = kPageTokens;
  } else {
    logical = static_cast<int64_t>(L.sealed) + (i - L.n_sel);
    const int64_t left = L.len - logical * kPageTokens;
    r.valid = left < kPageTokens ? static_cast<int>(left) : kPageTokens;
  }
  if (v.contig_tokens > 0) {
    r.page = logical;
    return r;
  }
  if (logical >= v.table_stride) {
    flag_status(v.status, kStatusBadBlock);
    r.valid = 0;
    return r;
  }
  const int64_t page = v.table[static_cast<int64_t>(b) * v.table_stride + logical];
  if (page < 0 || page >= v.num_pages) {
    flag_status(v.status, kStatusBadPage);
    r.valid = 0;
    return r;
  }
  r.page = page;
  return r;
}

// Per-lane offsets of this lane's slice of one KV head's rows.
struct LaneGeom {
  int row;
  int col;
  int64_t head_off;  // from a page's start to this lane's first K element
  int64_t v_off;     // K -> V of the same token
  int64_t step4;     // 4 tokens
};

__device__ inline LaneGeom lane_geom(const PoolView& v, int g, int lane) {
  LaneGeom lg;
  lg.row = lane / kLanesPerRow;
  lg.col = lane % kLanesPerRow;
  lg.head_off = static_cast<int64_t>(lg.row) * v.token_elems + g * D + lg.col * 8;
  lg.v_off = static_cast<int64_t>(v.kv_heads) * D;
  lg.step4 = static_cast<int64_t>(kRows) * v.token_elems;
  return lg;
}

// Issue the 16 dwordx4 loads of one page's K and V tiles (head g).  Rows past
// `valid` are not read (a contiguous buffer may end inside the last page).
__device__ inline void load_page(const PoolView& v, const PageRef& pr, const LaneGeom& lg, uint4 (&kr)[kIters],
                                 uint4 (&vr)[kIters]) {
  const uint16_t* kbase = v.pool + pr.page * v.page_elems + lg.head_off;
  if (pr.valid == kPageTokens) {
#pragma unroll
    for (int it = 0; it < kIters; ++it) kr[it] = load_stream16(kbase + it * lg.step4);
#pragma unroll
    for (int it = 0; it < kIters; ++it) vr[it] = load_stream16(kbase + it * lg.step4 + lg.v_off);
  } else {
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      if (it * kRows + lg.row < pr.valid) {
        kr[it] = load_stream16(kbase + it * lg.step4);
        vr[it] = load_stream16(kbase + it * lg.step4 + lg.v_off);
      } else {
        kr[it] = make_uint4(0, 0, 0, 0);
        vr[it] = make_uint4(0, 0, 0, 0);
      }
    }
  }
}

// Online-softmax state of one wave for the G query heads of a KV group.
template <int G>
struct WaveState {
  float qf[G][8];  // dims [8c, 8c+8) of each head, pre-scaled by scale*log2(e)
  float m[G];      // running max (log2 domain) of this lane's row
  float l[G];      // running denominator
  float acc[G][8];

  // q rows of the G heads of KV head g: query + (b*query_heads + g*G) * D.
  __device__ inline void init(const float* q_group, float qscale, int col) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float4* q4 = reinterpret_cast<const float4*>(q_group + h * D + col * 8);
      const float4 a = q4[0], c = q4[1];
      qf[h][0] = a.x * qscale;
      qf[h][1] = a.y * qscale;
      qf[h][2] = a.z * qscale;
      qf[h][3] = a.w * qscale;
      qf[h][4] = c.x * qscale;
      qf[h][5] = c.y * qscale;
      qf[h][6] = c.z * qscale;
      qf[h][7] = c.w * qscale;
      m[h] = kNegInf;
      l[h] = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[h][j] = 0.0f;
    }
  }

  // Online-softmax update with NIT 4-token row groups (a whole page when
  // NIT == kIters).  Rows at or past `valid` are masked.
  template <int NIT>
  __device__ inline void update(const uint4 (&kr)[NIT], const uint4 (&vr)[NIT], int valid, int row) {
    // logits (log2 domain) of this lane's tokens for every head
    float s[G][NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      float kf[8];
      unpack8(kr[it], kf);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) a = __builtin_fmaf(qf[h][j], kf[j], a);
        s[h][it] = row16_sum(a);
      }
    }
    // s becomes the probabilities relative to the new running max
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float pmax = kNegInf;
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        if (it * kRows + row >= valid) s[h][it] = kNegInf;
        pmax = fmaxf(pmax, s[h][it]);
      }
      pmax = fmaxf(pmax, shfl_xor_f(pmax, 16));
      pmax = fmaxf(pmax, shfl_xor_f(pmax, 32));
      const float mn = fmaxf(m[h], pmax);
      // mn == -inf only if nothing finite was seen: the state stays empty
      const float corr = (m[h] == mn) ? 1.0f : __builtin_amdgcn_exp2f(m[h] - mn);
      const float base = (mn == kNegInf) ? 0.0f : mn;
      m[h] = mn;
      float lsum = l[h] * corr;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[h][j] *= corr;
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        s[h][it] = __builtin_amdgcn_exp2f(s[h][it] - base);
        lsum += s[h][it];
      }
      l[h] = lsum;
    }
    // P.V, each V half converted at its use (v_fma_mix_f32)
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const uint32_t w[4] = {vr[it].x, vr[it].y, vr[it].z, vr[it].w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float vj = (j & 1) ? hi_h2f(w[j >> 1]) : lo_h2f(w[j >> 1]);
#pragma unroll
        for (int h = 0; h < G; ++h) acc[h][j] = __builtin_fmaf(s[h][it], vj, acc[h][j]);
      }
    }
  }

  __device__ inline void attend(const PoolView& v, const PageRef& pr, const LaneGeom& lg) {
    uint4 kr[kIters], vr[kIters];
    load_page(v, pr, lg, kr, vr);
    update<kIters>(kr, vr, pr.valid, lg.row);
  }

  // Sum the 4 rows of the wave (every row holds the same running max).
  __device__ inline void reduce_rows() {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      l[h] += shfl_xor_f(l[h], 16);
      l[h] += shfl_xor_f(l[h], 32);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc[h][j] += shfl_xor_f(acc[h][j], 16);
        acc[h][j] += shfl_xor_f(acc[h][j], 32);
      }
    }
  }
};

// LDS for combining the W waves of a workgroup.
template <int G, int W>
struct CombineSmem {
  float m[W][G];
  float l[W][G];
  float acc[W][G][D];
};

// After reduce_rows(): publish the wave's (m, l, acc) to LDS.  The caller
// synchronises the workgroup before combine_element().
template <int G, int W>
__device__ inline void publish_wave(const WaveState<G>& st, CombineSmem<G, W>& cs, int wave, int lane, int row,
                                    int col) {
  if (row == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int j = 0; j < 8; ++j) cs.acc[wave][h][col * 8 + j] = st.acc[h][j];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      cs.m[wave][h] = st.m[h];
      cs.l[wave][h] = st.l[h];
    }
  }
}

// Log-sum-exp combination of the W waves for head h, dim d: returns the
// merged max (log2 domain), denominator and accumulator.
template <int G, int W>
__device__ inline void combine_element(const CombineSmem<G, W>& cs, int h, int d, float& mx, float& lw, float& aw) {
  mx = kNegInf;
#pragma unroll
  for (int w = 0; w < W; ++w) mx = fmaxf(mx, cs.m[w][h]);
  lw = 0.0f;
  aw = 0.0f;
  if (mx != kNegInf) {
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float mw = cs.m[w][h];
      if (mw == kNegInf) continue;
      const float f = __builtin_amdgcn_exp2f(mw - mx);
      lw = __builtin_fmaf(cs.l[w][h], f, lw);
      aw = __builtin_fmaf(cs.acc[w][h][d], f, aw);
    }
  }
}

}  // namespace attn
}  // namespace sa
