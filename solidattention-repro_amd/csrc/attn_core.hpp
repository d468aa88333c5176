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
// from HBM once per group.  At G <= 2 everything runs on the VALU (decode
// attention is a matrix-vector product, about 2 flop per KV byte); at G = 4
// and 8 the pages are staged through LDS and q.K runs on the matrix cores
// (the staged section below), which halves the VALU work per page.
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

// ---- LDS-staged pages, q.K on the matrix cores (G = 4, 8) ------------------
// A wave copies its next page HBM -> LDS with 16 global_load_lds_dwordx4
// (nothing held in registers while in flight) while it computes the current
// page, so every wave keeps a page in flight through its arithmetic.  Lane
// l's 16 bytes of row group `it` land at stage[it*64 + l] (K row groups 0..7,
// then V 8..15).  V rows are staged as stored (chunk c of a 256 B row at
// position c): the P.V lanes read them back in the register layout above.
// K rows are staged swizzled: token tok keeps its 16-byte chunk c at
// position c ^ k_swizzle(tok), so that the 16 lanes of one matrix-core
// operand read (16 tokens, one chunk each) hit 16 distinct positions and no
// LDS bank twice; the DMA lanes fetch their chunks in that order.
constexpr int kStageVecs = 2 * kIters * kWave;  // 1024 x 16 B = 16 KiB per wave

typedef const void __attribute__((address_space(1)))* GlobalPtr;
typedef void __attribute__((address_space(3)))* LdsPtr;
constexpr int kDmaNontemporal = 2;  // cache policy of the staging loads: streamed (nt)

__device__ inline void dma16(const uint16_t* src, uint4* lds_row_group) {
  __builtin_amdgcn_global_load_lds((GlobalPtr)(src), (LdsPtr)(lds_row_group), 16, 0, kDmaNontemporal);
}

__device__ inline int k_swizzle(int tok) { return (tok & 3) | ((tok >> 3) << 2); }

// Per-lane element offsets (from a page's start) of the K chunk this lane
// stages in row groups 2u and 2u + 1: token 4 it + row, chunk
// col ^ k_swizzle(4 it + row) = col ^ (row + 4 u).
struct KStageOffsets {
  int32_t off[4];
};

__device__ inline KStageOffsets k_stage_offsets(const PoolView& v, int g, const LaneGeom& lg) {
  KStageOffsets k;
#pragma unroll
  for (int u = 0; u < 4; ++u) k.off[u] = lg.row * v.token_elems + g * D + ((lg.col ^ (lg.row + 4 * u)) * 8);
  return k;
}

// Issue the page's K (swizzled) and V rows of head g into `stage` (a
// wave-uniform LDS address).  Rows at or past `valid` are not read.
__device__ inline void stage_page(const PoolView& v, int64_t page, int valid, const LaneGeom& lg,
                                  const KStageOffsets& ko, uint4* stage) {
  const uint16_t* pbase = v.pool + page * v.page_elems;
  const uint16_t* vbase = pbase + lg.head_off + lg.v_off;
  if (valid == kPageTokens) {
#pragma unroll
    for (int it = 0; it < kIters; ++it) dma16(pbase + ko.off[it >> 1] + it * lg.step4, stage + it * kWave);
#pragma unroll
    for (int it = 0; it < kIters; ++it) dma16(vbase + it * lg.step4, stage + (kIters + it) * kWave);
  } else {
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      if (it * kRows + lg.row < valid) {
        dma16(pbase + ko.off[it >> 1] + it * lg.step4, stage + it * kWave);
        dma16(vbase + it * lg.step4, stage + (kIters + it) * kWave);
      }
    }
  }
}

// The staging loads count on vmcnt and retire in issue order with the
// wave's other vector loads; the LDS reads of a page wait for all of them.
__device__ inline void wait_staged() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// The next page may overwrite the slot only once its reads have returned.
__device__ inline void wait_lds_reads() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ inline int64_t readlane64(int64_t x, int k) {
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(x), k);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(static_cast<uint64_t>(x) >> 32), k);
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Pages start, start + step, ... (< end) of a page list, for the staged
// walk: the lanes resolve 64 positions at a time; positions that resolve to
// no page (flagged) are skipped.
struct ListPages {
  const PoolView& v;
  int b;
  const PageList& L;
  int pos;
  int end;
  int step;
  int lane;
  PageRef batch{0, 0};  // lane l: position pos_batch + l * step
  int k = 0;
  int n = 0;

  __device__ inline PageRef next(bool) {
    for (;;) {
      if (k >= n) {
        if (pos >= end) return PageRef{0, 0};
        const int i = pos + lane * step;
        batch = i < end ? resolve_page(v, b, i, L) : PageRef{0, 0};
        n = min(kWave, (end - pos + step - 1) / step);
        pos += kWave * step;
        k = 0;
      }
      PageRef r;
      r.valid = __builtin_amdgcn_readlane(batch.valid, k);
      r.page = readlane64(batch.page, k);
      ++k;
      if (r.valid > 0) return r;
    }
  }
};

// Online-softmax state of one wave for the G query heads of a KV group.
template <int G>
struct WaveState {
  float qf[G][8];  // dims [8c, 8c+8) of each head, pre-scaled by scale*log2(e)
  float m[G];      // running max (log2 domain) of this lane's row
  float l[G];      // running denominator
  float acc[G][8];

  // q rows of the G heads of KV head g: query + (b*query_heads + g*G) * D.
  __device__ inline void init(const float* q_group, float qscale, int col) {
    load_q(q_group, qscale, col);
    reset();
  }

  __device__ inline void load_q(const float* q_group, float qscale, int col) {
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
    }
  }

  __device__ inline void reset() {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      m[h] = kNegInf;
      l[h] = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[h][j] = 0.0f;
    }
  }

  // Online-softmax update with NIT 4-token row groups: row groups it0,
  // it0 + it_step, ... of a page (the whole page when NIT == kIters).  Rows
  // at or past `valid` are masked.
  template <int NIT>
  __device__ inline void update(const uint4 (&kr)[NIT], const uint4 (&vr)[NIT], int valid, int row, int it0 = 0,
                                int it_step = 1) {
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
        if ((it0 + it * it_step) * kRows + row >= valid) s[h][it] = kNegInf;
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

  // This wave's share of a partial page spread over the W waves of a
  // workgroup: row groups wave, wave + W, ...  The last page of a list is
  // usually partial; spread, it costs each wave 1/W of a page instead of
  // costing one wave a whole page.
  template <int W>
  __device__ inline void attend_rows(const PoolView& v, const PageRef& pr, const LaneGeom& lg, int wave) {
    static_assert(kIters % W == 0, "row groups split evenly over the waves");
    constexpr int NIT = kIters / W;
    uint4 kr[NIT], vr[NIT];
    const uint16_t* kbase = v.pool + pr.page * v.page_elems + lg.head_off;
#pragma unroll
    for (int j = 0; j < NIT; ++j) {
      const int it = wave + j * W;
      if (it * kRows + lg.row < pr.valid) {
        kr[j] = load_stream16(kbase + it * lg.step4);
        vr[j] = load_stream16(kbase + it * lg.step4 + lg.v_off);
      } else {
        kr[j] = make_uint4(0, 0, 0, 0);
        vr[j] = make_uint4(0, 0, 0, 0);
      }
    }
    update<NIT>(kr, vr, pr.valid, lg.row, wave, W);
  }

  // ---- q.K on the matrix cores (G = 4, 8), P.V on the VALU, pages staged ---
  // S = K q^T per 16-token tile with v_mfma_f32_16x16x32_f16: A = 16 staged
  // K rows x 32 dims (FP16 as stored), B = 32 dims x 16 columns holding the
  // G heads' high FP16 halves (columns 0..G-1) and low halves q - high
  // (columns G..2G-1); one DPP add joins the two partial products.  Every
  // product of two FP16 values is exact in fp32 and high + low equals q to
  // 2^-22.  Each head's q is first scaled by a power of two into
  // [2^13, 2^14) (exact, undone on S) so that neither half overflows or
  // loses bits to FP16 subnormals.
  // Token order: in tile t, A row m is token 8 (m/4) + 4 t + m%4, so D row
  // 4 (l/16) + i of lane l is token 8 (l/16) + 4 t + i and lane l holds
  // tokens 8 (l/16) + 0..7 of head column l % 16.
  // The probabilities reach the P.V lane order through `pbuf`, this wave's
  // LDS scratch of G*32 + G floats ([head][row][row group], then the G
  // rescale factors).
  __device__ inline void attend_staged_mfma(const PoolView& v, int b, const PageList& L, int start, int end,
                                            int step, const LaneGeom& lg, int lane, int g, uint4* stage,
                                            float* pbuf, const float* q_group, float qscale) {
    ListPages src{v, b, L, start, end, step, lane};
    attend_staged(v, src, lg, lane, g, stage, pbuf, q_group, qscale);
  }

  // The staged walk over the pages a source hands out: src.next(wait)
  // returns the next page to attend (valid > 0), valid == 0 when the source
  // is exhausted, or (only with wait == false) valid < 0 when the next page
  // is not known yet.  One page is in flight while the previous one is
  // computed.
  template <class Src>
  __device__ inline void attend_staged(const PoolView& v, Src& src, const LaneGeom& lg, int lane, int g,
                                       uint4* stage, float* pbuf, const float* q_group, float qscale) {
    static_assert(G == 4 || G == 8, "G high and G low head columns fill the 16 MFMA columns");
    typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
    typedef float f32x4_t __attribute__((ext_vector_type(4)));
    const int kq = lane >> 4;   // MFMA k group / D row group
    const int col = lane & 15;  // MFMA head column
    const int hd = col % G;

    // B operand: power-of-two scaled q of head hd, split into FP16 halves
    f16x8_t qb[4];
    float sinv;
    {
      float x[4][8];
      float amax = 0.0f;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const float4* q4 = reinterpret_cast<const float4*>(q_group + hd * D + 32 * kk + 8 * kq);
        const float4 a = q4[0], c = q4[1];
        const float e[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          x[kk][j] = e[j] * qscale;
          amax = fmaxf(amax, fabsf(x[kk][j]));
        }
      }
      amax = fmaxf(amax, shfl_xor_f(amax, 16));
      amax = fmaxf(amax, shfl_xor_f(amax, 32));
      const int ex = static_cast<int>((__float_as_uint(amax) >> 23) & 0xff);
      const int sh = ex == 0 ? 0 : min(126, max(-126, 140 - ex));  // amax * 2^sh in [2^13, 2^14)
      const float scale = __uint_as_float(static_cast<uint32_t>(127 + sh) << 23);
      sinv = __uint_as_float(static_cast<uint32_t>(127 - sh) << 23);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float xs = x[kk][j] * scale;
          const _Float16 hi = static_cast<_Float16>(xs);
          const _Float16 lo = static_cast<_Float16>(xs - static_cast<float>(hi));
          qb[kk][j] = col < G ? hi : (col < 2 * G ? lo : static_cast<_Float16>(0.0f));
        }
      }
    }
    // staged-K read positions (uint4 index in the slot) of A rows in tile t
    int kidx[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int tok = 8 * (col >> 2) + 4 * t + (col & 3);
      const int f = k_swizzle(tok);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) kidx[t][kk] = tok * 16 + ((4 * kk + kq) ^ f);
    }
    const KStageOffsets ko = k_stage_offsets(v, g, lg);

    // continue from the state in m/l (register layout: every row holds the
    // running max, row r the denominator share of row group r)
    float m_lane = m[0];  // running max of head column col (same in all 4 row groups)
    float l_lane = l[0];  // this lane's share of the denominator (its 8 tokens per page)
#pragma unroll
    for (int h = 1; h < G; ++h) {
      if (hd == h) {
        m_lane = m[h];
        l_lane = l[h];
      }
    }
    PageRef cur = src.next(true);
    if (cur.valid > 0) stage_page(v, cur.page, cur.valid, lg, ko, stage);
    while (cur.valid > 0) {
      const int valid = cur.valid;
      uint4 ka[2][4], vr[kIters];
      wait_staged();
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) ka[t][kk] = stage[kidx[t][kk]];
      }
#pragma unroll
      for (int it = 0; it < kIters; ++it) vr[it] = stage[(kIters + it) * kWave + lane];
      wait_lds_reads();
      PageRef nxt = src.next(false);
      if (nxt.valid > 0) stage_page(v, nxt.page, nxt.valid, lg, ko, stage);

      // S for this lane's 8 tokens 8 kq + 4 t + i (log2 domain)
      f32x4_t s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, ka[0][kk]), qb[kk], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, ka[1][kk]), qb[kk], s1, 0, 0, 0);
      }
      float sv[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sv[r] = (s0[r] + dpp_f<0x100 + G>(s0[r])) * sinv;  // row_shl:G: the low-half column
        sv[4 + r] = (s1[r] + dpp_f<0x100 + G>(s1[r])) * sinv;
      }
      if (valid < kPageTokens) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (8 * kq + 4 * (e >> 2) + (e & 3) >= valid) sv[e] = kNegInf;
        }
      }
      float pmax = kNegInf;
#pragma unroll
      for (int e = 0; e < 8; ++e) pmax = fmaxf(pmax, sv[e]);
      pmax = fmaxf(pmax, shfl_xor_f(pmax, 16));
      pmax = fmaxf(pmax, shfl_xor_f(pmax, 32));
      const float mn = fmaxf(m_lane, pmax);
      const float corr = (m_lane == mn) ? 1.0f : __builtin_amdgcn_exp2f(m_lane - mn);
      const float base_m = (mn == kNegInf) ? 0.0f : mn;
      m_lane = mn;
      float lsum = l_lane * corr;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sv[e] = __builtin_amdgcn_exp2f(sv[e] - base_m);
        lsum += sv[e];
      }
      l_lane = lsum;
      // probabilities to the P.V order: token 8 kq + 4 t + r is row r of
      // row group 2 kq + t
      if (col < G) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          *reinterpret_cast<float2*>(pbuf + (col * 4 + r) * kIters + 2 * kq) = make_float2(sv[r], sv[4 + r]);
      }
      // the wave's LDS operations complete in issue order: the reads below
      // see the writes above
      __builtin_amdgcn_wave_barrier();
      float p[G][kIters];
      float cr[G];
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float4 a = *reinterpret_cast<const float4*>(pbuf + (h * 4 + lg.row) * kIters);
        const float4 c = *reinterpret_cast<const float4*>(pbuf + (h * 4 + lg.row) * kIters + 4);
        p[h][0] = a.x; p[h][1] = a.y; p[h][2] = a.z; p[h][3] = a.w;
        p[h][4] = c.x; p[h][5] = c.y; p[h][6] = c.z; p[h][7] = c.w;
      }
      // head h's rescale factor is the one lane h (column h) computed
#pragma unroll
      for (int h = 0; h < G; ++h)
        cr[h] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, corr), h));
      __builtin_amdgcn_wave_barrier();
      if (valid < kPageTokens) {
        // rows past the tail were not staged: their slot holds stale bytes
#pragma unroll
        for (int it = 0; it < kIters; ++it) {
          if (it * kRows + lg.row >= valid) vr[it] = make_uint4(0, 0, 0, 0);
        }
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[h][j] *= cr[h];
      }
      // P.V, each V half converted at its use (v_fma_mix_f32)
#pragma unroll
      for (int it = 0; it < kIters; ++it) {
        const uint32_t w[4] = {vr[it].x, vr[it].y, vr[it].z, vr[it].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float vj = (j & 1) ? hi_h2f(w[j >> 1]) : lo_h2f(w[j >> 1]);
#pragma unroll
          for (int h = 0; h < G; ++h) acc[h][j] = __builtin_fmaf(p[h][it], vj, acc[h][j]);
        }
      }
      if (nxt.valid < 0) {
        nxt = src.next(true);
        if (nxt.valid > 0) stage_page(v, nxt.page, nxt.valid, lg, ko, stage);
      }
      cur = nxt;
    }
    // hand the statistics to the register layout: every row keeps the same
    // max; row r takes the denominator share of row group r, so that
    // reduce_rows() sums the four shares
#pragma unroll
    for (int h = 0; h < G; ++h) {
      m[h] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m_lane), h));
      l[h] = __shfl(l_lane, (lane & 48) | h, kWave);
    }
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

// The same combination without the cross-row shuffles of reduce_rows(): every
// lane publishes its own row's share (two 16-byte LDS writes per head) and
// the combine adds the kRows shares of each wave.  For the staged walk, whose
// rows all keep the same running max; 4x the LDS of CombineSmem.
template <int G, int W>
struct CombineRowsSmem {
  float m[W][G];
  float l[W][kRows][G];
  float acc[W][kRows][G][D];
};

template <int G, int W>
__device__ inline void publish_wave_rows(const WaveState<G>& st, CombineRowsSmem<G, W>& cs, int wave, int row,
                                         int col) {
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float4* dst = reinterpret_cast<float4*>(&cs.acc[wave][row][h][col * 8]);
    dst[0] = make_float4(st.acc[h][0], st.acc[h][1], st.acc[h][2], st.acc[h][3]);
    dst[1] = make_float4(st.acc[h][4], st.acc[h][5], st.acc[h][6], st.acc[h][7]);
  }
  if (col == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      cs.l[wave][row][h] = st.l[h];
      if (row == 0) cs.m[wave][h] = st.m[h];
    }
  }
}

template <int G, int W>
__device__ inline void combine_element_rows(const CombineRowsSmem<G, W>& cs, int h, int d, float& mx, float& lw,
                                            float& aw) {
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
      float lr = 0.0f, ar = 0.0f;
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        lr += cs.l[w][r][h];
        ar += cs.acc[w][r][h][d];
      }
      lw = __builtin_fmaf(lr, f, lw);
      aw = __builtin_fmaf(ar, f, aw);
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
