// attention_any.hip — attention of one query token over a contiguous
// token-major K/V buffer for head dimensions other than 128 (gfx950): any
// multiple of 8 up to 512, 1, 2, 4 or 8 query heads per KV head.  Semantics
// of the reference's attention_reference (cpp/src/attention_reference.cpp
// :55-96): per query head h of KV head g = h / group, logits q_h . K_t *
// scale over every token, softmax, and the weighted sum of V_t; the buffer
// is [tokens][K: kv_heads x head_dim][V: kv_heads x head_dim] FP16
// (backend.hpp:18-31).  The head_dim = 128 path is the paged attention
// kernel in contiguous mode (attention.hip); this one serves the others.
//
// Grid (kv_heads, splits): a workgroup takes one KV head's query heads over
// one contiguous token range.  Its 4 waves take 64-token tiles in turn:
//   * scores: lane = token; the lane reads its token's K row in 16-byte
//     pieces (eight in flight) against the query heads held in LDS;
//   * online softmax per head over the tile (log2 domain, wave reductions);
//   * P.V: lanes over d (two values of d per 4-byte load, 256 d per
//     instruction), 16 tokens' loads in flight (8 or 4 at 4 or 8 query heads
//     per KV head), the tile's probabilities
//     read back from LDS.
// The waves' states combine in LDS; with several splits each workgroup
// writes (max, denominator, accumulator) per head and a merge kernel adds
// the splits in split order (deterministic).
#include <algorithm>

#include "attn_rows.hpp"
#include "sa_device.hpp"
#include "sa_internal.hpp"

namespace sa {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxD = kAnyMaxHeadDim;
constexpr int kPairs = kMaxD / (2 * kWave);  // 4-byte V loads per lane per token
constexpr int kTile = kWave;                // tokens per wave tile
// P.V tokens whose V loads are in flight together: each lane's pieces are
// 4 bytes, so with 4 tokens a wave kept ~0.5 KiB in flight at head_dim 64
// and the walk was bound by load latency.  Fewer at 4 and 8 query heads per
// KV head, whose accumulators take the registers.
template <int G>
constexpr int pv_tokens() {
  return G <= 2 ? 16 : (G == 4 ? 8 : 4);
}
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

struct AnyParams {
  const uint16_t* kv;
  const float* query;
  float* out;
  float* part;  // [kv_heads][splits][group][head_dim + 2]: max, denominator, accumulator
  int64_t tokens;
  int64_t chunk;  // tokens per split
  int32_t kv_heads;
  int32_t head_dim;
  int32_t splits;
  float scale;
};

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

template <int G>
__global__ __launch_bounds__(kThreads) void attention_any_kernel(const AnyParams p) {
  __shared__ float q_s[G * kMaxD];
  __shared__ float p_s[kWaves][G][kTile];
  __shared__ float w_ml[kWaves][G][2];
  __shared__ float w_acc[kWaves][G][kMaxD];
  const int g = blockIdx.x;
  const int s = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int D = p.head_dim;
  const int64_t t_begin = static_cast<int64_t>(s) * p.chunk;
  const int64_t t_end = std::min<int64_t>(p.tokens, t_begin + p.chunk);
  const int64_t tok_elems = 2LL * p.kv_heads * D;
  const uint16_t* kbase = p.kv + static_cast<int64_t>(g) * D;
  const uint16_t* vbase = p.kv + static_cast<int64_t>(p.kv_heads + g) * D;
  const float* q = p.query + static_cast<int64_t>(g) * G * D;
  for (int i = tid; i < G * D; i += kThreads) q_s[(i / D) * kMaxD + i % D] = q[i];
  __syncthreads();

  const float sl2 = p.scale * kLog2e;
  float m[G], l[G], acc[G][2 * kPairs];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = kNegInf;
    l[h] = 0.0f;
#pragma unroll
    for (int j = 0; j < 2 * kPairs; ++j) acc[h][j] = 0.0f;
  }

  for (int64_t t0 = t_begin + static_cast<int64_t>(wave) * kTile; t0 < t_end; t0 += kWaves * kTile) {
    // scores of the tile's tokens, lane = token
    const int64_t t = t0 + lane;
    const bool valid = t < t_end;
    float sc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) sc[h] = 0.0f;
    if (valid) {
      const uint16_t* k = kbase + t * tok_elems;
      for (int d0 = 0; d0 < D; d0 += 64) {
        uint4 w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (d0 + 8 * u < D) w[u] = *reinterpret_cast<const uint4*>(k + d0 + 8 * u);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (d0 + 8 * u >= D) break;
          const uint32_t ww[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float kf = (e & 1) ? hi_h2f(ww[e >> 1]) : lo_h2f(ww[e >> 1]);
#pragma unroll
            for (int h = 0; h < G; ++h) sc[h] = __builtin_fmaf(q_s[h * kMaxD + d0 + 8 * u + e], kf, sc[h]);
          }
        }
      }
    }
    // online softmax per head over the tile
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float x = valid ? sc[h] * sl2 : kNegInf;
      const float mn = fmaxf(m[h], wave_max(x));
      const float corr = __builtin_amdgcn_exp2f(m[h] - mn);  // 0 while m is -inf
      const float pt = valid ? __builtin_amdgcn_exp2f(x - mn) : 0.0f;
      l[h] = l[h] * corr + wave_sum(pt);
      m[h] = mn;
#pragma unroll
      for (int j = 0; j < 2 * kPairs; ++j) acc[h][j] *= corr;
      p_s[wave][h][lane] = pt;
    }
    __builtin_amdgcn_wave_barrier();  // the wave's LDS writes precede its reads below
    // P.V: lane holds d = 2 (lane + 64 j) + {0, 1}
    const int n = static_cast<int>(std::min<int64_t>(kTile, t_end - t0));
    constexpr int kPvTokens = pv_tokens<G>();
    for (int i0 = 0; i0 < n; i0 += kPvTokens) {
      uint32_t vw[kPvTokens][kPairs];
#pragma unroll
      for (int i = 0; i < kPvTokens; ++i) {
        const uint16_t* v = vbase + (t0 + i0 + i) * tok_elems;
#pragma unroll
        for (int j = 0; j < kPairs; ++j) {
          const int d = 2 * (lane + kWave * j);
          vw[i][j] = 0u;
          if (i0 + i < n && d < D) vw[i][j] = *reinterpret_cast<const uint32_t*>(v + d);
        }
      }
#pragma unroll
      for (int i = 0; i < kPvTokens; ++i) {
        if (i0 + i >= n) break;
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const float pv = p_s[wave][h][i0 + i];
#pragma unroll
          for (int j = 0; j < kPairs; ++j) {
            acc[h][2 * j] = __builtin_fmaf(pv, lo_h2f(vw[i][j]), acc[h][2 * j]);
            acc[h][2 * j + 1] = __builtin_fmaf(pv, hi_h2f(vw[i][j]), acc[h][2 * j + 1]);
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // the tile's reads of p_s precede the next tile's writes
  }

  // combine the waves
#pragma unroll
  for (int h = 0; h < G; ++h) {
    if (lane == 0) {
      w_ml[wave][h][0] = m[h];
      w_ml[wave][h][1] = l[h];
    }
#pragma unroll
    for (int j = 0; j < kPairs; ++j) {
      const int d = 2 * (lane + kWave * j);
      if (d < D) {
        w_acc[wave][h][d] = acc[h][2 * j];
        w_acc[wave][h][d + 1] = acc[h][2 * j + 1];
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += kThreads) {
    const int h = i / D;
    const int d = i % D;
    float mx = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, w_ml[w][h][0]);
    float lw = 0.0f, aw = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = __builtin_amdgcn_exp2f(w_ml[w][h][0] - mx);  // waves without tokens: 0
      lw += w_ml[w][h][1] * f;
      aw += w_acc[w][h][d] * f;
    }
    if (p.splits == 1) {
      p.out[(static_cast<int64_t>(g) * G + h) * D + d] = lw > 0.0f ? aw / lw : 0.0f;
    } else {
      float* rec = p.part + ((static_cast<int64_t>(g) * p.splits + s) * G + h) * (D + 2);
      if (d == 0) {
        rec[0] = mx;
        rec[1] = lw;
      }
      rec[2 + d] = aw;
    }
  }
}

// out[h][d] from the splits' records of head h, added in split order.
__global__ __launch_bounds__(kThreads) void attention_any_merge_kernel(const AnyParams p, int group) {
  const int hq = blockIdx.x;
  const int g = hq / group;
  const int hh = hq % group;
  const int D = p.head_dim;
  const int64_t rec_stride = static_cast<int64_t>(group) * (D + 2);
  const float* first = p.part + (static_cast<int64_t>(g) * p.splits * group + hh) * (D + 2);
  float mx = kNegInf;
  for (int s = 0; s < p.splits; ++s) mx = fmaxf(mx, first[s * rec_stride]);
  for (int d = threadIdx.x; d < D; d += kThreads) {
    float lw = 0.0f, aw = 0.0f;
    for (int s = 0; s < p.splits; ++s) {
      const float* rec = first + s * rec_stride;
      const float f = __builtin_amdgcn_exp2f(rec[0] - mx);
      lw += rec[1] * f;
      aw += rec[2 + d] * f;
    }
    p.out[static_cast<int64_t>(hq) * D + d] = lw > 0.0f ? aw / lw : 0.0f;
  }
}

// ---- the paged form ------------------------------------------------------------
// Attention of sequence b's query heads of KV head g over the tokens of its
// list: the selected sealed blocks of g's selection group in list order,
// then every tail token (blocks sealed .. ceil(seq_len / 32) - 1), as the
// paged attention kernel (attention.hip) and the reference's
// attention_reference over the packed tokens (attention_reference.cpp
// :55-96).  Grid (kv_heads, splits, batch): split s takes a contiguous range
// of the list's token positions; position q is token q % 32 of the list's
// page q / 32.  A lane resolves its token's page (block id and table entry
// checked, out-of-range ones flagged in status and skipped) and keeps the
// row's element offset in LDS for the P.V loop, which skips invalid tokens.
// The tile arithmetic is attention_any_kernel's; records hold (max,
// denominator) then, after kPartPad floats, the accumulator.
struct PagedAnyParams {
  const uint16_t* pool;
  const int32_t* table;
  const int32_t* seq_len;
  const int32_t* sealed;
  const int32_t* selected;
  const int32_t* counts;
  const float* query;
  float* out;
  float* part;  // [batch][kv_heads][splits][group][part_stride(head_dim)]
  int32_t* status;
  int64_t num_pages;
  int32_t table_stride;
  int32_t sel_stride;
  int32_t select_groups;
  int32_t query_heads;
  int32_t kv_heads;
  int32_t head_dim;
  int32_t splits;
  float scale;
};

// Element offset of position q's K row in the pool (its KV head's slice
// added by the caller), or -1 when the token does not exist or its page is
// invalid.
__device__ inline int64_t paged_token(const PagedAnyParams& p, int b, const int32_t* sel, int n_sel, int sealed,
                                      int64_t len, int64_t q, int64_t tok_elems) {
  const int i = static_cast<int>(q / kPageTokens);
  const int t = static_cast<int>(q % kPageTokens);
  int64_t logical;
  if (i < n_sel) {
    logical = sel[i];
    if (logical < 0 || logical >= sealed) {
      flag_status(p.status, kStatusBadBlock);
      return -1;
    }
  } else {
    logical = static_cast<int64_t>(sealed) + (i - n_sel);
    if (logical * kPageTokens + t >= len) return -1;
  }
  if (logical >= p.table_stride) {
    flag_status(p.status, kStatusBadBlock);
    return -1;
  }
  const int64_t page = p.table[static_cast<int64_t>(b) * p.table_stride + logical];
  if (page < 0 || page >= p.num_pages) {
    flag_status(p.status, kStatusBadPage);
    return -1;
  }
  return (page * kPageTokens + t) * tok_elems;
}

template <int G>
__global__ __launch_bounds__(kThreads) void paged_any_kernel(const PagedAnyParams p) {
  __shared__ float q_s[G * kMaxD];
  __shared__ float p_s[kWaves][G][kTile];
  __shared__ int64_t off_s[kWaves][kTile];
  __shared__ float w_ml[kWaves][G][2];
  __shared__ float w_acc[kWaves][G][kMaxD];
  const int g = blockIdx.x;
  const int s = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int D = p.head_dim;
  const int sg = g / (p.kv_heads / p.select_groups);
  const int64_t list = static_cast<int64_t>(b) * p.select_groups + sg;
  const int32_t* sel = p.selected + list * p.sel_stride;
  int n_sel = p.counts[list];
  n_sel = n_sel < 0 ? 0 : (n_sel > p.sel_stride ? p.sel_stride : n_sel);
  const int64_t len = p.seq_len[b];
  const int sealed = p.sealed[b];
  const int64_t tail_tokens = len - static_cast<int64_t>(sealed) * kPageTokens;
  const int64_t tail_pages = tail_tokens > 0 ? (tail_tokens + kPageTokens - 1) / kPageTokens : 0;
  const int64_t positions = (n_sel + tail_pages) * kPageTokens;
  const int64_t chunk = (positions + p.splits - 1) / p.splits;
  const int64_t q_begin = static_cast<int64_t>(s) * chunk;
  const int64_t q_end = std::min<int64_t>(positions, q_begin + chunk);
  const int64_t tok_elems = 2LL * p.kv_heads * D;
  const uint16_t* kbase = p.pool + static_cast<int64_t>(g) * D;
  const uint16_t* vbase = p.pool + static_cast<int64_t>(p.kv_heads + g) * D;
  const float* q = p.query + (static_cast<int64_t>(b) * p.query_heads + static_cast<int64_t>(g) * G) * D;
  for (int i = tid; i < G * D; i += kThreads) q_s[(i / D) * kMaxD + i % D] = q[i];
  __syncthreads();

  const float sl2 = p.scale * kLog2e;
  float m[G], l[G], acc[G][2 * kPairs];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = kNegInf;
    l[h] = 0.0f;
#pragma unroll
    for (int j = 0; j < 2 * kPairs; ++j) acc[h][j] = 0.0f;
  }

  for (int64_t t0 = q_begin + static_cast<int64_t>(wave) * kTile; t0 < q_end; t0 += kWaves * kTile) {
    const int64_t t = t0 + lane;
    const int64_t off = t < q_end ? paged_token(p, b, sel, n_sel, sealed, len, t, tok_elems) : -1;
    const bool valid = off >= 0;
    off_s[wave][lane] = off;
    float sc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) sc[h] = 0.0f;
    if (valid) {
      const uint16_t* k = kbase + off;
      for (int d0 = 0; d0 < D; d0 += 64) {
        uint4 w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (d0 + 8 * u < D) w[u] = *reinterpret_cast<const uint4*>(k + d0 + 8 * u);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (d0 + 8 * u >= D) break;
          const uint32_t ww[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float kf = (e & 1) ? hi_h2f(ww[e >> 1]) : lo_h2f(ww[e >> 1]);
#pragma unroll
            for (int h = 0; h < G; ++h) sc[h] = __builtin_fmaf(q_s[h * kMaxD + d0 + 8 * u + e], kf, sc[h]);
          }
        }
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float x = valid ? sc[h] * sl2 : kNegInf;
      const float mn = fmaxf(m[h], wave_max(x));
      // a tile with no valid token leaves the state as it is (m stays -inf
      // until the first valid token: exp2(-inf - -inf) would be NaN)
      const float corr = mn == kNegInf ? 1.0f : __builtin_amdgcn_exp2f(m[h] - mn);
      const float pt = valid ? __builtin_amdgcn_exp2f(x - mn) : 0.0f;
      l[h] = l[h] * corr + wave_sum(pt);
      m[h] = mn;
#pragma unroll
      for (int j = 0; j < 2 * kPairs; ++j) acc[h][j] *= corr;
      p_s[wave][h][lane] = pt;
    }
    __builtin_amdgcn_wave_barrier();  // the wave's LDS writes precede its reads below
    const int n = static_cast<int>(std::min<int64_t>(kTile, q_end - t0));
    constexpr int kPvTokens = pv_tokens<G>();
    for (int i0 = 0; i0 < n; i0 += kPvTokens) {
      uint32_t vw[kPvTokens][kPairs];
#pragma unroll
      for (int i = 0; i < kPvTokens; ++i) {
        const int64_t o = i0 + i < n ? off_s[wave][i0 + i] : -1;
#pragma unroll
        for (int j = 0; j < kPairs; ++j) {
          const int d = 2 * (lane + kWave * j);
          vw[i][j] = 0u;
          if (o >= 0 && d < D) vw[i][j] = *reinterpret_cast<const uint32_t*>(vbase + o + d);
        }
      }
#pragma unroll
      for (int i = 0; i < kPvTokens; ++i) {
        if (i0 + i >= n) break;
        if (off_s[wave][i0 + i] < 0) continue;  // uniform: a token that does not exist adds nothing
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const float pv = p_s[wave][h][i0 + i];
#pragma unroll
          for (int j = 0; j < kPairs; ++j) {
            acc[h][2 * j] = __builtin_fmaf(pv, lo_h2f(vw[i][j]), acc[h][2 * j]);
            acc[h][2 * j + 1] = __builtin_fmaf(pv, hi_h2f(vw[i][j]), acc[h][2 * j + 1]);
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // the tile's reads of p_s / off_s precede the next tile's writes
  }

#pragma unroll
  for (int h = 0; h < G; ++h) {
    if (lane == 0) {
      w_ml[wave][h][0] = m[h];
      w_ml[wave][h][1] = l[h];
    }
#pragma unroll
    for (int j = 0; j < kPairs; ++j) {
      const int d = 2 * (lane + kWave * j);
      if (d < D) {
        w_acc[wave][h][d] = acc[h][2 * j];
        w_acc[wave][h][d + 1] = acc[h][2 * j + 1];
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += kThreads) {
    const int h = i / D;
    const int d = i % D;
    float mx = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, w_ml[w][h][0]);
    float lw = 0.0f, aw = 0.0f;
    if (mx != kNegInf) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float f = __builtin_amdgcn_exp2f(w_ml[w][h][0] - mx);  // waves without tokens: 0
        lw += w_ml[w][h][1] * f;
        aw += w_acc[w][h][d] * f;
      }
    }
    const int64_t hq = static_cast<int64_t>(b) * p.query_heads + static_cast<int64_t>(g) * G + h;
    if (p.splits == 1) {
      p.out[hq * D + d] = lw > 0.0f ? aw / lw : 0.0f;
    } else {
      float* rec = p.part + (((static_cast<int64_t>(b) * p.kv_heads + g) * p.splits + s) * G + h) * part_stride(D);
      if (d == 0) {
        rec[0] = mx;
        rec[1] = lw;
      }
      rec[kPartPad + d] = aw;
    }
  }
}

// ---- the paged form in token rows (head_dim up to 256) --------------------------
// The token-row walk of attn_rows.hpp over the list of (sequence b, KV head
// g).  Grid (kv_heads, splits, batch); split s takes a contiguous range of
// the list's pages (selected blocks, then the tail), its 4 waves every 4th
// unit (a page, or half a page at 32 lanes per row); the waves combine in
// LDS into the output or the split's record (the records and the merge of
// paged_any_kernel).
constexpr int kRowsWaves = 4;
constexpr int kRowsThreads = kRowsWaves * kWave;

// Tokens of page i of the list (selected blocks, then the tail) and its pool
// page; 0 when the page does not exist or is invalid (flagged as by
// paged_token()).
__device__ inline int list_page(const PagedAnyParams& p, int b, const int32_t* sel, int n_sel, int sealed,
                                int64_t len, int i, int64_t& page) {
  int64_t logical;
  int valid = kPageTokens;
  if (i < n_sel) {
    logical = sel[i];
    if (logical < 0 || logical >= sealed) {
      flag_status(p.status, kStatusBadBlock);
      return 0;
    }
  } else {
    logical = static_cast<int64_t>(sealed) + (i - n_sel);
    const int64_t left = len - logical * kPageTokens;
    if (left <= 0) return 0;
    valid = left < kPageTokens ? static_cast<int>(left) : kPageTokens;
  }
  if (logical >= p.table_stride) {
    flag_status(p.status, kStatusBadBlock);
    return 0;
  }
  page = p.table[static_cast<int64_t>(b) * p.table_stride + logical];
  if (page < 0 || page >= p.num_pages) {
    flag_status(p.status, kStatusBadPage);
    return 0;
  }
  return valid;
}

template <int G, int LPR>
__global__ __launch_bounds__(kRowsThreads) void paged_rows_kernel(const PagedAnyParams p) {
  using State = rows::RowsState<G, LPR>;
  __shared__ float w_ml[kRowsWaves][G][2];
  __shared__ float w_acc[kRowsWaves][G][LPR * 8];
  const int g = blockIdx.x;
  const int s = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int D = p.head_dim;
  const int sg = g / (p.kv_heads / p.select_groups);
  const int64_t list = static_cast<int64_t>(b) * p.select_groups + sg;
  const int32_t* sel = p.selected + list * p.sel_stride;
  int n_sel = p.counts[list];
  n_sel = n_sel < 0 ? 0 : (n_sel > p.sel_stride ? p.sel_stride : n_sel);
  const int64_t len = p.seq_len[b];
  const int sealed = p.sealed[b];
  const int64_t tail_tokens = len - static_cast<int64_t>(sealed) * kPageTokens;
  const int tail_pages = tail_tokens > 0 ? static_cast<int>((tail_tokens + kPageTokens - 1) / kPageTokens) : 0;
  const int total = n_sel + tail_pages;
  const int chunk = (total + p.splits - 1) / p.splits;
  const int i_begin = s * chunk;
  const int i_end = total < i_begin + chunk ? total : i_begin + chunk;

  State st;
  st.init(p.query + (static_cast<int64_t>(b) * p.query_heads + static_cast<int64_t>(g) * G) * D, D,
          p.scale * kLog2e, lane);
  const int64_t tok_elems = 2LL * p.kv_heads * D;
  const int64_t page_elems = kPageTokens * tok_elems;
  const int64_t lane_off = st.lane_offset(tok_elems, g, D);
  const int64_t v_off = static_cast<int64_t>(p.kv_heads) * D;
  for (int u = i_begin * State::kParts + wave; u < i_end * State::kParts; u += kRowsWaves) {
    const int i = u / State::kParts;
    const int part = u % State::kParts;
    int64_t page = 0;
    const int valid = list_page(p, b, sel, n_sel, sealed, len, i, page);
    if (valid <= part * State::NIT * State::kR) continue;  // no page, or no token in this unit
    st.attend_unit(p.pool + page * page_elems + lane_off, tok_elems, v_off, valid, part);
  }

  // the wave's rows added, then the waves combined
  st.finish();
#pragma unroll
  for (int h = 0; h < G; ++h) {
    if (lane == 0) {
      w_ml[wave][h][0] = st.m[h];
      w_ml[wave][h][1] = st.l[h];
    }
    if (st.row == 0 && st.dims) {
#pragma unroll
      for (int j = 0; j < 8; ++j) w_acc[wave][h][st.col * 8 + j] = st.acc[h][j];
    }
  }
  __syncthreads();
  for (int e = tid; e < G * D; e += kRowsThreads) {
    const int h = e / D;
    const int d = e % D;
    float mx = kNegInf;
#pragma unroll
    for (int w = 0; w < kRowsWaves; ++w) mx = fmaxf(mx, w_ml[w][h][0]);
    float lw = 0.0f, aw = 0.0f;
    if (mx != kNegInf) {
#pragma unroll
      for (int w = 0; w < kRowsWaves; ++w) {
        const float f = __builtin_amdgcn_exp2f(w_ml[w][h][0] - mx);  // waves without tokens: 0
        lw += w_ml[w][h][1] * f;
        aw += w_acc[w][h][d] * f;
      }
    }
    const int64_t hq = static_cast<int64_t>(b) * p.query_heads + static_cast<int64_t>(g) * G + h;
    if (p.splits == 1) {
      p.out[hq * D + d] = lw > 0.0f ? aw / lw : 0.0f;
    } else {
      float* rec = p.part + (((static_cast<int64_t>(b) * p.kv_heads + g) * p.splits + s) * G + h) * part_stride(D);
      if (d == 0) {
        rec[0] = mx;
        rec[1] = lw;
      }
      rec[kPartPad + d] = aw;
    }
  }
}

// out[b][hq][d] from the splits' records of (b, hq), added in split order.
__global__ __launch_bounds__(kThreads) void paged_any_merge_kernel(const PagedAnyParams p) {
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int group = p.query_heads / p.kv_heads;
  const int g = hq / group;
  const int hh = hq % group;
  const int D = p.head_dim;
  const int64_t rec_stride = static_cast<int64_t>(group) * part_stride(D);
  const float* first =
      p.part + ((static_cast<int64_t>(b) * p.kv_heads + g) * p.splits * group + hh) * part_stride(D);
  float mx = kNegInf;
  for (int s = 0; s < p.splits; ++s) mx = fmaxf(mx, first[s * rec_stride]);
  for (int d = threadIdx.x; d < D; d += kThreads) {
    float lw = 0.0f, aw = 0.0f;
    if (mx != kNegInf) {
      for (int s = 0; s < p.splits; ++s) {
        const float* rec = first + s * rec_stride;
        const float f = __builtin_amdgcn_exp2f(rec[0] - mx);
        lw += rec[1] * f;
        aw += rec[kPartPad + d] * f;
      }
    }
    p.out[(static_cast<int64_t>(b) * p.query_heads + hq) * D + d] = lw > 0.0f ? aw / lw : 0.0f;
  }
}

// head_dim the row layout takes (32 lanes x 8 dimensions); larger ones run
// paged_any_kernel.
constexpr int kMaxRowsHeadDim = rows::kMaxHeadDim;

template <int LPR>
hipError_t launch_rows(const PagedAnyParams& p, int group, dim3 grid, hipStream_t stream) {
  switch (group) {
    case 1: hipLaunchKernelGGL((paged_rows_kernel<1, LPR>), grid, dim3(kRowsThreads), 0, stream, p); break;
    case 2: hipLaunchKernelGGL((paged_rows_kernel<2, LPR>), grid, dim3(kRowsThreads), 0, stream, p); break;
    case 4: hipLaunchKernelGGL((paged_rows_kernel<4, LPR>), grid, dim3(kRowsThreads), 0, stream, p); break;
    default: hipLaunchKernelGGL((paged_rows_kernel<8, LPR>), grid, dim3(kRowsThreads), 0, stream, p); break;
  }
  return hipGetLastError();
}

// Splits that give every compute unit about two workgroups, each with at
// least 256 tokens (four tiles per wave), and no empty split.
void any_split(int64_t tokens, int32_t kv_heads, int32_t& splits, int64_t& chunk) {
  const int64_t want = std::max<int64_t>(1, 2LL * compute_units() / std::max(kv_heads, 1));
  const int64_t most = std::max<int64_t>(1, tokens / 256);
  int64_t n = std::min<int64_t>(std::min(want, most), 1024);
  chunk = (tokens + n - 1) / n;
  n = (tokens + chunk - 1) / chunk;
  splits = static_cast<int32_t>(n);
}

}  // namespace

bool attention_any_supported(int32_t query_heads, int32_t kv_heads, int32_t head_dim) {
  if (kv_heads <= 0 || query_heads <= 0 || query_heads % kv_heads != 0) return false;
  const int group = query_heads / kv_heads;
  return (group == 1 || group == 2 || group == 4 || group == 8) && head_dim > 0 && head_dim % 8 == 0 &&
         head_dim <= kAnyMaxHeadDim;
}

size_t attention_any_workspace_bytes(int64_t tokens, int32_t query_heads, int32_t kv_heads, int32_t head_dim) {
  if (tokens <= 0 || !attention_any_supported(query_heads, kv_heads, head_dim)) return 0;
  int32_t splits = 1;
  int64_t chunk = tokens;
  any_split(tokens, kv_heads, splits, chunk);
  if (splits == 1) return 0;
  return static_cast<size_t>(kv_heads) * splits * (query_heads / kv_heads) * (head_dim + 2) * sizeof(float);
}

hipError_t launch_paged_attention_any(const AttnLaunch& a, hipStream_t stream) {
  if (a.mode != 0 || a.chunk_pages != 0 || a.contig_tokens > 0 ||
      !attention_any_supported(a.query_heads, a.kv_heads, a.head_dim))
    return hipErrorInvalidValue;
  PagedAnyParams p{};
  p.pool = a.pool;
  p.table = a.table;
  p.seq_len = a.seq_len;
  p.sealed = a.sealed;
  p.selected = a.selected;
  p.counts = a.counts;
  p.query = a.query;
  p.out = a.out;
  p.part = a.part;
  p.status = a.status;
  p.num_pages = a.num_pages;
  p.table_stride = a.table_stride;
  p.sel_stride = a.sel_stride;
  p.select_groups = a.select_groups;
  p.query_heads = a.query_heads;
  p.kv_heads = a.kv_heads;
  p.head_dim = a.head_dim;
  p.splits = a.splits;
  p.scale = a.scale;
  const int group = a.query_heads / a.kv_heads;
  const dim3 grid(a.kv_heads, a.splits, a.batch);
  if (a.head_dim <= kMaxRowsHeadDim) {
    const int lpr = rows::lanes_per_row(a.head_dim);
    hipError_t e = hipSuccess;
    switch (lpr) {
      case 8: e = launch_rows<8>(p, group, grid, stream); break;
      case 16: e = launch_rows<16>(p, group, grid, stream); break;
      default: e = launch_rows<32>(p, group, grid, stream); break;
    }
    if (e != hipSuccess || p.splits == 1) return e;
    hipLaunchKernelGGL(paged_any_merge_kernel, dim3(a.query_heads, a.batch), dim3(kThreads), 0, stream, p);
    return hipGetLastError();
  }
  switch (group) {
    case 1: hipLaunchKernelGGL(paged_any_kernel<1>, grid, dim3(kThreads), 0, stream, p); break;
    case 2: hipLaunchKernelGGL(paged_any_kernel<2>, grid, dim3(kThreads), 0, stream, p); break;
    case 4: hipLaunchKernelGGL(paged_any_kernel<4>, grid, dim3(kThreads), 0, stream, p); break;
    default: hipLaunchKernelGGL(paged_any_kernel<8>, grid, dim3(kThreads), 0, stream, p); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.splits == 1) return e;
  hipLaunchKernelGGL(paged_any_merge_kernel, dim3(a.query_heads, a.batch), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_attention_any(const uint16_t* kv, const float* query, int64_t tokens, int32_t query_heads,
                                int32_t kv_heads, int32_t head_dim, float scale, float* out, void* workspace,
                                hipStream_t stream) {
  AnyParams p{};
  p.kv = kv;
  p.query = query;
  p.out = out;
  p.part = static_cast<float*>(workspace);
  p.tokens = tokens;
  p.kv_heads = kv_heads;
  p.head_dim = head_dim;
  p.scale = scale;
  any_split(tokens, kv_heads, p.splits, p.chunk);
  const int group = query_heads / kv_heads;
  const dim3 grid(kv_heads, p.splits);
  switch (group) {
    case 1: hipLaunchKernelGGL(attention_any_kernel<1>, grid, dim3(kThreads), 0, stream, p); break;
    case 2: hipLaunchKernelGGL(attention_any_kernel<2>, grid, dim3(kThreads), 0, stream, p); break;
    case 4: hipLaunchKernelGGL(attention_any_kernel<4>, grid, dim3(kThreads), 0, stream, p); break;
    default: hipLaunchKernelGGL(attention_any_kernel<8>, grid, dim3(kThreads), 0, stream, p); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.splits == 1) return e;
  hipLaunchKernelGGL(attention_any_merge_kernel, dim3(query_heads), dim3(kThreads), 0, stream, p, group);
  return hipGetLastError();
}

}  // namespace sa
