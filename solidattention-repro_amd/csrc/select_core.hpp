// select_core.hpp — device building blocks of block-representative scoring
// and budgeted top-k selection (gfx950), bit-exact with the reference's
// select_shared_blocks (cpp/src/selection.cpp:96-147) applied to each
// selection group.  Shared by the selection kernel and the fused
// select + attend kernel.  The including translation unit must be compiled
// with -ffp-contract=off (every product and sum rounded separately, as in the
// g++-built reference, which contains no FMA).
//
// Scoring: one lane per block.  Representatives are stored head_dim-major
// ([rep head][d][block]), so for a fixed d the lanes of a wave read 64
// consecutive floats (coalesced) while each lane keeps the reference's
// sequential per-(head, block) dot order (selection.cpp:108-118).
//
// Selection: scores become order-preserving 32-bit keys (with -0.0 folded
// onto +0.0, since the reference's `>` comparator treats them as equal).  A
// 4-pass 8-bit radix select (or, for one wave and up to 1024 blocks, a
// bit-by-bit search over keys held in registers) finds the key T of the k-th
// best candidate; all
// candidates above T are taken plus the lowest-id candidates equal to T, which
// is exactly what a stable descending sort followed by a greedy fill picks
// (selection.cpp:128-142).  Output ids are compacted in ascending order with
// wave ballots (selection.cpp:143-145).
#pragma once

#include "sa_device.hpp"
#include "sa_internal.hpp"

namespace sa {
namespace sel {

constexpr int D = kHeadDim;

__device__ inline uint32_t order_key(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u << 1) == 0u) u = 0u;  // -0.0 and +0.0 compare equal
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Where the representatives and query of one (sequence, selection group) are.
struct ScoreArgs {
  const float* query;   // [batch][query_heads][D]
  const float* reps;    // [batch][rep_heads][D][rep_stride]
  int32_t b;
  int32_t h_first;      // first query head of the group
  int32_t heads_per_sel;
  int32_t query_heads;
  int32_t group;        // query heads per KV head
  int32_t rep_heads;
  int32_t rep_stride;
};

// q rows of the group's heads into LDS (q_s: heads_per_sel * D floats).
template <int kThreads>
__device__ inline void load_query(const ScoreArgs& a, float* q_s) {
  const float* q = a.query + (static_cast<int64_t>(a.b) * a.query_heads + a.h_first) * D;
  for (int e = threadIdx.x; e < a.heads_per_sel * D; e += kThreads) q_s[e] = q[e];
}

constexpr int kScoreBatch = 64;

// Issue the first batch of representative loads of block `blk` (d 0..63 of
// the group's first representative row) before the query is in LDS, so the
// representative stream starts while the caller does other work.
__device__ inline void score_prefetch(const ScoreArgs& a, int blk, float (&rv)[kScoreBatch]) {
  const int rh = a.rep_heads == a.query_heads ? a.h_first : a.h_first / a.group;
  const float* r = a.reps + (static_cast<int64_t>(a.b) * a.rep_heads + rh) * D * a.rep_stride + blk;
#pragma unroll
  for (int k = 0; k < kScoreBatch; ++k) rv[k] = load_stream_f32(r + static_cast<int64_t>(k) * a.rep_stride);
}

// Score of block blk (sequential fp32, no contraction).  FIRST: the block is
// this thread's first, whose first batch lives in rv0 (loaded here unless
// have_pre says score_prefetch() already issued it).
template <int GR, bool FIRST>
__device__ inline float score_one(const ScoreArgs& a, const float* q_s, int blk, float (&rv0)[kScoreBatch],
                                  bool have_pre) {
  // An opaque zero offset keeps the query reads inside the block loop:
  // hoisted out of it, the heads_per_sel x 128 query values would be held in
  // registers (and spilled) across all blocks of the lane.
  int qoff = 0;
  asm volatile("" : "+s"(qoff));
  const float heads_f = static_cast<float>(a.heads_per_sel);
  float score = 0.0f;
  for (int h0 = 0; h0 < a.heads_per_sel; h0 += GR) {
    const int h = a.h_first + h0;
    const int rh = a.rep_heads == a.query_heads ? h : h / a.group;
    const float* r = a.reps + (static_cast<int64_t>(a.b) * a.rep_heads + rh) * D * a.rep_stride + blk;
    float dot[GR];
#pragma unroll
    for (int j = 0; j < GR; ++j) dot[j] = 0.0f;
#pragma unroll
    for (int d0 = 0; d0 < D; d0 += kScoreBatch) {
      if (FIRST && d0 == 0 && h0 == 0) {
        if (!have_pre) {
#pragma unroll
          for (int k = 0; k < kScoreBatch; ++k) rv0[k] = load_stream_f32(r + static_cast<int64_t>(k) * a.rep_stride);
        }
#pragma unroll
        for (int k = 0; k < kScoreBatch; ++k) {
#pragma unroll
          for (int j = 0; j < GR; ++j) dot[j] = dot[j] + q_s[qoff + (h0 + j) * D + k] * rv0[k];
        }
      } else {
        float rv[kScoreBatch];
#pragma unroll
        for (int k = 0; k < kScoreBatch; ++k) rv[k] = load_stream_f32(r + static_cast<int64_t>(d0 + k) * a.rep_stride);
#pragma unroll
        for (int k = 0; k < kScoreBatch; ++k) {
#pragma unroll
          for (int j = 0; j < GR; ++j) dot[j] = dot[j] + q_s[qoff + (h0 + j) * D + d0 + k] * rv[k];
        }
      }
    }
#pragma unroll
    for (int j = 0; j < GR; ++j) score = score + dot[j] / heads_f;
  }
  return score;
}

// score_one() for the separate selection kernels, with the loads of the
// next 32 representative values in flight while the current 32 are summed
// (two 32-value buffers): memory and arithmetic overlap within each wave
// instead of alternating across the whole workgroup.  Same operations in the
// same order as score_one().
constexpr int kPipeBatch = 32;

template <int GR>
__device__ inline void dot_batch(const float* q_s, int qoff, int h0, int d0, const float (&rv)[kPipeBatch],
                                 float (&dot)[GR]) {
#pragma unroll
  for (int k = 0; k < kPipeBatch; ++k) {
#pragma unroll
    for (int j = 0; j < GR; ++j) dot[j] = dot[j] + q_s[qoff + (h0 + j) * D + d0 + k] * rv[k];
  }
}

__device__ inline void load_batch(const float* r, int64_t stride, int d0, float (&rv)[kPipeBatch]) {
#pragma unroll
  for (int k = 0; k < kPipeBatch; ++k) rv[k] = load_stream_f32(r + static_cast<int64_t>(d0 + k) * stride);
}

template <int GR>
__device__ inline float score_one_pipelined(const ScoreArgs& a, const float* q_s, int blk) {
  static_assert(D == 4 * kPipeBatch, "four batches per representative row");
  int qoff = 0;
  asm volatile("" : "+s"(qoff));
  const float heads_f = static_cast<float>(a.heads_per_sel);
  const int64_t stride = a.rep_stride;
  float score = 0.0f;
  for (int h0 = 0; h0 < a.heads_per_sel; h0 += GR) {
    const int h = a.h_first + h0;
    const int rh = a.rep_heads == a.query_heads ? h : h / a.group;
    const float* r = a.reps + (static_cast<int64_t>(a.b) * a.rep_heads + rh) * D * stride + blk;
    float dot[GR];
#pragma unroll
    for (int j = 0; j < GR; ++j) dot[j] = 0.0f;
    float ra[kPipeBatch], rb[kPipeBatch];
    load_batch(r, stride, 0, ra);
    load_batch(r, stride, kPipeBatch, rb);
    dot_batch<GR>(q_s, qoff, h0, 0, ra, dot);
    load_batch(r, stride, 2 * kPipeBatch, ra);
    dot_batch<GR>(q_s, qoff, h0, kPipeBatch, rb, dot);
    load_batch(r, stride, 3 * kPipeBatch, rb);
    dot_batch<GR>(q_s, qoff, h0, 2 * kPipeBatch, ra, dot);
    dot_batch<GR>(q_s, qoff, h0, 3 * kPipeBatch, rb, dot);
#pragma unroll
    for (int j = 0; j < GR; ++j) score = score + dot[j] / heads_f;
  }
  return score;
}

// The same scoring with the query staged transposed: q_t[d * heads_per_sel
// + h], so the GR heads that share a representative row are adjacent and one
// broadcast LDS read per d feeds all of them (with q_s[h * D + d] each d
// costs GR reads, each waited on before its multiply).  Same operations in
// the same order as score_one(): bit-identical scores.
template <int kThreads>
__device__ inline void load_query_t(const ScoreArgs& a, float* q_t) {
  const float* q = a.query + (static_cast<int64_t>(a.b) * a.query_heads + a.h_first) * D;
  for (int e = threadIdx.x; e < a.heads_per_sel * D; e += kThreads) q_t[(e % D) * a.heads_per_sel + e / D] = q[e];
}

template <int GR>
__device__ inline void read_q_t(const float* p, float (&qv)[GR]) {
  if constexpr (GR == 4) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    qv[0] = v.x;
    qv[1] = v.y;
    qv[2] = v.z;
    qv[3] = v.w;
  } else if constexpr (GR == 2) {
    const float2 v = *reinterpret_cast<const float2*>(p);
    qv[0] = v.x;
    qv[1] = v.y;
  } else {
#pragma unroll
    for (int j = 0; j < GR; ++j) qv[j] = p[j];
  }
}

template <int GR>
__device__ inline void dot_batch_t(const float* q_t, int qoff, int hps, int h0, int d0,
                                   const float (&rv)[kPipeBatch], float (&dot)[GR]) {
#pragma unroll
  for (int k = 0; k < kPipeBatch; ++k) {
    float qv[GR];
    read_q_t<GR>(q_t + qoff + (d0 + k) * hps + h0, qv);
#pragma unroll
    for (int j = 0; j < GR; ++j) dot[j] = dot[j] + qv[j] * rv[k];
  }
}

template <int GR>
__device__ inline float score_one_t(const ScoreArgs& a, const float* q_t, int blk) {
  static_assert(D == 4 * kPipeBatch, "four batches per representative row");
  int qoff = 0;
  asm volatile("" : "+s"(qoff));
  const float heads_f = static_cast<float>(a.heads_per_sel);
  const int hps = a.heads_per_sel;
  const int64_t stride = a.rep_stride;
  float score = 0.0f;
  for (int h0 = 0; h0 < hps; h0 += GR) {
    const int h = a.h_first + h0;
    const int rh = a.rep_heads == a.query_heads ? h : h / a.group;
    const float* r = a.reps + (static_cast<int64_t>(a.b) * a.rep_heads + rh) * D * stride + blk;
    float dot[GR];
#pragma unroll
    for (int j = 0; j < GR; ++j) dot[j] = 0.0f;
    float ra[kPipeBatch], rb[kPipeBatch];
    load_batch(r, stride, 0, ra);
    load_batch(r, stride, kPipeBatch, rb);
    dot_batch_t<GR>(q_t, qoff, hps, h0, 0, ra, dot);
    load_batch(r, stride, 2 * kPipeBatch, ra);
    dot_batch_t<GR>(q_t, qoff, hps, h0, kPipeBatch, rb, dot);
    load_batch(r, stride, 3 * kPipeBatch, rb);
    dot_batch_t<GR>(q_t, qoff, hps, h0, 2 * kPipeBatch, ra, dot);
    dot_batch_t<GR>(q_t, qoff, hps, h0, 3 * kPipeBatch, rb, dot);
#pragma unroll
    for (int j = 0; j < GR; ++j) score = score + dot[j] / heads_f;
  }
  return score;
}

template <int GR, int kThreads>
__device__ inline void score_blocks_t(const ScoreArgs& a, const float* q_t, int n, uint32_t* keys, float* scores) {
  for (int blk = threadIdx.x; blk < n; blk += kThreads) {
    const float score = score_one_t<GR>(a, q_t, blk);
    keys[blk] = order_key(score);
    if (scores) scores[blk] = score;
  }
}

// NB (2 or 4) consecutive blocks per lane: one 8- or 16-byte load per d
// fetches the lane's NB representative values (rows of rep_stride floats,
// rep_stride a multiple of NB, reps aligned to 4 NB bytes), so a wave reads
// 512 B or 1 KiB per load instruction instead of 256 B.  On the Qwen3-8B
// selection layout (256 lists x 128 rows x 1024 blocks) the loads alone take
// 18 us with 4 blocks per lane (4 waves per list), 22 us with 2 (8 waves)
// and 29 us with one (probe).  Each block's dot is still the sequential fp32
// sum over d per head, in the same order: bit-identical scores.  Batches of
// 8 rows, double-buffered (three batches ahead measured no faster).
constexpr int kVecBatch = 8;

template <int NB>
struct RepVec {
  typedef float type __attribute__((ext_vector_type(NB)));
};

template <int NB, int KB = kVecBatch>
__device__ inline void load_vecs(const float* r, int64_t stride, int d0, typename RepVec<NB>::type (&rv)[KB]) {
  typedef typename RepVec<NB>::type vec_t;
#pragma unroll
  for (int k = 0; k < KB; ++k)
    rv[k] = __builtin_nontemporal_load(reinterpret_cast<const vec_t*>(r + static_cast<int64_t>(d0 + k) * stride));
}

template <int GR, int NB, int KB = kVecBatch>
__device__ inline void dot_vecs(const float* q_t, int qoff, int hps, int h0, int d0,
                                const typename RepVec<NB>::type (&rv)[KB], float (&dot)[GR][NB]) {
#pragma unroll
  for (int k = 0; k < KB; ++k) {
    float qv[GR];
    read_q_t<GR>(q_t + qoff + (d0 + k) * hps + h0, qv);
#pragma unroll
    for (int j = 0; j < GR; ++j) {
#pragma unroll
      for (int c = 0; c < NB; ++c) dot[j][c] = dot[j][c] + qv[j] * rv[k][c];
    }
  }
}

template <int GR, int NB>
__device__ inline void score_vec(const ScoreArgs& a, const float* q_t, int blk0, float (&score)[NB]) {
  static_assert(D % (2 * kVecBatch) == 0, "whole double batches per representative row");
  typedef typename RepVec<NB>::type vec_t;
  int qoff = 0;
  asm volatile("" : "+s"(qoff));
  const float heads_f = static_cast<float>(a.heads_per_sel);
  // opaque like qoff: with the head count known at compile time (the fused
  // kernel) the allocator spilled hundreds of registers
  int hps = a.heads_per_sel;
  asm volatile("" : "+s"(hps));
  int64_t stride = a.rep_stride;
  asm volatile("" : "+s"(stride));
#pragma unroll
  for (int c = 0; c < NB; ++c) score[c] = 0.0f;
  for (int h0 = 0; h0 < hps; h0 += GR) {
    const int h = a.h_first + h0;
    const int rh = a.rep_heads == a.query_heads ? h : h / a.group;
    const float* r = a.reps + (static_cast<int64_t>(a.b) * a.rep_heads + rh) * D * stride + blk0;
    float dot[GR][NB];
#pragma unroll
    for (int j = 0; j < GR; ++j) {
#pragma unroll
      for (int c = 0; c < NB; ++c) dot[j][c] = 0.0f;
    }
    vec_t ra[kVecBatch], rb[kVecBatch];
    load_vecs<NB>(r, stride, 0, ra);
#pragma unroll
    for (int d0 = 0; d0 < D; d0 += 2 * kVecBatch) {
      load_vecs<NB>(r, stride, d0 + kVecBatch, rb);
      dot_vecs<GR, NB>(q_t, qoff, hps, h0, d0, ra, dot);
      if (d0 + 2 * kVecBatch < D) load_vecs<NB>(r, stride, d0 + 2 * kVecBatch, ra);
      dot_vecs<GR, NB>(q_t, qoff, hps, h0, d0 + kVecBatch, rb, dot);
    }
#pragma unroll
    for (int j = 0; j < GR; ++j) {
#pragma unroll
      for (int c = 0; c < NB; ++c) score[c] = score[c] + dot[j][c] / heads_f;
    }
  }
}

// The GR per-head dots of one representative row (the row of query heads
// h_first + h0 .. + GR - 1 within the group) for blocks blk0 .. blk0 + NB - 1:
// the inner loop of score_vec() for one h0, the same operations in the same
// order, so that summing dot[j][c] / heads in head order gives score_vec()'s
// scores bit for bit.
// KB rows per load batch, two batches in flight: the batches follow each
// other on the lane's own latency, so deep batches keep the chain short.
template <int GR, int NB, int KB>
__device__ inline void row_dots(const ScoreArgs& a, const float* q_t, int blk0, int h0, float (&dot)[GR][NB]) {
  static_assert(D % (2 * KB) == 0, "whole double batches per representative row");
  typedef typename RepVec<NB>::type vec_t;
  int qoff = 0;
  asm volatile("" : "+s"(qoff));
  int hps = a.heads_per_sel;
  asm volatile("" : "+s"(hps));
  int64_t stride = a.rep_stride;
  asm volatile("" : "+s"(stride));
  const int h = a.h_first + h0;
  const int rh = a.rep_heads == a.query_heads ? h : h / a.group;
  const float* r = a.reps + (static_cast<int64_t>(a.b) * a.rep_heads + rh) * D * stride + blk0;
#pragma unroll
  for (int j = 0; j < GR; ++j) {
#pragma unroll
    for (int c = 0; c < NB; ++c) dot[j][c] = 0.0f;
  }
  vec_t ra[KB], rb[KB];
  load_vecs<NB, KB>(r, stride, 0, ra);
#pragma unroll
  for (int d0 = 0; d0 < D; d0 += 2 * KB) {
    load_vecs<NB, KB>(r, stride, d0 + KB, rb);
    dot_vecs<GR, NB, KB>(q_t, qoff, hps, h0, d0, ra, dot);
    if (d0 + 2 * KB < D) load_vecs<NB, KB>(r, stride, d0 + 2 * KB, ra);
    dot_vecs<GR, NB, KB>(q_t, qoff, hps, h0, d0 + KB, rb, dot);
  }
}

// keys/scores of blocks [0, n), NB per lane, by the kThreads threads with
// index tid; the loads of a lane's last group may cover blocks
// n..rep_stride-1 (inside the row, discarded).
// Blocks [lo, n) (lo a multiple of NB).
template <int GR, int NB, int kThreads>
__device__ inline void score_blocks_vec(const ScoreArgs& a, const float* q_t, int n, uint32_t* keys, float* scores,
                                        int tid, int lo = 0) {
  for (int blk0 = lo + NB * tid; blk0 < n; blk0 += NB * kThreads) {
    float sc[NB];
    score_vec<GR, NB>(a, q_t, blk0, sc);
#pragma unroll
    for (int c = 0; c < NB; ++c) {
      if (blk0 + c < n) {
        keys[blk0 + c] = order_key(sc[c]);
        if (scores) scores[blk0 + c] = sc[c];
      }
    }
  }
}

// The representative layout allows NB-wide loads.
template <int NB>
__host__ __device__ inline bool vec_layout(const float* reps, int rep_stride) {
  return (reinterpret_cast<uintptr_t>(reps) & (4u * NB - 1u)) == 0 && rep_stride % NB == 0;
}

// keys[blk] = order_key(score of block blk) for blk < n; scores (optional)
// receives the fp32 scores.  GR = query heads sharing one representative row
// (the group size when representatives are per KV head, else 1).  q_s must
// be visible to the workgroup.  One block per lane; the 128 representative
// values of a block are loaded in two batches of 64 independent loads before
// the sequential chains run, so the latency of the HBM reads is paid twice
// per block, not per d.  rv0 holds the first batch of the thread's first
// block when have_pre (see score_prefetch()).
template <int GR, int kThreads>
__device__ inline void score_blocks(const ScoreArgs& a, const float* q_s, int n, uint32_t* keys, float* scores,
                                    float (&rv0)[kScoreBatch], bool have_pre) {
  int blk = threadIdx.x;
  if (blk < n) {
    const float score = score_one<GR, true>(a, q_s, blk, rv0, have_pre);
    keys[blk] = order_key(score);
    if (scores) scores[blk] = score;
  }
  for (blk += kThreads; blk < n; blk += kThreads) {
    const float score = score_one<GR, false>(a, q_s, blk, rv0, false);
    keys[blk] = order_key(score);
    if (scores) scores[blk] = score;
  }
}

template <int GR, int kThreads>
__device__ inline void score_blocks(const ScoreArgs& a, const float* q_s, int n, uint32_t* keys, float* scores) {
  for (int blk = threadIdx.x; blk < n; blk += kThreads) {
    const float score = score_one_pipelined<GR>(a, q_s, blk);
    keys[blk] = order_key(score);
    if (scores) scores[blk] = score;
  }
}

// The budget split of one selection: forced blocks [0, init_n) and
// [local_first, n), k dynamic picks among the rest (0 when all are taken).
struct Budget {
  int init_n;
  int local_first;
  int k;
  bool take_all;
  bool bad;  // per-sequence budget outside [init + local, sel_stride]
};

__device__ inline Budget budget_split(int n, int budget, const int32_t* budgets, int b, int init_blocks,
                                      int local_blocks, int sel_stride) {
  Budget r{};
  if (budgets) {
    budget = budgets[b];
    if (budget < init_blocks + local_blocks || budget > sel_stride || budget <= 0) {
      r.bad = true;
      return r;
    }
  }
  r.init_n = init_blocks < n ? init_blocks : n;
  const int local_n = local_blocks < n ? local_blocks : n;
  r.local_first = n - local_n;
  r.take_all = budget >= n;
  const int overlap = r.init_n > r.local_first ? r.init_n - r.local_first : 0;
  const int forced = r.init_n + local_n - overlap;
  r.k = r.take_all ? 0 : budget - forced;
  return r;
}

// LDS of the radix select and the compaction.
template <int kWaves>
struct SelectSmem {
  uint32_t hist[2][256];
  int counts[2][2][kWaves];
  uint32_t prefix;
  uint32_t remaining;
};

// Key T of the k-th best candidate among blocks [init_n, local_first)
// (k > 0) and how many candidates equal to T the selection takes.  4 passes
// of 8 bits; the histogram of the next pass is cleared while the current
// one fills, so each pass costs two workgroup barriers.  All threads call it.
template <int kThreads>
__device__ inline void radix_threshold(const uint32_t* keys, const Budget& bs, SelectSmem<kThreads / kWave>& sm,
                                       uint32_t& threshold, uint32_t& equal_take) {
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  for (int e = tid; e < 256; e += kThreads) sm.hist[0][e] = 0;
  __syncthreads();
  uint32_t prefix = 0, mask = 0, remaining = static_cast<uint32_t>(bs.k);
  int buf = 0;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int blk = bs.init_n + tid; blk < bs.local_first; blk += kThreads) {
      const uint32_t key = keys[blk];
      if ((key & mask) == prefix) atomicAdd(&sm.hist[buf][(key >> shift) & 255u], 1u);
    }
    for (int e = tid; e < 256; e += kThreads) sm.hist[buf ^ 1][e] = 0;
    __syncthreads();
    if (tid < kWave) {
      // lane covers digits 255-4*lane .. 252-4*lane (descending)
      uint32_t c[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) c[q] = sm.hist[buf][255 - 4 * lane - q];
      const uint32_t mine = c[0] + c[1] + c[2] + c[3];
      uint32_t incl = mine;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const uint32_t t = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += t;
      }
      uint32_t before = incl - mine;  // candidates in higher digits
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (before < remaining && before + c[q] >= remaining) {
          sm.prefix = prefix | (static_cast<uint32_t>(255 - 4 * lane - q) << shift);
          sm.remaining = remaining - before;
        }
        before += c[q];
      }
    }
    __syncthreads();
    prefix = sm.prefix;
    remaining = sm.remaining;
    mask |= 255u << shift;
    buf ^= 1;
  }
  threshold = prefix;
  equal_take = remaining;
}

// Ascending compaction of the selected ids into out_ids (global, row of
// sel_stride) and, when lds_ids is non-null, into lds_ids as well (which may
// alias keys: an id is written at a position <= its block, after every key
// of its 512-block chunk has been read).  One barrier per chunk.  Returns the
// number of selected blocks (clamped to sel_stride).  All threads call it.
template <int kThreads>
__device__ inline int compact_ids(const uint32_t* keys, int n, const Budget& bs, uint32_t threshold,
                                  uint32_t equal_take, int32_t* out_ids, int sel_stride, int32_t* lds_ids,
                                  SelectSmem<kThreads / kWave>& sm) {
  constexpr int kWaves = kThreads / kWave;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  int taken_eq = 0, written = 0, par = 0;
  for (int base = 0; base < n; base += kThreads) {
    const int blk = base + tid;
    const bool valid = blk < n;
    const bool is_forced = valid && (bs.take_all || blk < bs.init_n || blk >= bs.local_first);
    const uint32_t key = valid ? keys[blk] : 0u;
    const bool cand = valid && !is_forced && bs.k > 0;
    const bool is_eq = cand && key == threshold;
    const bool sure = is_forced || (cand && key > threshold);
    const uint64_t m_sure = __ballot(sure);
    const uint64_t m_eq = __ballot(is_eq);
    if (lane == 0) {
      sm.counts[par][0][wave] = __popcll(m_sure);
      sm.counts[par][1][wave] = __popcll(m_eq);
    }
    __syncthreads();
    // every wave derives every wave's take count: the sure blocks plus as
    // many of its equal-key blocks as the lowest-id-first rule leaves room for
    int eq_off = 0, take_off = 0, eq_tot = 0, take_tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const int cs = sm.counts[par][0][w];
      const int ce = sm.counts[par][1][w];
      int room = static_cast<int>(equal_take) - taken_eq - eq_tot;
      room = room < 0 ? 0 : (room > ce ? ce : room);
      const int tw = cs + room;
      if (w < wave) {
        eq_off += ce;
        take_off += tw;
      }
      eq_tot += ce;
      take_tot += tw;
    }
    const uint64_t below = (1ull << lane) - 1ull;
    const int eq_rank = taken_eq + eq_off + __popcll(m_eq & below);
    const bool take = sure || (is_eq && eq_rank < static_cast<int>(equal_take));
    const uint64_t m_take = __ballot(take);
    const int pos = written + take_off + __popcll(m_take & below);
    if (take && pos < sel_stride) {
      out_ids[pos] = blk;
      if (lds_ids) lds_ids[pos] = blk;
    }
    taken_eq += eq_tot;
    written += take_tot;
    par ^= 1;
  }
  return written < sel_stride ? written : sel_stride;
}

// ---- single-wave variants ----------------------------------------------------
// The same radix select and compaction run by ONE wave with no workgroup
// barrier, so the other waves of the workgroup can stream pages meanwhile.
// LDS operations of one wave execute in program order; the workgroup fences
// below only make the compiler wait for them.

__device__ inline void lds_order() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup"); }

__device__ inline void radix_threshold_wave(const uint32_t* keys, const Budget& bs, uint32_t* hist,
                                            uint32_t& threshold, uint32_t& equal_take) {
  const int lane = threadIdx.x % kWave;
  uint32_t prefix = 0, mask = 0, remaining = static_cast<uint32_t>(bs.k);
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int e = lane; e < 256; e += kWave) hist[e] = 0;
    lds_order();
    for (int blk = bs.init_n + lane; blk < bs.local_first; blk += kWave) {
      const uint32_t key = keys[blk];
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    lds_order();
    // lane covers digits 255-4*lane .. 252-4*lane (descending)
    uint32_t c[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) c[q] = hist[255 - 4 * lane - q];
    const uint32_t mine = c[0] + c[1] + c[2] + c[3];
    uint32_t incl = mine;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const uint32_t t = __shfl_up(incl, off, kWave);
      if (lane >= off) incl += t;
    }
    uint32_t before = incl - mine;
    uint32_t digit = 0, rem = 0;
    bool found = false;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (before < remaining && before + c[q] >= remaining) {
        digit = 255 - 4 * lane - q;
        rem = remaining - before;
        found = true;
      }
      before += c[q];
    }
    // exactly one lane finds the digit (0 < remaining <= candidates left)
    const uint64_t fm = __ballot(found);
    const int src = fm ? __builtin_ctzll(fm) : 0;
    prefix |= static_cast<uint32_t>(__shfl(static_cast<int>(digit), src, kWave)) << shift;
    remaining = static_cast<uint32_t>(__shfl(static_cast<int>(rem), src, kWave));
    mask |= 255u << shift;
    lds_order();
  }
  threshold = prefix;
  equal_take = remaining;
}

// Single-wave ascending compaction; lds_ids may alias keys (an id lands at a
// position <= its block after the keys of its 64-block chunk were read).
__device__ inline int compact_ids_wave(const uint32_t* keys, int n, const Budget& bs, uint32_t threshold,
                                       uint32_t equal_take, int32_t* out_ids, int sel_stride, int32_t* lds_ids) {
  const int lane = threadIdx.x % kWave;
  const uint64_t below = (1ull << lane) - 1ull;
  int taken_eq = 0, written = 0;
  for (int base = 0; base < n; base += kWave) {
    const int blk = base + lane;
    const bool valid = blk < n;
    const bool is_forced = valid && (bs.take_all || blk < bs.init_n || blk >= bs.local_first);
    const uint32_t key = valid ? keys[blk] : 0u;
    const bool cand = valid && !is_forced && bs.k > 0;
    const bool is_eq = cand && key == threshold;
    const bool sure = is_forced || (cand && key > threshold);
    const uint64_t m_eq = __ballot(is_eq);
    const int eq_rank = taken_eq + __popcll(m_eq & below);
    const bool take = sure || (is_eq && eq_rank < static_cast<int>(equal_take));
    const uint64_t m_take = __ballot(take);
    const int pos = written + __popcll(m_take & below);
    if (take && pos < sel_stride) {
      if (out_ids) out_ids[pos] = blk;
      lds_ids[pos] = blk;
    }
    taken_eq += __popcll(m_eq);
    written += __popcll(m_take);
  }
  return written < sel_stride ? written : sel_stride;
}

// ---- single-wave selection with the keys in registers (n <= 64 NC) ----------
// Lane l holds the keys of blocks l + 64 i (i < NC), each key that is not a
// dynamic candidate replaced by 0, so one LDS read per key is all the LDS
// traffic.  The k-th largest candidate key T is built from the top bit down:
// T takes bit b when at least k candidates have keys >= T | 2^b, counted with
// one wave ballot per register and scalar popcounts.  Every test value is
// >= 1, so the masked zeros are never counted and a candidate whose key is 0
// is ranked correctly.  The take and the ascending compaction are those of
// compact_ids_wave.
//
// The compares of eight (or four) registers are issued back to back (one asm
// block) before their scalar popcounts: compiled from ballots, each popcount
// directly followed the compare it reads and waited out the vector pipeline
// (about 500 cycles per step against 290 so, measured at 16 registers).
__device__ inline int count_at_least8(uint32_t x, const uint32_t* k) {
  uint64_t m0, m1, m2, m3, m4, m5, m6, m7;
  asm volatile(
      "v_cmp_le_u32_e64 %0, %8, %9\n"
      "v_cmp_le_u32_e64 %1, %8, %10\n"
      "v_cmp_le_u32_e64 %2, %8, %11\n"
      "v_cmp_le_u32_e64 %3, %8, %12\n"
      "v_cmp_le_u32_e64 %4, %8, %13\n"
      "v_cmp_le_u32_e64 %5, %8, %14\n"
      "v_cmp_le_u32_e64 %6, %8, %15\n"
      "v_cmp_le_u32_e64 %7, %8, %16\n"
      : "=&s"(m0), "=&s"(m1), "=&s"(m2), "=&s"(m3), "=&s"(m4), "=&s"(m5), "=&s"(m6), "=&s"(m7)
      : "s"(x), "v"(k[0]), "v"(k[1]), "v"(k[2]), "v"(k[3]), "v"(k[4]), "v"(k[5]), "v"(k[6]), "v"(k[7]));
  return __popcll(m0) + __popcll(m1) + __popcll(m2) + __popcll(m3) + __popcll(m4) + __popcll(m5) + __popcll(m6) +
         __popcll(m7);
}

__device__ inline int count_at_least4(uint32_t x, uint32_t k0, uint32_t k1, uint32_t k2, uint32_t k3) {
  uint64_t m0, m1, m2, m3;
  asm volatile(
      "v_cmp_le_u32_e64 %0, %4, %5\n"
      "v_cmp_le_u32_e64 %1, %4, %6\n"
      "v_cmp_le_u32_e64 %2, %4, %7\n"
      "v_cmp_le_u32_e64 %3, %4, %8\n"
      : "=&s"(m0), "=&s"(m1), "=&s"(m2), "=&s"(m3)
      : "s"(x), "v"(k0), "v"(k1), "v"(k2), "v"(k3));
  return __popcll(m0) + __popcll(m1) + __popcll(m2) + __popcll(m3);
}

template <int NC>
__device__ inline int count_at_least(const uint32_t (&kr)[NC], uint32_t x) {
  static_assert(NC % 4 == 0, "keys per lane in fours");
  int c = 0;
#pragma unroll
  for (int i = 0; i + 8 <= NC; i += 8) c += count_at_least8(x, kr + i);
  if constexpr (NC % 8 != 0) c += count_at_least4(x, kr[NC - 4], kr[NC - 3], kr[NC - 2], kr[NC - 1]);
  return c;
}

// keys must hold at least 64 NC entries (entries past n are read, not used).
template <int NC>
__device__ inline int select_ids_wave_regs(const uint32_t* keys, int n, const Budget& bs, int32_t* out_ids,
                                           int sel_stride, int32_t* lds_ids) {
  const int lane = threadIdx.x % kWave;
  const bool dynamic = bs.k > 0 && !bs.take_all;
  uint32_t kr[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) kr[i] = keys[i * kWave + lane];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int blk = i * kWave + lane;
    const bool cand = dynamic && blk >= bs.init_n && blk < bs.local_first;
    kr[i] = cand ? kr[i] : 0u;
  }
  uint32_t threshold = 0xffffffffu;
  int equal_take = 0;
  if (dynamic) {
    uint32_t t = 0;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t c = t | (1u << bit);
      if (count_at_least<NC>(kr, c) >= bs.k) t = c;
    }
    threshold = t;
    equal_take = bs.k - (t == 0xffffffffu ? 0 : count_at_least<NC>(kr, t + 1u));
  }
  const uint64_t below = (1ull << lane) - 1ull;
  int taken_eq = 0, written = 0;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int blk = i * kWave + lane;
    const bool valid = blk < n;
    const bool is_forced = valid && (bs.take_all || blk < bs.init_n || blk >= bs.local_first);
    const bool cand = valid && !is_forced && dynamic;
    const bool is_eq = cand && kr[i] == threshold;
    const bool sure = is_forced || (cand && kr[i] > threshold);
    const uint64_t m_eq = __ballot(is_eq);
    const int eq_rank = taken_eq + __popcll(m_eq & below);
    const bool take = sure || (is_eq && eq_rank < equal_take);
    const uint64_t m_take = __ballot(take);
    const int pos = written + __popcll(m_take & below);
    if (take && pos < sel_stride) {
      if (out_ids) out_ids[pos] = blk;
      lds_ids[pos] = blk;
    }
    taken_eq += __popcll(m_eq);
    written += __popcll(m_take);
  }
  return written < sel_stride ? written : sel_stride;
}

// ---- workgroup selection with the keys in registers (n <= kThreads NC) -------
// For one list per workgroup with the workgroup to itself (the split
// selection's second launch), of any whole number of waves up to kThreads
// (blockDim.x).  Thread t holds the keys of blocks NC t .. NC t + NC - 1
// (contiguous, so that the ascending compaction is one scan).
//
// Threshold: the same 4 passes of 8 bits as radix_threshold(), with the
// histogram of each pass spread over kRadixCopies copies (lane l adds into
// copy l % 16, copies 4 banks apart): scores from a narrow range share their
// top digits, and 64 lanes adding into one LDS word serialise.  Each pass has
// its own histogram set (zeroed once), so a pass costs two barriers; wave 0
// sums the copies and scans the digits.
constexpr int kRadixPad = 260;  // words per copy: 256 bins, 16-byte rows, 4 banks apart

// kCopies histogram copies per pass: 16 where the workgroup has the compute
// unit to itself (66.5 KB), fewer where the LDS bounds the workgroups a CU
// holds (4 copies: 16.6 KB, up to 16 lanes per word in one instruction).
template <int kThreads, int kCopies = 16>
struct RegsSelectSmem {
  uint32_t hist[4][kCopies * kRadixPad];
  uint32_t prefix[4];
  uint32_t remaining[4];
  uint32_t wave_sum[kThreads / kWave];
};

template <int kThreads, int kCopies>
__device__ inline void clear_regs_select(RegsSelectSmem<kThreads, kCopies>& sm) {
  uint4* h = reinterpret_cast<uint4*>(&sm.hist[0][0]);
  for (int e = threadIdx.x; e < 4 * kCopies * kRadixPad / 4; e += blockDim.x) h[e] = make_uint4(0, 0, 0, 0);
}

// k-th largest key among the candidates (cand[i]) and how many keys equal
// to it are taken; k > 0.  clear_regs_select() and a barrier must precede.
template <int kThreads, int NC, int kCopies>
__device__ inline void radix_threshold_regs(const uint32_t (&kr)[NC], const bool (&cand)[NC], int k,
                                            RegsSelectSmem<kThreads, kCopies>& sm, uint32_t& threshold,
                                            uint32_t& equal_take) {
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  uint32_t prefix = 0, mask = 0, remaining = static_cast<uint32_t>(k);
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    uint32_t* h = sm.hist[pass] + (lane % kCopies) * kRadixPad;
#pragma unroll
    for (int i = 0; i < NC; ++i)
      if (cand[i] && (kr[i] & mask) == prefix) atomicAdd(&h[(kr[i] >> shift) & 255u], 1u);
    __syncthreads();
    if (tid < kWave) {
      // lane covers digits 255-4*lane .. 252-4*lane (descending)
      uint32_t c[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int cp = 0; cp < kCopies; ++cp) {
        const uint4 v = *reinterpret_cast<const uint4*>(sm.hist[pass] + cp * kRadixPad + 252 - 4 * lane);
        c[3] += v.x;
        c[2] += v.y;
        c[1] += v.z;
        c[0] += v.w;
      }
      const uint32_t mine = c[0] + c[1] + c[2] + c[3];
      uint32_t before = wave_prefix_sum(mine) - mine;  // candidates in higher digits
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (before < remaining && before + c[q] >= remaining) {
          sm.prefix[pass] = prefix | (static_cast<uint32_t>(255 - 4 * lane - q) << shift);
          sm.remaining[pass] = remaining - before;
        }
        before += c[q];
      }
    }
    __syncthreads();
    prefix = sm.prefix[pass];
    remaining = sm.remaining[pass];
    mask |= 255u << shift;
  }
  threshold = prefix;
  equal_take = remaining;
}

// Ascending compaction of the selected ids of blocks [0, n) (thread t holds
// blocks NC t ..): forced blocks, candidates above the threshold, and the
// lowest-id candidates equal to it up to equal_take.  One scan of the
// per-thread (sure, equal) counts.  Returns the count (clamped to
// sel_stride).
template <int kThreads, int NC, int kCopies>
__device__ inline int compact_ids_regs(const uint32_t (&kr)[NC], const bool (&cand)[NC], int n, const Budget& bs,
                                       uint32_t threshold, uint32_t equal_take, int32_t* out_ids, int sel_stride,
                                       RegsSelectSmem<kThreads, kCopies>& sm) {
  const int waves = static_cast<int>(blockDim.x) / kWave;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int base = NC * tid;
  bool sure[NC], eq[NC];
  uint32_t sure_c = 0, eq_c = 0;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int blk = base + i;
    const bool forced = blk < n && (bs.take_all || blk < bs.init_n || blk >= bs.local_first);
    eq[i] = cand[i] && kr[i] == threshold;
    sure[i] = forced || (cand[i] && kr[i] > threshold);
    sure_c += sure[i];
    eq_c += eq[i];
  }
  // (sure, equal) counts packed in 16-bit halves: each at most 8192
  const uint32_t packed = (sure_c << 16) | eq_c;
  const uint32_t incl = wave_prefix_sum(packed);
  if (lane == kWave - 1) sm.wave_sum[wave] = incl;
  __syncthreads();
  uint32_t before = incl - packed, total = 0;
  for (int w = 0; w < waves; ++w) {
    const uint32_t s = sm.wave_sum[w];
    if (w < wave) before += s;
    total += s;
  }
  const int take_eq = static_cast<int>(equal_take);
  int eq_seen = static_cast<int>(before & 0xffffu);
  int pos = static_cast<int>(before >> 16) + (eq_seen < take_eq ? eq_seen : take_eq);
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    bool take = sure[i];
    if (eq[i]) take = eq_seen++ < take_eq;
    if (take) {
      if (pos < sel_stride) out_ids[pos] = base + i;
      ++pos;
    }
  }
  const int tot_eq = static_cast<int>(total & 0xffffu);
  const int count = static_cast<int>(total >> 16) + (tot_eq < take_eq ? tot_eq : take_eq);
  return count < sel_stride ? count : sel_stride;
}

// The selection of one list whose keys are in LDS (keys[0, n), n <= kThreads
// NC): each thread takes NC contiguous keys into registers, then
// radix_threshold_regs() and compact_ids_regs().  The histograms must be
// zeroed (clear_regs_select() and a barrier, once per kernel) and keys[]
// complete (a barrier).  Returns the count.
template <int kThreads, int NC, int kCopies>
__device__ inline int select_from_keys_regs(const uint32_t* keys, int n, const Budget& bs, int32_t* out_ids,
                                            int sel_stride, RegsSelectSmem<kThreads, kCopies>& sm) {
  const int base = NC * static_cast<int>(threadIdx.x);
  const bool dynamic = bs.k > 0 && !bs.take_all;
  uint32_t kr[NC];
  bool cand[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int blk = base + i;
    kr[i] = blk < n ? keys[blk] : 0u;
    cand[i] = dynamic && blk >= bs.init_n && blk < bs.local_first;
  }
  uint32_t threshold = 0xffffffffu, equal_take = 0;
  if (dynamic) radix_threshold_regs<kThreads, NC, kCopies>(kr, cand, bs.k, sm, threshold, equal_take);
  return compact_ids_regs<kThreads, NC, kCopies>(kr, cand, n, bs, threshold, equal_take, out_ids, sel_stride, sm);
}

// select_from_keys_regs() with NC = 4 or 8, the smaller that covers n;
// longer lists (more than 8 keys per thread) take the LDS radix select and
// compaction (radix_threshold, compact_ids), so that the register form
// does not raise the kernel's register count.  The same ids either way.
template <int kThreads, int kCopies>
__device__ inline int select_from_keys(const uint32_t* keys, int n, const Budget& bs, int32_t* out_ids, int sel_stride,
                                       RegsSelectSmem<kThreads, kCopies>& sm, SelectSmem<kThreads / kWave>& lds) {
  if (n <= kThreads * 4) return select_from_keys_regs<kThreads, 4, kCopies>(keys, n, bs, out_ids, sel_stride, sm);
  if (n <= kThreads * 8) return select_from_keys_regs<kThreads, 8, kCopies>(keys, n, bs, out_ids, sel_stride, sm);
  uint32_t threshold = 0xffffffffu, equal_take = 0;
  if (bs.k > 0) radix_threshold<kThreads>(keys, bs, lds, threshold, equal_take);
  return compact_ids<kThreads>(keys, n, bs, threshold, equal_take, out_ids, sel_stride, nullptr, lds);
}

// Single-wave selection of one list: forced blocks plus the k best
// candidates (lowest id first among equal keys), ids ascending into out_ids
// (null: none) and lds_ids (which may alias keys).  Up to 1024 blocks the
// keys are held in registers (keys must hold n rounded up to a multiple of
// 256 entries); longer lists take the LDS radix select.  Returns the count.
__device__ inline int select_ids_wave(const uint32_t* keys, int n, const Budget& bs, uint32_t* hist,
                                      int32_t* out_ids, int sel_stride, int32_t* lds_ids) {
  if (n <= 4 * kWave) return select_ids_wave_regs<4>(keys, n, bs, out_ids, sel_stride, lds_ids);
  if (n <= 8 * kWave) return select_ids_wave_regs<8>(keys, n, bs, out_ids, sel_stride, lds_ids);
  if (n <= 12 * kWave) return select_ids_wave_regs<12>(keys, n, bs, out_ids, sel_stride, lds_ids);
  if (n <= 16 * kWave) return select_ids_wave_regs<16>(keys, n, bs, out_ids, sel_stride, lds_ids);
  uint32_t threshold = 0xffffffffu, equal_take = 0;
  if (bs.k > 0) radix_threshold_wave(keys, bs, hist, threshold, equal_take);
  return compact_ids_wave(keys, n, bs, threshold, equal_take, out_ids, sel_stride, lds_ids);
}

}  // namespace sel
}  // namespace sa
