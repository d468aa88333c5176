// select.hip — block-representative scoring and budgeted top-k selection
// (gfx950), bit-exact with the reference's select_shared_blocks
// (cpp/src/selection.cpp:96-147) applied to each selection group.  The
// scoring, radix select and compaction are in select_core.hpp; this kernel
// runs them with one workgroup per (sequence, selection group) of 8 or 16
// waves.  A lane scores its blocks one after the other, and every workgroup
// waits for its slowest lane, so the launch picks the width with the fewer
// (rounds of resident workgroups) x (blocks per lane): 8 waves (two
// workgroups per CU) at B=64 / 16K, 16 waves (one per CU, one block per
// lane) at B=32 / 32K.  This file is compiled with -ffp-contract=off.
#include "schedule.hpp"
#include "select_core.hpp"

namespace sa {
namespace {

using namespace sel;

struct Params {
  const float* query;
  const float* reps;
  const int32_t* sealed;
  int32_t* selected;
  int32_t* counts;
  float* scores;
  int32_t* status;
  int32_t query_heads;
  int32_t group;          // query heads per KV head
  int32_t rep_heads;
  int32_t rep_stride;
  int32_t select_groups;
  int32_t heads_per_sel;
  int32_t budget;
  const int32_t* budgets;  // optional per-sequence budgets
  int32_t init_blocks;
  int32_t local_blocks;
  int32_t sel_stride;
  // chunked selection, lists longest first (schedule.hpp): workgroup w takes
  // chunk sched[slots + w] of list sched[w] = b * select_groups + sg (-1: none)
  const int32_t* sched;
};

// QUAD: four blocks per lane with 16-byte representative loads (reps 16-byte
// aligned, rep_stride a multiple of 4); else one block per lane.
// LDS: the group's query rows and one key per block, sized by the launch
// (select_smem_bytes) to the group's heads and min(rep_stride, 8192) keys, so
// that short representative rows leave room for more resident workgroups.
template <int GR, int kThreads, bool QUAD>
__global__ __launch_bounds__(kThreads) void score_select_kernel(const Params p) {
  const int sg = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;

  extern __shared__ __align__(16) float dyn_smem[];
  float* q_s = dyn_smem;                                                   // heads_per_sel * D
  uint32_t* keys = reinterpret_cast<uint32_t*>(dyn_smem + p.heads_per_sel * D);  // min(rep_stride, 8192)
  __shared__ __align__(16) RegsSelectSmem<kThreads, 4> sm;
  __shared__ SelectSmem<kThreads / kWave> lds;

  const int64_t out_row = static_cast<int64_t>(b) * p.select_groups + sg;
  int32_t* out_ids = p.selected + out_row * p.sel_stride;

  const int n = p.sealed[b];
  if (n < 0 || n > p.rep_stride || n > kMaxSelectBlocks) {
    if (tid == 0) {
      flag_status(p.status, kStatusCapacity);
      p.counts[out_row] = 0;
    }
    return;
  }

  const Budget bs = budget_split(n, p.budget, p.budgets, b, p.init_blocks, p.local_blocks, p.sel_stride);
  if (bs.take_all && !bs.bad && !p.scores) {
    // the budget takes every block: no score can change the ids
    const int count = n < p.sel_stride ? n : p.sel_stride;
    for (int i = tid; i < count; i += kThreads) out_ids[i] = i;
    if (tid == 0) p.counts[out_row] = count;
    return;
  }

  ScoreArgs a{};
  a.query = p.query;
  a.reps = p.reps;
  a.b = b;
  a.h_first = sg * p.heads_per_sel;
  a.heads_per_sel = p.heads_per_sel;
  a.query_heads = p.query_heads;
  a.group = p.group;
  a.rep_heads = p.rep_heads;
  a.rep_stride = p.rep_stride;
  clear_regs_select(sm);
  load_query_t<kThreads>(a, q_s);
  __syncthreads();
  float* scores_row = p.scores ? p.scores + out_row * p.rep_stride : nullptr;
  if constexpr (QUAD) {
    score_blocks_vec<GR, 4, kThreads>(a, q_s, n, keys, scores_row, tid);
  } else {
    score_blocks_t<GR, kThreads>(a, q_s, n, keys, scores_row);
  }
  __syncthreads();

  if (bs.bad) {
    if (tid == 0) {
      flag_status(p.status, kStatusBadBudget);
      p.counts[out_row] = 0;
    }
    return;
  }
  const int count = select_from_keys(keys, n, bs, out_ids, p.sel_stride, sm, lds);
  if (tid == 0) p.counts[out_row] = count;
}

// ---- split selection: scoring spread over chunks of blocks -------------------
// For few or very long lists, one workgroup per (sequence, selection group)
// leaves most of the device idle while its lanes walk hundreds of blocks each.
// The split form scores kChunkBlocks blocks per workgroup (one per lane, the
// same score_one() arithmetic) into the fp32 scores row, then a second kernel
// per (sequence, selection group) turns the row into keys and selects exactly
// as score_select_kernel does.
constexpr int kChunkBlocks = 256;

template <int GR>
__global__ __launch_bounds__(kChunkBlocks) void score_chunk_kernel(const Params p) {
  const int sg = blockIdx.x;
  const int b = blockIdx.y;
  const int first = blockIdx.z * kChunkBlocks;
  const int n = p.sealed[b];
  // invalid lengths are flagged by the selection kernel
  if (n < 0 || n > p.rep_stride || n > kMaxSelectBlocks || first >= n) return;
  __shared__ __align__(16) float q_s[kMaxSelectHeads * D];
  ScoreArgs a{};
  a.query = p.query;
  a.reps = p.reps;
  a.b = b;
  a.h_first = sg * p.heads_per_sel;
  a.heads_per_sel = p.heads_per_sel;
  a.query_heads = p.query_heads;
  a.group = p.group;
  a.rep_heads = p.rep_heads;
  a.rep_stride = p.rep_stride;
  load_query_t<kChunkBlocks>(a, q_s);
  __syncthreads();
  const int blk = first + static_cast<int>(threadIdx.x);
  if (blk < n) {
    const float score = score_one_t<GR>(a, q_s, blk);
    p.scores[(static_cast<int64_t>(b) * p.select_groups + sg) * p.rep_stride + blk] = score;
  }
}

// ---- scoring at a head_dim other than 128 -------------------------------------
// One lane per block, 256 blocks of one list per workgroup, the group's query
// rows in LDS: score = the sum over the group's query heads, in head order,
// of (the sequential fp32 dot over head_dim) / heads: the reference's
// select_shared_blocks arithmetic (selection.cpp:108-119) for any head_dim.
// The lanes read consecutive blocks of each d-row of the d-major
// representatives (coalesced).  GR query heads share a representative row
// (the group, with a row per KV head): their dots run side by side over one
// pass of the row, in batches of 32 rows, the next batch's loads in flight
// while one is summed.  The selection launch of the split form follows.
constexpr int kAnyRowBatch = 32;

template <int GR>
__global__ __launch_bounds__(kChunkBlocks) void score_any_kernel(const Params p, int head_dim) {
  extern __shared__ __align__(16) float q_any[];  // [heads_per_sel][head_dim]
  const int sg = blockIdx.x;
  const int b = blockIdx.y;
  const int first = blockIdx.z * kChunkBlocks;
  const int n = p.sealed[b];
  // invalid lengths are flagged by the selection kernel
  if (n < 0 || n > p.rep_stride || n > kMaxSelectBlocks || first >= n) return;
  const int hps = p.heads_per_sel;
  const int h_first = sg * hps;
  const float* q = p.query + (static_cast<int64_t>(b) * p.query_heads + h_first) * head_dim;
  for (int e = threadIdx.x; e < hps * head_dim; e += kChunkBlocks) q_any[e] = q[e];
  __syncthreads();
  const int blk = first + static_cast<int>(threadIdx.x);
  if (blk >= n) return;
  const float heads_f = static_cast<float>(hps);
  const int64_t stride = p.rep_stride;
  float score = 0.0f;
  for (int j0 = 0; j0 < hps; j0 += GR) {  // GR divides hps
    const int h = h_first + j0;
    const int rh = p.rep_heads == p.query_heads ? h : h / p.group;
    const float* r = p.reps + (static_cast<int64_t>(b) * p.rep_heads + rh) * head_dim * stride + blk;
    float dot[GR];
#pragma unroll
    for (int j = 0; j < GR; ++j) dot[j] = 0.0f;
    // two batches of rows in flight: the next batch loads while this one is summed
    auto load = [&](int d0, float (&rv)[kAnyRowBatch]) {
#pragma unroll
      for (int k = 0; k < kAnyRowBatch; ++k)
        rv[k] = d0 + k < head_dim ? load_stream_f32(r + static_cast<int64_t>(d0 + k) * stride) : 0.0f;
    };
    auto sum = [&](int d0, const float (&rv)[kAnyRowBatch]) {
#pragma unroll
      for (int k = 0; k < kAnyRowBatch; ++k) {
        if (d0 + k >= head_dim) break;
#pragma unroll
        for (int j = 0; j < GR; ++j) dot[j] = dot[j] + q_any[(j0 + j) * head_dim + d0 + k] * rv[k];
      }
    };
    float ra[kAnyRowBatch], rb[kAnyRowBatch];
    load(0, ra);
    for (int d0 = 0; d0 < head_dim; d0 += 2 * kAnyRowBatch) {
      const bool second = d0 + kAnyRowBatch < head_dim;
      if (second) load(d0 + kAnyRowBatch, rb);
      sum(d0, ra);
      if (d0 + 2 * kAnyRowBatch < head_dim) load(d0 + 2 * kAnyRowBatch, ra);
      if (second) sum(d0 + kAnyRowBatch, rb);
    }
#pragma unroll
    for (int j = 0; j < GR; ++j) score = score + dot[j] / heads_f;
  }
  p.scores[(static_cast<int64_t>(b) * p.select_groups + sg) * p.rep_stride + blk] = score;
}

// ---- split scoring of a group with several representative rows -----------
// A selection group whose query heads read several representative rows (the
// reference's shared mode: one block set over every query head, a row per KV
// head) spreads the rows over the waves: workgroup (group, sequence, chunk of
// 64 NB blocks), wave w computes the per-head dots of rows w, w + 8, ... for
// the chunk (NB blocks per lane, row_dots(): each dot the sequential fp32 sum
// over d), the dots meet in LDS, and one lane per block adds dot / heads in
// head order.  The same operations in the same order as score_vec(), so the
// scores are bit-identical; each lane holds one row's chains instead of every
// row's, and the launch has rows x more lanes in flight.
constexpr int kRowWaves = 8;
constexpr int kRowThreads = kRowWaves * kWave;

template <int GR, int NB, int KB>
__global__ __launch_bounds__(kRowThreads) void score_rows_kernel(const Params p) {
  constexpr int kBlocks = kWave * NB;
  const int sg = blockIdx.x;
  const int b = blockIdx.y;
  const int first = blockIdx.z * kBlocks;
  const int n = p.sealed[b];
  // invalid lengths are flagged by the selection kernel
  if (n < 0 || n > p.rep_stride || n > kMaxSelectBlocks || first >= n) return;
  __shared__ __align__(16) float q_t[kMaxSelectHeads * D];
  __shared__ float dots[kMaxSelectHeads][kBlocks + 1];
  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  ScoreArgs a{};
  a.query = p.query;
  a.reps = p.reps;
  a.b = b;
  a.h_first = sg * p.heads_per_sel;
  a.heads_per_sel = p.heads_per_sel;
  a.query_heads = p.query_heads;
  a.group = p.group;
  a.rep_heads = p.rep_heads;
  a.rep_stride = p.rep_stride;
  load_query_t<kRowThreads>(a, q_t);
  __syncthreads();
  const int blk0 = first + lane * NB;
  if (blk0 < n) {
    // blk0 + NB <= rep_stride: rep_stride is a multiple of NB
    for (int h0 = wave * GR; h0 < p.heads_per_sel; h0 += kRowWaves * GR) {
      float dot[GR][NB];
      row_dots<GR, NB, KB>(a, q_t, blk0, h0, dot);
#pragma unroll
      for (int j = 0; j < GR; ++j) {
#pragma unroll
        for (int c = 0; c < NB; ++c) dots[h0 + j][lane * NB + c] = dot[j][c];
      }
    }
  }
  __syncthreads();
  const float heads_f = static_cast<float>(p.heads_per_sel);
  // dot / heads for a power-of-two head count (every shape here): the
  // product with the exact reciprocal rounds the same exact value once, as
  // the division does, so the bits are the division's
  const bool pow2 = (p.heads_per_sel & (p.heads_per_sel - 1)) == 0;
  const float inv = 1.0f / heads_f;
  float* row = p.scores + (static_cast<int64_t>(b) * p.select_groups + sg) * p.rep_stride;
  for (int t = tid; t < kBlocks; t += kRowThreads) {
    if (first + t >= n) break;
    float score = 0.0f;
    if (pow2) {
      for (int h = 0; h < p.heads_per_sel; ++h) score = score + dots[h][t] * inv;
    } else {
      for (int h = 0; h < p.heads_per_sel; ++h) score = score + dots[h][t] / heads_f;
    }
    row[first + t] = score;
  }
}

// ---- chunked selection: long lists spread over workgroups, one launch -------
// One workgroup scores kThreads x NB consecutive blocks of a list (NB per
// lane, 4 NB-byte representative loads, the score_select_kernel arithmetic;
// NB = 4, or 2 for 8 heads per representative row, where the compiler
// cannot place 4 x 8 dot chains).
// A list of one chunk selects on the spot; the chunks of a longer list hand
// their keys over through the workspace and the last chunk to arrive (an
// arrival counter per list, left at zero) selects from all of them.  Lists
// of mixed lengths then spread over the device in pieces of at most one
// chunk instead of one workgroup per list, and a budget that takes every
// block skips the scoring (no score can change its ids).
template <int GR, int kThreads, int NB>
__global__ __launch_bounds__(kThreads) void score_select_chunked_kernel(const Params p, uint32_t* ws_keys,
                                                                        int32_t* ws_arrive, int32_t key_stride) {
  constexpr int kChunk = NB * kThreads;
  int sg = blockIdx.x;
  int b = blockIdx.y;
  int z = blockIdx.z;
  if (p.sched) {
    const int64_t w = blockIdx.x + static_cast<int64_t>(gridDim.x) * (blockIdx.y + static_cast<int64_t>(gridDim.y) *
                                                                                     blockIdx.z);
    const int32_t l = p.sched[w];
    if (l < 0) return;
    b = l / p.select_groups;
    sg = l % p.select_groups;
    z = p.sched[static_cast<int64_t>(gridDim.x) * gridDim.y * gridDim.z + w];
  }
  const int tid = threadIdx.x;

  extern __shared__ __align__(16) float dyn_smem[];
  float* q_s = dyn_smem;                                                   // heads_per_sel * D
  uint32_t* keys = reinterpret_cast<uint32_t*>(dyn_smem + p.heads_per_sel * D);  // min(rep_stride, 8192)
  __shared__ __align__(16) RegsSelectSmem<kThreads, 4> sm;
  __shared__ SelectSmem<kThreads / kWave> lds;
  __shared__ int s_last;

  const int64_t out_row = static_cast<int64_t>(b) * p.select_groups + sg;
  int32_t* out_ids = p.selected + out_row * p.sel_stride;
  const int n = p.sealed[b];
  if (n < 0 || n > p.rep_stride || n > kMaxSelectBlocks) {
    if (z == 0 && tid == 0) {
      flag_status(p.status, kStatusCapacity);
      p.counts[out_row] = 0;
    }
    return;
  }
  const Budget bs = budget_split(n, p.budget, p.budgets, b, p.init_blocks, p.local_blocks, p.sel_stride);
  if (bs.bad || bs.take_all) {
    if (z != 0) return;
    if (bs.bad) {
      if (tid == 0) {
        flag_status(p.status, kStatusBadBudget);
        p.counts[out_row] = 0;
      }
      return;
    }
    // the budget takes every block: no score can change the ids
    const int count = n < p.sel_stride ? n : p.sel_stride;
    for (int i = tid; i < count; i += kThreads) out_ids[i] = i;
    if (tid == 0) p.counts[out_row] = count;
    return;
  }
  const int chunks = (n + kChunk - 1) / kChunk;
  if (z >= chunks) return;
  const int lo = z * kChunk;
  const int hi = lo + kChunk < n ? lo + kChunk : n;

  ScoreArgs a{};
  a.query = p.query;
  a.reps = p.reps;
  a.b = b;
  a.h_first = sg * p.heads_per_sel;
  a.heads_per_sel = p.heads_per_sel;
  a.query_heads = p.query_heads;
  a.group = p.group;
  a.rep_heads = p.rep_heads;
  a.rep_stride = p.rep_stride;
  clear_regs_select(sm);
  load_query_t<kThreads>(a, q_s);
  __syncthreads();
  score_blocks_vec<GR, NB, kThreads>(a, q_s, hi, keys, nullptr, tid, lo);
  uint32_t* ws_row = ws_keys + out_row * key_stride;
  if (chunks > 1) {
    // hand the keys over (each thread its own, no barrier needed); the last
    // chunk of the list selects
    for (int blk0 = lo + NB * tid; blk0 < hi; blk0 += NB * kThreads) {
#pragma unroll
      for (int c = 0; c < NB; ++c) {
        if (blk0 + c < hi) store_agent(ws_row + blk0 + c, keys[blk0 + c]);
      }
    }
    if (!last_arrival(ws_arrive + out_row, chunks, &s_last)) return;
    for (int blk = tid; blk < n; blk += kThreads) {
      if (blk < lo || blk >= hi) keys[blk] = load_agent(ws_row + blk);
    }
  }
  __syncthreads();
  const int count = select_from_keys(keys, n, bs, out_ids, p.sel_stride, sm, lds);
  if (tid == 0) p.counts[out_row] = count;
}

// The selection of the split form: one workgroup per list, the list's
// scores held in registers, radix_threshold_regs() and compact_ids_regs();
// the same ids as score_select_kernel.  The workgroup is sized by the launch
// to the representative row at 4 blocks per thread, at most 1024 threads;
// a list longer than 4 per thread (rows past 4096 blocks) takes 8 per
// thread (8192 blocks).  More threads with fewer keys each measured faster:
// the radix passes and the compaction cost each thread's keys in turn (8
// lists of 4096 blocks: 5.9-6.0 us at 4 per thread, 6.6-6.7 at 8, 8.7 at
// 16, 12.8 at 32).
constexpr int kRegsThreads = 1024;
constexpr int kRegsKeys = 4;
static_assert(kRegsThreads * 2 * kRegsKeys >= kMaxSelectBlocks, "every selectable block in registers");

template <int kThreads, int NC>
__device__ inline int select_scores_regs(const Params& p, const float* row, int n, const Budget& bs,
                                         int32_t* out_ids, RegsSelectSmem<kThreads, 16>& sm) {
  const int tid = threadIdx.x;
  const int base = NC * tid;
  uint32_t kr[NC];
  if (base + NC <= n && (reinterpret_cast<uintptr_t>(row) & 15u) == 0) {
#pragma unroll
    for (int i = 0; i < NC; i += 4) {
      const float4 v = *reinterpret_cast<const float4*>(row + base + i);
      kr[i] = order_key(v.x);
      kr[i + 1] = order_key(v.y);
      kr[i + 2] = order_key(v.z);
      kr[i + 3] = order_key(v.w);
    }
  } else {
#pragma unroll
    for (int i = 0; i < NC; ++i) kr[i] = base + i < n ? order_key(row[base + i]) : 0u;
  }
  const bool dynamic = bs.k > 0 && !bs.take_all;
  bool cand[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) cand[i] = dynamic && base + i >= bs.init_n && base + i < bs.local_first;
  __syncthreads();  // histograms zeroed
  uint32_t threshold = 0xffffffffu, equal_take = 0;
  if (dynamic) radix_threshold_regs<kThreads, NC, 16>(kr, cand, bs.k, sm, threshold, equal_take);
  return compact_ids_regs<kThreads, NC, 16>(kr, cand, n, bs, threshold, equal_take, out_ids, p.sel_stride, sm);
}

template <int kThreads, int NC>
__global__ __launch_bounds__(kThreads) void select_scores_regs_kernel(const Params p) {
  const int sg = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  __shared__ __align__(16) RegsSelectSmem<kThreads, 16> sm;
  const int64_t out_row = static_cast<int64_t>(b) * p.select_groups + sg;
  int32_t* out_ids = p.selected + out_row * p.sel_stride;
  clear_regs_select(sm);
  const int n = p.sealed[b];
  if (n < 0 || n > p.rep_stride || n > static_cast<int>(blockDim.x) * 2 * NC) {
    if (tid == 0) {
      flag_status(p.status, kStatusCapacity);
      p.counts[out_row] = 0;
    }
    return;
  }
  const Budget bs = budget_split(n, p.budget, p.budgets, b, p.init_blocks, p.local_blocks, p.sel_stride);
  if (bs.bad) {
    if (tid == 0) {
      flag_status(p.status, kStatusBadBudget);
      p.counts[out_row] = 0;
    }
    return;
  }
  const float* row = p.scores + out_row * p.rep_stride;
  // uniform per list: NC keys per thread when they cover it, else 2 NC
  const int count = n <= static_cast<int>(blockDim.x) * NC
                        ? select_scores_regs<kThreads, NC>(p, row, n, bs, out_ids, sm)
                        : select_scores_regs<kThreads, 2 * NC>(p, row, n, bs, out_ids, sm);
  if (tid == 0) p.counts[out_row] = count;
}

// 16 waves when (rounds x blocks per lane) is smaller than with 8 waves;
// resident workgroups per CU: two of 8 waves, one of 16.
bool wide_select(int64_t workgroups, int64_t blocks) {
  const int64_t cus = compute_units();
  const int64_t narrow = ((workgroups + 2 * cus - 1) / (2 * cus)) * ((blocks + 511) / 512);
  const int64_t wide = ((workgroups + cus - 1) / cus) * ((blocks + 1023) / 1024);
  return wide < narrow;
}

size_t select_smem_bytes(const Params& p) {
  const int keys = p.rep_stride < kMaxSelectBlocks ? p.rep_stride : kMaxSelectBlocks;
  return (static_cast<size_t>(p.heads_per_sel) * D + (keys + 3) / 4 * 4) * sizeof(float);
}

template <int GR>
void launch_gr(const Params& p, dim3 grid, hipStream_t stream) {
  const size_t smem = select_smem_bytes(p);
  if (vec_layout<4>(p.reps, p.rep_stride)) {
    // 4 waves score 1024 blocks per pass
    hipLaunchKernelGGL((score_select_kernel<GR, 256, true>), grid, dim3(256), smem, stream, p);
  } else if (wide_select(static_cast<int64_t>(grid.x) * grid.y, p.rep_stride)) {
    hipLaunchKernelGGL((score_select_kernel<GR, 1024, false>), grid, dim3(1024), smem, stream, p);
  } else {
    hipLaunchKernelGGL((score_select_kernel<GR, 512, false>), grid, dim3(512), smem, stream, p);
  }
}

Params make_params(const SelectLaunch& s) {
  Params p{};
  p.query = s.query;
  p.reps = s.reps;
  p.sealed = s.sealed;
  p.selected = s.selected;
  p.counts = s.counts;
  p.scores = s.scores;
  p.status = s.status;
  p.query_heads = s.query_heads;
  p.group = s.query_heads / s.kv_heads;
  p.rep_heads = s.rep_heads;
  p.rep_stride = s.rep_stride;
  p.select_groups = s.select_groups;
  p.heads_per_sel = s.query_heads / s.select_groups;
  p.budget = s.budget;
  p.budgets = s.budgets;
  p.init_blocks = s.init_blocks;
  p.local_blocks = s.local_blocks;
  p.sel_stride = s.sel_stride;
  return p;
}

}  // namespace

int compute_units() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

hipError_t launch_score_select(const SelectLaunch& s, hipStream_t stream) {
  const Params p = make_params(s);
  const dim3 grid(s.select_groups, s.batch);
  const int gr = s.rep_heads == s.query_heads ? 1 : p.group;
  switch (gr) {
    case 1: launch_gr<1>(p, grid, stream); break;
    case 2: launch_gr<2>(p, grid, stream); break;
    case 4: launch_gr<4>(p, grid, stream); break;
    case 8: launch_gr<8>(p, grid, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Smallest chunk of any width (256 threads x 2 blocks): bounds the schedule.
constexpr int kMinSelectChunk = 512;

size_t score_select_chunked_workspace_bytes(int64_t batch, int32_t select_groups, int32_t rep_stride) {
  const int64_t lists = batch * select_groups;
  const int64_t key_stride = (rep_stride < kMaxSelectBlocks ? rep_stride : kMaxSelectBlocks);
  const int64_t sched = 2 * lists * ((key_stride + kMinSelectChunk - 1) / kMinSelectChunk);
  return static_cast<size_t>((lists * 4 + 255) / 256 * 256 + lists * key_stride * 4 + sched * 4);
}

bool score_select_chunked_supported(const SelectLaunch& s) { return sel::vec_layout<4>(s.reps, s.rep_stride); }

// The chunked selection's workgroups, lists longest first (schedule.hpp):
// the length key is the list's block count when it is scored; a list whose
// budget takes every block (or is invalid) does no scoring and sorts last.
__global__ __launch_bounds__(kSchedThreads) void select_schedule_kernel(const Params p, int batch, int chunk,
                                                                         int max_chunks, int32_t* sched) {
  const int lists = batch * p.select_groups;
  build_list_schedule(lists, static_cast<int64_t>(lists) * max_chunks, sched, [&](int l, int& key, int& chunks) {
    const int b = l / p.select_groups;
    const int n = p.sealed[b];
    key = 0;
    chunks = 1;
    if (n < 0 || n > p.rep_stride || n > kMaxSelectBlocks) return;
    const Budget bs = budget_split(n, p.budget, p.budgets, b, p.init_blocks, p.local_blocks, p.sel_stride);
    if (bs.bad || bs.take_all) return;
    key = n;
    chunks = (n + chunk - 1) / chunk;
  });
}

template <int GR, int kThreads, int NB>
void launch_chunked(const Params& p, int batch, int32_t* arrive, uint32_t* keys, int32_t key_stride,
                    int32_t* sched, hipStream_t stream) {
  constexpr int kChunk = NB * kThreads;
  const int max_chunks = (key_stride + kChunk - 1) / kChunk;
  const dim3 grid(p.select_groups, batch, max_chunks);
  Params q = p;
  if (sched && static_cast<int64_t>(batch) * p.select_groups <= kSchedMaxLists) {
    hipLaunchKernelGGL(select_schedule_kernel, dim3(1), dim3(kSchedThreads), 0, stream, p, batch, kChunk,
                       max_chunks, sched);
    q.sched = sched;
  }
  hipLaunchKernelGGL((score_select_chunked_kernel<GR, kThreads, NB>), grid, dim3(kThreads), select_smem_bytes(q),
                     stream, q, keys, arrive, key_stride);
}

template <int GR, int NB>
void launch_chunked_width(const Params& p, int batch, bool many_lists, int32_t* arrive, uint32_t* keys,
                          int32_t key_stride, int32_t* sched, hipStream_t stream) {
  // with a list per compute unit or more, 16-wave workgroups (chunks of 2048
  // blocks) pull the most per list; with fewer lists, 4-wave workgroups
  // (chunks of 1024) spread each list over more compute units.  Measured on
  // the mixed B=128 workload (1024 lists of 61-2038 blocks): 512 threads
  // 80.9 us, 256 threads 82.8 us, 128 threads 91.8 us.
  if (many_lists) {
    launch_chunked<GR, 512, NB>(p, batch, arrive, keys, key_stride, sched, stream);
  } else {
    launch_chunked<GR, 256, NB>(p, batch, arrive, keys, key_stride, sched, stream);
  }
}

hipError_t launch_score_select_chunked(const SelectLaunch& s, void* workspace, hipStream_t stream) {
  const Params p = make_params(s);
  const int64_t lists = static_cast<int64_t>(s.batch) * s.select_groups;
  const bool many = lists >= compute_units();
  const int32_t key_stride = s.rep_stride < kMaxSelectBlocks ? s.rep_stride : kMaxSelectBlocks;
  int32_t* arrive = static_cast<int32_t*>(workspace);
  uint32_t* keys = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + (lists * 4 + 255) / 256 * 256);
  int32_t* sched = reinterpret_cast<int32_t*>(keys + lists * key_stride);  // rewritten by every call
  const int gr = s.rep_heads == s.query_heads ? 1 : p.group;
  switch (gr) {
    case 1: launch_chunked_width<1, 4>(p, s.batch, many, arrive, keys, key_stride, sched, stream); break;
    case 2: launch_chunked_width<2, 4>(p, s.batch, many, arrive, keys, key_stride, sched, stream); break;
    case 4: launch_chunked_width<4, 4>(p, s.batch, many, arrive, keys, key_stride, sched, stream); break;
    case 8: launch_chunked_width<8, 2>(p, s.batch, many, arrive, keys, key_stride, sched, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Two blocks per lane (8-byte loads) where the layout allows: measured at
// the long-context shared selection (8 lists x 4096 blocks x 8 rows), two
// blocks per lane with 8-row load batches 23.1 us, one block per lane with
// 16-row batches 23.1-23.8 us, four blocks per lane 29 us (half the
// workgroups), 32- and 64-row batches 24-36 us (fewer resident waves).
template <int GR>
void launch_rows(const Params& p, int batch, hipStream_t stream) {
  if (vec_layout<2>(p.reps, p.rep_stride)) {
    const dim3 grid(p.select_groups, batch, (p.rep_stride + 2 * kWave - 1) / (2 * kWave));
    hipLaunchKernelGGL((score_rows_kernel<GR, 2, 8>), grid, dim3(kRowThreads), 0, stream, p);
  } else {
    const dim3 grid(p.select_groups, batch, (p.rep_stride + kWave - 1) / kWave);
    hipLaunchKernelGGL((score_rows_kernel<GR, 1, 16>), grid, dim3(kRowThreads), 0, stream, p);
  }
}

hipError_t launch_score_select_split(const SelectLaunch& s, hipStream_t stream) {
  const Params p = make_params(s);
  const int chunks = (s.rep_stride + kChunkBlocks - 1) / kChunkBlocks;
  const dim3 grid(s.select_groups, s.batch, chunks);
  const int gr = s.rep_heads == s.query_heads ? 1 : p.group;
  if (general_head_dim(s.head_dim)) {
    const size_t smem = static_cast<size_t>(p.heads_per_sel) * s.head_dim * sizeof(float);
    switch (gr) {
      case 1: hipLaunchKernelGGL(score_any_kernel<1>, grid, dim3(kChunkBlocks), smem, stream, p, s.head_dim); break;
      case 2: hipLaunchKernelGGL(score_any_kernel<2>, grid, dim3(kChunkBlocks), smem, stream, p, s.head_dim); break;
      case 4: hipLaunchKernelGGL(score_any_kernel<4>, grid, dim3(kChunkBlocks), smem, stream, p, s.head_dim); break;
      case 8: hipLaunchKernelGGL(score_any_kernel<8>, grid, dim3(kChunkBlocks), smem, stream, p, s.head_dim); break;
      default: return hipErrorInvalidValue;
    }
  } else if (p.heads_per_sel / gr >= kRowWaves / 2) {
    // a group over four or more representative rows: a wave per row
    switch (gr) {
      case 1: launch_rows<1>(p, s.batch, stream); break;
      case 2: launch_rows<2>(p, s.batch, stream); break;
      case 4: launch_rows<4>(p, s.batch, stream); break;
      case 8: launch_rows<8>(p, s.batch, stream); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (gr) {
      case 1: hipLaunchKernelGGL(score_chunk_kernel<1>, grid, dim3(kChunkBlocks), 0, stream, p); break;
      case 2: hipLaunchKernelGGL(score_chunk_kernel<2>, grid, dim3(kChunkBlocks), 0, stream, p); break;
      case 4: hipLaunchKernelGGL(score_chunk_kernel<4>, grid, dim3(kChunkBlocks), 0, stream, p); break;
      case 8: hipLaunchKernelGGL(score_chunk_kernel<8>, grid, dim3(kChunkBlocks), 0, stream, p); break;
      default: return hipErrorInvalidValue;
    }
  }
  const hipError_t e0 = hipGetLastError();
  if (e0 != hipSuccess) return e0;
  // enough whole waves for every block of the row at kRegsKeys per thread,
  // at most 16 (the kernel takes twice as many per thread beyond 4096 blocks
  // and refuses the blocks past 8192)
  const int keys = s.rep_stride < kMaxSelectBlocks ? s.rep_stride : kMaxSelectBlocks;
  int waves = (keys + kRegsKeys * kWave - 1) / (kRegsKeys * kWave);
  if (waves > kRegsThreads / kWave) waves = kRegsThreads / kWave;
  hipLaunchKernelGGL((select_scores_regs_kernel<kRegsThreads, kRegsKeys>), dim3(s.select_groups, s.batch),
                     dim3(waves * kWave), 0, stream, p);
  return hipGetLastError();
}

}  // namespace sa
