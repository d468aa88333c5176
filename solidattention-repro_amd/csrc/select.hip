// select.hip — block-representative scoring and budgeted top-k selection
// (gfx950), bit-exact with the reference's select_shared_blocks
// (cpp/src/selection.cpp:96-147) applied to each selection group.
//
// Scoring: one lane per block.  Representatives are stored head_dim-major
// ([rep head][d][block]), so for a fixed d the lanes of a wave read 64
// consecutive floats (coalesced) while each lane keeps the reference's
// sequential per-(head, block) dot order.  The workgroup is 8 waves, so
// 512 blocks (a 16K-token sequence) are scored in one pass.  This file is compiled with
// -ffp-contract=off: every product and sum is rounded separately, as in the
// g++-built reference (which contains no FMA).
//
// Selection: scores become order-preserving 32-bit keys (with -0.0 folded
// onto +0.0, since the reference's `>` comparator treats them as equal).  A
// 4-pass 8-bit radix select finds the key T of the k-th best candidate; all
// candidates above T are taken plus the lowest-id candidates equal to T, which
// is exactly what a stable descending sort followed by a greedy fill picks.
// Output ids are compacted in ascending order with wave ballots.
#include "sa_device.hpp"
#include "sa_internal.hpp"

namespace sa {
namespace {

constexpr int D = kHeadDim;
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;

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
};

__device__ inline uint32_t order_key(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u << 1) == 0u) u = 0u;  // -0.0 and +0.0 compare equal
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive prefix count of `pred` over the workgroup in thread order, and
// the workgroup total.  Uses `scratch[kWaves]`.
__device__ inline int block_prefix(bool pred, int* scratch, int* total) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const uint64_t mask = __ballot(pred);
  const int below = __popcll(mask & ((1ull << lane) - 1ull));
  if (lane == 0) scratch[wave] = __popcll(mask);
  __syncthreads();
  int offset = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int c = scratch[w];
    offset += w < wave ? c : 0;
    sum += c;
  }
  __syncthreads();
  *total = sum;
  return offset + below;
}

// GR = query heads of the selection group that share one representative row
// (the group size when representatives are per KV head, else 1).
template <int GR>
__global__ __launch_bounds__(kThreads) void score_select_kernel(const Params p) {
  const int sg = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;

  __shared__ float q_s[kMaxSelectHeads * D];
  __shared__ uint32_t keys[kMaxSelectBlocks];
  __shared__ uint32_t hist[256];
  __shared__ int scratch[kWaves];
  __shared__ uint32_t s_prefix, s_remaining;

  const int64_t out_row = static_cast<int64_t>(b) * p.select_groups + sg;
  int32_t* out_ids = p.selected + out_row * p.sel_stride;

  int n = p.sealed[b];
  if (n < 0 || n > p.rep_stride || n > kMaxSelectBlocks) {
    if (tid == 0) {
      flag_status(p.status, kStatusCapacity);
      p.counts[out_row] = 0;
    }
    return;
  }

  // ---- query heads of the selection group into LDS ------------------------
  const int h_first = sg * p.heads_per_sel;
  for (int e = tid; e < p.heads_per_sel * D; e += kThreads)
    q_s[e] = p.query[(static_cast<int64_t>(b) * p.query_heads + h_first) * D + e];
  __syncthreads();

  // ---- scores (sequential fp32, no contraction) ----------------------------
  // One block per lane.  The 128 representative values of a block are loaded
  // in two batches of 64 independent loads before the sequential chains run,
  // so the latency of the HBM reads is paid twice per block, not per d.
  const float heads_f = static_cast<float>(p.heads_per_sel);
  constexpr int kBatch = 64;
  for (int blk = tid; blk < n; blk += kThreads) {
    float score = 0.0f;
    for (int h0 = 0; h0 < p.heads_per_sel; h0 += GR) {
      const int h = h_first + h0;
      const int rh = p.rep_heads == p.query_heads ? h : h / p.group;
      const float* r = p.reps + (static_cast<int64_t>(b) * p.rep_heads + rh) * D * p.rep_stride + blk;
      float dot[GR];
#pragma unroll
      for (int j = 0; j < GR; ++j) dot[j] = 0.0f;
#pragma unroll
      for (int d0 = 0; d0 < D; d0 += kBatch) {
        float rv[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) rv[k] = load_stream_f32(r + static_cast<int64_t>(d0 + k) * p.rep_stride);
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
#pragma unroll
          for (int j = 0; j < GR; ++j) dot[j] = dot[j] + q_s[(h0 + j) * D + d0 + k] * rv[k];
        }
      }
#pragma unroll
      for (int j = 0; j < GR; ++j) score = score + dot[j] / heads_f;
    }
    keys[blk] = order_key(score);
    if (p.scores) p.scores[out_row * p.rep_stride + blk] = score;
  }
  __syncthreads();

  // ---- forced blocks and the dynamic count --------------------------------
  const int init_n = p.init_blocks < n ? p.init_blocks : n;
  const int local_n = p.local_blocks < n ? p.local_blocks : n;
  const int local_first = n - local_n;
  int budget = p.budget;
  if (p.budgets) {
    budget = p.budgets[b];
    if (budget < p.init_blocks + p.local_blocks || budget > p.sel_stride || budget <= 0) {
      if (tid == 0) {
        flag_status(p.status, kStatusBadBudget);
        p.counts[out_row] = 0;
      }
      return;
    }
  }
  const bool take_all = budget >= n;
  const int overlap = init_n > local_first ? init_n - local_first : 0;
  const int forced = init_n + local_n - overlap;
  const int k = take_all ? 0 : budget - forced;

  // ---- radix select of the k-th best candidate key ------------------------
  uint32_t threshold = 0xffffffffu;
  uint32_t equal_take = 0;  // candidates equal to the threshold to take
  if (k > 0) {
    uint32_t prefix = 0, mask = 0, remaining = static_cast<uint32_t>(k);
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int e = tid; e < 256; e += kThreads) hist[e] = 0;
      __syncthreads();
      for (int blk = tid; blk < n; blk += kThreads) {
        if (blk < init_n || blk >= local_first) continue;
        const uint32_t key = keys[blk];
        if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid < kWave) {
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
        uint32_t before = incl - mine;  // candidates in higher digits
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (before < remaining && before + c[q] >= remaining) {
            s_prefix = prefix | (static_cast<uint32_t>(255 - 4 * lane - q) << shift);
            s_remaining = remaining - before;
          }
          before += c[q];
        }
      }
      __syncthreads();
      prefix = s_prefix;
      remaining = s_remaining;
      mask |= 255u << shift;
    }
    threshold = prefix;
    equal_take = remaining;
  }

  // ---- mark and compact in ascending block order --------------------------
  int taken_eq = 0, written = 0;
  for (int base = 0; base < n; base += kThreads) {
    const int blk = base + tid;
    const bool valid = blk < n;
    const bool is_forced = valid && (take_all || blk < init_n || blk >= local_first);
    const uint32_t key = valid ? keys[blk] : 0u;
    const bool cand = valid && !is_forced && k > 0;
    const bool is_eq = cand && key == threshold;
    int eq_total;
    const int eq_rank = block_prefix(is_eq, scratch, &eq_total);
    const bool take = is_forced || (cand && key > threshold) ||
                      (is_eq && static_cast<uint32_t>(taken_eq + eq_rank) < equal_take);
    int take_total;
    const int pos = block_prefix(take, scratch, &take_total);
    if (take && written + pos < p.sel_stride) out_ids[written + pos] = blk;
    taken_eq += eq_total;
    written += take_total;
  }
  if (tid == 0) p.counts[out_row] = written < p.sel_stride ? written : p.sel_stride;
  (void)lane;
}

template <int GR>
void launch_gr(const Params& p, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL(score_select_kernel<GR>, grid, dim3(kThreads), 0, stream, p);
}

}  // namespace

hipError_t launch_score_select(const SelectLaunch& s, hipStream_t stream) {
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

}  // namespace sa
