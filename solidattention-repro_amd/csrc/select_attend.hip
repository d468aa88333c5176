// select_attend.hip — one launch per layer for the decode step's KV work
// (gfx950): an 8-wave workgroup per (sequence, KV head g)
//   1. (decode step only) appends head g of the new token to its page and,
//      while the tail holds >= local + 32 tokens, seals the oldest tail block
//      for head g: its mean-key representative (sum of the 32 keys in token
//      order / 32, the reference's build_local_causal_representatives with
//      window 1 and top-k 32, cpp/src/selection.cpp:12-94) is written to the
//      representative array (tail lifecycle of kv_lifecycle_main.cpp:31-45,
//      92-113; append_fp16_kv of qwen_layer_main.cpp:270-281);
//   2. scores every sealed block against the G query heads of the group and
//      selects init + local + dynamic blocks, bit-exact with
//      select_shared_blocks (selection.cpp:96-147) applied to the group;
//   3. attends the selected blocks plus the unsealed tail
//      (attention_reference semantics, attention_reference.cpp:55-96).
// The result equals append_seal, score_select and sparse_decode_attention
// (splits 1) in sequence: the same bytes, representatives, counters and ids,
// and the same attention output within fp32 rounding (the waves visit the
// pages in another order).
//
// Wave roles after scoring: wave 0 runs the radix select and the compaction
// alone (no workgroup barrier) while waves 1..7 attend the last local blocks,
// which are selected whatever the scores; then all 8 waves attend the rest
// of the selected blocks and the tail, round robin starting at wave 0.
//
// Sequence counters: the 8 workgroups of a sequence all read seq_len,
// sealed and generation; the last of them to arrive (a per-sequence arrival
// counter in the caller's workspace, left at zero) writes the new values,
// so no workgroup can read an updated counter.
//
// This file is compiled with -ffp-contract=off (scoring and seal sums are
// bit-exact); the attention writes its fused multiply-adds explicitly.
#include "attn_core.hpp"
#include "online_seal.hpp"
#include "select_core.hpp"

namespace sa {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int D = kHeadDim;
constexpr int kStagedIds = kMaxStagedSelected;
constexpr int kMaxPrePages = kWaves - 1;  // forced blocks attended during the selection (G = 4)

struct Params {
  attn::PoolView v;
  int32_t* seq_len;
  int32_t* sealed;
  int32_t* generation;
  float* reps;
  const float* query;
  int32_t* selected;
  int32_t* counts;
  float* out;
  const float* k;        // new token K/V [batch][kv_heads][D] (fp32, converted RNE) ...
  const float* vv;
  const uint16_t* k16;   // ... or raw FP16 bits
  const uint16_t* v16;
  int32_t* arrive;       // [batch] arrival counters (decode step only)
  int32_t query_heads;
  int32_t rep_heads;
  int32_t rep_stride;
  int32_t budget;
  const int32_t* budgets;
  int32_t init_blocks;
  int32_t local_blocks;
  int32_t sel_stride;
  int32_t local_tokens;
  float qscale;  // softmax scale * log2(e)
  online::Args online;  // InfLLM online seal (ring non-null)
};

__device__ inline int64_t table_page(const attn::PoolView& v, int b, int64_t logical) {
  if (logical < 0 || logical >= v.table_stride) return -1;
  const int64_t page = v.table[static_cast<int64_t>(b) * v.table_stride + logical];
  return (page >= 0 && page < v.num_pages) ? page : -1;
}

// Append head g of the new token and seal filled blocks for head g.  Returns
// whether the token was appended (false: no page for it, nothing changes);
// len and n are advanced in place.  ONLINE: the decode queries of the
// group's heads are kept in the ring and a sealed block's representative of
// each of them is the local-causal builder over the block (seal_smem: LDS
// the caller does not use yet, online::kSmemFloats floats).
template <int G, bool F16, bool ONLINE = false>
__device__ inline bool append_seal_head(const Params& p, int b, int g, int64_t& len, int& n, int& added,
                                        float* seal_smem = nullptr) {
  const int tid = threadIdx.x;
  const int64_t page = table_page(p.v, b, len / kPageTokens);
  if (page < 0) {
    if (tid == 0) flag_status(p.v.status, kStatusCapacity);
    return false;
  }
  if (tid < kWave) {
    // lanes 0..31: 4 K values each, lanes 32..63: 4 V values each
    const int is_v = tid / 32;
    const int e = (tid % 32) * 4;
    const int64_t src = (static_cast<int64_t>(b) * p.v.kv_heads + g) * D + e;
    ushort4 h;
    if (F16) {
      h = *reinterpret_cast<const ushort4*>((is_v ? p.v16 : p.k16) + src);
    } else {
      const float4 f = *reinterpret_cast<const float4*>((is_v ? p.vv : p.k) + src);
      h = make_ushort4(f2h_rne(f.x), f2h_rne(f.y), f2h_rne(f.z), f2h_rne(f.w));
    }
    uint16_t* dst = const_cast<uint16_t*>(p.v.pool) + page * p.v.page_elems +
                    (len % kPageTokens) * p.v.token_elems + is_v * p.v.kv_heads * D + g * D + e;
    *reinterpret_cast<ushort4*>(dst) = h;
  }
  if (ONLINE) online::store_queries(p.online, p.query, b, g * G, G, len, tid, kThreads);
  len += 1;
  __syncthreads();  // the new token (and its queries) visible to the seal below
  const int rg = p.rep_heads == p.v.kv_heads ? 1 : G;  // representative rows of head g
  while (len >= static_cast<int64_t>(n + 1) * kPageTokens + p.local_tokens) {
    const int64_t sp = n < p.rep_stride ? table_page(p.v, b, n) : -1;
    if (sp < 0) {
      if (tid == 0) flag_status(p.v.status, kStatusCapacity);
      break;
    }
    if (ONLINE) {
      // rep_heads == query_heads: one representative per query head
      for (int j = 0; j < G; ++j) {
        const int h = g * G + j;
        online::seal_head<kThreads>(p.online, b, h, p.v.pool + sp * p.v.page_elems + g * D, p.v.token_elems,
                                    static_cast<int64_t>(n) * kPageTokens,
                                    p.reps + (static_cast<int64_t>(b) * p.rep_heads + h) * D * p.rep_stride + n,
                                    p.rep_stride, seal_smem);
      }
    } else if (tid < D) {
      const uint16_t* src = p.v.pool + sp * p.v.page_elems + g * D + tid;
      float sum = 0.0f;
#pragma unroll 8
      for (int t = 0; t < kPageTokens; ++t) sum = sum + h2f(src[t * p.v.token_elems]);
      const float rep = sum / static_cast<float>(kPageTokens);
      for (int j = 0; j < rg; ++j)
        p.reps[((static_cast<int64_t>(b) * p.rep_heads + g * rg + j) * D + tid) * p.rep_stride + n] = rep;
    }
    ++n;
    ++added;
  }
  return true;
}

// G = query heads per KV head; GR = query heads sharing one representative
// row (G for per-KV-head representatives, 1 for per-query-head ones);
// APPEND: decode step (append + seal first); F16: raw FP16 K/V input.
template <int G, int GR, bool APPEND, bool F16, bool ONLINE = false>
__global__ __launch_bounds__(kThreads, 4) void decode_kernel(const Params p) {
  const int g = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;

  __shared__ float q_s[G * D];
  __shared__ uint32_t keys[kMaxSelectBlocks];  // block keys, then the selected ids
  __shared__ uint32_t hist[256];
  __shared__ attn::CombineSmem<G, kWaves> cs;
  __shared__ int s_count;

  const int64_t out_row = static_cast<int64_t>(b) * p.v.kv_heads + g;
  int64_t len = p.seq_len[b];
  int n = p.sealed[b];

  // ---- 0. start the representative stream: the first batch of this thread's
  // first block, for blocks sealed before this step (a seal below only adds
  // blocks, whose representatives are loaded after it) --------------------------
  sel::ScoreArgs a{};
  a.query = p.query;
  a.reps = p.reps;
  a.b = b;
  a.h_first = g * G;
  a.heads_per_sel = G;
  a.query_heads = p.query_heads;
  a.group = G;
  a.rep_heads = p.rep_heads;
  a.rep_stride = p.rep_stride;
  // (with one representative row per query head the group's G rows would
  // keep the prefetched batch live across the second row: not prefetched)
  constexpr bool kPrefetch = GR == G;
  const bool have_pre = kPrefetch && n >= 0 && n <= p.rep_stride && n <= kMaxSelectBlocks && tid < n;
  float pre[sel::kScoreBatch];
  if (have_pre) sel::score_prefetch(a, tid, pre);

  // ---- 1. append + seal (decode step) ---------------------------------------
  if (APPEND) {
    const int gen = p.generation ? p.generation[b] : 0;
    int added = 0;
    const bool appended =
        append_seal_head<G, F16, ONLINE>(p, b, g, len, n, added, reinterpret_cast<float*>(keys));
    __syncthreads();  // representatives visible to the scoring below
    if (tid == 0 && atomicAdd(&p.arrive[b], 1) == p.v.kv_heads - 1) {
      if (appended) {
        p.seq_len[b] = static_cast<int32_t>(len);
        p.sealed[b] = n;
        if (p.generation) p.generation[b] = gen + added;
      }
      p.arrive[b] = 0;
    }
  }

  attn::WaveState<G> st;
  const attn::LaneGeom lg = attn::lane_geom(p.v, g, lane);

  // ---- 2. score + select ------------------------------------------------------
  int pre_pages = 0;  // local blocks [n - pre_pages, n) attended by waves 1.. during the selection
  if (n < 0 || n > p.rep_stride || n > kMaxSelectBlocks) {
    st.init(p.query + (static_cast<int64_t>(b) * p.query_heads + g * G) * D, p.qscale, lg.col);
    if (tid == 0) {
      flag_status(p.v.status, kStatusCapacity);
      p.counts[out_row] = 0;
      s_count = 0;
    }
  } else {
    sel::load_query<kThreads>(a, q_s);
    __syncthreads();
    if (kPrefetch) {
      sel::score_blocks<GR, kThreads>(a, q_s, n, keys, nullptr, pre, have_pre);
    } else {
      sel::score_blocks<GR, kThreads>(a, q_s, n, keys, nullptr);
    }
    __syncthreads();
    st.init(p.query + (static_cast<int64_t>(b) * p.query_heads + g * G) * D, p.qscale, lg.col);
    const sel::Budget bs =
        sel::budget_split(n, p.budget, p.budgets, b, p.init_blocks, p.local_blocks, p.sel_stride);
    if (bs.bad) {
      if (tid == 0) {
        flag_status(p.v.status, kStatusBadBudget);
        p.counts[out_row] = 0;
        s_count = 0;
      }
    } else {
      const int local_n = p.local_blocks < n ? p.local_blocks : n;
      pre_pages = local_n < kWaves - 1 ? local_n : kWaves - 1;
      if (wave == 0) {
        const int count = sel::select_ids_wave(keys, n, bs, hist, p.selected + out_row * p.sel_stride,
                                               p.sel_stride, reinterpret_cast<int32_t*>(keys));
        if (lane == 0) {
          p.counts[out_row] = count;
          s_count = count;
        }
      } else if (wave <= pre_pages) {
        // forced local block n - wave: selected whatever the scores
        const int64_t logical = n - wave;
        const int64_t page = table_page(p.v, b, logical);
        if (page < 0) {
          flag_status(p.v.status, logical >= p.v.table_stride ? kStatusBadBlock : kStatusBadPage);
        } else {
          st.attend(p.v, attn::PageRef{page, kPageTokens}, lg);
        }
      }
    }
  }
  __syncthreads();

  // ---- 3. attend the other selected blocks and the tail ---------------------------
  attn::PageList L{reinterpret_cast<const int32_t*>(keys), 0, 0, 0, 0};
  L.len = len;
  L.sealed = n;
  L.n_sel = s_count - pre_pages;  // the last pre_pages ids are n - pre_pages .. n - 1, already attended
  if (L.sealed < 0 || L.len < static_cast<int64_t>(L.sealed) * kPageTokens) {
    flag_status(p.v.status, kStatusBadLength);
    if (L.sealed < 0) L.sealed = 0;
    L.len = static_cast<int64_t>(L.sealed) * kPageTokens;
  }
  const int64_t tail_tokens = L.len - static_cast<int64_t>(L.sealed) * kPageTokens;
  L.total = L.n_sel + static_cast<int>((tail_tokens + kPageTokens - 1) / kPageTokens);
  for (int i = wave; i < L.total; i += kWaves) {
    const attn::PageRef pr = attn::resolve_page(p.v, b, i, L);
    if (pr.valid <= 0) continue;
    st.attend(p.v, pr, lg);
  }

  st.reduce_rows();
  attn::publish_wave<G, kWaves>(st, cs, wave, lane, lg.row, lg.col);
  __syncthreads();
  for (int o = tid; o < G * D; o += kThreads) {
    const int h = o / D;
    const int d = o % D;
    float mx, lw, aw;
    attn::combine_element<G, kWaves>(cs, h, d, mx, lw, aw);
    p.out[(static_cast<int64_t>(b) * p.query_heads + g * G + h) * D + d] = lw > 0.0f ? aw / lw : 0.0f;
  }
}


// ---- 4 query heads per KV head: LDS-staged pages, q.K on the matrix cores --
// One 8-wave workgroup per (sequence, KV head), one per CU (the eight 16 KiB
// page slots).  After append + seal, all 512 threads score two blocks per lane
// (8-byte representative loads); the keys borrow the page slots of waves 0
// and 1.  Wave 0 then selects while waves 1..7 (2..7 when the keys reach into
// wave 1's slot) attend one forced block each (the last local blocks, then
// init blocks: selected whatever the scores) through their own slots; then
// all waves attend the rest of the selected blocks and the tail
// with the staged walk of attn_core.hpp (pages HBM -> LDS by DMA, q.K on
// v_mfma_f32_16x16x32_f16).
template <int GR, bool APPEND, bool F16, bool ONLINE = false>
__global__ __launch_bounds__(kThreads) void decode_kernel_staged(const Params p) {
  constexpr int G = 4;
  constexpr int kStageBytes = kWaves * attn::kStageVecs * 16;
  constexpr int kPbufFloats = (G * 32 + G + 3) / 4 * 4;
  static_assert(kMaxSelectBlocks * 4 <= 2 * attn::kStageVecs * 16, "keys fit the page slots of waves 0 and 1");
  static_assert(sizeof(attn::CombineRowsSmem<G, kWaves>) <= kStageBytes, "combine fits the page slots");
  const int g = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;

  __shared__ __align__(16) unsigned char smem[kStageBytes + kWaves * kPbufFloats * 4];
  __shared__ __align__(16) float q_t[G * D];
  __shared__ uint32_t hist[256];
  __shared__ int32_t ids[kStagedIds];
  __shared__ int32_t pre_ids[kMaxPrePages];
  __shared__ int s_count;
  uint32_t* keys = reinterpret_cast<uint32_t*>(smem);
  uint4* stage = reinterpret_cast<uint4*>(smem) + wave * attn::kStageVecs;
  float* pbuf = reinterpret_cast<float*>(smem + kStageBytes) + wave * kPbufFloats;
  const float* q_group = p.query + (static_cast<int64_t>(b) * p.query_heads + g * G) * D;

  const int64_t out_row = static_cast<int64_t>(b) * p.v.kv_heads + g;
  int64_t len = p.seq_len[b];
  int n = p.sealed[b];

  // ---- 1. append + seal (decode step) ---------------------------------------
  if (APPEND) {
    const int gen = p.generation ? p.generation[b] : 0;
    int added = 0;
    const bool appended =
        append_seal_head<G, F16, ONLINE>(p, b, g, len, n, added, reinterpret_cast<float*>(smem));
    __syncthreads();  // representatives visible to the scoring below
    if (tid == 0 && atomicAdd(&p.arrive[b], 1) == p.v.kv_heads - 1) {
      if (appended) {
        p.seq_len[b] = static_cast<int32_t>(len);
        p.sealed[b] = n;
        if (p.generation) p.generation[b] = gen + added;
      }
      p.arrive[b] = 0;
    }
  }

  attn::WaveState<G> st;
  st.reset();
  const attn::LaneGeom lg = attn::lane_geom(p.v, g, lane);

  // ---- 2. score + select; waves 1.. attend forced blocks meanwhile -----------
  // pre_init init blocks [0, pre_init) and pre_local local blocks
  // [n - pre_local, n) are attended during the selection: in the ascending
  // selection they are the first pre_init and the last pre_local ids.
  int pre_init = 0, pre_local = 0;
  if (n < 0 || n > p.rep_stride || n > kMaxSelectBlocks) {
    if (tid == 0) {
      flag_status(p.v.status, kStatusCapacity);
      p.counts[out_row] = 0;
      s_count = 0;
    }
  } else {
    sel::ScoreArgs a{};
    a.query = p.query;
    a.reps = p.reps;
    a.b = b;
    a.h_first = g * G;
    a.heads_per_sel = G;
    a.query_heads = p.query_heads;
    a.group = G;
    a.rep_heads = p.rep_heads;
    a.rep_stride = p.rep_stride;
    sel::load_query_t<kThreads>(a, q_t);
    __syncthreads();
    sel::score_blocks_vec<GR, 2, kThreads>(a, q_t, n, keys, nullptr, tid);
    const sel::Budget bs =
        sel::budget_split(n, p.budget, p.budgets, b, p.init_blocks, p.local_blocks, p.sel_stride);
    // one forced page per wave that has a free slot: wave 1's slot is free
    // unless the keys (4 bytes per block) reach into it (a second page per
    // wave measured slower: each wave keeps one page in flight, so it costs a
    // whole load latency while the selection has already ended)
    const int pre_first = n * 4 <= attn::kStageVecs * 16 ? 1 : 2;
    const int pre_cap = kWaves - pre_first;
    if (!bs.bad) {
      // local blocks not already init blocks, then init blocks
      const int local_n = n - (bs.local_first > bs.init_n ? bs.local_first : bs.init_n);
      pre_local = local_n < pre_cap ? local_n : pre_cap;
      pre_init = bs.init_n < pre_cap - pre_local ? bs.init_n : pre_cap - pre_local;
      if (tid < pre_init + pre_local) pre_ids[tid] = tid < pre_init ? tid : n - pre_local + (tid - pre_init);
    }
    __syncthreads();  // keys and pre_ids visible
    if (bs.bad) {
      if (tid == 0) {
        flag_status(p.v.status, kStatusBadBudget);
        p.counts[out_row] = 0;
        s_count = 0;
      }
    } else {
      const int pre_pages = pre_init + pre_local;
      if (wave == 0) {
        const int count =
            sel::select_ids_wave(keys, n, bs, hist, p.selected + out_row * p.sel_stride, p.sel_stride, ids);
        if (lane == 0) {
          p.counts[out_row] = count;
          s_count = count;
        }
      } else if (wave >= pre_first && wave - pre_first < pre_pages) {
        const attn::PageList Lp{pre_ids, static_cast<int64_t>(n) * kPageTokens, n, pre_pages, pre_pages};
        st.attend_staged_mfma(p.v, b, Lp, wave - pre_first, pre_pages, kWaves - pre_first, lg, lane, g, stage,
                              pbuf, q_group, p.qscale);
      }
    }
  }
  __syncthreads();

  // ---- 3. attend the other selected blocks and the tail ---------------------------
  attn::PageList L{ids + pre_init, 0, 0, 0, 0};
  L.len = len;
  L.sealed = n;
  L.n_sel = s_count - pre_init - pre_local;
  if (L.n_sel < 0) L.n_sel = 0;
  if (L.sealed < 0 || L.len < static_cast<int64_t>(L.sealed) * kPageTokens) {
    flag_status(p.v.status, kStatusBadLength);
    if (L.sealed < 0) L.sealed = 0;
    L.len = static_cast<int64_t>(L.sealed) * kPageTokens;
  }
  const int64_t tail_tokens = L.len - static_cast<int64_t>(L.sealed) * kPageTokens;
  L.total = L.n_sel + static_cast<int>((tail_tokens + kPageTokens - 1) / kPageTokens);
  st.attend_staged_mfma(p.v, b, L, wave, L.total, kWaves, lg, lane, g, stage, pbuf, q_group, p.qscale);
  __syncthreads();  // every wave is done with its slot before the combine reuses the area

  attn::CombineRowsSmem<G, kWaves>& cs = *reinterpret_cast<attn::CombineRowsSmem<G, kWaves>*>(smem);
  attn::publish_wave_rows<G, kWaves>(st, cs, wave, lg.row, lg.col);
  __syncthreads();
  for (int o = tid; o < G * D; o += kThreads) {
    const int h = o / D;
    const int d = o % D;
    float mx, lw, aw;
    attn::combine_element_rows<G, kWaves>(cs, h, d, mx, lw, aw);
    p.out[(static_cast<int64_t>(b) * p.query_heads + g * G + h) * D + d] = lw > 0.0f ? aw / lw : 0.0f;
  }
}

// Decode step with the InfLLM online seal (fp32 K/V, one representative per
// query head).
hipError_t launch_online(const Params& p, int batch, hipStream_t stream) {
  const int group = p.query_heads / p.v.kv_heads;
  const dim3 grid(p.v.kv_heads, batch);
  if (p.rep_heads != p.query_heads) return hipErrorInvalidValue;
  if (group == 4) {
    hipLaunchKernelGGL((decode_kernel_staged<1, true, false, true>), grid, dim3(kThreads), 0, stream, p);
  } else if (group == 1) {
    hipLaunchKernelGGL((decode_kernel<1, 1, true, false, true>), grid, dim3(kThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((decode_kernel<2, 1, true, false, true>), grid, dim3(kThreads), 0, stream, p);
  }
  return hipGetLastError();
}

template <bool APPEND, bool F16>
hipError_t launch_mode(const Params& p, int batch, hipStream_t stream) {
  const int group = p.query_heads / p.v.kv_heads;
  const bool per_query_reps = p.rep_heads == p.query_heads;
  const dim3 grid(p.v.kv_heads, batch);
  if (group == 4) {
    if (per_query_reps) {
      hipLaunchKernelGGL((decode_kernel_staged<1, APPEND, F16>), grid, dim3(kThreads), 0, stream, p);
    } else {
      hipLaunchKernelGGL((decode_kernel_staged<4, APPEND, F16>), grid, dim3(kThreads), 0, stream, p);
    }
  } else if (group == 1) {
    hipLaunchKernelGGL((decode_kernel<1, 1, APPEND, F16>), grid, dim3(kThreads), 0, stream, p);
  } else if (per_query_reps) {
    hipLaunchKernelGGL((decode_kernel<2, 1, APPEND, F16>), grid, dim3(kThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((decode_kernel<2, 2, APPEND, F16>), grid, dim3(kThreads), 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace

bool select_attend_supported(int32_t query_heads, int32_t kv_heads, int32_t select_groups, int32_t sel_stride,
                             const float* reps, int32_t rep_stride) {
  const int group = kv_heads > 0 ? query_heads / kv_heads : 0;
  if (select_groups != kv_heads) return false;
  if (group == 1 || group == 2) return true;
  // 4: the selected ids are held in LDS; two-block representative loads
  return group == 4 && sel_stride <= kStagedIds && sel::vec_layout<2>(reps, rep_stride);
}

int select_attend_per_cu(int32_t query_heads, int32_t kv_heads) {
  return kv_heads > 0 && query_heads / kv_heads == 4 ? 1 : 2;
}

hipError_t launch_select_attend(const SelectAttendLaunch& s, hipStream_t stream) {
  if (!select_attend_supported(s.query_heads, s.kv_heads, s.kv_heads, s.sel_stride, s.reps, s.rep_stride))
    return hipErrorInvalidValue;
  if (s.append && !s.arrive) return hipErrorInvalidValue;
  Params p{};
  p.v.pool = s.pool;
  p.v.table = s.table;
  p.v.status = s.status;
  p.v.num_pages = s.num_pages;
  p.v.contig_tokens = 0;
  p.v.token_elems = 2 * s.kv_heads * D;
  p.v.page_elems = static_cast<int64_t>(kPageTokens) * p.v.token_elems;
  p.v.table_stride = s.table_stride;
  p.v.kv_heads = s.kv_heads;
  p.seq_len = s.seq_len;
  p.sealed = s.sealed;
  p.generation = s.generation;
  p.reps = s.reps;
  p.query = s.query;
  p.selected = s.selected;
  p.counts = s.counts;
  p.out = s.out;
  p.k = s.k;
  p.vv = s.v;
  p.k16 = s.k16;
  p.v16 = s.v16;
  p.arrive = s.arrive;
  p.query_heads = s.query_heads;
  p.rep_heads = s.rep_heads;
  p.rep_stride = s.rep_stride;
  p.budget = s.budget;
  p.budgets = s.budgets;
  p.init_blocks = s.init_blocks;
  p.local_blocks = s.local_blocks;
  p.sel_stride = s.sel_stride;
  p.local_tokens = s.local_tokens;
  p.qscale = s.scale * attn::kLog2e;
  if (s.ring) {
    if (!s.append || s.k16) return hipErrorInvalidValue;
    p.online = online::Args{s.ring, s.ring_tokens, s.window, s.topk, s.query_heads, s.seal_scale};
    return launch_online(p, s.batch, stream);
  }
  if (!s.append) return launch_mode<false, false>(p, s.batch, stream);
  return s.k16 ? launch_mode<true, true>(p, s.batch, stream) : launch_mode<true, false>(p, s.batch, stream);
}

}  // namespace sa
