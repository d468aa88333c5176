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
// Wave roles after scoring: wave 0 selects alone (no workgroup barrier) while
// waves 1..7 attend the forced blocks (init and local, selected whatever the
// scores); then every wave attends its planned share of the other selected
// blocks and the tail (the planned walk, below).
//
// Sequence counters: the 8 workgroups of a sequence all read seq_len,
// sealed and generation; the last of them to arrive (a per-sequence arrival
// counter in the caller's workspace, left at zero) writes the new values at
// its end, so no workgroup can read an updated counter.
//
// This file is compiled with -ffp-contract=off (scoring and seal sums are
// bit-exact); the attention writes its fused multiply-adds explicitly.
#include <type_traits>

#include "attn_core.hpp"
#include "attn_rows.hpp"
#include "online_seal.hpp"
#include "qkv_epilogue.hpp"
#include "select_core.hpp"

namespace sa {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int D = kHeadDim;
constexpr int kStagedIds = kMaxStagedSelected;

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
// Head g of the new token as FP16 bits, four values per lane of one wave:
// lanes 0..31 hold K values 4 l .. 4 l + 3, lanes 32..63 the V values.
template <bool F16>
__device__ inline ushort4 token_quad(const Params& p, int b, int g, int lane) {
  const int is_v = lane / 32;
  const int e = (lane % 32) * 4;
  const int64_t src = (static_cast<int64_t>(b) * p.v.kv_heads + g) * D + e;
  if (F16) return *reinterpret_cast<const ushort4*>((is_v ? p.v16 : p.k16) + src);
  const float4 f = *reinterpret_cast<const float4*>((is_v ? p.vv : p.k) + src);
  return make_ushort4(f2h_rne(f.x), f2h_rne(f.y), f2h_rne(f.z), f2h_rne(f.w));
}

__device__ inline void store_token_quad(const Params& p, int64_t page, int64_t pos, int g, int lane, ushort4 h) {
  const int is_v = lane / 32;
  const int e = (lane % 32) * 4;
  uint16_t* dst = const_cast<uint16_t*>(p.v.pool) + page * p.v.page_elems + (pos % kPageTokens) * p.v.token_elems +
                  is_v * p.v.kv_heads * D + g * D + e;
  *reinterpret_cast<ushort4*>(dst) = h;
}

// Whether appending one token at position len seals a block (len + 1 tokens
// reach block n's end plus the local tail).
__device__ inline bool append_seals(const Params& p, int64_t len, int n) {
  return len + 1 >= static_cast<int64_t>(n + 1) * kPageTokens + p.local_tokens;
}

// TOK_W1: the token is not read from p.k/p.vv but given, in token_quad()'s
// layout, by the lanes of wave 1 (tok).
template <int G, bool F16, bool ONLINE = false, bool TOK_W1 = false>
__device__ inline bool append_seal_head(const Params& p, int b, int g, int64_t& len, int& n, int& added,
                                        float* seal_smem = nullptr, ushort4 tok = {}) {
  const int tid = threadIdx.x;
  const int64_t page = table_page(p.v, b, len / kPageTokens);
  if (page < 0) {
    if (tid == 0) flag_status(p.v.status, kStatusCapacity);
    return false;
  }
  if (TOK_W1) {
    if (tid >= kWave && tid < 2 * kWave) store_token_quad(p, page, len, g, tid - kWave, tok);
  } else if (tid < kWave) {
    store_token_quad(p, page, len, g, tid, token_quad<F16>(p, b, g, tid));
  }
  if (ONLINE) online::store_queries(p.online, p.query, b, g * G, G, len, tid, kThreads);
  len += 1;
  // the new token (and its queries) visible to the seal below; without a
  // seal nothing in this workgroup reads them
  if (len >= static_cast<int64_t>(n + 1) * kPageTokens + p.local_tokens) __syncthreads();
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

// Sequence counters of one decode step.  Every workgroup of sequence b reads
// seq_len, sealed and generation at its start and adds 1 to arrive[b] after
// its append; the workgroup that brings the count to kv_heads (all others
// have read the counters by then) writes the new values and clears the count.
struct SeqCommit {
  int gen = 0;
  int added = 0;
  int arrived = -1;
  bool appended = false;
};

__device__ inline void commit_sequence(const Params& p, int b, int64_t len, int n, const SeqCommit& c) {
  if (c.arrived != p.v.kv_heads - 1) return;
  if (c.appended) {
    p.seq_len[b] = static_cast<int32_t>(len);
    p.sealed[b] = n;
    if (p.generation) p.generation[b] = c.gen + c.added;
  }
  p.arrive[b] = 0;
}

// ---- the planned page walk (both fused kernels) ------------------------------
// After the scoring every wave walks its own positions of one list:
//   * positions [0, F): the forced blocks (init, then local: selected
//     whatever the scores; at most kEarly), whose pages the last wave looked
//     up while it scored; waves 1..7 take them round robin while wave 0
//     selects;
//   * positions [F, F + late): the other selected blocks, then the tail
//     pages, listed by wave 0 after its selection and split into contiguous
//     ranges so that every wave's total count of positions is balanced
//     (wave 0's selection counting as kSelectPages positions).
// A wave that reaches the late positions before the list is out waits for it
// (an LDS flag that wave 0 sets on every path).  No wave idles at a barrier
// between the selection and the walk, and the plan depends only on the list:
// every run attends the same pages in the same order on the same waves, so
// the outputs are reproducible bit for bit.
constexpr int kEarly = 64;      // forced blocks looked up before the selection
constexpr int kTailPages = 64;  // tail pages listed by wave 0 (more are looked up when reached)
// Wave 0's selection takes about as long as two pages of the walk (measured
// at 16K-32K contexts), so its planned share is two positions smaller.
constexpr int kSelectPages = 2;

// Page of logical block blk of sequence b, or -1 (flagged) if there is none.
__device__ inline int64_t lookup_page(const attn::PoolView& v, int b, int64_t blk) {
  if (v.contig_tokens > 0) return blk;
  if (blk < 0 || blk >= v.table_stride) {
    flag_status(v.status, kStatusBadBlock);
    return -1;
  }
  const int64_t page = v.table[static_cast<int64_t>(b) * v.table_stride + blk];
  if (page < 0 || page >= v.num_pages) {
    flag_status(v.status, kStatusBadPage);
    return -1;
  }
  return page;
}

// LDS state of the planned walk (the late pages live in the caller's id array).
struct ClaimSmem {
  int late_ready;   // 1 once wave 0 has listed the late positions
  int late_n;       // late positions: selected blocks, then tail pages
  int late_mid;     // of which selected blocks
  int tail_listed;  // tail pages with their page in the list (the rest looked up when reached)
  int32_t early[kEarly];
};

__device__ inline void wait_late(ClaimSmem& cs) {
  while (__hip_atomic_load(&cs.late_ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0)
    __builtin_amdgcn_s_sleep(1);
}

// The forced blocks listed early: [0, e_init) and [n - e_local, n).
struct Forced {
  int e_init;
  int e_local;
  int F;
};

__device__ inline Forced forced_blocks(const sel::Budget& bs, int n) {
  int init_f = 0, local_f = 0;  // every block is forced when the budget takes all
  if (!bs.bad) {
    init_f = bs.take_all ? n : bs.init_n;
    local_f = bs.take_all ? 0 : n - (bs.local_first > bs.init_n ? bs.local_first : bs.init_n);
  }
  Forced f;
  f.e_init = init_f < kEarly ? init_f : kEarly;
  f.e_local = local_f < kEarly - f.e_init ? local_f : kEarly - f.e_init;
  f.F = f.e_init + f.e_local;
  return f;
}

// Lane `lane` of the looking-up wave: the page of forced position `lane`.
__device__ inline int32_t early_page(const Params& p, int b, int n, const Forced& f, int lane) {
  if (lane >= f.F) return -1;
  return static_cast<int32_t>(lookup_page(p.v, b, lane < f.e_init ? lane : n - f.e_local + (lane - f.e_init)));
}

// Wave 0, after its selection (count ids ascending in late[]): the late
// positions in place over the ids (position j reads id e_init + j >= j, all
// lanes read before any writes), at most late_cap entries, then the flag.
__device__ inline void list_late(const Params& p, int b, ClaimSmem& cl, int32_t* late, int late_cap, int count,
                                 const Forced& f, int wn, int tail_pages, int lane) {
  const int mid = count - f.F > 0 ? count - f.F : 0;
  int tail_listed = tail_pages < kTailPages ? tail_pages : kTailPages;
  if (mid + tail_listed > late_cap) tail_listed = late_cap - mid;
  const int listed = mid + tail_listed;
  for (int j0 = 0; j0 < listed; j0 += kWave) {
    const int j = j0 + lane;
    int64_t page = -1;
    if (j < mid) {
      page = lookup_page(p.v, b, late[f.e_init + j]);
    } else if (j < listed) {
      page = lookup_page(p.v, b, static_cast<int64_t>(wn) + (j - mid));
    }
    __builtin_amdgcn_wave_barrier();  // every lane has read its id before any lane writes
    if (j < listed) late[j] = static_cast<int32_t>(page);
  }
  if (lane == 0) {
    cl.late_mid = mid;
    cl.late_n = mid + tail_pages;
    cl.tail_listed = tail_listed;
  }
  // the wave's stores (an appended token among them) and LDS writes are
  // complete before any wave can reach the late positions
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  if (lane == 0) __hip_atomic_store(&cl.late_ready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Page source of the walk: this wave's planned positions (see above); all
// values wave-uniform.
struct PlanPages {
  ClaimSmem& cs;
  const int32_t* late;
  const attn::PoolView& v;
  int b;
  int wave;
  int F;        // forced positions listed early
  int n;        // sealed blocks
  int64_t len;  // tokens (after this step's append)
  int e_next;   // next forced position of this wave (F when done)
  int l_next = 0;
  int l_end = 0;
  bool ready = false;

  __device__ PlanPages(ClaimSmem& cs_, const int32_t* late_, const attn::PoolView& v_, int b_, int wave_, int F_,
                       int n_, int64_t len_)
      : cs(cs_), late(late_), v(v_), b(b_), wave(wave_), F(F_), n(n_), len(len_) {
    e_next = wave == 0 ? F : wave - 1;
  }

  // Forced positions of wave w (>= 1): w - 1, w - 1 + 7, ... below F.
  __device__ static int forced_count(int w, int F) {
    if (w == 0 || w - 1 >= F) return 0;
    return (F - (w - 1) + kWaves - 2) / (kWaves - 1);
  }

  // This wave's contiguous range of the late positions: every wave's total
  // (forced + late) is T / 8 or T / 8 + 1 with T = positions + kSelectPages,
  // wave 0 counting its selection as kSelectPages positions; the waves in
  // order, wave 7 taking any remainder.
  __device__ inline void plan_late(int late_n) {
    const int total = F + late_n + kSelectPages;
    int begin = 0;
    for (int w = 0; w <= wave; ++w) {
      const int target = total / kWaves + (w < total % kWaves ? 1 : 0);
      const int want = target - (w == 0 ? kSelectPages : forced_count(w, F));
      const int take = want > 0 ? want : 0;
      if (w == wave) {
        l_next = begin < late_n ? begin : late_n;
        const int end = begin + take;
        l_end = wave == kWaves - 1 ? late_n : (end < late_n ? end : late_n);
      }
      begin += take;
    }
  }

  __device__ inline attn::PageRef next(bool wait) {
    while (e_next < F) {
      const int c = e_next;
      e_next += kWaves - 1;
      const int32_t page = __builtin_amdgcn_readfirstlane(cs.early[c]);
      if (page >= 0) return attn::PageRef{page, kPageTokens};
    }
    if (!ready) {
      if (!wait && __hip_atomic_load(&cs.late_ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == 0)
        return attn::PageRef{0, -1};
      wait_late(cs);
      ready = true;
      plan_late(__builtin_amdgcn_readfirstlane(cs.late_n));
    }
    const int mid = __builtin_amdgcn_readfirstlane(cs.late_mid);
    const int tail_listed = __builtin_amdgcn_readfirstlane(cs.tail_listed);
    while (l_next < l_end) {
      const int j = l_next++;
      if (j < mid) {
        const int32_t page = __builtin_amdgcn_readfirstlane(late[j]);
        if (page >= 0) return attn::PageRef{page, kPageTokens};
        continue;
      }
      const int k = j - mid;
      const int64_t left = len - static_cast<int64_t>(n + k) * kPageTokens;
      const int valid = left < kPageTokens ? static_cast<int>(left) : kPageTokens;
      const int64_t page = k < tail_listed ? static_cast<int64_t>(__builtin_amdgcn_readfirstlane(late[j]))
                                           : lookup_page(v, b, static_cast<int64_t>(n) + k);
      if (page >= 0 && valid > 0) return attn::PageRef{page, valid};
    }
    return attn::PageRef{0, 0};
  }
};

// G = query heads per KV head; GR = query heads sharing one representative
// row (G for per-KV-head representatives, 1 for per-query-head ones);
// APPEND: decode step (append + seal first); F16: raw FP16 K/V input.
// No q/k/v producer: the step's query and token are inputs.
struct NoProducer {};

// Prod = qkv::ReduceParams: the step takes the q/k/v projection's K-slice
// partials instead of q, k and v, and runs their epilogue (qkv_epilogue.hpp)
// for its own heads at entry: wave 0 the group's query heads (32 lanes each),
// wave 1 KV head g's k (lanes 0..31) and v (lanes 32..63), the layout in which
// wave 1 appends the token.  q, k and v are also written out, the values the
// producer's reduce launch would write.
template <int G, int GR, bool APPEND, bool F16, bool ONLINE, class Prod>
__device__ inline void decode_body(const Params& p, const Prod& qp) {
  constexpr bool kProd = !std::is_same<Prod, NoProducer>::value;
  static_assert(!kProd || (G <= 2 && APPEND && !F16 && !ONLINE), "the producer epilogue: 1-2 heads, fp32 token");
  const int g = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;

  __shared__ float q_s[G * D];
  __shared__ uint32_t keys[kMaxSelectBlocks];  // block keys, then the selected ids, then the late pages
  __shared__ uint32_t hist[256];
  __shared__ attn::CombineSmem<G, kWaves> cs;
  __shared__ ClaimSmem cl;

  const int64_t out_row = static_cast<int64_t>(b) * p.v.kv_heads + g;
  // the group's query rows, loaded at entry (their latency overlaps the append)
  const float* q_group = p.query + (static_cast<int64_t>(b) * p.query_heads + g * G) * D;
  float q_entry = 0.0f;
  if constexpr (!kProd) q_entry = tid < G * D ? q_group[tid] : 0.0f;
  int64_t len = p.seq_len[b];
  int n = p.sealed[b];

  ushort4 tok{};
  if constexpr (kProd) {
    if (wave < 2) {
      const int half = lane / 32;
      const int j = lane % 32;
      // (with one query head, wave 0's upper half repeats it and stores nothing)
      const int hh = wave == 0 ? g * G + (half < G ? half : 0) : qp.q_heads + half * qp.kv_heads + g;
      const qkv::f32x4_t val = qkv::head_value(qp, hh, b, j);
      if (wave == 1 || half < G) *reinterpret_cast<qkv::f32x4_t*>(qkv::head_dst(qp, hh, b) + 4 * j) = val;
      if (wave == 0 && half < G) {
#pragma unroll
        for (int e = 0; e < 4; ++e) q_s[half * D + 4 * j + e] = val[e];
      }
      if (wave == 1) tok = make_ushort4(f2h_rne(val[0]), f2h_rne(val[1]), f2h_rne(val[2]), f2h_rne(val[3]));
    }
    // (no barrier: waves 2 and 3 go on to their prefetch; q_s is read after
    // the scoring's barrier, or the one before st.init)
  }

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
  // The arrival count is read at the end of the kernel, so that its round
  // trip overlaps the scoring; the representatives a seal wrote are visible
  // to the scoring after the query barrier below.
  SeqCommit commit{};
  if (APPEND) {
    commit.gen = p.generation ? p.generation[b] : 0;
    commit.appended = append_seal_head<G, F16, ONLINE, kProd>(p, b, g, len, n, commit.added,
                                                              reinterpret_cast<float*>(keys), tok);
    if (tid == 0) commit.arrived = atomicAdd(&p.arrive[b], 1);
  }

  attn::WaveState<G> st;
  const attn::LaneGeom lg = attn::lane_geom(p.v, g, lane);

  // ---- 2. score; the forced blocks' pages looked up meanwhile ----------------
  const bool n_ok = n >= 0 && n <= p.rep_stride && n <= kMaxSelectBlocks;
  const sel::Budget bs =
      n_ok ? sel::budget_split(n, p.budget, p.budgets, b, p.init_blocks, p.local_blocks, p.sel_stride)
           : sel::Budget{0, 0, 0, false, true};
  const Forced fb = forced_blocks(bs, n);
  const int32_t early = wave == kWaves - 1 ? early_page(p, b, n, fb, lane) : -1;
  if (n_ok && !bs.take_all) {  // (a budget that takes every block needs no scores)
    if (!kProd && tid < G * D) q_s[tid] = q_entry;
    __syncthreads();
    if (kPrefetch) {
      sel::score_blocks<GR, kThreads>(a, q_s, n, keys, nullptr, pre, have_pre);
    } else {
      sel::score_blocks<GR, kThreads>(a, q_s, n, keys, nullptr);
    }
  }
  if (wave == kWaves - 1) cl.early[lane] = early;
  if (tid == 0) cl.late_ready = 0;
  if (kProd && !(n_ok && !bs.take_all)) __syncthreads();  // q_s complete (no scoring barrier)
  st.init(kProd ? q_s : q_group, p.qscale, lg.col);
  // the walk's view of the sequence (a length below the sealed blocks is
  // flagged and walked as no tail)
  int wn = n;
  int64_t wlen = len;
  if (wn < 0 || wlen < static_cast<int64_t>(wn) * kPageTokens) {
    if (tid == 0) flag_status(p.v.status, kStatusBadLength);
    if (wn < 0) wn = 0;
    wlen = static_cast<int64_t>(wn) * kPageTokens;
  }
  const int tail_pages = static_cast<int>((wlen - static_cast<int64_t>(wn) * kPageTokens + kPageTokens - 1) /
                                          kPageTokens);
  __syncthreads();  // keys, the early pages and the flag visible

  // ---- 3. select (wave 0) and walk (every wave, planned positions) -------------
  int32_t* late = reinterpret_cast<int32_t*>(keys);  // the selected ids, then the late pages
  if (wave == 0) {
    int count = 0;
    if (!n_ok || bs.bad) {
      if (lane == 0) {
        flag_status(p.v.status, n_ok ? kStatusBadBudget : kStatusCapacity);
        p.counts[out_row] = 0;
      }
    } else {
      count = sel::select_ids_wave(keys, n, bs, hist, p.selected + out_row * p.sel_stride, p.sel_stride, late);
      if (lane == 0) p.counts[out_row] = count;
    }
    list_late(p, b, cl, late, kMaxSelectBlocks, count, fb, wn, tail_pages, lane);
  }
  PlanPages src(cl, late, p.v, b, wave, fb.F, wn, wlen);
  for (;;) {
    const attn::PageRef pr = src.next(true);
    if (pr.valid <= 0) break;
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
  if (APPEND && tid == 0) commit_sequence(p, b, len, n, commit);
}

// (the online seal's builder state takes more registers: 2 resident
// workgroups per compute unit, the fused grid's usual count, without spills)
template <int G, int GR, bool APPEND, bool F16, bool ONLINE = false>
__global__ __launch_bounds__(kThreads, ONLINE ? 2 : 4) void decode_kernel(const Params p) {
  decode_body<G, GR, APPEND, F16, ONLINE>(p, NoProducer{});
}

// The decode step fed by the q/k/v projection's partials (fp32 token).
template <int G, int GR>
__global__ __launch_bounds__(kThreads, 4) void decode_kernel_qkv(const Params p, const qkv::ReduceParams qp) {
  decode_body<G, GR, true, false, false>(p, qp);
}

// ---- shared selection: one block set per sequence over every query head -----
// The reference's shared mode (select_shared_blocks over all heads,
// selection.cpp:96-147, as its selection and pipeline drivers call it,
// selection_main.cpp:178-181, pipeline_main.cpp:480-499) as one launch.
// Every workgroup of a sequence (one per KV head) scores the whole shared set
// itself, so that no workgroup waits on another: a wave per representative
// row computes its query heads' dots (each the sequential fp32 sum over d),
// the dots meet in LDS, and one lane per block adds dot / heads in head
// order: the arithmetic of the split scoring (score_rows_kernel), so the
// scores are bit-identical.  Every workgroup then selects the same ids; the
// workgroup of KV head 0 writes them.  Each workgroup reads the sequence's
// representatives once per KV head, so the launch takes short lists only
// (select_attend_shared_supported()).
//
// A step that seals a block computes every KV head's representative of it in
// every workgroup and writes them all (the values are identical: the same
// sums of the same FP16 keys in token order; the new token's key comes from
// the step's input, as its own workgroup stores it to the page in this
// launch), so the scoring reads only representatives written by its own
// workgroup or by earlier launches.
template <bool F16>
__device__ inline bool append_seal_shared(const Params& p, int b, int g, int64_t& len, int& n, int& added) {
  const int tid = threadIdx.x;
  const int64_t page = table_page(p.v, b, len / kPageTokens);
  if (page < 0) {
    if (tid == 0) flag_status(p.v.status, kStatusCapacity);
    return false;
  }
  if (tid < kWave) store_token_quad(p, page, len, g, tid, token_quad<F16>(p, b, g, tid));
  const int64_t pos = len;  // the new token
  len += 1;
  const int kv = p.v.kv_heads;
  while (len >= static_cast<int64_t>(n + 1) * kPageTokens + p.local_tokens) {
    const int64_t sp = n < p.rep_stride ? table_page(p.v, b, n) : -1;
    if (sp < 0) {
      if (tid == 0) flag_status(p.v.status, kStatusCapacity);
      break;
    }
    const int64_t first = static_cast<int64_t>(n) * kPageTokens;
    for (int e = tid; e < kv * D; e += kThreads) {
      const int h = e / D;
      const int d = e % D;
      const int64_t in = (static_cast<int64_t>(b) * kv + h) * D + d;
      const uint16_t fresh = F16 ? p.k16[in] : f2h_rne(p.k[in]);
      const uint16_t* src = p.v.pool + sp * p.v.page_elems + h * D + d;
      float sum = 0.0f;
#pragma unroll 8
      for (int t = 0; t < kPageTokens; ++t) sum = sum + h2f(first + t == pos ? fresh : src[t * p.v.token_elems]);
      p.reps[((static_cast<int64_t>(b) * p.rep_heads + h) * D + d) * p.rep_stride + n] =
          sum / static_cast<float>(kPageTokens);
    }
    ++n;
    ++added;
  }
  return true;
}

// G = query heads per KV head (1, 2 or 4; representatives per KV head, G
// heads per representative row; the pages walked in registers); APPEND:
// decode step; F16: raw FP16 K/V input.
template <int G, bool APPEND, bool F16>
__global__ __launch_bounds__(kThreads) void decode_kernel_shared(const Params p) {
  const int g = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;

  __shared__ __align__(16) float q_t[kMaxSelectHeads * D];
  __shared__ float dots[kMaxSelectHeads][kWave + 1];
  // block keys, then the selected ids, then the late pages; the register
  // selection reads n rounded up to a multiple of 256 keys
  constexpr int kKeys = (kMaxSharedFusedBlocks + 255) / 256 * 256 + kTailPages;
  __shared__ uint32_t keys[kKeys];
  __shared__ uint32_t hist[256];
  __shared__ attn::CombineSmem<G, kWaves> cs;
  __shared__ ClaimSmem cl;

  const float* q_group = p.query + (static_cast<int64_t>(b) * p.query_heads + g * G) * D;
  int64_t len = p.seq_len[b];
  int n = p.sealed[b];

  SeqCommit commit{};
  if (APPEND) {
    commit.gen = p.generation ? p.generation[b] : 0;
    commit.appended = append_seal_shared<F16>(p, b, g, len, n, commit.added);
    if (tid == 0) commit.arrived = atomicAdd(&p.arrive[b], 1);
  }

  attn::WaveState<G> st;
  const attn::LaneGeom lg = attn::lane_geom(p.v, g, lane);

  // ---- score the shared set (every query head); forced pages looked up -------
  const bool n_ok = n >= 0 && n <= p.rep_stride && n <= kMaxSharedFusedBlocks;
  const sel::Budget bs =
      n_ok ? sel::budget_split(n, p.budget, p.budgets, b, p.init_blocks, p.local_blocks, p.sel_stride)
           : sel::Budget{0, 0, 0, false, true};
  const Forced fb = forced_blocks(bs, n);
  const int32_t early = wave == kWaves - 1 ? early_page(p, b, n, fb, lane) : -1;
  if (n_ok && !bs.take_all) {  // (a budget that takes every block needs no scores)
    sel::ScoreArgs a{};
    a.query = p.query;
    a.reps = p.reps;
    a.b = b;
    a.h_first = 0;
    a.heads_per_sel = p.query_heads;
    a.query_heads = p.query_heads;
    a.group = G;
    a.rep_heads = p.rep_heads;
    a.rep_stride = p.rep_stride;
    sel::load_query_t<kThreads>(a, q_t);
    __syncthreads();  // the query, and the representatives this workgroup sealed
    const int hps = p.query_heads;
    const float heads_f = static_cast<float>(hps);
    // dot / heads for a power-of-two head count: the product with the exact
    // reciprocal rounds the same exact value once, as the division does
    const bool pow2 = (hps & (hps - 1)) == 0;
    const float inv = 1.0f / heads_f;
    for (int c0 = 0; c0 < n; c0 += kWave) {
      const int blk = c0 + lane;
      if (blk < n) {
        for (int h0 = wave * G; h0 < hps; h0 += kWaves * G) {
          float dot[G][1];
          sel::row_dots<G, 1, 32>(a, q_t, blk, h0, dot);
#pragma unroll
          for (int j = 0; j < G; ++j) dots[h0 + j][lane] = dot[j][0];
        }
      }
      __syncthreads();
      if (tid < kWave && c0 + tid < n) {
        float score = 0.0f;
        if (pow2) {
          for (int h = 0; h < hps; ++h) score = score + dots[h][tid] * inv;
        } else {
          for (int h = 0; h < hps; ++h) score = score + dots[h][tid] / heads_f;
        }
        keys[c0 + tid] = sel::order_key(score);
      }
      __syncthreads();
    }
  }
  if (wave == kWaves - 1) cl.early[lane] = early;
  if (tid == 0) cl.late_ready = 0;
  st.init(q_group, p.qscale, lg.col);
  int wn = n;
  int64_t wlen = len;
  if (wn < 0 || wlen < static_cast<int64_t>(wn) * kPageTokens) {
    if (tid == 0) flag_status(p.v.status, kStatusBadLength);
    if (wn < 0) wn = 0;
    wlen = static_cast<int64_t>(wn) * kPageTokens;
  }
  const int tail_pages = static_cast<int>((wlen - static_cast<int64_t>(wn) * kPageTokens + kPageTokens - 1) /
                                          kPageTokens);
  __syncthreads();  // keys, the early pages and the flag visible

  // ---- select (wave 0; the workgroup of KV head 0 writes the ids) and walk ----
  int32_t* late = reinterpret_cast<int32_t*>(keys);
  if (wave == 0) {
    int count = 0;
    if (!n_ok || bs.bad) {
      if (lane == 0) {
        flag_status(p.v.status, n_ok ? kStatusBadBudget : kStatusCapacity);
        if (g == 0) p.counts[b] = 0;
      }
    } else {
      count = sel::select_ids_wave(keys, n, bs, hist, g == 0 ? p.selected + static_cast<int64_t>(b) * p.sel_stride
                                                              : nullptr,
                                   p.sel_stride, late);
      if (lane == 0 && g == 0) p.counts[b] = count;
    }
    list_late(p, b, cl, late, kKeys, count, fb, wn, tail_pages, lane);
  }
  PlanPages src(cl, late, p.v, b, wave, fb.F, wn, wlen);
  for (;;) {
    const attn::PageRef pr = src.next(true);
    if (pr.valid <= 0) break;
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
  if (APPEND && tid == 0) commit_sequence(p, b, len, n, commit);
}


// ---- one launch at a head_dim other than 128 (up to 256) -----------------------
// decode_kernel's step with the head_dim at run time (hd): append + seal of
// KV head g (the new token as hd / 4 four-value pieces of K and of V; the
// seal's mean key summed in token order by hd threads), the group's scoring
// with one lane per block (the GR = G query heads sharing the KV head's
// representative row summed side by side over one pass of it, the
// reference's sequential dots, then dot / heads in head order: the
// arithmetic of score_any_kernel, bit-identical scores), wave 0's selection
// and the planned walk of the forced, selected and tail pages, each page
// with the token-row walk of attn_rows.hpp (LPR lanes per token row).
// Representatives per KV head only.
constexpr int kRowsMaxG = 4;

template <bool F16>
__device__ inline bool append_seal_head_any(const Params& p, int b, int g, int hd, int64_t& len, int& n,
                                            int& added) {
  const int tid = threadIdx.x;
  const int64_t page = table_page(p.v, b, len / kPageTokens);
  if (page < 0) {
    if (tid == 0) flag_status(p.v.status, kStatusCapacity);
    return false;
  }
  const int pieces = hd / 4;  // four values each, of K then of V
  for (int u = tid; u < 2 * pieces; u += kThreads) {
    const int is_v = u / pieces;
    const int e = (u % pieces) * 4;
    const int64_t src = (static_cast<int64_t>(b) * p.v.kv_heads + g) * hd + e;
    ushort4 h;
    if constexpr (F16) {
      h = *reinterpret_cast<const ushort4*>((is_v ? p.v16 : p.k16) + src);
    } else {
      const float4 f = *reinterpret_cast<const float4*>((is_v ? p.vv : p.k) + src);
      h = make_ushort4(f2h_rne(f.x), f2h_rne(f.y), f2h_rne(f.z), f2h_rne(f.w));
    }
    uint16_t* dst = const_cast<uint16_t*>(p.v.pool) + page * p.v.page_elems +
                    (len % kPageTokens) * p.v.token_elems + static_cast<int64_t>(is_v) * p.v.kv_heads * hd +
                    static_cast<int64_t>(g) * hd + e;
    *reinterpret_cast<ushort4*>(dst) = h;
  }
  len += 1;
  // the new token visible to the seal below; without a seal nothing in this
  // workgroup reads it
  if (len >= static_cast<int64_t>(n + 1) * kPageTokens + p.local_tokens) __syncthreads();
  while (len >= static_cast<int64_t>(n + 1) * kPageTokens + p.local_tokens) {
    const int64_t sp = n < p.rep_stride ? table_page(p.v, b, n) : -1;
    if (sp < 0) {
      if (tid == 0) flag_status(p.v.status, kStatusCapacity);
      break;
    }
    if (tid < hd) {
      const uint16_t* src = p.v.pool + sp * p.v.page_elems + static_cast<int64_t>(g) * hd + tid;
      float sum = 0.0f;
#pragma unroll 8
      for (int t = 0; t < kPageTokens; ++t) sum = sum + h2f(src[t * p.v.token_elems]);
      p.reps[((static_cast<int64_t>(b) * p.rep_heads + g) * hd + tid) * p.rep_stride + n] =
          sum / static_cast<float>(kPageTokens);
    }
    ++n;
    ++added;
  }
  return true;
}

// Score of block blk for the group's G heads (one representative row),
// q_s = the G query rows of hd floats in LDS.
template <int G>
__device__ inline float score_block_any(const Params& p, const float* q_s, int b, int g, int hd, int blk) {
  constexpr int kBatch = 32;
  const int64_t stride = p.rep_stride;
  const float* r = p.reps + (static_cast<int64_t>(b) * p.rep_heads + g) * hd * stride + blk;
  float dot[G];
#pragma unroll
  for (int j = 0; j < G; ++j) dot[j] = 0.0f;
  for (int d0 = 0; d0 < hd; d0 += kBatch) {
    float rv[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k)
      rv[k] = d0 + k < hd ? load_stream_f32(r + static_cast<int64_t>(d0 + k) * stride) : 0.0f;
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      if (d0 + k >= hd) break;
#pragma unroll
      for (int j = 0; j < G; ++j) dot[j] = dot[j] + q_s[j * hd + d0 + k] * rv[k];
    }
  }
  const float heads_f = static_cast<float>(G);
  float score = 0.0f;
#pragma unroll
  for (int j = 0; j < G; ++j) score = score + dot[j] / heads_f;
  return score;
}

template <int G, int LPR, bool F16>
__global__ __launch_bounds__(kThreads) void decode_kernel_rows(const Params p, int hd) {
  static_assert(G <= kRowsMaxG, "1, 2 or 4 query heads per KV head");
  using State = rows::RowsState<G, LPR>;
  const int g = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;

  __shared__ __align__(16) float q_s[G * rows::kMaxHeadDim];
  __shared__ uint32_t keys[kMaxSelectBlocks];  // block keys, then the selected ids, then the late pages
  __shared__ uint32_t hist[256];
  __shared__ ClaimSmem cl;
  __shared__ float w_ml[kWaves][G][2];
  __shared__ float w_acc[kWaves][G][LPR * 8];

  const int64_t out_row = static_cast<int64_t>(b) * p.v.kv_heads + g;
  const float* q_group = p.query + (static_cast<int64_t>(b) * p.query_heads + g * G) * hd;
  for (int e = tid; e < G * hd; e += kThreads) q_s[e] = q_group[e];
  int64_t len = p.seq_len[b];
  int n = p.sealed[b];

  SeqCommit commit{};
  commit.gen = p.generation ? p.generation[b] : 0;
  commit.appended = append_seal_head_any<F16>(p, b, g, hd, len, n, commit.added);
  if (tid == 0) commit.arrived = atomicAdd(&p.arrive[b], 1);

  State st;
  st.init(q_group, hd, p.qscale, lane);

  // ---- score; the forced blocks' pages looked up meanwhile ----------------
  const bool n_ok = n >= 0 && n <= p.rep_stride && n <= kMaxSelectBlocks;
  const sel::Budget bs =
      n_ok ? sel::budget_split(n, p.budget, p.budgets, b, p.init_blocks, p.local_blocks, p.sel_stride)
           : sel::Budget{0, 0, 0, false, true};
  const Forced fb = forced_blocks(bs, n);
  const int32_t early = wave == kWaves - 1 ? early_page(p, b, n, fb, lane) : -1;
  __syncthreads();  // the query rows, and the representatives this workgroup sealed
  if (n_ok && !bs.take_all) {  // (a budget that takes every block needs no scores)
    for (int blk = tid; blk < n; blk += kThreads) keys[blk] = sel::order_key(score_block_any<G>(p, q_s, b, g, hd, blk));
  }
  if (wave == kWaves - 1) cl.early[lane] = early;
  if (tid == 0) cl.late_ready = 0;
  int wn = n;
  int64_t wlen = len;
  if (wn < 0 || wlen < static_cast<int64_t>(wn) * kPageTokens) {
    if (tid == 0) flag_status(p.v.status, kStatusBadLength);
    if (wn < 0) wn = 0;
    wlen = static_cast<int64_t>(wn) * kPageTokens;
  }
  const int tail_pages = static_cast<int>((wlen - static_cast<int64_t>(wn) * kPageTokens + kPageTokens - 1) /
                                          kPageTokens);
  __syncthreads();  // keys, the early pages and the flag visible

  // ---- select (wave 0) and walk (every wave, planned positions) -------------
  int32_t* late = reinterpret_cast<int32_t*>(keys);
  if (wave == 0) {
    int count = 0;
    if (!n_ok || bs.bad) {
      if (lane == 0) {
        flag_status(p.v.status, n_ok ? kStatusBadBudget : kStatusCapacity);
        p.counts[out_row] = 0;
      }
    } else {
      count = sel::select_ids_wave(keys, n, bs, hist, p.selected + out_row * p.sel_stride, p.sel_stride, late);
      if (lane == 0) p.counts[out_row] = count;
    }
    list_late(p, b, cl, late, kMaxSelectBlocks, count, fb, wn, tail_pages, lane);
  }
  const int64_t lane_off = st.lane_offset(p.v.token_elems, g, hd);
  const int64_t v_off = static_cast<int64_t>(p.v.kv_heads) * hd;
  PlanPages src(cl, late, p.v, b, wave, fb.F, wn, wlen);
  for (;;) {
    const attn::PageRef pr = src.next(true);
    if (pr.valid <= 0) break;
    st.attend_page(p.v.pool + pr.page * p.v.page_elems + lane_off, p.v.token_elems, v_off, pr.valid);
  }

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
  for (int e = tid; e < G * hd; e += kThreads) {
    const int h = e / hd;
    const int d = e % hd;
    float mx = rows::kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, w_ml[w][h][0]);
    float lw = 0.0f, aw = 0.0f;
    if (mx != rows::kNegInf) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float f = __builtin_amdgcn_exp2f(w_ml[w][h][0] - mx);  // waves without tokens: 0
        lw += w_ml[w][h][1] * f;
        aw += w_acc[w][h][d] * f;
      }
    }
    p.out[(static_cast<int64_t>(b) * p.query_heads + g * G + h) * hd + d] = lw > 0.0f ? aw / lw : 0.0f;
  }
  if (tid == 0) commit_sequence(p, b, len, n, commit);
}


// ---- 4 query heads per KV head: LDS-staged pages, q.K on the matrix cores --
// One 8-wave workgroup per (sequence, KV head), one per CU (the eight 16 KiB
// page slots).  After append + seal, all 512 threads score two blocks per lane
// (8-byte representative loads); the keys borrow the page slots of waves 0
// and 1.  Then every wave walks its planned positions (the planned walk
// above) with the staged walk of attn_core.hpp (pages HBM -> LDS by DMA, q.K
// on v_mfma_f32_16x16x32_f16), one page in flight while the previous one is
// computed.  A step that seals nothing stores its token at the start of the
// walk phase (wave 0, before it lists the tail).
template <int GR, bool APPEND, bool F16, bool ONLINE = false>
__global__ __launch_bounds__(kThreads) void decode_kernel_staged(const Params p) {
  constexpr int G = 4;
  constexpr int kStageBytes = kWaves * attn::kStageVecs * 16;
  constexpr int kPbufFloats = (G * 32 + G + 3) / 4 * 4;
  constexpr int kSlotBytes = attn::kStageVecs * 16;
  static_assert(kMaxSelectBlocks * 4 <= 2 * kSlotBytes, "keys fit the page slots of waves 0 and 1");
  static_assert(sizeof(attn::CombineRowsSmem<G, kWaves>) <= kStageBytes, "combine fits the page slots");
  static_assert(kEarly <= kWave, "one lane per early lookup");
  const int g = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;

  // The probabilities' LDS buffer is its own variable: the compiler then
  // knows the staging loads in flight (into smem) do not write it, and its
  // stores need not wait for them (one variable for both made every page's
  // P.V wait for the next page's staging loads to land).
  __shared__ __align__(16) unsigned char smem[kStageBytes];
  __shared__ __align__(16) float pbuf_s[kWaves * kPbufFloats];
  __shared__ __align__(16) float q_t[G * D];
  __shared__ uint32_t hist[256];
  __shared__ ClaimSmem cl;
  __shared__ int32_t late_ids[kStagedIds + kTailPages];  // the selected ids, then (in place) the late pages
  uint32_t* keys = reinterpret_cast<uint32_t*>(smem);
  uint4* stage = reinterpret_cast<uint4*>(smem) + wave * attn::kStageVecs;
  float* pbuf = pbuf_s + wave * kPbufFloats;
  const float* q_group = p.query + (static_cast<int64_t>(b) * p.query_heads + g * G) * D;

  const int64_t out_row = static_cast<int64_t>(b) * p.v.kv_heads + g;
  // the group's query rows, loaded at entry (their latency overlaps the append)
  const float q_entry = q_group[tid % (G * D)];
  int64_t len = p.seq_len[b];
  int n = p.sealed[b];

  // ---- 1. append + seal (decode step; arrival read at the end, as above) ------
  // A step that seals a block appends and seals here, before the scoring.
  // Otherwise nothing reads the new token before the page walk: wave 0
  // stores it at the start of the walk phase, before it lists the tail (the
  // tail page's id and the token are loaded now; their latency overlaps the
  // scoring).
  SeqCommit commit{};
  bool deferred = false;
  int64_t tail_page = -1;
  ushort4 token{};
  if (APPEND) {
    commit.gen = p.generation ? p.generation[b] : 0;
    if (append_seals(p, len, n)) {
      commit.appended =
          append_seal_head<G, F16, ONLINE>(p, b, g, len, n, commit.added, reinterpret_cast<float*>(smem));
    } else {
      deferred = true;
      tail_page = table_page(p.v, b, len / kPageTokens);
      if (wave == 0) token = token_quad<F16>(p, b, g, lane);
    }
    if (tid == 0) commit.arrived = atomicAdd(&p.arrive[b], 1);
  }

  attn::WaveState<G> st;
  st.reset();
  const attn::LaneGeom lg = attn::lane_geom(p.v, g, lane);

  // ---- 2. score; the forced blocks' pages looked up meanwhile ----------------
  const bool n_ok = n >= 0 && n <= p.rep_stride && n <= kMaxSelectBlocks;
  const sel::Budget bs =
      n_ok ? sel::budget_split(n, p.budget, p.budgets, b, p.init_blocks, p.local_blocks, p.sel_stride)
           : sel::Budget{0, 0, 0, false, true};
  const Forced fb = forced_blocks(bs, n);
  const int32_t early = wave == kWaves - 1 ? early_page(p, b, n, fb, lane) : -1;
  if (n_ok && !bs.take_all) {  // (a budget that takes every block needs no scores)
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
    static_assert(G * D == kThreads, "one query element per thread");
    q_t[(tid % D) * G + tid / D] = q_entry;
    __syncthreads();
    sel::score_blocks_vec<GR, 2, kThreads>(a, q_t, n, keys, nullptr, tid);
  }
  if (ONLINE && deferred && tail_page >= 0) {
    // the group's query rows of this step to the ring (read by later seals)
    const int64_t slot = len % p.online.ring_tokens;
    const int h = g * G + tid / D;
    p.online.ring[((static_cast<int64_t>(b) * p.online.query_heads + h) * p.online.ring_tokens + slot) * D +
                  tid % D] = q_entry;
  }
  if (wave == kWaves - 1) cl.early[lane] = early;
  if (tid == 0) cl.late_ready = 0;
  if (deferred && tail_page >= 0) {
    commit.appended = true;
    len += 1;
  }
  // the tail after this step's append (the walk's view: a length below the
  // sealed blocks is flagged and walked as no tail)
  int wn = n;
  int64_t wlen = len;
  if (wn < 0 || wlen < static_cast<int64_t>(wn) * kPageTokens) {
    if (tid == 0) flag_status(p.v.status, kStatusBadLength);
    if (wn < 0) wn = 0;
    wlen = static_cast<int64_t>(wn) * kPageTokens;
  }
  const int64_t tail_tokens = wlen - static_cast<int64_t>(wn) * kPageTokens;
  const int tail_pages = static_cast<int>((tail_tokens + kPageTokens - 1) / kPageTokens);
  __syncthreads();  // keys, the early pages and the flag visible

  // ---- 3. select (wave 0) and walk (every wave, planned positions) -------------
  if (wave == 0) {
    if (deferred) {
      if (tail_page >= 0) store_token_quad(p, tail_page, len - 1, g, lane, token);
      else if (lane == 0) flag_status(p.v.status, kStatusCapacity);
    }
    int count = 0;
    if (!n_ok || bs.bad) {
      if (lane == 0) {
        flag_status(p.v.status, n_ok ? kStatusBadBudget : kStatusCapacity);
        p.counts[out_row] = 0;
      }
    } else {
      count = sel::select_ids_wave(keys, n, bs, hist, p.selected + out_row * p.sel_stride, p.sel_stride, late_ids);
      if (lane == 0) p.counts[out_row] = count;
    }
    list_late(p, b, cl, late_ids, kStagedIds + kTailPages, count, fb, wn, tail_pages, lane);
  }
  const bool waits = wave != 0 && wave * kSlotBytes < n * 4;  // the keys reach into this wave's page slot
  if (waits) wait_late(cl);
  PlanPages src(cl, late_ids, p.v, b, wave, fb.F, wn, wlen);
  st.attend_staged(p.v, src, lg, lane, g, stage, pbuf, q_group, p.qscale);
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
  if (APPEND && tid == 0) commit_sequence(p, b, len, n, commit);
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

// Representative bytes the shared one-launch step may read beyond the split
// scoring's single pass (each of a sequence's kv_heads workgroups reads all
// of them): 32 MiB, a few microseconds of HBM.
constexpr int64_t kSharedRepeatBytes = int64_t{32} << 20;

bool select_attend_shared_supported(int32_t batch, int32_t query_heads, int32_t kv_heads, int32_t rep_heads,
                                    int32_t select_groups, int32_t rep_stride) {
  if (select_groups != 1 || kv_heads <= 1 || rep_heads != kv_heads || query_heads > kMaxSelectHeads) return false;
  const int group = query_heads / kv_heads;
  if (group != 1 && group != 2 && group != 4) return false;
  if (rep_stride < 0 || rep_stride > kMaxSharedFusedBlocks) return false;
  const int64_t repeat = static_cast<int64_t>(batch) * kv_heads * (kv_heads - 1) * rep_stride * D * sizeof(float);
  return repeat <= kSharedRepeatBytes;
}

template <bool APPEND, bool F16>
hipError_t launch_shared(const Params& p, int batch, hipStream_t stream) {
  const dim3 grid(p.v.kv_heads, batch);
  const int group = p.query_heads / p.v.kv_heads;
  if (group == 1) {
    hipLaunchKernelGGL((decode_kernel_shared<1, APPEND, F16>), grid, dim3(kThreads), 0, stream, p);
  } else if (group == 2) {
    hipLaunchKernelGGL((decode_kernel_shared<2, APPEND, F16>), grid, dim3(kThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((decode_kernel_shared<4, APPEND, F16>), grid, dim3(kThreads), 0, stream, p);
  }
  return hipGetLastError();
}

bool select_attend_rows_supported(int32_t query_heads, int32_t kv_heads, int32_t rep_heads, int32_t select_groups,
                                  int32_t head_dim) {
  if (kv_heads <= 0 || select_groups != kv_heads || rep_heads != kv_heads) return false;
  const int group = query_heads / kv_heads;
  return (group == 1 || group == 2 || group == 4) && head_dim > 0 && head_dim % 8 == 0 &&
         head_dim <= rows::kMaxHeadDim && head_dim != kHeadDim;
}

template <int LPR, bool F16>
hipError_t launch_rows_step(const Params& p, int batch, int hd, hipStream_t stream) {
  const dim3 grid(p.v.kv_heads, batch);
  switch (p.query_heads / p.v.kv_heads) {
    case 1: hipLaunchKernelGGL((decode_kernel_rows<1, LPR, F16>), grid, dim3(kThreads), 0, stream, p, hd); break;
    case 2: hipLaunchKernelGGL((decode_kernel_rows<2, LPR, F16>), grid, dim3(kThreads), 0, stream, p, hd); break;
    default: hipLaunchKernelGGL((decode_kernel_rows<4, LPR, F16>), grid, dim3(kThreads), 0, stream, p, hd); break;
  }
  return hipGetLastError();
}

template <bool F16>
hipError_t launch_rows_lpr(const Params& p, int batch, int hd, hipStream_t stream) {
  switch (rows::lanes_per_row(hd)) {
    case 8: return launch_rows_step<8, F16>(p, batch, hd, stream);
    case 16: return launch_rows_step<16, F16>(p, batch, hd, stream);
    default: return launch_rows_step<32, F16>(p, batch, hd, stream);
  }
}

namespace {

Params step_params(const SelectAttendLaunch& s, int hd) {
  Params p{};
  p.v.pool = s.pool;
  p.v.table = s.table;
  p.v.status = s.status;
  p.v.num_pages = s.num_pages;
  p.v.contig_tokens = 0;
  p.v.token_elems = 2 * s.kv_heads * hd;
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
  return p;
}

}  // namespace

hipError_t launch_select_attend(const SelectAttendLaunch& s, hipStream_t stream) {
  const int hd = s.head_dim > 0 ? s.head_dim : kHeadDim;
  if (hd != kHeadDim) {
    // another head_dim: the decode step only, representatives per KV head
    if (!s.append || !s.arrive || s.ring ||
        !select_attend_rows_supported(s.query_heads, s.kv_heads, s.rep_heads, s.select_groups, hd))
      return hipErrorInvalidValue;
    const Params p = step_params(s, hd);
    return s.k16 ? launch_rows_lpr<true>(p, s.batch, hd, stream) : launch_rows_lpr<false>(p, s.batch, hd, stream);
  }
  const bool shared = s.select_groups != s.kv_heads;
  if (shared ? !select_attend_shared_supported(s.batch, s.query_heads, s.kv_heads, s.rep_heads, s.select_groups,
                                               s.rep_stride)
             : !select_attend_supported(s.query_heads, s.kv_heads, s.select_groups, s.sel_stride, s.reps,
                                        s.rep_stride))
    return hipErrorInvalidValue;
  if (s.append && !s.arrive) return hipErrorInvalidValue;
  Params p = step_params(s, D);
  if (shared) {
    if (s.ring) return hipErrorInvalidValue;
    if (!s.append) return launch_shared<false, false>(p, s.batch, stream);
    return s.k16 ? launch_shared<true, true>(p, s.batch, stream) : launch_shared<true, false>(p, s.batch, stream);
  }
  if (s.ring) {
    if (!s.append || s.k16) return hipErrorInvalidValue;
    p.online = online::Args{s.ring, s.ring_tokens, s.window, s.topk, s.query_heads, s.seal_scale};
    return launch_online(p, s.batch, stream);
  }
  if (!s.append) return launch_mode<false, false>(p, s.batch, stream);
  return s.k16 ? launch_mode<true, true>(p, s.batch, stream) : launch_mode<true, false>(p, s.batch, stream);
}

bool decode_step_qkv_supported(int32_t query_heads, int32_t kv_heads, int32_t select_groups, int32_t head_dim) {
  if (kv_heads <= 0 || select_groups != kv_heads || (head_dim != 0 && head_dim != kHeadDim)) return false;
  const int group = query_heads / kv_heads;
  return group == 1 || group == 2;
}

hipError_t launch_decode_step_qkv(const SelectAttendLaunch& s, const qkv::ReduceParams& r, hipStream_t stream) {
  if (!s.append || !s.arrive || s.ring || s.k16 || !s.k || !s.v || r.rows != s.batch ||
      r.q_heads != s.query_heads || r.kv_heads != s.kv_heads || r.q != s.query ||
      !decode_step_qkv_supported(s.query_heads, s.kv_heads, s.select_groups, s.head_dim))
    return hipErrorInvalidValue;
  const Params p = step_params(s, D);
  const dim3 grid(s.kv_heads, s.batch);
  const int group = s.query_heads / s.kv_heads;
  if (group == 1) {
    hipLaunchKernelGGL((decode_kernel_qkv<1, 1>), grid, dim3(kThreads), 0, stream, p, r);
  } else if (s.rep_heads == s.query_heads) {
    hipLaunchKernelGGL((decode_kernel_qkv<2, 1>), grid, dim3(kThreads), 0, stream, p, r);
  } else {
    hipLaunchKernelGGL((decode_kernel_qkv<2, 2>), grid, dim3(kThreads), 0, stream, p, r);
  }
  return hipGetLastError();
}

}  // namespace sa
