// represent.hip — InfLLM local-causal block representatives of a prefill on
// the GPU (gfx950): the reference's build_local_causal_representatives
// (cpp/src/selection.cpp:12-94).
//
//   1. window_softmax_kernel: for every (query head h, query position q) the
//      logits of the keys [max(0, q+1-W), q] of h's KV head (sequential fp32
//      dot over head_dim, no contraction, times 1/sqrt(head_dim)), their max,
//      exp(logit - max) and the sequential denominator, and the
//      probabilities p = e / denominator.  Lanes: WL lanes per query (WL the
//      power of two >= W / 4, at most 64); lane l of a query takes the four
//      window positions w = l, l + WL, l + 2 WL, l + 3 WL, so each query value
//      read from LDS serves four keys; the denominator is summed in window
//      order by every lane of the query from the exponentials staged in LDS.
//   2. block_topk_kernel: per (h, 32-token block), each token's received
//      mass (the sum over the queries whose window holds it, in ascending
//      query order, as the reference accumulates it), a stable descending
//      rank (ties keep token order), the top-k token offsets, and the
//      representative = sum of the chosen keys in rank order / k.
// Those two kernels are tiled for head_dim 128, 32-token blocks and windows
// up to 256; window_softmax_any_kernel and block_topk_any_kernel (below)
// take any head_dim, block size and window with the same arithmetic.
//
// The exponential is expf_glibc(): the method of glibc 2.35's expf, which is
// what the reference's std::exp(float) runs (a 32-entry 2^(i/32) table, a
// degree-3 polynomial in double, and the fused multiply-adds of glibc's
// x86-64 FMA build), so the probabilities, received masses, chosen tokens and
// representatives equal the reference's bit for bit.  Compiled with
// -ffp-contract=off: every float product and sum is rounded separately, as in
// the reference, and the double steps fuse exactly where written.
#include "expf_glibc.hpp"
#include "sa_device.hpp"
#include "sa_internal.hpp"

namespace sa {
namespace {

constexpr int D = kHeadDim;
constexpr int kMaxKeysPerLane = 4;  // window <= 4 x 64
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// Workgroup of the window kernel: 256 threads, at most 64 queries (33 KB of
// staged queries).
template <int WL>
constexpr int window_threads() { return WL >= 4 ? 256 : 64 * WL; }

// The rounded product q * k of an FP16 key: fma(q, k, +0) rounds q * k once,
// exactly as a separate multiply does (the sum +0 only turns a -0 product into
// +0, which no later addition to the running dot can tell apart), and lets
// the compiler read the FP16 operand directly (v_fma_mix_f32).
__device__ inline float mul_h(float q, uint32_t w, int hi) {
  return __builtin_fmaf(q, hi ? hi_h2f(w) : lo_h2f(w), 0.0f);
}

struct Params {
  const float* pq;      // [hq][tokens][D] prompt queries
  const uint16_t* kv;   // [tokens][2][hkv][D] FP16 bits
  float* prob;          // [hq][tokens][window] probabilities (workspace)
  float* received;      // [hq][tokens]
  float* values;        // [hq][blocks][D] or null
  float* reps;          // [hq][D][rep_stride] or null
  int32_t* offsets;     // [hq][blocks][topk] or null
  int64_t tokens;
  int32_t hq;
  int32_t hkv;
  int32_t head_dim;      // the general kernels' (the tiled ones are built for D)
  int32_t block_tokens;  // the general kernels' (the tiled ones: 32)
  int32_t window;
  int32_t topk;
  int32_t rep_stride;
  float scale;
};

// Workgroup -> (tile x, query head y) of a grid (nx tiles, hq heads).
// Workgroups are dispatched in order x fastest and handed to the 8 XCDs
// round robin; when their count is a multiple of 8, dispatch number i is
// given the (i mod 8)-th eighth of the order (KV group, tile, query head in
// the group), so that each XCD's L2 sees consecutive tiles, whose key rows
// and probability rows overlap, and the query heads that share a KV head,
// next to each other.
__device__ inline void xcd_tile(int hq, int hkv, int& x, int& y) {
  const int nx = static_cast<int>(gridDim.x);
  const int group = hq / hkv;
  const int id = static_cast<int>(blockIdx.x) + static_cast<int>(blockIdx.y) * nx;
  const int total = nx * hq;
  const int v = total % 8 == 0 ? (id % 8) * (total / 8) + id / 8 : id;
  const int per_kv = nx * group;
  const int rem = v % per_kv;
  x = rem / group;
  y = (v / per_kv) * group + rem % group;
}

// Lanes per query: WL (a power of two, 1..64); queries per wave 64 / WL.
// STAGE: the keys of the workgroup's windows are staged in LDS (rows padded
// by 16 bytes so the lanes of a query, reading consecutive rows, hit
// different banks); without it every lane reads its own 4 KiB-strided key
// row from global memory, which the address units serialise.
template <int WL, bool STAGE>
__global__ __launch_bounds__(window_threads<WL>()) void window_softmax_kernel(const Params p) {
  constexpr int kWindowThreads = window_threads<WL>();
  constexpr int kQueriesPerGroup = kWindowThreads / WL;
  constexpr int kRowVecs = D / 8;                              // 16 uint4 per key row
  constexpr int kMaxRows = STAGE ? kQueriesPerGroup + kMaxKeysPerLane * WL - 1 : 1;
  int tile, h;
  xcd_tile(p.hq, p.hkv, tile, h);
  const int tid = threadIdx.x;
  const int qi = tid / WL;          // query within the workgroup
  const int wl = tid % WL;          // window lane within the query
  const int g = h / (p.hq / p.hkv);
  const int64_t q0 = static_cast<int64_t>(tile) * kQueriesPerGroup;
  const int64_t q = q0 + qi;
  const int64_t token_elems = 2LL * p.hkv * D;

  // query rows padded by 16 bytes: the 64 / WL queries of a wave read the
  // same column at once, which unpadded 512-byte rows put in one bank group
  __shared__ __align__(16) float q_s[kQueriesPerGroup][D + 4];
  __shared__ uint4 k_s[kMaxRows][kRowVecs + 1];
  __shared__ __align__(16) float e_s[kQueriesPerGroup][kMaxKeysPerLane * WL];
  // staging: per pass each thread issues a batch of query loads and a batch
  // of key loads (4 pieces of 16 bytes each) before its first LDS store, so
  // a pass costs one memory round trip.  Offsets are 32-bit from
  // per-workgroup bases; pieces past the end are read from a clamped
  // address (queries past the last token are never used, and a clamped key
  // piece rewrites its own value).
  constexpr int kQVecs = kQueriesPerGroup * D / 4;
  constexpr int kBatch = 4;
  constexpr int kQPasses = (kQVecs + kBatch * kWindowThreads - 1) / (kBatch * kWindowThreads);
  const int q_rows = p.tokens - q0 < kQueriesPerGroup ? static_cast<int>(p.tokens - q0) : kQueriesPerGroup;
  const int q_last_vec = q_rows * (D / 4) - 1;
  const u32x4_t* qbase = reinterpret_cast<const u32x4_t*>(p.pq + (static_cast<int64_t>(h) * p.tokens + q0) * D);
  // key rows [row0, row0 + rows): every window of the workgroup's queries
  const int64_t row0 = q0 + 1 > p.window ? q0 + 1 - p.window : 0;
  const int64_t q_last = q0 + kQueriesPerGroup - 1 < p.tokens - 1 ? q0 + kQueriesPerGroup - 1 : p.tokens - 1;
  const int rows = static_cast<int>(q_last - row0 + 1);
  const int k_pieces = STAGE ? rows * kRowVecs : 0;
  const u32x4_t* kbase = reinterpret_cast<const u32x4_t*>(p.kv + row0 * token_elems + g * D);
  const int row_vecs = static_cast<int>(token_elems / 8);  // 16-byte pieces per token row of the pool
  for (int pass = 0;; ++pass) {
    const bool do_q = pass < kQPasses;                      // uniform
    const bool do_k = pass * kBatch * kWindowThreads < k_pieces;  // uniform
    if (!do_q && !do_k) break;
    const int e0 = tid + pass * kBatch * kWindowThreads;
    u32x4_t qv[kBatch];  // the float bits
    u32x4_t kv[kBatch];
    if (do_q) {
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int e = e0 + i * kWindowThreads;
        qv[i] = qbase[e < q_last_vec ? e : q_last_vec];
      }
    }
    if (do_k) {
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int e = e0 + i * kWindowThreads;
        const int r = e / kRowVecs < rows ? e / kRowVecs : rows - 1;
        kv[i] = kbase[r * row_vecs + e % kRowVecs];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (do_q) {
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        // a piece past the tile rewrites the last query's slot with the
        // value its owner writes (or the slot of a query past the last token)
        const int e = e0 + i * kWindowThreads < kQVecs ? e0 + i * kWindowThreads : kQVecs - 1;
        *reinterpret_cast<u32x4_t*>(&q_s[e / (D / 4)][(e % (D / 4)) * 4]) = qv[i];
      }
    }
    if (do_k) {
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int e = e0 + i * kWindowThreads;
        const int r = e / kRowVecs < rows ? e / kRowVecs : rows - 1;
        *reinterpret_cast<u32x4_t*>(&k_s[r][e % kRowVecs]) = kv[i];
      }
    }
  }
  __syncthreads();
  if (q >= p.tokens) return;  // whole query groups leave together

  const int64_t start = q + 1 > p.window ? q + 1 - p.window : 0;
  const int count = static_cast<int>(q - start + 1);

  // logits of this lane's keys w = wl + j * WL: sequential dots, no
  // contraction, the four keys' chains side by side over each query chunk
  float dot[kMaxKeysPerLane];
  int rowk[kMaxKeysPerLane];
  const uint4* kg[kMaxKeysPerLane];
#pragma unroll
  for (int j = 0; j < kMaxKeysPerLane; ++j) {
    const int w = wl + j * WL;
    const int wc = w < count ? w : count - 1;  // clamp: its result is dropped
    dot[j] = 0.0f;
    rowk[j] = static_cast<int>(start + wc - row0);
    kg[j] = reinterpret_cast<const uint4*>(p.kv + (start + wc) * token_elems + g * D);
  }
#pragma unroll 2
  for (int c = 0; c < kRowVecs; ++c) {
    float qv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[e] = q_s[qi][c * 8 + e];
#pragma unroll
    for (int j = 0; j < kMaxKeysPerLane; ++j) {
      const uint4 kk = STAGE ? k_s[rowk[j]][c] : kg[j][c];
      const uint32_t kw[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) dot[j] = dot[j] + mul_h(qv[e], kw[e >> 1], e & 1);
    }
  }
  float logit[kMaxKeysPerLane];
  float maximum = -__builtin_huge_valf();
#pragma unroll
  for (int j = 0; j < kMaxKeysPerLane; ++j) {
    logit[j] = -__builtin_huge_valf();
    if (wl + j * WL < count) {
      logit[j] = dot[j] * p.scale;
      if (logit[j] > maximum) maximum = logit[j];
    }
  }
  // max over the query's lanes (exact in any order)
#pragma unroll
  for (int off = 1; off < WL; off <<= 1) maximum = fmaxf(maximum, __shfl_xor(maximum, off, kWave));

  float e[kMaxKeysPerLane];
#pragma unroll
  for (int j = 0; j < kMaxKeysPerLane; ++j) {
    const float ej = expf_glibc(logit[j] - maximum);  // every key: the table reads go out together
    e[j] = wl + j * WL < count ? ej : 0.0f;
  }

  // denominator summed in window order, w = 0 .. count-1: the query's lanes
  // put their exponentials in LDS (the query's lanes are in one wave, whose
  // LDS operations execute in order) and every lane reads them back four at
  // a time.  The slots past count hold +0, and adding +0 leaves the running
  // sum (which starts at +0) unchanged, so every lane adds all 4 WL slots
  // with no per-slot test.
#pragma unroll
  for (int j = 0; j < kMaxKeysPerLane; ++j) e_s[qi][wl + j * WL] = e[j];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float denominator = 0.0f;
  const float4* e4 = reinterpret_cast<const float4*>(e_s[qi]);
#pragma unroll 8
  for (int w4 = 0; w4 < kMaxKeysPerLane * WL / 4; ++w4) {
    const float4 v = e4[w4];
    denominator = denominator + v.x;
    denominator = denominator + v.y;
    denominator = denominator + v.z;
    denominator = denominator + v.w;
  }

  float* row = p.prob + (static_cast<int64_t>(h) * p.tokens + q) * p.window;
#pragma unroll
  for (int j = 0; j < kMaxKeysPerLane; ++j) {
    const int w = wl + j * WL;
    const float pr = e[j] / denominator;
    if (w < count) row[w] = pr;
  }
}

// block_topk_kernel stages, per block, the probabilities of the queries whose
// windows reach it (32 + W - 1 rows) in LDS, in one of two layouts:
//   * per token column (any W): row r holds the 32 probabilities query
//     t0 + r gives the block's tokens, plus one column of padding, so that
//     lane j reading (row j + i, column j) hits bank 34 j mod 64;
//   * whole rows (W a power of two, 4..64, 16-byte aligned probabilities):
//     the block's query rows are one contiguous span of the workspace, copied
//     in 16-byte pieces (stored as two 8-byte halves) into rows of W + 2
//     floats, so that lane j reading (row j + i, column W - 1 - i) hits bank
//     pair (W + 2) j mod 64, distinct for the 32 lanes.
constexpr int kStageCols = kPageTokens + 1;
constexpr int kMaxWholeRowWindow = 64;
static_assert(D == 2 * kWave, "block_topk_kernel: a lane per pair of dimensions");

bool block_topk_whole_rows(int window, const float* prob) {
  return window >= 4 && window <= kMaxWholeRowWindow && (window & (window - 1)) == 0 &&
         reinterpret_cast<uintptr_t>(prob) % 16 == 0;
}

// Blocks per workgroup of block_topk_kernel with whole rows.
constexpr int kWholeRowBlocks = 4;

size_t block_topk_lds_bytes(int window, bool whole_rows) {
  const int blocks = whole_rows ? kWholeRowBlocks : 1;
  return static_cast<size_t>(blocks * kPageTokens + window - 1) * (whole_rows ? window + 2 : kStageCols) *
         sizeof(float);
}

// One wave per (block, head): received mass, stable rank, top-k, representative.
// BPW blocks per workgroup, one wave each: with whole rows the BPW blocks'
// query rows overlap (32 BPW + W - 1 rows for BPW blocks, against 32 + W - 1
// each), so the waves stage them once together and more blocks fit in LDS at
// once; the per-column layout holds one block's columns (BPW = 1).
template <bool WHOLE_ROWS, int BPW>
__global__ __launch_bounds__(BPW * kWave) void block_topk_kernel(const Params p) {
  constexpr int kThreads = BPW * kWave;
  int tile, h;
  xcd_tile(p.hq, p.hkv, tile, h);
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int g = h / (p.hq / p.hkv);
  const int64_t blocks = p.tokens / kPageTokens;
  const int b = tile * BPW + wave;
  const bool valid = b < blocks;  // a wave past the last block only joins the staging and the barriers
  const int64_t tt = static_cast<int64_t>(tile) * BPW * kPageTokens;  // first token of the tile
  const int64_t t0 = static_cast<int64_t>(b) * kPageTokens;
  const int W = p.window;
  __shared__ int order[BPW][kPageTokens];
  extern __shared__ float stage_s[];

  // the queries tt .. q_last, whose rows start at prob_b; the window of query
  // tt + r starts at tt + r + 1 - W (at 0 for the first W - 1 queries)
  const int64_t q_last = tt + BPW * kPageTokens - 1 + W - 1 < p.tokens - 1 ? tt + BPW * kPageTokens - 1 + W - 1
                                                                           : p.tokens - 1;
  const int rows = static_cast<int>(q_last - tt + 1);
  const float* prob_b = p.prob + (static_cast<int64_t>(h) * p.tokens + tt) * W;
  if (WHOLE_ROWS) {
    // rows x W floats from prob_b, W / 4 pieces per row (a power of two)
    const int pieces = rows * (W / 4);
    const int shift = __builtin_ctz(W / 4);
    const u32x4_t* src = reinterpret_cast<const u32x4_t*>(prob_b);
    constexpr int kBatch = 8;
    for (int e0 = tid; e0 < pieces; e0 += kBatch * kThreads) {
      u32x4_t v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) v[i] = src[e0 + i * kThreads < pieces ? e0 + i * kThreads : pieces - 1];
      __builtin_amdgcn_sched_barrier(0);  // every load of the batch ahead of the stores
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int e = e0 + i * kThreads < pieces ? e0 + i * kThreads : pieces - 1;  // a clamped piece rewrites its value
        u32x2_t* dst = reinterpret_cast<u32x2_t*>(stage_s + (e >> shift) * (W + 2) + (e & (W / 4 - 1)) * 4);
        dst[0] = u32x2_t{v[i].x, v[i].y};
        dst[1] = u32x2_t{v[i].z, v[i].w};
      }
    }
  } else {
    static_assert(WHOLE_ROWS || BPW == 1, "the per-column layout holds one block");
    // (row r, column j) = the probability query t0 + r gives token t0 + j:
    // each row's 32 columns are contiguous in the query's window row, so a
    // load instruction covers two rows; entries outside a query's window are
    // loaded from a clamped column and never read
    const int pieces = rows * kPageTokens;
    const int first_full = static_cast<int>(t0 + 1 >= W ? 0 : W - 1 - t0);  // first row whose start > 0
    constexpr int kBatch = 16;
    for (int e0 = lane; e0 < pieces; e0 += kBatch * kWave) {
      float v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int e = e0 + i * kWave < pieces ? e0 + i * kWave : pieces - 1;
        const int r = e / kPageTokens;
        const int j = e % kPageTokens;
        int col = r >= first_full ? j - r + W - 1 : static_cast<int>(t0) + j;
        col = col < 0 ? 0 : (col >= W ? W - 1 : col);
        v[i] = prob_b[r * W + col];
      }
      __builtin_amdgcn_sched_barrier(0);  // every load of the batch ahead of the stores
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int e = e0 + i * kWave < pieces ? e0 + i * kWave : pieces - 1;  // a clamped piece rewrites its value
        stage_s[(e / kPageTokens) * kStageCols + e % kPageTokens] = v[i];
      }
    }
  }
  __syncthreads();

  // received mass of token t = t0 + lane: the probabilities of the queries
  // t .. min(t + W - 1, tokens - 1) summed in query order
  float r = 0.0f;
  if (valid && lane < kPageTokens) {
    const int64_t t = t0 + lane;
    const int n = static_cast<int>((t + W - 1 < p.tokens - 1 ? t + W - 1 : p.tokens - 1) - t + 1);
    const int row_t = static_cast<int>(t - tt);  // the stage row of query t
    // stage index of query t + i's probability of token t
    auto at = [&](int i) {
      if (WHOLE_ROWS) {
        const int64_t start = t + i + 1 > W ? t + i + 1 - W : 0;
        return (row_t + i) * (W + 2) + static_cast<int>(t - start);
      }
      return (row_t + i) * kStageCols + lane;
    };
    constexpr int kReads = 8;  // LDS reads issued together, then added in order
    for (int i0 = 0; i0 < n; i0 += kReads) {
      float c[kReads];
#pragma unroll
      for (int i = 0; i < kReads; ++i) c[i] = stage_s[at(i0 + i < n ? i0 + i : n - 1)];
#pragma unroll
      for (int i = 0; i < kReads; ++i)
        if (i0 + i < n) r = r + c[i];
    }
    p.received[static_cast<int64_t>(h) * p.tokens + t] = r;
  }
  // stable descending rank (mass_before / mass_tied: greater ones first,
  // equal ones in token order, NaN last); lane j's mass broadcast by
  // readlane, the tests combined without branches
  int rank = 0;
#pragma unroll
  for (int j = 0; j < kPageTokens; ++j) {
    const float rj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, r), j));
    rank += static_cast<int>(mass_before(rj, r)) | (static_cast<int>(mass_tied(rj, r)) & static_cast<int>(j < lane));
  }
  if (valid && lane < kPageTokens && rank < p.topk) {
    order[wave][rank] = lane;
    if (p.offsets) p.offsets[(static_cast<int64_t>(h) * blocks + b) * p.topk + rank] = lane;
  }
  __syncthreads();
  if (!valid) return;

  // representative: lane d-pair (2 lane, 2 lane + 1); the chosen keys' words
  // loaded 8 at a time, summed in rank order
  const int64_t token_elems = 2LL * p.hkv * D;
  const uint32_t* kblock =
      reinterpret_cast<const uint32_t*>(p.kv + t0 * token_elems + g * D) + lane;  // word lane of each key row
  float sum0 = 0.0f;
  float sum1 = 0.0f;
  constexpr int kKeys = 8;
  for (int rk0 = 0; rk0 < p.topk; rk0 += kKeys) {
    uint32_t w[kKeys];
#pragma unroll
    for (int i = 0; i < kKeys; ++i) {
      const int rk = rk0 + i < p.topk ? rk0 + i : p.topk - 1;
      w[i] = kblock[order[wave][rk] * (token_elems / 2)];
    }
#pragma unroll
    for (int i = 0; i < kKeys; ++i) {
      if (rk0 + i < p.topk) {
        sum0 = sum0 + lo_h2f(w[i]);
        sum1 = sum1 + hi_h2f(w[i]);
      }
    }
  }
  const float k = static_cast<float>(p.topk);
  const float v0 = sum0 / k;
  const float v1 = sum1 / k;
  const int d = 2 * lane;
  if (p.values) {
    float* out = p.values + (static_cast<int64_t>(h) * blocks + b) * D + d;
    out[0] = v0;
    out[1] = v1;
  }
  if (p.reps) {
    p.reps[(static_cast<int64_t>(h) * D + d) * p.rep_stride + b] = v0;
    p.reps[(static_cast<int64_t>(h) * D + d + 1) * p.rep_stride + b] = v1;
  }
}

// ---- general shapes: any head_dim, block size and window ------------------
//
// window_softmax_any_kernel: one wave per (query head h, query position q),
// four per workgroup; lane l takes the window positions w = l, l + 64, ...
//   1. each logit (sequential fp32 dot over head_dim, no contraction, times
//      the scale) goes to the query's probability row, and the lanes' maxima
//      are combined;
//   2. in chunks of kAnyChunk positions the row's logits become
//      exponentials (a lane rereads only the entries it wrote), the chunk is
//      staged in LDS and every lane adds it to the denominator in window
//      order;
//   3. each entry is divided by the denominator.
// VEC: head_dim a multiple of 8, rows read 16 bytes at a time.
constexpr int kAnyWaves = 4;
constexpr int kAnyChunk = 1024;

template <bool VEC>
__global__ __launch_bounds__(kAnyWaves * kWave) void window_softmax_any_kernel(const Params p) {
  __shared__ __align__(16) float e_s[kAnyWaves][kAnyChunk];
  int tile, h;
  xcd_tile(p.hq, p.hkv, tile, h);
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int64_t q = static_cast<int64_t>(tile) * kAnyWaves + wave;
  if (q >= p.tokens) return;  // a whole wave leaves; the kernel has no workgroup barrier
  const int dim = p.head_dim;
  const int g = h / (p.hq / p.hkv);
  const int64_t token_elems = 2LL * p.hkv * dim;
  const int64_t start = q + 1 > p.window ? q + 1 - p.window : 0;
  const int count = static_cast<int>(q - start + 1);
  const float* qrow = p.pq + (static_cast<int64_t>(h) * p.tokens + q) * dim;
  float* row = p.prob + (static_cast<int64_t>(h) * p.tokens + q) * p.window;

  float maximum = -__builtin_huge_valf();
  for (int w = lane; w < count; w += kWave) {
    const uint16_t* krow = p.kv + (start + w) * token_elems + static_cast<int64_t>(g) * dim;
    float dot = 0.0f;
    if (VEC) {
      for (int d = 0; d < dim; d += 8) {
        const uint4 kk = *reinterpret_cast<const uint4*>(krow + d);
        const float4 qa = *reinterpret_cast<const float4*>(qrow + d);
        const float4 qb = *reinterpret_cast<const float4*>(qrow + d + 4);
        dot = dot + mul_h(qa.x, kk.x, 0);
        dot = dot + mul_h(qa.y, kk.x, 1);
        dot = dot + mul_h(qa.z, kk.y, 0);
        dot = dot + mul_h(qa.w, kk.y, 1);
        dot = dot + mul_h(qb.x, kk.z, 0);
        dot = dot + mul_h(qb.y, kk.z, 1);
        dot = dot + mul_h(qb.z, kk.w, 0);
        dot = dot + mul_h(qb.w, kk.w, 1);
      }
    } else {
      for (int d = 0; d < dim; ++d) dot = dot + mul_h(qrow[d], krow[d], 0);
    }
    const float logit = dot * p.scale;
    row[w] = logit;
    if (logit > maximum) maximum = logit;
  }
  // max over the wave (exact in any order)
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) maximum = fmaxf(maximum, __shfl_xor(maximum, off, kWave));

  float denominator = 0.0f;
  float* es = e_s[wave];
  for (int c0 = 0; c0 < count; c0 += kAnyChunk) {
    const int n = count - c0 < kAnyChunk ? count - c0 : kAnyChunk;
    for (int i = lane; i < n; i += kWave) {  // c0 is a multiple of 64: entry c0 + i is this lane's
      const float e = expf_glibc(row[c0 + i] - maximum);
      row[c0 + i] = e;
      es[i] = e;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll 8
    for (int i = 0; i < n; ++i) denominator = denominator + es[i];
    // every lane has read the chunk before the next one overwrites it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  for (int w = lane; w < count; w += kWave) row[w] = row[w] / denominator;
}

// block_topk_any_kernel: one wave per (query head, block) of any size.
// Each token's received mass is summed over the queries whose window holds
// it, in ascending query order, and written to `received`; after a
// workgroup barrier (which makes those writes visible to the whole wave)
// each token's stable descending rank is counted against every token of
// the block (mass_before / mass_tied: greater first, equal ones in token
// order, NaN last), the top-k offsets are placed in LDS by rank, and the
// representative of each head dimension is the sum of the chosen keys in
// rank order / topk.
__global__ __launch_bounds__(kWave) void block_topk_any_kernel(const Params p) {
  extern __shared__ int order_s[];  // [topk]
  int b, h;
  xcd_tile(p.hq, p.hkv, b, h);
  const int lane = threadIdx.x;
  const int dim = p.head_dim;
  const int bt = p.block_tokens;
  const int W = p.window;
  const int g = h / (p.hq / p.hkv);
  const int64_t blocks = p.tokens / bt;
  const int64_t t0 = static_cast<int64_t>(b) * bt;
  float* rec = p.received + static_cast<int64_t>(h) * p.tokens;
  const float* prob_h = p.prob + static_cast<int64_t>(h) * p.tokens * W;
  for (int i = lane; i < bt; i += kWave) {
    const int64_t t = t0 + i;
    const int64_t q_end = t + W - 1 < p.tokens - 1 ? t + W - 1 : p.tokens - 1;
    float r = 0.0f;
    for (int64_t q = t; q <= q_end; ++q) {
      const int64_t start = q + 1 > W ? q + 1 - W : 0;
      r = r + prob_h[q * W + (t - start)];
    }
    rec[t] = r;
  }
  __syncthreads();
  for (int i = lane; i < bt; i += kWave) {
    const float ri = rec[t0 + i];
    int rank = 0;
    for (int j = 0; j < bt; ++j) {
      const float rj = rec[t0 + j];
      rank += static_cast<int>(mass_before(rj, ri)) | (static_cast<int>(mass_tied(rj, ri)) & static_cast<int>(j < i));
    }
    if (rank < p.topk) {
      order_s[rank] = i;
      if (p.offsets) p.offsets[(static_cast<int64_t>(h) * blocks + b) * p.topk + rank] = i;
    }
  }
  __syncthreads();
  const int64_t token_elems = 2LL * p.hkv * dim;
  const uint16_t* kblock = p.kv + t0 * token_elems + static_cast<int64_t>(g) * dim;
  const float k = static_cast<float>(p.topk);
  for (int d = lane; d < dim; d += kWave) {
    float sum = 0.0f;
    for (int rk = 0; rk < p.topk; ++rk) sum = sum + lo_h2f(kblock[order_s[rk] * token_elems + d]);
    const float v = sum / k;
    if (p.values) p.values[(static_cast<int64_t>(h) * blocks + b) * dim + d] = v;
    if (p.reps) p.reps[(static_cast<int64_t>(h) * dim + d) * p.rep_stride + b] = v;
  }
}

template <int WL>
void launch_window(const Params& p, hipStream_t stream) {
  constexpr int kQueriesPerGroup = window_threads<WL>() / WL;
  const dim3 grid(static_cast<unsigned>((p.tokens + kQueriesPerGroup - 1) / kQueriesPerGroup), p.hq);
  if constexpr (WL <= 32) {
    hipLaunchKernelGGL((window_softmax_kernel<WL, true>), grid, dim3(window_threads<WL>()), 0, stream, p);
  } else {
    hipLaunchKernelGGL((window_softmax_kernel<WL, false>), grid, dim3(window_threads<WL>()), 0, stream, p);
  }
}

}  // namespace

size_t local_causal_workspace_bytes(int64_t tokens, int32_t query_heads, int32_t window) {
  size_t rows = 0;
  size_t floats = 0;
  size_t bytes = 0;
  if (__builtin_mul_overflow(static_cast<size_t>(tokens), static_cast<size_t>(query_heads), &rows) ||
      __builtin_mul_overflow(rows, static_cast<size_t>(window) + 1, &floats) ||
      __builtin_mul_overflow(floats, sizeof(float), &bytes))
    return 0;  // too large to allocate
  return bytes;
}

hipError_t launch_local_causal_representatives(const RepresentativeLaunch& r, hipStream_t stream) {
  Params p{};
  p.pq = r.prompt_queries;
  p.kv = r.kv;
  p.prob = r.workspace;
  p.received = r.received ? r.received : r.workspace + static_cast<int64_t>(r.tokens) * r.query_heads * r.window;
  p.values = r.values;
  p.reps = r.reps;
  p.offsets = r.offsets;
  p.tokens = r.tokens;
  p.hq = r.query_heads;
  p.hkv = r.kv_heads;
  p.head_dim = r.head_dim;
  p.block_tokens = r.block_tokens;
  p.window = r.window;
  p.topk = r.topk;
  p.rep_stride = r.rep_stride;
  p.scale = r.scale;
  if (r.head_dim != D || r.block_tokens != kPageTokens || r.window > kMaxTiledLocalWindow) {
    const int64_t blocks = r.tokens / r.block_tokens;
    const bool vec = r.head_dim % 8 == 0 && reinterpret_cast<uintptr_t>(r.prompt_queries) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(r.kv) % 16 == 0;
    const dim3 grid(static_cast<unsigned>((r.tokens + kAnyWaves - 1) / kAnyWaves), r.query_heads);
    if (vec) hipLaunchKernelGGL((window_softmax_any_kernel<true>), grid, dim3(kAnyWaves * kWave), 0, stream, p);
    else hipLaunchKernelGGL((window_softmax_any_kernel<false>), grid, dim3(kAnyWaves * kWave), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(block_topk_any_kernel, dim3(static_cast<unsigned>(blocks), r.query_heads), dim3(kWave),
                       static_cast<size_t>(r.topk) * sizeof(int), stream, p);
    return hipGetLastError();
  }
  const int w = r.window;  // lanes per query: the power of two >= w / 4
  if (w <= 4) launch_window<1>(p, stream);
  else if (w <= 8) launch_window<2>(p, stream);
  else if (w <= 16) launch_window<4>(p, stream);
  else if (w <= 32) launch_window<8>(p, stream);
  else if (w <= 64) launch_window<16>(p, stream);
  else if (w <= 128) launch_window<32>(p, stream);
  else launch_window<64>(p, stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t blocks = r.tokens / kPageTokens;
  if (block_topk_whole_rows(r.window, p.prob)) {
    const dim3 grid(static_cast<unsigned>((blocks + kWholeRowBlocks - 1) / kWholeRowBlocks), r.query_heads);
    hipLaunchKernelGGL((block_topk_kernel<true, kWholeRowBlocks>), grid, dim3(kWholeRowBlocks * kWave),
                       block_topk_lds_bytes(r.window, true), stream, p);
  } else {
    const dim3 grid(static_cast<unsigned>(blocks), r.query_heads);
    hipLaunchKernelGGL((block_topk_kernel<false, 1>), grid, dim3(kWave), block_topk_lds_bytes(r.window, false), stream,
                       p);
  }
  return hipGetLastError();
}

}  // namespace sa
