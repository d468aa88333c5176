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

// Workgroup of the window kernel: 256 threads, at most 64 queries (32 KB of
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
  int32_t window;
  int32_t topk;
  int32_t rep_stride;
  float scale;
};

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
  const int h = blockIdx.y;
  const int tid = threadIdx.x;
  const int qi = tid / WL;          // query within the workgroup
  const int wl = tid % WL;          // window lane within the query
  const int g = h / (p.hq / p.hkv);
  const int64_t q0 = static_cast<int64_t>(blockIdx.x) * kQueriesPerGroup;
  const int64_t q = q0 + qi;
  const int64_t token_elems = 2LL * p.hkv * D;

  __shared__ float q_s[kQueriesPerGroup][D];
  __shared__ uint4 k_s[kMaxRows][kRowVecs + 1];
  __shared__ __align__(16) float e_s[kQueriesPerGroup][kMaxKeysPerLane * WL];
  for (int e = tid; e < kQueriesPerGroup * D; e += kWindowThreads) {
    const int64_t qq = q0 + e / D;
    q_s[e / D][e % D] = qq < p.tokens ? p.pq[(static_cast<int64_t>(h) * p.tokens + qq) * D + e % D] : 0.0f;
  }
  // key rows [row0, row0 + rows): every window of the workgroup's queries
  const int64_t row0 = q0 + 1 > p.window ? q0 + 1 - p.window : 0;
  if (STAGE) {
    const int64_t q_last = q0 + kQueriesPerGroup - 1 < p.tokens - 1 ? q0 + kQueriesPerGroup - 1 : p.tokens - 1;
    const int rows = static_cast<int>(q_last - row0 + 1);
    for (int e = tid; e < rows * kRowVecs; e += kWindowThreads) {
      const int r = e / kRowVecs;
      const int c = e % kRowVecs;
      k_s[r][c] = reinterpret_cast<const uint4*>(p.kv + (row0 + r) * token_elems + g * D)[c];
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
  for (int j = 0; j < kMaxKeysPerLane; ++j) e[j] = (wl + j * WL < count) ? expf_glibc(logit[j] - maximum) : 0.0f;

  // denominator summed in window order, w = 0 .. count-1: the query's lanes
  // put their exponentials in LDS (the query's lanes are in one wave, whose
  // LDS operations execute in order) and every lane reads them back four at
  // a time
#pragma unroll
  for (int j = 0; j < kMaxKeysPerLane; ++j) e_s[qi][wl + j * WL] = e[j];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float denominator = 0.0f;
  const float4* e4 = reinterpret_cast<const float4*>(e_s[qi]);
  for (int w = 0; w < count; w += 4) {
    const float4 v = e4[w / 4];
    denominator = denominator + v.x;
    if (w + 1 < count) denominator = denominator + v.y;
    if (w + 2 < count) denominator = denominator + v.z;
    if (w + 3 < count) denominator = denominator + v.w;
  }

  float* row = p.prob + (static_cast<int64_t>(h) * p.tokens + q) * p.window;
#pragma unroll
  for (int j = 0; j < kMaxKeysPerLane; ++j) {
    const int w = wl + j * WL;
    if (w < count) row[w] = e[j] / denominator;
  }
}

// One wave per (block, head): received mass, stable rank, top-k, representative.
__global__ __launch_bounds__(kWave) void block_topk_kernel(const Params p) {
  const int b = blockIdx.x;
  const int h = blockIdx.y;
  const int lane = threadIdx.x;
  const int g = h / (p.hq / p.hkv);
  const int64_t blocks = p.tokens / kPageTokens;
  __shared__ int order[kPageTokens];

  // received mass: the probabilities of the queries t .. t+W-1 in query
  // order, loaded 16 at a time before the sequential sum
  float r = 0.0f;
  if (lane < kPageTokens) {
    const int64_t t = static_cast<int64_t>(b) * kPageTokens + lane;
    const int64_t q_end = t + p.window - 1 < p.tokens - 1 ? t + p.window - 1 : p.tokens - 1;
    constexpr int kBatch = 16;
    for (int64_t q0 = t; q0 <= q_end; q0 += kBatch) {
      float v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int64_t q = q0 + i;
        const int64_t start = q + 1 > p.window ? q + 1 - p.window : 0;
        v[i] = q <= q_end ? p.prob[(static_cast<int64_t>(h) * p.tokens + q) * p.window + (t - start)] : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i)
        if (q0 + i <= q_end) r = r + v[i];
    }
    p.received[static_cast<int64_t>(h) * p.tokens + t] = r;
  }
  // stable descending rank: greater ones first, equal ones in token order
  int rank = 0;
  for (int j = 0; j < kPageTokens; ++j) {
    const float rj = __shfl(r, j, kWave);
    rank += (rj > r || (!(r > rj) && !(rj > r) && j < lane)) ? 1 : 0;
  }
  if (lane < kPageTokens && rank < p.topk) {
    order[rank] = lane;
    if (p.offsets) p.offsets[(static_cast<int64_t>(h) * blocks + b) * p.topk + rank] = lane;
  }
  __syncthreads();

  const int64_t token_elems = 2LL * p.hkv * D;
  const uint16_t* kblock = p.kv + static_cast<int64_t>(b) * kPageTokens * token_elems + g * D;
  for (int d = lane; d < D; d += kWave) {
    float sum = 0.0f;
    for (int rk = 0; rk < p.topk; ++rk) sum = sum + h2f(kblock[order[rk] * token_elems + d]);
    const float v = sum / static_cast<float>(p.topk);
    if (p.values) p.values[(static_cast<int64_t>(h) * blocks + b) * D + d] = v;
    if (p.reps) p.reps[(static_cast<int64_t>(h) * D + d) * p.rep_stride + b] = v;
  }
}

// Windows up to 128 keys stage their key rows in LDS (at most 135 padded
// rows, 37 KB); longer ones read them from memory.
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
  return static_cast<size_t>(tokens) * query_heads * (static_cast<size_t>(window) + 1) * sizeof(float);
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
  p.window = r.window;
  p.topk = r.topk;
  p.rep_stride = r.rep_stride;
  p.scale = r.scale;
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
  const dim3 grid(static_cast<unsigned>(r.tokens / kPageTokens), r.query_heads);
  hipLaunchKernelGGL(block_topk_kernel, grid, dim3(kWave), 0, stream, p);
  return hipGetLastError();
}

}  // namespace sa
