// represent.hip — InfLLM local-causal block representatives of a prefill on
// the GPU (gfx950): the reference's build_local_causal_representatives
// (cpp/src/selection.cpp:12-94).
//
//   1. window_softmax_kernel: for every (query head h, query position q) the
//      logits of the keys [max(0, q+1-W), q] of h's KV head (sequential fp32
//      dot over head_dim, no contraction, times 1/sqrt(head_dim)), their max,
//      exp(logit - max) and the sequential denominator, and the
//      probabilities p = e / denominator.  Lanes: WL lanes per query (WL the
//      power of two >= W, at most 64); lane l of a query takes the window
//      positions w = l, l + WL, ...; the denominator is summed in window
//      order by every lane of the query through cross-lane reads.
//   2. block_topk_kernel: per (h, 32-token block), each token's received
//      mass (the sum over the queries whose window holds it, in ascending
//      query order, as the reference accumulates it), a stable descending
//      rank (ties keep token order), the top-k token offsets, and the
//      representative = sum of the chosen keys in rank order / k.
//
// The exponential is exp_det(): fixed double-precision operations (the same
// as the oracle's sao_exp_det), not the reference's glibc expf, which the GPU
// cannot reproduce; the two agree on nearly every argument and the chosen
// tokens on every committed golden case (see the oracle's tests).  Compiled
// with -ffp-contract=off: every float product and sum is rounded separately,
// as in the reference.
#include "sa_device.hpp"
#include "sa_internal.hpp"

namespace sa {
namespace {

constexpr int D = kHeadDim;
constexpr int kMaxKeysPerLane = 4;  // window <= 256

// Workgroup of the window kernel: 256 threads, at most 64 queries (32 KB of
// staged queries).
template <int WL>
constexpr int window_threads() { return WL >= 4 ? 256 : 64 * WL; }

// exp(x) rounded to float through fixed double operations: Cody-Waite
// reduction (fdlibm's ln2 split), degree-13 Taylor polynomial in Horner form,
// scaling by 2^k.
__device__ inline float exp_det(float x) {
  constexpr double kLn2Hi = 6.93147180369123816490e-01;
  constexpr double kLn2Lo = 1.90821492927058770002e-10;
  constexpr double kLog2e = 1.44269504088896338700e+00;
  constexpr double kInvFact[14] = {
      1.0, 1.0, 0.5, 1.0 / 6.0, 1.0 / 24.0, 1.0 / 120.0, 1.0 / 720.0, 1.0 / 5040.0, 1.0 / 40320.0,
      1.0 / 362880.0, 1.0 / 3628800.0, 1.0 / 39916800.0, 1.0 / 479001600.0, 1.0 / 6227020800.0};
  if (x != x) return x;
  if (x < -104.0f) return 0.0f;
  if (x > 89.0f) return __builtin_huge_valf();
  const double xd = static_cast<double>(x);
  const double k = __builtin_rint(xd * kLog2e);
  const double r = (xd - k * kLn2Hi) - k * kLn2Lo;
  double poly = kInvFact[13];
#pragma unroll
  for (int i = 12; i >= 0; --i) poly = poly * r + kInvFact[i];
  return static_cast<float>(__builtin_ldexp(poly, static_cast<int>(k)));
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
template <int WL>
__global__ __launch_bounds__(window_threads<WL>()) void window_softmax_kernel(const Params p) {
  constexpr int kWindowThreads = window_threads<WL>();
  constexpr int kQueriesPerGroup = kWindowThreads / WL;
  const int h = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int qi = tid / WL;          // query within the workgroup
  const int wl = tid % WL;          // window lane within the query
  const int g = h / (p.hq / p.hkv);
  const int64_t q = static_cast<int64_t>(blockIdx.x) * kQueriesPerGroup + qi;

  __shared__ float q_s[kQueriesPerGroup][D];
  for (int e = tid; e < kQueriesPerGroup * D; e += kWindowThreads) {
    const int64_t qq = static_cast<int64_t>(blockIdx.x) * kQueriesPerGroup + e / D;
    q_s[e / D][e % D] = qq < p.tokens ? p.pq[(static_cast<int64_t>(h) * p.tokens + qq) * D + e % D] : 0.0f;
  }
  __syncthreads();
  if (q >= p.tokens) return;  // whole query groups leave together

  const int64_t start = q + 1 > p.window ? q + 1 - p.window : 0;
  const int count = static_cast<int>(q - start + 1);
  const int64_t token_elems = 2LL * p.hkv * D;

  // logits of this lane's keys w = wl + j * WL (sequential dot, no contraction)
  float logit[kMaxKeysPerLane];
  float maximum = -__builtin_huge_valf();
#pragma unroll
  for (int j = 0; j < kMaxKeysPerLane; ++j) {
    const int w = wl + j * WL;
    logit[j] = -__builtin_huge_valf();
    if (w < count) {
      const uint4* k4 = reinterpret_cast<const uint4*>(p.kv + (start + w) * token_elems + g * D);
      float dot = 0.0f;
#pragma unroll 4
      for (int c = 0; c < D / 8; ++c) {
        const uint4 kk = k4[c];
        const uint32_t kw[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float kf = (e & 1) ? hi_h2f(kw[e >> 1]) : lo_h2f(kw[e >> 1]);
          dot = dot + q_s[qi][c * 8 + e] * kf;
        }
      }
      logit[j] = dot * p.scale;
      if (logit[j] > maximum) maximum = logit[j];
    }
  }
  // max over the query's lanes (exact in any order)
#pragma unroll
  for (int off = 1; off < WL; off <<= 1) maximum = fmaxf(maximum, __shfl_xor(maximum, off, kWave));

  float e[kMaxKeysPerLane];
#pragma unroll
  for (int j = 0; j < kMaxKeysPerLane; ++j) e[j] = (wl + j * WL < count) ? exp_det(logit[j] - maximum) : 0.0f;

  // denominator summed in window order, w = 0 .. count-1: key w is e[w / WL]
  // of lane w % WL of the query (every lane of the query picks the same j)
  const int base = lane - wl;  // first lane of this query in the wave
  float denominator = 0.0f;
  for (int w = 0; w < count; ++w) {
    const int j = w / WL;
    float src = e[0];
#pragma unroll
    for (int jj = 1; jj < kMaxKeysPerLane; ++jj)
      if (j == jj) src = e[jj];
    denominator = denominator + __shfl(src, base + (w % WL), kWave);
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

  float r = 0.0f;
  if (lane < kPageTokens) {
    const int64_t t = static_cast<int64_t>(b) * kPageTokens + lane;
    const int64_t q_end = t + p.window - 1 < p.tokens - 1 ? t + p.window - 1 : p.tokens - 1;
    for (int64_t q = t; q <= q_end; ++q) {
      const int64_t start = q + 1 > p.window ? q + 1 - p.window : 0;
      r = r + p.prob[(static_cast<int64_t>(h) * p.tokens + q) * p.window + (t - start)];
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

template <int WL>
void launch_window(const Params& p, hipStream_t stream) {
  constexpr int kQueriesPerGroup = window_threads<WL>() / WL;
  const dim3 grid(static_cast<unsigned>((p.tokens + kQueriesPerGroup - 1) / kQueriesPerGroup), p.hq);
  hipLaunchKernelGGL(window_softmax_kernel<WL>, grid, dim3(window_threads<WL>()), 0, stream, p);
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
  const int w = r.window;
  if (w <= 1) launch_window<1>(p, stream);
  else if (w <= 2) launch_window<2>(p, stream);
  else if (w <= 4) launch_window<4>(p, stream);
  else if (w <= 8) launch_window<8>(p, stream);
  else if (w <= 16) launch_window<16>(p, stream);
  else if (w <= 32) launch_window<32>(p, stream);
  else launch_window<64>(p, stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 grid(static_cast<unsigned>(r.tokens / kPageTokens), r.query_heads);
  hipLaunchKernelGGL(block_topk_kernel, grid, dim3(kWave), 0, stream, p);
  return hipGetLastError();
}

}  // namespace sa
