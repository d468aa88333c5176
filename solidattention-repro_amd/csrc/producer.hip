// producer.hip — the query producer and output consumer around the decode
// attention (gfx950): RMSNorm, the [out][in] fp32 projections on the matrix
// cores, and the per-head RMS norm + rotary embedding fused into the
// projection's epilogue.  Semantics of the reference's rms_norm, head_rms,
// rope and cublasSgemm(CUBLAS_OP_T) calls (cpp/src/qwen_layer_main.cpp
// :125-172, :576-584, :640-645; cpp/src/qwen_chain_main.cpp:365-399) for a
// batch of decode tokens (one row per sequence).
//
// Projection (linear_partial_kernel): y[r][o] = sum_i x[r][i] w[o][i].  At
// decode the rows are few (the batch) and the weights are the traffic, so a
// workgroup takes a 64-column slab of w and a slice of the K range, streams
// that slice of w exactly once with non-temporal 16-byte loads, and runs
// v_mfma_f32_16x16x4f32 over up to 64 rows (4 tiles of 16).  A lane loads 4
// consecutive k of one w row and of one x row; the four MFMA steps of a
// 16-wide k chunk consume one component each (any order of the k sum is a
// valid fp32 sum; lane l supplies k = 4 (l / 16) + j to step j).  The K
// slices write fp32 partial sums that the epilogue adds in a fixed order,
// so results are deterministic.
#include <algorithm>

#include "sa_device.hpp"
#include "sa_internal.hpp"

namespace sa {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kSlab = 64;       // output columns per workgroup (16 per wave)
constexpr int kMTile = 16;
constexpr int kMTiles = 4;      // rows per workgroup: 64
constexpr int kKStep = 16;      // k per MFMA group (4 steps of 4)

__device__ inline f32x4_t load_nt4(const float* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
}

__device__ inline float block_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) red[wave] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int w = 0; w < kThreads / kWave; ++w) s += red[w];
  return s;
}

__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const float* x, const float* w, float* out, int width,
                                                            float eps) {
  __shared__ float red[kThreads / kWave];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * width;
  float ss = 0.0f;
  for (int i = threadIdx.x * 4; i < width; i += kThreads * 4) {
    const float4 v = *reinterpret_cast<const float4*>(xr + i);
    ss = __builtin_fmaf(v.x, v.x, ss);
    ss = __builtin_fmaf(v.y, v.y, ss);
    ss = __builtin_fmaf(v.z, v.z, ss);
    ss = __builtin_fmaf(v.w, v.w, ss);
  }
  ss = block_sum(ss, red);
  const float inv = 1.0f / __builtin_sqrtf(ss / static_cast<float>(width) + eps);
  for (int i = threadIdx.x * 4; i < width; i += kThreads * 4) {
    const float4 v = *reinterpret_cast<const float4*>(xr + i);
    const float4 g = *reinterpret_cast<const float4*>(w + i);
    float4 o;
    o.x = v.x * inv * g.x;
    o.y = v.y * inv * g.y;
    o.z = v.z * inv * g.z;
    o.w = v.w * inv * g.w;
    *reinterpret_cast<float4*>(out + row * width + i) = o;
  }
}

struct LinearParams {
  const float* x;       // [rows][in]
  const float* w[3];    // [out][in] row-major; up to three stacked weights (column ranges below)
  int32_t w_end[3];     // weight j covers output columns [w_end[j-1], w_end[j])
  float* part;          // [ksplit][rows][out] partial sums
  int32_t rows;
  int32_t in;
  int32_t out;
  int32_t kslice;       // k per workgroup
};

// Rows of x staged in LDS per workgroup: 64 x (kslice + 4) floats; kslice
// at most kMaxKSlice (the 4-float pad spreads the rows over the banks).
constexpr int kMaxKSlice = 256;
constexpr int kXPad = 4;

template <int KS>
__global__ __launch_bounds__(kThreads) void linear_partial_kernel(const LinearParams p) {
  static_assert(KS % 64 == 0 && KS <= kMaxKSlice, "K slice of 64..256");
  __shared__ f32x4_t xs[kMTile * kMTiles * (KS + kXPad) / 4];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int n0 = blockIdx.x * kSlab;
  const int ks = blockIdx.y;
  const int m0 = blockIdx.z * (kMTile * kMTiles);
  const int k_begin = ks * KS;
  constexpr int xs_stride = (KS + kXPad) / 4;  // in float4
  // this wave's whole w slice, issued first: 16 columns x kslice
  int wi = 0;
  if (n0 >= p.w_end[0]) wi = n0 >= p.w_end[1] ? 2 : 1;
  const int col0 = wi == 0 ? 0 : p.w_end[wi - 1];
  const int n = n0 + wave * 16 + lane % 16;  // this lane's output column (B operand column)
  const float* wrow = p.w[wi] + static_cast<int64_t>(n - col0) * p.in + k_begin + 4 * (lane / 16);
  // x rows [m0, m0 + 64) x [k_begin, k_begin + KS): all loads in flight at
  // once (coalesced, from L2), then the w slice from HBM, then x to LDS
  constexpr int vecs = KS / 4;
  constexpr int kXPerThread = kMTile * kMTiles * vecs / kThreads;
  f32x4_t xr[kXPerThread];
#pragma unroll
  for (int i = 0; i < kXPerThread; ++i) {
    const int e = i * kThreads + threadIdx.x;
    const int m = m0 + e / vecs;
    xr[i] = m < p.rows ? *reinterpret_cast<const f32x4_t*>(p.x + static_cast<int64_t>(m) * p.in + k_begin +
                                                           4 * (e % vecs))
                       : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  }
  f32x4_t wv[KS / kKStep];
#pragma unroll
  for (int s = 0; s < KS / kKStep; ++s) wv[s] = load_nt4(wrow + s * kKStep);
#pragma unroll
  for (int i = 0; i < kXPerThread; ++i) {
    const int e = i * kThreads + threadIdx.x;
    xs[(e / vecs) * xs_stride + e % vecs] = xr[i];
  }
  __syncthreads();

  f32x4_t c[kMTiles];
#pragma unroll
  for (int t = 0; t < kMTiles; ++t) c[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < KS / kKStep; ++s) {
#pragma unroll
    for (int t = 0; t < kMTiles; ++t) {
      // A operand: row 16 t + lane % 16, k = 16 s + 4 (lane / 16) + j
      const f32x4_t xa = xs[(t * kMTile + lane % 16) * xs_stride + 4 * s + lane / 16];
#pragma unroll
      for (int j = 0; j < 4; ++j) c[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[j], wv[s][j], c[t], 0, 0, 0);
    }
  }
  // D layout: lane holds rows 4 (lane / 16) + i of the tile, column lane % 16
  float* part = p.part + static_cast<int64_t>(ks) * p.rows * p.out;
#pragma unroll
  for (int t = 0; t < kMTiles; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + t * kMTile + 4 * (lane / 16) + i;
      if (m < p.rows) part[static_cast<int64_t>(m) * p.out + n] = c[t][i];
    }
  }
}

// out[r][o] = sum of the K-slice partials (in slice order) + residual[r][o];
// 4 consecutive elements per thread, the slices' loads issued 8 at a time
__global__ __launch_bounds__(kThreads) void linear_epilogue_kernel(const float* part, const float* residual,
                                                                   float* out, int64_t elems, int ksplit) {
  const int64_t e = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * 4;
  if (e >= elems) return;
  f32x4_t s = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  int k = 0;
  for (; k + 8 <= ksplit; k += 8) {
    f32x4_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const f32x4_t*>(part + (k + i) * elems + e);
#pragma unroll
    for (int i = 0; i < 8; ++i) s += v[i];
  }
  for (; k < ksplit; ++k) s += *reinterpret_cast<const f32x4_t*>(part + k * elems + e);
  if (residual) s += *reinterpret_cast<const f32x4_t*>(residual + e);
  *reinterpret_cast<f32x4_t*>(out + e) = s;
}

struct QkvEpilogue {
  const float* part;   // [ksplit][rows][q_heads*128 + 2*kv_heads*128]
  const float* q_norm;
  const float* k_norm;
  const int32_t* positions;
  float* q;            // [rows][q_heads][128]
  float* k;            // [rows][kv_heads][128]
  float* v;
  int32_t rows;
  int32_t q_heads;
  int32_t kv_heads;
  int32_t ksplit;
  float eps;
  float inv_freq[64];  // theta^(-2i/128), correctly rounded
};

// One wave per (row, head) of q, k and v: lane holds dims (lane, lane + 64),
// the RoPE pair.  head_rms then rope for q and k; v as projected.
__global__ __launch_bounds__(kThreads) void qkv_epilogue_kernel(const QkvEpilogue p) {
  const int lane = threadIdx.x % kWave;
  const int heads = p.q_heads + 2 * p.kv_heads;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
  if (item >= static_cast<int64_t>(p.rows) * heads) return;
  const int row = static_cast<int>(item / heads);
  const int h = static_cast<int>(item % heads);
  const int width = heads * kHeadDim;
  const int64_t elems = static_cast<int64_t>(p.rows) * width;
  const int64_t base = static_cast<int64_t>(row) * width + h * kHeadDim;
  float a = 0.0f, b = 0.0f;
  for (int k = 0; k < p.ksplit; ++k) {
    a += p.part[k * elems + base + lane];
    b += p.part[k * elems + base + lane + 64];
  }
  float* dst;
  const float* norm;
  if (h < p.q_heads) {
    dst = p.q + (static_cast<int64_t>(row) * p.q_heads + h) * kHeadDim;
    norm = p.q_norm;
  } else if (h < p.q_heads + p.kv_heads) {
    dst = p.k + (static_cast<int64_t>(row) * p.kv_heads + (h - p.q_heads)) * kHeadDim;
    norm = p.k_norm;
  } else {
    dst = p.v + (static_cast<int64_t>(row) * p.kv_heads + (h - p.q_heads - p.kv_heads)) * kHeadDim;
    dst[lane] = a;
    dst[lane + 64] = b;
    return;
  }
  float ss = a * a + b * b;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, kWave);
  const float inv = 1.0f / __builtin_sqrtf(ss / static_cast<float>(kHeadDim) + p.eps);
  a = a * inv * norm[lane];
  b = b * inv * norm[lane + 64];
  const float angle = static_cast<float>(p.positions[row]) * p.inv_freq[lane];
  float sn, cs;
  sincosf(angle, &sn, &cs);
  dst[lane] = a * cs - b * sn;
  dst[lane + 64] = b * cs + a * sn;
}

int slabs_for(int out) { return out / kSlab; }

}  // namespace

int linear_ksplit(int64_t rows, int64_t in, int64_t out) {
  // the fewest K slices (partial sums are extra traffic) that give about one
  // workgroup per CU, with slices of 64..256 k
  const int64_t mtiles = (rows + kMTile * kMTiles - 1) / (kMTile * kMTiles);
  const int64_t blocks = (out / kSlab) * mtiles;
  int64_t ks = 1;
  while (in / ks > kMaxKSlice || (ks * blocks < compute_units() && in / (ks * 2) >= 64)) ks *= 2;
  return static_cast<int>(ks);
}

hipError_t launch_rms_norm(const float* x, const float* w, float* out, int rows, int width, float eps,
                           hipStream_t stream) {
  hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(kThreads), 0, stream, x, w, out, width, eps);
  return hipGetLastError();
}

static hipError_t launch_partials(const LinearParams& lp, hipStream_t stream) {
  const int mtiles = (lp.rows + kMTile * kMTiles - 1) / (kMTile * kMTiles);
  const dim3 grid(slabs_for(lp.out), lp.in / lp.kslice, mtiles);
  switch (lp.kslice) {
    case 64: hipLaunchKernelGGL(linear_partial_kernel<64>, grid, dim3(kThreads), 0, stream, lp); break;
    case 128: hipLaunchKernelGGL(linear_partial_kernel<128>, grid, dim3(kThreads), 0, stream, lp); break;
    case 256: hipLaunchKernelGGL(linear_partial_kernel<256>, grid, dim3(kThreads), 0, stream, lp); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_linear(const LinearLaunch& l, hipStream_t stream) {
  const int ks = linear_ksplit(l.rows, l.in, l.out);
  LinearParams lp{};
  lp.x = l.x;
  lp.w[0] = lp.w[1] = lp.w[2] = l.w;
  lp.w_end[0] = lp.w_end[1] = lp.w_end[2] = l.out;
  lp.part = l.workspace;
  lp.rows = l.rows;
  lp.in = l.in;
  lp.out = l.out;
  lp.kslice = l.in / ks;
  hipError_t e = launch_partials(lp, stream);
  if (e != hipSuccess) return e;
  const int64_t elems = static_cast<int64_t>(l.rows) * l.out;  // a multiple of 64
  const int blocks = static_cast<int>((elems / 4 + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(linear_epilogue_kernel, dim3(blocks), dim3(kThreads), 0, stream, l.workspace, l.residual,
                     l.y, elems, ks);
  return hipGetLastError();
}

hipError_t launch_qkv_project(const QkvLaunch& q, hipStream_t stream) {
  const int qw = q.q_heads * kHeadDim, kw = q.kv_heads * kHeadDim;
  const int out = qw + 2 * kw;
  const int ks = linear_ksplit(q.rows, q.hidden, out);
  LinearParams lp{};
  lp.x = q.x;
  lp.w[0] = q.wq;
  lp.w[1] = q.wk;
  lp.w[2] = q.wv;
  lp.w_end[0] = qw;
  lp.w_end[1] = qw + kw;
  lp.w_end[2] = out;
  lp.part = q.workspace;
  lp.rows = q.rows;
  lp.in = q.hidden;
  lp.out = out;
  lp.kslice = q.hidden / ks;
  hipError_t e = launch_partials(lp, stream);
  if (e != hipSuccess) return e;
  QkvEpilogue ep{};
  ep.part = q.workspace;
  ep.q_norm = q.q_norm;
  ep.k_norm = q.k_norm;
  ep.positions = q.positions;
  ep.q = q.q;
  ep.k = q.k;
  ep.v = q.v;
  ep.rows = q.rows;
  ep.q_heads = q.q_heads;
  ep.kv_heads = q.kv_heads;
  ep.ksplit = ks;
  ep.eps = q.eps;
  for (int i = 0; i < 64; ++i) ep.inv_freq[i] = q.inv_freq[i];
  const int64_t items = static_cast<int64_t>(q.rows) * (q.q_heads + 2 * q.kv_heads);
  const int64_t blocks = (items + kThreads / kWave - 1) / (kThreads / kWave);
  hipLaunchKernelGGL(qkv_epilogue_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, stream, ep);
  return hipGetLastError();
}

}  // namespace sa
