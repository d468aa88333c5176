// producer.hip — the query producer and output consumer around the decode
// attention (gfx950): RMSNorm, the [out][in] fp32 projections on the matrix
// cores, the per-head RMS norm + rotary embedding, and the residual add.
// Semantics of the reference's rms_norm, head_rms, rope and
// cublasSgemm(CUBLAS_OP_T) calls (cpp/src/qwen_layer_main.cpp:125-172,
// :576-584, :640-645; cpp/src/qwen_chain_main.cpp:365-399) for a batch of
// decode tokens (one row per sequence).
//
// Projections: y[r][o] = sum_i x[r][i] w[o][i].  At decode the rows are few
// (the batch) and the weights are the traffic.  Two launches:
//   * proj_split_kernel<C, KS>: a workgroup of 4 waves takes 64 rows x C
//     columns (64 or 32) over one K slice of KS = 256 or 128 (two
//     workgroups per compute unit at 1024 -> 4096, one at 2048 -> 1024;
//     split_shape()).  It issues all its
//     loads at once in 32-k units, stores each
//     unit to its LDS region as it arrives and runs that unit's
//     v_mfma_f32_16x16x4f32 steps (wave t: rows 16 t .. + 15) while later
//     units are in flight; the partial tile goes to the workspace.  With
//     the input RMSNorm folded in, x is multiplied by the norm weight as it
//     is staged and the slice's sum of squares of x per row is kept.
//   * the reduce launch adds the slices in slice order (any order of the k
//     sum is a valid fp32 sum; this one is fixed: deterministic) and applies
//     the epilogue: the residual (linear), or the row's RMSNorm scale, then
//     head RMS norm + RoPE for q/k heads (qkv).
#include <algorithm>

#include "qkv_epilogue.hpp"
#include "sa_device.hpp"
#include "sa_internal.hpp"

namespace sa {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kMTile = 16;
constexpr int kMTiles = 4;
constexpr int kRowsPerWg = kMTile * kMTiles;  // 64

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

// ---- split-K projections ------------------------------------------------------
// A workgroup takes 64 rows x C columns over one K slice of KS.  All its
// loads (x times the input gain, and w: up to 32 float4 per thread) are
// issued at once, in 32-k units; each unit goes to
// its own LDS region as it arrives and its matrix steps run while the later
// units are still in flight.  A second launch adds the slices in slice order
// and applies the epilogue.  Against whole-K columns of 16 this cuts what a
// compute unit pulls from L2 (x is read once per slice and column block, not
// once per 16 columns) and gives each LDS read of x C / 16 matrix steps.
constexpr int kUnitK = 32;
constexpr int kWideTileMaxSlices = 8;  // 64-column tiles only up to this many K slices

struct SplitParams {
  const float* x;          // [rows][in]
  const float* w[3];       // [out][in]; weight j covers columns [w_end[j-1], w_end[j])
  int32_t w_end[3];
  const float* gain;       // optional input RMSNorm weight [in]: x * gain is projected
  float* part;             // [slices][rows_pad][out]
  float* ss;               // [slices][rows_pad]: partial sums of squares of x (gain only)
  int32_t rows;
  int32_t rows_pad;
  int32_t in;
  int32_t out;
};

template <int C, int KS, bool GAIN>
__global__ __launch_bounds__(kThreads) void proj_split_kernel(const SplitParams p) {
  constexpr int kNU = KS / kUnitK;                        // units
  constexpr int kXU = kRowsPerWg * kUnitK / 4 / kThreads;  // 2 float4 of x per thread and unit
  constexpr int kWU = C * kUnitK / 4 / kThreads;          // C / 32 float4 of w
  constexpr int kCT = C / 16;                             // column tiles
  constexpr int kStr = KS + 4;                            // padded LDS row (floats)
  static_assert(kXU * kNU + kWU * kNU <= 32, "the whole tile in registers");
  __shared__ __align__(16) float xs[kRowsPerWg * kStr];
  __shared__ __align__(16) float ws[C * kStr];
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  // the K slice is the fastest-varying workgroup index: workgroups are
  // dealt to the XCDs round robin, so each XCD's L2 holds the activation
  // columns of one or two slices instead of all of them
  const int z = blockIdx.x;
  const int cb = blockIdx.y;
  const int mb = blockIdx.z;
  const int n0 = cb * C;
  const int m0 = mb * kRowsPerWg;
  int wi = 0;
  if (n0 >= p.w_end[0]) wi = n0 >= p.w_end[1] ? 2 : 1;
  const int col0 = wi == 0 ? 0 : p.w_end[wi - 1];
  const float* wbase = p.w[wi] + static_cast<int64_t>(n0 - col0) * p.in;
  const int k0 = z * KS;
  const int c4 = tid % 8;  // float4 e of a thread covers k 4 c4 .. + 3 of its unit; row / column e / 8

  f32x4_t xr[kNU][kXU], wr[kNU][kWU], g4[kNU];
#pragma unroll
  for (int u = 0; u < kNU; ++u) {
    const int kc = k0 + u * kUnitK + 4 * c4;
#pragma unroll
    for (int i = 0; i < kXU; ++i) {
      const int m = m0 + (i * kThreads + tid) / 8;
      const int mm = m < p.rows ? m : p.rows - 1;  // rows past the batch read row rows-1, never used
      xr[u][i] = *reinterpret_cast<const f32x4_t*>(p.x + static_cast<int64_t>(mm) * p.in + kc);
    }
#pragma unroll
    for (int i = 0; i < kWU; ++i)
      wr[u][i] = load_nt4(wbase + static_cast<int64_t>((i * kThreads + tid) / 8) * p.in + kc);
    if (GAIN) g4[u] = *reinterpret_cast<const f32x4_t*>(p.gain + kc);
  }
  __builtin_amdgcn_sched_barrier(0);

  f32x4_t acc[kCT];
#pragma unroll
  for (int t = 0; t < kCT; ++t) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float ss[kXU];
#pragma unroll
  for (int i = 0; i < kXU; ++i) ss[i] = 0.0f;
  // wave: rows 16 wave .. + 15 against the C columns; step s of a unit covers
  // k = 16 s + [0, 16), lane l supplying k = 16 s + 4 (l / 16) + e to matrix step 4 s + e
  const float* xa = &xs[(wave * kMTile + lane % 16) * kStr + 4 * (lane / 16)];
  const float* wb = &ws[(lane % 16) * kStr + 4 * (lane / 16)];
  // unit u's x (times the gain) and w into its own LDS region
  auto stage = [&](int u) {
#pragma unroll
    for (int i = 0; i < kXU; ++i) {
      f32x4_t v = xr[u][i];
      if (GAIN) {
#pragma unroll
        for (int e = 0; e < 4; ++e) ss[i] = __builtin_fmaf(v[e], v[e], ss[i]);
        v = v * g4[u];
      }
      *reinterpret_cast<f32x4_t*>(&xs[((i * kThreads + tid) / 8) * kStr + u * kUnitK + 4 * c4]) = v;
    }
#pragma unroll
    for (int i = 0; i < kWU; ++i)
      *reinterpret_cast<f32x4_t*>(&ws[((i * kThreads + tid) / 8) * kStr + u * kUnitK + 4 * c4]) = wr[u][i];
  };
  auto mfma_step = [&](const f32x4_t& a, const f32x4_t* b) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int t = 0; t < kCT; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[t][e], acc[t], 0, 0, 0);
    }
  };
  // Two steps per unit.  The operands of each step are read from LDS one step
  // ahead, and unit u + 1 is staged among the matrix steps of unit u's first
  // step, so its barrier passes between unit u's two steps and no LDS
  // latency or barrier wait sits between matrix steps.
  static_assert(kUnitK == 32, "two 16-k steps per unit");
  // instruction classes of __builtin_amdgcn_sched_group_barrier
  constexpr int kSgMfma = 0x008, kSgDsRead = 0x100, kSgDsWrite = 0x200;
  constexpr int kSteps = 4 * kCT;       // matrix steps per step
  constexpr int kReads = 1 + kCT;       // LDS reads of one step's operands
  constexpr int kWrites = kXU + kWU;    // LDS writes of one unit
  stage(0);
  __syncthreads();
  f32x4_t a0 = *reinterpret_cast<const f32x4_t*>(xa), b0[kCT];
#pragma unroll
  for (int t = 0; t < kCT; ++t) b0[t] = *reinterpret_cast<const f32x4_t*>(wb + t * 16 * kStr);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < kNU; ++u) {
    const int k1 = u * kUnitK + 16;
    const f32x4_t a1 = *reinterpret_cast<const f32x4_t*>(xa + k1);
    f32x4_t b1[kCT];
#pragma unroll
    for (int t = 0; t < kCT; ++t) b1[t] = *reinterpret_cast<const f32x4_t*>(wb + t * 16 * kStr + k1);
    mfma_step(a0, b0);
    if (u + 1 < kNU) stage(u + 1);
    // reads of step 1, then the writes of unit u + 1, spread over step 0's matrix steps
    __builtin_amdgcn_sched_group_barrier(kSgDsRead, kReads, 0);
    __builtin_amdgcn_sched_group_barrier(kSgMfma, 2, 0);
#pragma unroll
    for (int r = 0; r < kWrites; ++r) {
      __builtin_amdgcn_sched_group_barrier(kSgDsWrite, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSgMfma, (kSteps - 2) / kWrites > 0 ? (kSteps - 2) / kWrites : 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (u + 1 < kNU) {
      __syncthreads();
      const int k2 = (u + 1) * kUnitK;
      a0 = *reinterpret_cast<const f32x4_t*>(xa + k2);
#pragma unroll
      for (int t = 0; t < kCT; ++t) b0[t] = *reinterpret_cast<const f32x4_t*>(wb + t * 16 * kStr + k2);
    }
    mfma_step(a1, b1);
    // reads of unit u + 1's step 0 spread over step 1's matrix steps
    __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 1);
#pragma unroll
    for (int r = 0; r < kReads; ++r) {
      __builtin_amdgcn_sched_group_barrier(kSgDsRead, 1, 1);
      __builtin_amdgcn_sched_group_barrier(kSgMfma, (kSteps - 1) / kReads > 0 ? (kSteps - 1) / kReads : 1, 1);
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  // D layout: lane holds rows 16 wave + 4 (lane / 16) + i, column 16 t + lane % 16
  float* part = p.part + static_cast<int64_t>(z) * p.rows_pad * p.out;
#pragma unroll
  for (int t = 0; t < kCT; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = m0 + wave * kMTile + 4 * (lane / 16) + i;
      __builtin_nontemporal_store(acc[t][i], &part[static_cast<int64_t>(row) * p.out + n0 + 16 * t + lane % 16]);
    }
  }
  if (GAIN && cb == 0) {
    // the slice's sum of squares of x per row: row (i * 256 + tid) / 8 is
    // held by 8 consecutive threads
#pragma unroll
    for (int i = 0; i < kXU; ++i) {
      float v = ss[i];
#pragma unroll
      for (int off = 4; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
      if (c4 == 0) p.ss[static_cast<int64_t>(z) * p.rows_pad + m0 + (i * kThreads + tid) / 8] = v;
    }
  }
}

using QkvReduceParams = qkv::ReduceParams;

// The K-slice partials at offset off of each slice (slice_stride floats
// apart), added in slice order from zero; each batch of 8 slices' loads is
// issued before its adds.
__device__ inline f32x4_t sum_slices4(const float* part, int slices, int64_t slice_stride, int64_t off) {
  constexpr int kBatch = 8;
  f32x4_t v = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  for (int z0 = 0; z0 < slices; z0 += kBatch) {
    f32x4_t s[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int z = z0 + i < slices ? z0 + i : slices - 1;
      s[i] = *reinterpret_cast<const f32x4_t*>(part + z * slice_stride + off);
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      if (z0 + i < slices) v += s[i];
  }
  return v;
}

// Workgroup (head, 8-row block): the slices of the head's 128 columns added
// in slice order, times the row's input RMSNorm scale; q and k heads then
// take the head RMS norm and RoPE (qkv::head_value).  Thread t: row t / 32,
// d = 4 (t % 32) .. + 3; d and d + 64 sit 16 threads apart.
__device__ inline void qkv_reduce_rows(const QkvReduceParams& p, int hh, int rb) {
  const int tid = threadIdx.x;
  const int row = rb * 8 + tid / 32;
  const int rr = row < p.rows ? row : p.rows - 1;  // rows past the batch compute row rows-1, not stored
  const int j = tid % 32;
  const qkv::f32x4_t o = qkv::head_value(p, hh, rr, j);
  if (row < p.rows) *reinterpret_cast<qkv::f32x4_t*>(qkv::head_dst(p, hh, row) + 4 * j) = o;
}

__global__ __launch_bounds__(kThreads) void qkv_reduce_kernel(const QkvReduceParams p) {
  for (int rb = blockIdx.y; rb * 8 < p.rows; rb += gridDim.y) qkv_reduce_rows(p, blockIdx.x, rb);
}

// y[row][c..c+3] = the slices added in slice order (+ residual).
__global__ __launch_bounds__(kWave) void linear_reduce_kernel(const float* part, int slices, int rows,
                                                              int rows_pad, int out, const float* residual,
                                                              float* y) {
  const int c = (blockIdx.x * kWave + threadIdx.x) * 4;
  if (c >= out) return;
  for (int row = blockIdx.y; row < rows; row += gridDim.y) {
    const int64_t o = static_cast<int64_t>(row) * out + c;
    const f32x4_t r = residual ? *reinterpret_cast<const f32x4_t*>(residual + o) : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    f32x4_t v = sum_slices4(part, slices, static_cast<int64_t>(rows_pad) * out, o);
    if (residual) v += r;
    *reinterpret_cast<f32x4_t*>(y + o) = v;
  }
}

}  // namespace

// Tile of a split projection: K slices of 256 k (no upper bound: the reduce
// adds any number of slices in slice order), with 64 columns per workgroup
// when the slices number at most 8 and the 64-column grid still gives every
// compute unit a workgroup, else 32 columns (2048 -> 1024: 256 workgroups, 8
// slices; 4096 -> 4096, the Qwen3-8B o-projection: 2048 workgroups, 16
// slices).  A 64-column tile of at most 4 slices takes 128 k instead (twice
// the slices): its 66 KB of LDS lets two workgroups share a compute unit, one
// staging while the other runs its matrix steps (1024 -> 4096: 512
// workgroups, 8 slices; 10.0 against 10.9 us for 4 slices of 256 k, the
// epilogue's loads of the extra slices issued together).  The workspace holds
// slices x rows x out partial sums.
SplitShape split_shape(int64_t rows, int64_t in, int64_t out) {
  const int64_t rb = (rows + kRowsPerWg - 1) / kRowsPerWg;
  SplitShape sh{64, static_cast<int32_t>(in / 256), 256};
  if (sh.slices > kWideTileMaxSlices || (out / 64) * sh.slices * rb < compute_units()) {
    sh.cols = 32;
  } else if (2 * sh.slices <= kWideTileMaxSlices) {
    sh.slices *= 2;
    sh.ks = 128;
  }
  return sh;
}

size_t split_part_bytes(int64_t rows, int64_t in, int64_t out, bool with_ss) {
  const SplitShape sh = split_shape(rows, in, out);
  const int64_t rows_pad = (rows + kRowsPerWg - 1) / kRowsPerWg * kRowsPerWg;
  const size_t part = static_cast<size_t>(sh.slices) * rows_pad * out * sizeof(float);
  return part + (with_ss ? static_cast<size_t>(sh.slices) * rows_pad * sizeof(float) : 0);
}

namespace {

hipError_t launch_split(const SplitParams& p, const SplitShape& sh, int rb, hipStream_t stream) {
  const dim3 grid(sh.slices, p.out / sh.cols, rb);
  if (sh.cols == 64 && sh.ks == 128) {
    if (p.gain) hipLaunchKernelGGL((proj_split_kernel<64, 128, true>), grid, dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((proj_split_kernel<64, 128, false>), grid, dim3(kThreads), 0, stream, p);
  } else if (sh.cols == 64) {
    if (p.gain) hipLaunchKernelGGL((proj_split_kernel<64, 256, true>), grid, dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((proj_split_kernel<64, 256, false>), grid, dim3(kThreads), 0, stream, p);
  } else {
    if (p.gain) hipLaunchKernelGGL((proj_split_kernel<32, 256, true>), grid, dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((proj_split_kernel<32, 256, false>), grid, dim3(kThreads), 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_rms_norm(const float* x, const float* w, float* out, int rows, int width, float eps,
                           hipStream_t stream) {
  hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(kThreads), 0, stream, x, w, out, width, eps);
  return hipGetLastError();
}

hipError_t launch_linear(const LinearLaunch& l, hipStream_t stream) {
  const SplitShape sh = split_shape(l.rows, l.in, l.out);
  const int rb = (l.rows + kRowsPerWg - 1) / kRowsPerWg;
  SplitParams p{};
  p.x = l.x;
  p.w[0] = p.w[1] = p.w[2] = l.w;
  p.w_end[0] = p.w_end[1] = p.w_end[2] = l.out;
  p.part = l.workspace;
  p.rows = l.rows;
  p.rows_pad = rb * kRowsPerWg;
  p.in = l.in;
  p.out = l.out;
  hipError_t e = launch_split(p, sh, rb, stream);
  if (e != hipSuccess) return e;
  const dim3 grid((l.out / 4 + kWave - 1) / kWave, std::min(l.rows, 65535));
  hipLaunchKernelGGL(linear_reduce_kernel, grid, dim3(kWave), 0, stream, p.part, sh.slices, l.rows, p.rows_pad,
                     l.out, l.residual, l.y);
  return hipGetLastError();
}

hipError_t launch_qkv_partials(const QkvLaunch& q, qkv::ReduceParams* r, hipStream_t stream) {
  const int qw = q.q_heads * kHeadDim, kw = q.kv_heads * kHeadDim;
  const int out = qw + 2 * kw;
  const SplitShape sh = split_shape(q.rows, q.hidden, out);
  const int rb = (q.rows + kRowsPerWg - 1) / kRowsPerWg;
  SplitParams p{};
  p.x = q.x;
  p.w[0] = q.wq;
  p.w[1] = q.wk;
  p.w[2] = q.wv;
  p.w_end[0] = qw;
  p.w_end[1] = qw + kw;
  p.w_end[2] = out;
  p.gain = q.gain;
  p.part = q.workspace;
  p.rows = q.rows;
  p.rows_pad = rb * kRowsPerWg;
  p.ss = q.workspace + static_cast<int64_t>(sh.slices) * p.rows_pad * out;
  p.in = q.hidden;
  p.out = out;
  hipError_t e = launch_split(p, sh, rb, stream);
  if (e != hipSuccess) return e;
  *r = qkv::ReduceParams{};
  r->part = p.part;
  r->ss = q.gain ? p.ss : nullptr;
  r->slices = sh.slices;
  r->rows = q.rows;
  r->rows_pad = p.rows_pad;
  r->in = q.hidden;
  r->out = out;
  r->in_eps = q.in_eps;
  r->q_norm = q.q_norm;
  r->k_norm = q.k_norm;
  r->positions = q.positions;
  r->q = q.q;
  r->k = q.k;
  r->v = q.v;
  r->q_heads = q.q_heads;
  r->kv_heads = q.kv_heads;
  r->eps = q.eps;
  for (int i = 0; i < 64; ++i) r->inv_freq[i] = q.inv_freq[i];
  return hipSuccess;
}

hipError_t launch_qkv_project(const QkvLaunch& q, hipStream_t stream) {
  QkvReduceParams r;
  hipError_t e = launch_qkv_partials(q, &r, stream);
  if (e != hipSuccess) return e;
  const dim3 grid(q.q_heads + 2 * q.kv_heads, std::min((q.rows + 7) / 8, 65535));
  hipLaunchKernelGGL(qkv_reduce_kernel, grid, dim3(kThreads), 0, stream, r);
  return hipGetLastError();
}

}  // namespace sa
