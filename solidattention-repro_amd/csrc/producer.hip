// producer.hip — the query producer and output consumer around the decode
// attention (gfx950): RMSNorm, the [out][in] fp32 projections on the matrix
// cores, the per-head RMS norm + rotary embedding, and the residual add.
// Semantics of the reference's rms_norm, head_rms, rope and
// cublasSgemm(CUBLAS_OP_T) calls (cpp/src/qwen_layer_main.cpp:125-172,
// :576-584, :640-645; cpp/src/qwen_chain_main.cpp:365-399) for a batch of
// decode tokens (one row per sequence).
//
// Projection (proj_kernel): y[r][o] = sum_i x[r][i] w[o][i].  At decode the
// rows are few (the batch) and the weights are the traffic.  A workgroup of
// 4 waves owns 16 output columns and up to 64 rows over a K range (all of K,
// or 1/ks of it), taken in 128-k chunks that all 256 threads stage in LDS
// with row-contiguous loads (two chunks ahead); wave t then runs the
// v_mfma_f32_16x16x4f32 steps of rows 16 t .. 16 t + 15 against the 16
// columns (any order of the k sum is a valid fp32 sum, and the order is
// fixed: deterministic).  Epilogues run in the same launch:
//   * linear: with ks > 1 the K slices write partial tiles; the last slice to
//     arrive (an arrival counter per column slab, left at zero) adds them in
//     slice order plus the residual;
//   * q/k/v: the optional input RMSNorm folds into a per-row scale (every
//     workgroup sees whole rows: ks is 1), v columns are written directly,
//     and the last of a q/k head's 8 slabs to arrive applies head RMS + RoPE.
#include <algorithm>

#include "sa_device.hpp"
#include "sa_internal.hpp"

namespace sa {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;  // 4
constexpr int kCols = 16;                 // output columns per workgroup
constexpr int kMTile = 16;
constexpr int kMTiles = 4;
constexpr int kRowsPerWg = kMTile * kMTiles;  // 64
constexpr int kChunk = 64;                // k per pipeline stage and wave
constexpr int kKPerWgUnit = kWaves * kChunk;  // 256: K per workgroup is a multiple

__device__ inline f32x4_t load_nt4(const float* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
}

// Values handed from one workgroup to another (possibly on another XCD) go
// through agent-scope atomic stores and loads: coherent single accesses, with
// no L2 writeback or invalidate (an agent-scope fence would write back and
// invalidate the whole L2 of the XCD, and with it the x rows every other
// workgroup is reading).  The writer waits for its stores to complete before
// the arrival counter is incremented.
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

struct ProjParams {
  const float* x;          // [rows][in]
  const float* w[3];       // [out][in]; weight j covers output columns [w_end[j-1], w_end[j])
  int32_t w_end[3];
  const float* gain;       // q/k/v: optional input RMSNorm weight [in]
  float in_eps;
  const float* residual;   // linear: optional [rows][out]
  float* y;                // linear: [rows][out]
  float* part;             // linear: [ks][rows][out] slice tiles (ks > 1); q/k/v: [rows][out] before the head epilogue
  int32_t* counters;       // arrival counters, zero between launches
  int32_t rows;
  int32_t in;
  int32_t out;
  int32_t ks;
  // q/k/v epilogue
  const float* q_norm;
  const float* k_norm;
  const int32_t* positions;
  float* q;                // [rows][q_heads][128]
  float* k;                // [rows][kv_heads][128]
  float* v;
  int32_t q_heads;
  int32_t kv_heads;
  float eps;
  float inv_freq[64];
};

// One thread's share of a 128-k chunk: x [64 rows][128] is 2048 float4 (8 per
// thread), w [16 columns][128] is 512 float4 (2 per thread); thread e of a
// float4 index reads row e / 32, float4 e % 32 of that row, so a wave's load
// covers two whole 512-byte row segments.
constexpr int kKC = 128;
constexpr int kLdsStride = kKC + 4;  // padded LDS rows (floats)
constexpr int kXVecs = kRowsPerWg * kKC / 4 / kThreads;  // 8
constexpr int kWVecs = kCols * kKC / 4 / kThreads;       // 2

struct ChunkRegs {
  f32x4_t x[kXVecs];
  f32x4_t w[kWVecs];
  f32x4_t g;
};

template <bool GAIN>
__device__ inline void chunk_load(ChunkRegs& r, const ProjParams& p, const float* wbase, int m0, int kc) {
  const int tid = threadIdx.x;
  const int c4 = tid % 32;
#pragma unroll
  for (int i = 0; i < kWVecs; ++i) {
    const int col = (i * kThreads + tid) / 32;
    r.w[i] = load_nt4(wbase + static_cast<int64_t>(col) * p.in + kc + 4 * c4);
  }
#pragma unroll
  for (int i = 0; i < kXVecs; ++i) {
    const int m = m0 + (i * kThreads + tid) / 32;
    const int mm = m < p.rows ? m : p.rows - 1;  // rows past the batch read row rows-1, never stored
    r.x[i] = *reinterpret_cast<const f32x4_t*>(p.x + static_cast<int64_t>(mm) * p.in + kc + 4 * c4);
  }
  if (GAIN) r.g = *reinterpret_cast<const f32x4_t*>(p.gain + kc + 4 * c4);
}

template <bool GAIN>
__device__ inline void chunk_store(const ChunkRegs& r, float* xs, float* ws, float (&ss)[kXVecs]) {
  const int tid = threadIdx.x;
  const int c4 = tid % 32;
#pragma unroll
  for (int i = 0; i < kWVecs; ++i) {
    const int col = (i * kThreads + tid) / 32;
    *reinterpret_cast<f32x4_t*>(ws + col * kLdsStride + 4 * c4) = r.w[i];
  }
#pragma unroll
  for (int i = 0; i < kXVecs; ++i) {
    const int row = (i * kThreads + tid) / 32;
    f32x4_t v = r.x[i];
    if (GAIN) {
#pragma unroll
      for (int e = 0; e < 4; ++e) ss[i] = __builtin_fmaf(v[e], v[e], ss[i]);
      v = v * r.g;
    }
    *reinterpret_cast<f32x4_t*>(xs + row * kLdsStride + 4 * c4) = v;
  }
}

// Wave t: rows 16 t .. 16 t + 15 of the chunk against its 16 columns; step s
// covers k = 16 s + [0, 16), lane l supplying k = 16 s + 4 (l / 16) + e to
// MFMA 4 s + e.
__device__ inline void chunk_mfma(const float* xs, const float* ws, int wave, int lane, f32x4_t& acc) {
  const float* xa = xs + (wave * kMTile + lane % 16) * kLdsStride + 4 * (lane / 16);
  const float* wb = ws + (lane % 16) * kLdsStride + 4 * (lane / 16);
#pragma unroll
  for (int s = 0; s < kKC / 16; ++s) {
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(xa + 16 * s);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(wb + 16 * s);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], acc, 0, 0, 0);
  }
}

// The head RMS norm then RoPE (NeoX pairs d, d + 64) of rows [m0, m0 + 64) of
// q/k head hh (hh < q_heads: q) from the pre-epilogue values in part.  Wave w
// takes rows m0 + w + 4 i, i < 16, lane l holding d = l and l + 64; the 16
// rows are independent, so their loads, reductions, sincos and stores are
// issued together (fully unrolled, no early exit).
__device__ inline void qk_head_epilogue(const ProjParams& p, int m0, int hh) {
  constexpr int kRowsPerWave = kRowsPerWg / kWaves;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const bool is_q = hh < p.q_heads;
  const float* norm = is_q ? p.q_norm : p.k_norm;
  const float n_lo = norm[lane], n_hi = norm[lane + 64];
  const float f = p.inv_freq[lane];
  float a[kRowsPerWave], b[kRowsPerWave], ss[kRowsPerWave], angle[kRowsPerWave];
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const int row = m0 + wave + kWaves * i;
    const int rr = row < p.rows ? row : m0;
    const float* src = p.part + static_cast<int64_t>(rr) * p.out + hh * kHeadDim;
    a[i] = load_agent(src + lane);
    b[i] = load_agent(src + lane + 64);
    angle[i] = static_cast<float>(p.positions[rr]) * f;
  }
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) ss[i] = a[i] * a[i] + b[i] * b[i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
#pragma unroll
    for (int i = 0; i < kRowsPerWave; ++i) ss[i] += __shfl_xor(ss[i], off, kWave);
  }
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const int row = m0 + wave + kWaves * i;
    const float inv = 1.0f / __builtin_sqrtf(ss[i] / static_cast<float>(kHeadDim) + p.eps);
    const float x0 = a[i] * inv * n_lo;
    const float x1 = b[i] * inv * n_hi;
    float sn, cs;
    sincosf(angle[i], &sn, &cs);
    if (row < p.rows) {
      float* dst = is_q ? p.q + (static_cast<int64_t>(row) * p.q_heads + hh) * kHeadDim
                        : p.k + (static_cast<int64_t>(row) * p.kv_heads + (hh - p.q_heads)) * kHeadDim;
      dst[lane] = x0 * cs - x1 * sn;
      dst[lane + 64] = x1 * cs + x0 * sn;
    }
  }
}

// QKV: q/k/v producer (ks 1); else the linear (ks K slices).  Chunks of the
// workgroup's K range are staged in LDS two ahead (registers, then one of two
// LDS buffers); the chunk order starts at the slab's index so that the
// workgroups, which read the same x, do not all read the same addresses at
// the same time.
template <bool QKV, bool GAIN>
__global__ __launch_bounds__(kThreads) void proj_kernel(const ProjParams p) {
  __shared__ __align__(16) float xs[2][kRowsPerWg * kLdsStride];
  __shared__ __align__(16) float ws[2][kCols * kLdsStride];
  __shared__ float ss_s[kRowsPerWg];
  __shared__ int s_last;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int slab = blockIdx.x;
  const int z = blockIdx.y;
  const int mb = blockIdx.z;
  const int n0 = slab * kCols;
  const int m0 = mb * kRowsPerWg;
  const int kslice = p.in / p.ks;
  const int chunks = kslice / kKC;  // even, >= 2
  const int rot = slab % chunks;

  int wi = 0;
  if (n0 >= p.w_end[0]) wi = n0 >= p.w_end[1] ? 2 : 1;
  const int col0 = wi == 0 ? 0 : p.w_end[wi - 1];
  const float* wbase = p.w[wi] + static_cast<int64_t>(n0 - col0) * p.in;
  auto kc_of = [&](int c) { return z * kslice + ((c + rot) % chunks) * kKC; };

  f32x4_t acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float ss[kXVecs];
#pragma unroll
  for (int i = 0; i < kXVecs; ++i) ss[i] = 0.0f;
  if (chunks % 4 == 0) {
    // four chunks in flight (registers r0..r3), two in LDS: at the top of
    // an iteration chunk c is in LDS buffer 0 and r1, r2, r3 hold c + 1 ..
    // c + 3; the loads of the steady state are unconditional
    ChunkRegs r0, r1, r2, r3;
    chunk_load<GAIN>(r0, p, wbase, m0, kc_of(0));
    chunk_load<GAIN>(r1, p, wbase, m0, kc_of(1));
    chunk_load<GAIN>(r2, p, wbase, m0, kc_of(2));
    chunk_load<GAIN>(r3, p, wbase, m0, kc_of(3));
    chunk_store<GAIN>(r0, xs[0], ws[0], ss);
    __syncthreads();
    int c = 0;
    for (; c + 7 < chunks; c += 4) {
      chunk_load<GAIN>(r0, p, wbase, m0, kc_of(c + 4));
      __builtin_amdgcn_sched_barrier(0);
      chunk_mfma(xs[0], ws[0], wave, lane, acc);
      chunk_store<GAIN>(r1, xs[1], ws[1], ss);
      __syncthreads();
      chunk_load<GAIN>(r1, p, wbase, m0, kc_of(c + 5));
      __builtin_amdgcn_sched_barrier(0);
      chunk_mfma(xs[1], ws[1], wave, lane, acc);
      chunk_store<GAIN>(r2, xs[0], ws[0], ss);
      __syncthreads();
      chunk_load<GAIN>(r2, p, wbase, m0, kc_of(c + 6));
      __builtin_amdgcn_sched_barrier(0);
      chunk_mfma(xs[0], ws[0], wave, lane, acc);
      chunk_store<GAIN>(r3, xs[1], ws[1], ss);
      __syncthreads();
      chunk_load<GAIN>(r3, p, wbase, m0, kc_of(c + 7));
      __builtin_amdgcn_sched_barrier(0);
      chunk_mfma(xs[1], ws[1], wave, lane, acc);
      chunk_store<GAIN>(r0, xs[0], ws[0], ss);
      __syncthreads();
    }
    // the last four chunks
    chunk_mfma(xs[0], ws[0], wave, lane, acc);
    chunk_store<GAIN>(r1, xs[1], ws[1], ss);
    __syncthreads();
    chunk_mfma(xs[1], ws[1], wave, lane, acc);
    chunk_store<GAIN>(r2, xs[0], ws[0], ss);
    __syncthreads();
    chunk_mfma(xs[0], ws[0], wave, lane, acc);
    chunk_store<GAIN>(r3, xs[1], ws[1], ss);
    __syncthreads();
    chunk_mfma(xs[1], ws[1], wave, lane, acc);
  } else {
  ChunkRegs r0, r1;
  chunk_load<GAIN>(r0, p, wbase, m0, kc_of(0));
  chunk_load<GAIN>(r1, p, wbase, m0, kc_of(1));
  chunk_store<GAIN>(r0, xs[0], ws[0], ss);
  __syncthreads();
  // iteration c: chunk c in LDS buffer 0, chunk c + 1 in registers r1.  The
  // loads of the steady state are unconditional: a load under a branch makes
  // the compiler wait for it at the next use of the other buffer, which would
  // expose the whole latency once per chunk.
  // (the scheduling barriers keep each chunk's loads ahead of the matrix
  // work instead of sunk next to their LDS stores)
  int c = 0;
  for (; c + 3 < chunks; c += 2) {
    chunk_load<GAIN>(r0, p, wbase, m0, kc_of(c + 2));
    __builtin_amdgcn_sched_barrier(0);
    chunk_mfma(xs[0], ws[0], wave, lane, acc);
    chunk_store<GAIN>(r1, xs[1], ws[1], ss);
    __syncthreads();
    chunk_load<GAIN>(r1, p, wbase, m0, kc_of(c + 3));
    __builtin_amdgcn_sched_barrier(0);
    chunk_mfma(xs[1], ws[1], wave, lane, acc);
    chunk_store<GAIN>(r0, xs[0], ws[0], ss);
    __syncthreads();
  }
  // the last two chunks
  chunk_mfma(xs[0], ws[0], wave, lane, acc);
  chunk_store<GAIN>(r1, xs[1], ws[1], ss);
  __syncthreads();
  chunk_mfma(xs[1], ws[1], wave, lane, acc);
  }

  // D layout: lane holds rows 16 wave + 4 (lane / 16) + i, column lane % 16
  float inv[4] = {1.0f, 1.0f, 1.0f, 1.0f};
  if (GAIN) {
    // ss[i] of row (i * 256 + tid) / 32: the 32 threads of a row are half a wave
#pragma unroll
    for (int i = 0; i < kXVecs; ++i) {
      float v = ss[i];
#pragma unroll
      for (int off = 16; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
      if (tid % 32 == 0) ss_s[(i * kThreads + tid) / 32] = v;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float tot = ss_s[wave * kMTile + 4 * (lane / 16) + i];
      inv[i] = 1.0f / __builtin_sqrtf(tot / static_cast<float>(p.in) + p.in_eps);
    }
  }
  const int col = n0 + lane % 16;

  if (QKV) {
    const bool is_v = n0 >= p.w_end[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = m0 + wave * kMTile + 4 * (lane / 16) + i;
      if (row >= p.rows) continue;
      const float val = acc[i] * inv[i];
      if (is_v) {
        p.v[static_cast<int64_t>(row) * p.kv_heads * kHeadDim + (col - p.w_end[1])] = val;
      } else {
        store_agent(p.part + static_cast<int64_t>(row) * p.out + col, val);
      }
    }
    if (is_v) return;
    // the last of the head's 8 slabs applies head RMS + RoPE
    const int hh = n0 / kHeadDim;
    if (!last_arrival(p.counters + mb * (p.q_heads + p.kv_heads) + hh, kHeadDim / kCols, &s_last)) return;
    qk_head_epilogue(p, m0, hh);
    return;
  }

  // linear
  const int64_t slice = static_cast<int64_t>(p.rows) * p.out;
  if (p.ks == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = m0 + wave * kMTile + 4 * (lane / 16) + i;
      if (row >= p.rows) continue;
      const int64_t o = static_cast<int64_t>(row) * p.out + col;
      p.y[o] = p.residual ? acc[i] + p.residual[o] : acc[i];
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = m0 + wave * kMTile + 4 * (lane / 16) + i;
    if (row < p.rows) store_agent(p.part + z * slice + static_cast<int64_t>(row) * p.out + col, acc[i]);
  }
  if (!last_arrival(p.counters + mb * (p.out / kCols) + slab, p.ks, &s_last)) return;
  // the slices in slice order, then the residual: thread e sums row e / 4,
  // columns 4 (e % 4) .. + 3
  const int row = m0 + tid / 4;
  if (row >= p.rows) return;
  const int64_t o = static_cast<int64_t>(row) * p.out + n0 + 4 * (tid % 4);
  // the slices' values loaded together (up to 8 at a time), then added in order
  float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int z0 = 0; z0 < p.ks; z0 += 8) {
    float v[8][4];
#pragma unroll
    for (int zz = 0; zz < 8; ++zz) {
#pragma unroll
      for (int j = 0; j < 4; ++j) v[zz][j] = z0 + zz < p.ks ? load_agent(p.part + (z0 + zz) * slice + o + j) : 0.0f;
    }
#pragma unroll
    for (int zz = 0; zz < 8; ++zz) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (z0 + zz < p.ks) sum[j] += v[zz][j];
    }
  }
  f32x4_t v4{sum[0], sum[1], sum[2], sum[3]};
  if (p.residual) v4 += *reinterpret_cast<const f32x4_t*>(p.residual + o);
  *reinterpret_cast<f32x4_t*>(p.y + o) = v4;
}

}  // namespace

int linear_ksplit(int64_t rows, int64_t in, int64_t out) {
  // K slices so that the workgroups (16 columns x 64 rows each) about fill
  // the compute units, each slice a multiple of 256 k (4 waves x 64)
  const int64_t mblocks = (rows + kRowsPerWg - 1) / kRowsPerWg;
  const int64_t blocks = (out / kCols) * mblocks;
  int64_t ks = 1;
  while (blocks * ks * 2 <= compute_units() && (in / (ks * 2)) % kKPerWgUnit == 0) ks *= 2;
  return static_cast<int>(ks);
}

size_t linear_counter_bytes(int64_t rows, int64_t out) {
  const int64_t mblocks = (rows + kRowsPerWg - 1) / kRowsPerWg;
  return static_cast<size_t>((mblocks * (out / kCols) * 4 + 255) / 256 * 256);
}

size_t qkv_counter_bytes(int64_t rows, int q_heads, int kv_heads) {
  const int64_t mblocks = (rows + kRowsPerWg - 1) / kRowsPerWg;
  return static_cast<size_t>((mblocks * (q_heads + kv_heads) * 4 + 255) / 256 * 256);
}

hipError_t launch_rms_norm(const float* x, const float* w, float* out, int rows, int width, float eps,
                           hipStream_t stream) {
  hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(kThreads), 0, stream, x, w, out, width, eps);
  return hipGetLastError();
}

hipError_t launch_linear(const LinearLaunch& l, hipStream_t stream) {
  const int ks = linear_ksplit(l.rows, l.in, l.out);
  ProjParams p{};
  p.x = l.x;
  p.w[0] = p.w[1] = p.w[2] = l.w;
  p.w_end[0] = p.w_end[1] = p.w_end[2] = l.out;
  p.residual = l.residual;
  p.y = l.y;
  p.counters = reinterpret_cast<int32_t*>(l.workspace);
  p.part = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(l.workspace) + linear_counter_bytes(l.rows, l.out));
  p.rows = l.rows;
  p.in = l.in;
  p.out = l.out;
  p.ks = ks;
  const dim3 grid(l.out / kCols, ks, (l.rows + kRowsPerWg - 1) / kRowsPerWg);
  hipLaunchKernelGGL((proj_kernel<false, false>), grid, dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_qkv_project(const QkvLaunch& q, hipStream_t stream) {
  const int qw = q.q_heads * kHeadDim, kw = q.kv_heads * kHeadDim;
  const int out = qw + 2 * kw;
  ProjParams p{};
  p.x = q.x;
  p.w[0] = q.wq;
  p.w[1] = q.wk;
  p.w[2] = q.wv;
  p.w_end[0] = qw;
  p.w_end[1] = qw + kw;
  p.w_end[2] = out;
  p.gain = q.gain;
  p.in_eps = q.in_eps;
  p.counters = reinterpret_cast<int32_t*>(q.workspace);
  p.part = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(q.workspace) +
                                    qkv_counter_bytes(q.rows, q.q_heads, q.kv_heads));
  p.rows = q.rows;
  p.in = q.hidden;
  p.out = out;
  p.ks = 1;
  p.q_norm = q.q_norm;
  p.k_norm = q.k_norm;
  p.positions = q.positions;
  p.q = q.q;
  p.k = q.k;
  p.v = q.v;
  p.q_heads = q.q_heads;
  p.kv_heads = q.kv_heads;
  p.eps = q.eps;
  for (int i = 0; i < 64; ++i) p.inv_freq[i] = q.inv_freq[i];
  const dim3 grid(out / kCols, 1, (q.rows + kRowsPerWg - 1) / kRowsPerWg);
  if (q.gain) {
    hipLaunchKernelGGL((proj_kernel<true, true>), grid, dim3(kThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((proj_kernel<true, false>), grid, dim3(kThreads), 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace sa
