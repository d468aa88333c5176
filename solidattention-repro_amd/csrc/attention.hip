// attention.hip — GQA sparse decode attention over paged FP16 KV (gfx950).
//
// Semantics: attention_reference (reference cpp/src/attention_reference.cpp
// :55-96) applied, per (sequence, KV head g), to the tokens of the selected
// sealed blocks followed by the unsealed tail, for each of the G query heads
// of g.  Softmax is computed online in the log2 domain and split over
// `splits` workgroups per (sequence, KV head); partial results are merged
// with log-sum-exp by a second, small kernel.  fp32 arithmetic on exact FP16
// decodes; the reference's two-pass order is not reproduced
// (tolerance-checked, not bit-exact).
//
// Mapping (head_dim 128): one wave64 walks whole 32-token pages.  A 16-byte
// load per lane covers 4 rows of 256 B (16 lanes per K or V row of one KV
// head), so a page's K and V tiles for head g are 8 + 8 dwordx4 loads per
// lane.  Lane (row r, column c) owns dims [8c, 8c+8) of tokens {r, r+4, ...}.
// q.k partial dots are reduced across the 16 lanes of a row with DPP; the G
// query heads of the group reuse every K/V register (v_fma_mix_f32 consumes
// the FP16 halves directly), so KV bytes are read from HBM once per group.
// No MFMA: decode attention is a matrix-vector product (about 2 flop per KV
// byte at G=2).  Measured on MI355X at B=64/16K: one workgroup of 8 waves per
// (sequence, KV head), ~8 pages per wave, with non-temporal page loads
// streams the selected pages at ~6.1 TB/s (plain loads: 5.3 TB/s; a plain
// contiguous read of the pool: 6.4 TB/s); a register-prefetch variant and a
// fused last-workgroup merge were both slower.
#include "sa_device.hpp"
#include "sa_internal.hpp"

namespace sa {
namespace {

constexpr int D = kHeadDim;
// Waves per workgroup: 8 for G <= 2 (123 VGPRs: two 8-wave workgroups per
// CU); 4 for G >= 4, whose larger accumulator sets (161+ VGPRs) would leave
// room for only one 8-wave workgroup per CU.
template <int G>
constexpr int waves_per_group() { return G >= 4 ? 4 : 8; }
constexpr int kMergeThreads = 256;
constexpr int kLanesPerRow = D / 8;               // 16 lanes x 8 halves = one 256 B row
constexpr int kRows = kWave / kLanesPerRow;       // 4 rows per wave-wide load
constexpr int kIters = kPageTokens / kRows;       // 8 tokens per lane per page
constexpr float kNegInf = -__builtin_huge_valf();

struct Params {
  const uint16_t* pool;
  const int32_t* table;
  const int32_t* seq_len;
  const int32_t* sealed;
  const int32_t* selected;
  const int32_t* counts;
  const float* query;
  float* out;
  float* part;
  int32_t* status;
  int64_t num_pages;
  int64_t contig_tokens;
  int64_t page_elems;
  int32_t token_elems;
  int32_t table_stride;
  int32_t sel_stride;
  int32_t select_groups;
  int32_t kv_per_sel;
  int32_t query_heads;
  int32_t kv_heads;
  int32_t splits;        // workgroups per (sequence, KV head) in this launch
  int32_t part_base;     // first partial record written by this launch
  int32_t part_total;    // partial records per (sequence, KV head) in the workspace
  int32_t include_tail;  // attend the unsealed tail too
  int32_t direct;        // write the normalised output instead of a partial record
  float qscale;          // softmax scale * log2(e)
};

__device__ inline void unpack8(const uint4& w, float (&f)[8]) {
  f[0] = lo_h2f(w.x);
  f[1] = hi_h2f(w.x);
  f[2] = lo_h2f(w.y);
  f[3] = hi_h2f(w.y);
  f[4] = lo_h2f(w.z);
  f[5] = hi_h2f(w.z);
  f[6] = lo_h2f(w.w);
  f[7] = hi_h2f(w.w);
}

// Page `i` of the (sequence, KV head) list: selected sealed blocks first,
// then the tail pages.  valid = number of tokens to read (0 = skip).
struct PageRef {
  int64_t page;
  int valid;
};

struct PageList {
  const int32_t* sel;
  int64_t len;
  int sealed;
  int n_sel;
  int total;
};

__device__ inline PageRef resolve_page(const Params& p, int b, int i, const PageList& L) {
  PageRef r{0, 0};
  if (i >= L.total) return r;
  int64_t logical;
  if (i < L.n_sel) {
    logical = L.sel[i];
    if (logical < 0 || logical >= L.sealed) {
      flag_status(p.status, kStatusBadBlock);
      return r;
    }
    r.valid = kPageTokens;
  } else {
    logical = static_cast<int64_t>(L.sealed) + (i - L.n_sel);
    const int64_t left = L.len - logical * kPageTokens;
    r.valid = left < kPageTokens ? static_cast<int>(left) : kPageTokens;
  }
  if (p.contig_tokens > 0) {
    r.page = logical;
    return r;
  }
  if (logical >= p.table_stride) {
    flag_status(p.status, kStatusBadBlock);
    r.valid = 0;
    return r;
  }
  const int64_t page = p.table[static_cast<int64_t>(b) * p.table_stride + logical];
  if (page < 0 || page >= p.num_pages) {
    flag_status(p.status, kStatusBadPage);
    r.valid = 0;
    return r;
  }
  r.page = page;
  return r;
}

// Issue the 16 dwordx4 loads of one page's K and V tiles (head g).  Rows past
// `valid` are not read (a contiguous buffer may end inside the last page).
__device__ inline void load_page(const Params& p, const PageRef& pr, int64_t head_off, int64_t v_off,
                                 int64_t step4, int row, uint4 (&kr)[kIters], uint4 (&vr)[kIters]) {
  const uint16_t* kbase = p.pool + pr.page * p.page_elems + head_off;
  if (pr.valid == kPageTokens) {
#pragma unroll
    for (int it = 0; it < kIters; ++it) kr[it] = load_stream16(kbase + it * step4);
#pragma unroll
    for (int it = 0; it < kIters; ++it) vr[it] = load_stream16(kbase + it * step4 + v_off);
  } else {
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      if (it * kRows + row < pr.valid) {
        kr[it] = load_stream16(kbase + it * step4);
        vr[it] = load_stream16(kbase + it * step4 + v_off);
      } else {
        kr[it] = make_uint4(0, 0, 0, 0);
        vr[it] = make_uint4(0, 0, 0, 0);
      }
    }
  }
}

// Online-softmax update of the wave state with one page.
template <int G>
__device__ inline void process_page(const uint4 (&kr)[kIters], const uint4 (&vr)[kIters], int valid, int row,
                                    const float (&qf)[G][8], float (&m)[G], float (&l)[G],
                                    float (&acc)[G][8]) {
  // logits (log2 domain) of this lane's 8 tokens for every head
  float s[G][kIters];
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    float kf[8];
    unpack8(kr[it], kf);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float a = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) a = __builtin_fmaf(qf[h][j], kf[j], a);
      s[h][it] = row16_sum(a);
    }
  }
  // s becomes the page's probabilities relative to the new running max
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float pmax = kNegInf;
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      if (it * kRows + row >= valid) s[h][it] = kNegInf;
      pmax = fmaxf(pmax, s[h][it]);
    }
    pmax = fmaxf(pmax, shfl_xor_f(pmax, 16));
    pmax = fmaxf(pmax, shfl_xor_f(pmax, 32));
    const float mn = fmaxf(m[h], pmax);
    // mn == -inf only if nothing finite was seen: the state stays empty
    const float corr = (m[h] == mn) ? 1.0f : __builtin_amdgcn_exp2f(m[h] - mn);
    const float base = (mn == kNegInf) ? 0.0f : mn;
    m[h] = mn;
    float lsum = l[h] * corr;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[h][j] *= corr;
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      s[h][it] = __builtin_amdgcn_exp2f(s[h][it] - base);
      lsum += s[h][it];
    }
    l[h] = lsum;
  }
  // P.V, each V half converted at its use (v_fma_mix_f32)
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const uint32_t w[4] = {vr[it].x, vr[it].y, vr[it].z, vr[it].w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float vj = (j & 1) ? hi_h2f(w[j >> 1]) : lo_h2f(w[j >> 1]);
#pragma unroll
      for (int h = 0; h < G; ++h) acc[h][j] = __builtin_fmaf(s[h][it], vj, acc[h][j]);
    }
  }
}

template <int G>
__global__ __launch_bounds__(waves_per_group<G>() * kWave) void sparse_decode_attention_kernel(const Params p) {
  constexpr int kWavesPerGroup = waves_per_group<G>();
  constexpr int kThreads = kWavesPerGroup * kWave;
  const int g = blockIdx.x;
  const int b = blockIdx.y;
  const int z = blockIdx.z;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int row = lane / kLanesPerRow;
  const int col = lane % kLanesPerRow;

  // ---- page list of this (sequence, KV head) -------------------------------
  PageList L{nullptr, 0, 0, 0, 0};
  if (p.contig_tokens > 0) {
    L.len = p.contig_tokens;
  } else {
    L.len = p.seq_len[b];
    L.sealed = p.sealed[b];
    const int sg = g / p.kv_per_sel;
    L.n_sel = p.counts[b * p.select_groups + sg];
    L.sel = p.selected + static_cast<int64_t>(b * p.select_groups + sg) * p.sel_stride;
    if (L.sealed < 0 || L.len < static_cast<int64_t>(L.sealed) * kPageTokens || L.n_sel < 0 ||
        L.n_sel > p.sel_stride) {
      flag_status(p.status, kStatusBadLength);
      if (L.sealed < 0) L.sealed = 0;
      L.len = static_cast<int64_t>(L.sealed) * kPageTokens;
      if (L.n_sel < 0 || L.n_sel > p.sel_stride) L.n_sel = 0;
    }
  }
  const int64_t tail_tokens = p.include_tail ? L.len - static_cast<int64_t>(L.sealed) * kPageTokens : 0;
  L.total = L.n_sel + static_cast<int>((tail_tokens + kPageTokens - 1) / kPageTokens);

  // ---- query: dims [8c, 8c+8) of each head of the group, pre-scaled -------
  float qf[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float4* q4 = reinterpret_cast<const float4*>(
        p.query + (static_cast<int64_t>(b) * p.query_heads + g * G + h) * D + col * 8);
    const float4 a = q4[0], c = q4[1];
    qf[h][0] = a.x * p.qscale;
    qf[h][1] = a.y * p.qscale;
    qf[h][2] = a.z * p.qscale;
    qf[h][3] = a.w * p.qscale;
    qf[h][4] = c.x * p.qscale;
    qf[h][5] = c.y * p.qscale;
    qf[h][6] = c.z * p.qscale;
    qf[h][7] = c.w * p.qscale;
  }

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = kNegInf;
    l[h] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[h][j] = 0.0f;
  }

  const int64_t head_off = static_cast<int64_t>(row) * p.token_elems + g * D + col * 8;
  const int64_t v_off = static_cast<int64_t>(p.kv_heads) * D;
  const int64_t step4 = static_cast<int64_t>(kRows) * p.token_elems;
  const int stride = p.splits * kWavesPerGroup;
  int i = z * kWavesPerGroup + wave;

  {
    for (; i < L.total; i += stride) {
      const PageRef pr = resolve_page(p, b, i, L);
      if (pr.valid <= 0) continue;
      uint4 kr[kIters], vr[kIters];
      load_page(p, pr, head_off, v_off, step4, row, kr, vr);
      process_page<G>(kr, vr, pr.valid, row, qf, m, l, acc);
    }
  }

  // ---- combine the 4 rows of the wave (same running max in every row) ----
#pragma unroll
  for (int h = 0; h < G; ++h) {
    l[h] += shfl_xor_f(l[h], 16);
    l[h] += shfl_xor_f(l[h], 32);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc[h][j] += shfl_xor_f(acc[h][j], 16);
      acc[h][j] += shfl_xor_f(acc[h][j], 32);
    }
  }

  // ---- combine the waves of the workgroup through LDS ----------------------
  __shared__ float sm_m[kWavesPerGroup][G];
  __shared__ float sm_l[kWavesPerGroup][G];
  __shared__ float sm_acc[kWavesPerGroup][G][D];
  if (row == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int j = 0; j < 8; ++j) sm_acc[wave][h][col * 8 + j] = acc[h][j];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      sm_m[wave][h] = m[h];
      sm_l[wave][h] = l[h];
    }
  }
  __syncthreads();

  for (int o = threadIdx.x; o < G * D; o += kThreads) {
    const int h = o / D;
    const int d = o % D;
    float mx = kNegInf;
#pragma unroll
    for (int w = 0; w < kWavesPerGroup; ++w) mx = fmaxf(mx, sm_m[w][h]);
    float lw = 0.0f, aw = 0.0f;
    if (mx != kNegInf) {
#pragma unroll
      for (int w = 0; w < kWavesPerGroup; ++w) {
        const float mw = sm_m[w][h];
        if (mw == kNegInf) continue;
        const float f = __builtin_amdgcn_exp2f(mw - mx);
        lw = __builtin_fmaf(sm_l[w][h], f, lw);
        aw = __builtin_fmaf(sm_acc[w][h][d], f, aw);
      }
    }
    const int qh = g * G + h;
    if (p.direct) {
      p.out[(static_cast<int64_t>(b) * p.query_heads + qh) * D + d] = lw > 0.0f ? aw / lw : 0.0f;
    } else {
      float* rec = p.part + (((static_cast<int64_t>(b) * p.kv_heads + g) * p.part_total + p.part_base + z) * G + h) *
                                part_stride(D);
      if (d == 0) {
        rec[0] = mx;
        rec[1] = lw;
      }
      rec[kPartPad + d] = aw;
    }
  }
}

// Log-sum-exp merge of the split partial results of one (sequence, KV head).
template <int G>
__global__ __launch_bounds__(kMergeThreads) void merge_partials_kernel(const Params p) {
  constexpr int kThreads = kMergeThreads;
  const int g = blockIdx.x;
  const int b = blockIdx.y;
  const float* base =
      p.part + ((static_cast<int64_t>(b) * p.kv_heads + g) * p.part_total) * G * part_stride(D);
  for (int o = threadIdx.x; o < G * D; o += kThreads) {
    const int h = o / D;
    const int d = o % D;
    float mx = kNegInf;
    for (int zz = 0; zz < p.part_total; ++zz) mx = fmaxf(mx, base[(zz * G + h) * part_stride(D)]);
    float lw = 0.0f, aw = 0.0f;
    if (mx != kNegInf) {
      for (int zz = 0; zz < p.part_total; ++zz) {
        const float* rec = base + (zz * G + h) * part_stride(D);
        if (rec[0] == kNegInf) continue;
        const float f = __builtin_amdgcn_exp2f(rec[0] - mx);
        lw = __builtin_fmaf(rec[1], f, lw);
        aw = __builtin_fmaf(rec[kPartPad + d], f, aw);
      }
    }
    p.out[(static_cast<int64_t>(b) * p.query_heads + g * G + h) * D + d] = lw > 0.0f ? aw / lw : 0.0f;
  }
}

// mode 0: attention (+ merge when split); 1: partial records only; 2: merge only.
template <int G>
hipError_t launch_g(const Params& p, int batch, int mode, hipStream_t stream) {
  if (mode != 2) {
    const dim3 grid(p.kv_heads, batch, p.splits);
    hipLaunchKernelGGL(sparse_decode_attention_kernel<G>, grid, dim3(waves_per_group<G>() * kWave), 0, stream, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || mode == 1 || p.direct) return e;
  }
  hipLaunchKernelGGL(merge_partials_kernel<G>, dim3(p.kv_heads, batch), dim3(kMergeThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_sparse_decode_attention(const AttnLaunch& a, hipStream_t stream) {
  Params p{};
  p.pool = a.pool;
  p.table = a.table;
  p.seq_len = a.seq_len;
  p.sealed = a.sealed;
  p.selected = a.selected;
  p.counts = a.counts;
  p.query = a.query;
  p.out = a.out;
  p.part = a.part;
  p.status = a.status;
  p.num_pages = a.num_pages;
  p.contig_tokens = a.contig_tokens;
  p.token_elems = 2 * a.kv_heads * D;
  p.page_elems = static_cast<int64_t>(kPageTokens) * p.token_elems;
  p.table_stride = a.table_stride;
  p.sel_stride = a.sel_stride;
  p.select_groups = a.select_groups > 0 ? a.select_groups : 1;
  p.kv_per_sel = a.kv_heads / p.select_groups;
  p.query_heads = a.query_heads;
  p.kv_heads = a.kv_heads;
  p.splits = a.splits;
  if (a.mode == 0) {
    p.part_base = 0;
    p.part_total = a.splits;
    p.include_tail = 1;
    p.direct = a.splits == 1;
  } else {
    p.part_base = a.part_base;
    p.part_total = a.part_total;
    p.include_tail = a.include_tail;
    p.direct = 0;
  }
  p.qscale = a.scale * 1.4426950408889634f;
  const int group = a.query_heads / a.kv_heads;
  switch (group) {
    case 1: return launch_g<1>(p, a.batch, a.mode, stream);
    case 2: return launch_g<2>(p, a.batch, a.mode, stream);
    case 4: return launch_g<4>(p, a.batch, a.mode, stream);
    case 8: return launch_g<8>(p, a.batch, a.mode, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace sa
