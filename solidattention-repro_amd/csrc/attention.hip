// attention.hip — GQA sparse decode attention over paged FP16 KV (gfx950).
//
// One launch attends, per (sequence, KV head g), the selected sealed blocks
// followed by the unsealed tail, for the G query heads of g (the lane
// mapping and the online softmax are in attn_core.hpp).  The page list of a
// (sequence, KV head) is split over `splits` workgroups; with splits > 1 each
// writes a partial (max, sum, acc) record and a small second kernel merges
// them with log-sum-exp.
//
// With chunk_pages > 0 the list is instead cut into chunks of that many
// pages, one workgroup each (mixed lengths and budgets: a 2048-page list and
// a 16-page one cost by their length).
//
// Measured on MI355X at B=64/16K (512 (sequence, KV head) pairs, 64 selected
// pages + a partial tail page each): one workgroup of 8 waves per pair,
// ~8 pages per wave, with non-temporal page loads streams the selected
// pages at ~6.0 TB/s (plain loads: 5.3 TB/s).  Reads of 16 KiB page slices
// in random page order peak at 6.3-6.5 TB/s on this pool layout (a
// contiguous stream: 7.2 TB/s).  Rejected variants at G <= 2, measured:
// register prefetch of the next page, a fused last-workgroup merge,
// prefetching the page ids of a wave's pages into lanes, and spreading the
// partial tail page over all waves (all within run-to-run noise or slower).
//
// G = 4 (Qwen3-8B shape, B=32/32K, 256 pairs): LDS-staged pages with q.K on
// the matrix cores, one 8-wave workgroup per pair and no merge, runs within
// ~3% of the same kernel with its arithmetic removed (timing probe); the
// register kernel with splits of 2 + merge ran ~13% slower on the same box.
#include "attn_core.hpp"
#include "schedule.hpp"

namespace sa {
namespace {

using namespace attn;

// Waves per workgroup: 8 for G <= 4 (G <= 2: 123 VGPRs, two 8-wave
// workgroups per CU; G = 4: one 8-wave workgroup per CU, bound by its
// 8 x 16 KiB LDS page slots); 4 for G = 8, whose registers (~300) allow one
// wave per SIMD.
template <int G>
constexpr int waves_per_group() { return G >= 8 ? 4 : 8; }
constexpr int kMergeThreads = 256;

struct Params {
  PoolView v;
  const int32_t* seq_len;
  const int32_t* sealed;
  const int32_t* selected;
  const int32_t* counts;
  const float* query;
  float* out;
  float* part;
  int32_t sel_stride;
  int32_t select_groups;
  int32_t kv_per_sel;
  int32_t query_heads;
  int32_t splits;        // workgroups per (sequence, KV head) in this launch
  int32_t part_base;     // first partial record written by this launch
  int32_t part_total;    // partial records per (sequence, KV head) in the workspace
  int32_t include_tail;  // attend the unsealed tail too
  int32_t direct;        // write the normalised output instead of a partial record
  int32_t chunk_pages;   // > 0: workgroup z attends list positions [z*chunk, (z+1)*chunk)
  float qscale;          // softmax scale * log2(e)
  // chunked, lists longest first: workgroup w (dispatch order) attends
  // chunk sched[slots + w] of list sched[w] = b * kv_heads + g (-1: none)
  const int32_t* sched;
};

// The page list of (sequence b, KV head g): selected sealed blocks, then the
// unsealed tail (when included).  Inconsistent lengths or counts are flagged
// and clamped to what can be read safely.
__device__ inline PageList page_list(const Params& p, int b, int g) {
  PageList L{nullptr, 0, 0, 0, 0};
  if (p.v.contig_tokens > 0) {
    L.len = p.v.contig_tokens;
  } else {
    L.len = p.seq_len[b];
    L.sealed = p.sealed[b];
    const int sg = g / p.kv_per_sel;
    L.n_sel = p.counts[b * p.select_groups + sg];
    L.sel = p.selected + static_cast<int64_t>(b * p.select_groups + sg) * p.sel_stride;
    if (L.sealed < 0 || L.len < static_cast<int64_t>(L.sealed) * kPageTokens || L.n_sel < 0 ||
        L.n_sel > p.sel_stride) {
      flag_status(p.v.status, kStatusBadLength);
      if (L.sealed < 0) L.sealed = 0;
      L.len = static_cast<int64_t>(L.sealed) * kPageTokens;
      if (L.n_sel < 0 || L.n_sel > p.sel_stride) L.n_sel = 0;
    }
  }
  const int64_t tail_tokens = p.include_tail ? L.len - static_cast<int64_t>(L.sealed) * kPageTokens : 0;
  L.total = L.n_sel + static_cast<int>((tail_tokens + kPageTokens - 1) / kPageTokens);
  return L;
}

template <int G>
__global__ __launch_bounds__(waves_per_group<G>() * kWave) void sparse_decode_attention_kernel(const Params p) {
  constexpr int kWavesPerGroup = waves_per_group<G>();
  constexpr int kThreads = kWavesPerGroup * kWave;
  int g = blockIdx.x;
  int b = blockIdx.y;
  int z = blockIdx.z;
  if (p.sched) {
    const int64_t w = blockIdx.x + static_cast<int64_t>(gridDim.x) * (blockIdx.y + static_cast<int64_t>(gridDim.y) *
                                                                                     blockIdx.z);
    const int32_t l = p.sched[w];
    if (l < 0) return;
    b = l / p.v.kv_heads;
    g = l % p.v.kv_heads;
    z = p.sched[static_cast<int64_t>(gridDim.x) * gridDim.y * gridDim.z + w];
  }
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;

  const PageList L = page_list(p, b, g);
  // chunked: a chunk past the end of a short list has nothing to attend and
  // writes no record (the merge reads only the records of existing chunks)
  if (p.chunk_pages > 0 && z > 0 && static_cast<int64_t>(z) * p.chunk_pages >= L.total) return;

  const LaneGeom lg = lane_geom(p.v, g, lane);
  const float* q_group = p.query + (static_cast<int64_t>(b) * p.query_heads + g * G) * D;
  WaveState<G> st;

  // G = 4, 8: pages staged through LDS (a 16 KiB slot per wave, reused for
  // the combine below) and q.K on the matrix cores; G <= 2 keeps pages in
  // registers (two 8-wave workgroups per CU already keep enough pages in
  // flight and the arithmetic per page is half or less)
  constexpr bool kStaged = G == 4 || G == 8;
  constexpr int kStageBytes = kWavesPerGroup * kStageVecs * 16;
  constexpr int kPbufFloats = (G * 32 + G + 3) / 4 * 4;
  constexpr int kSmemBytes = kStaged ? kStageBytes : static_cast<int>(sizeof(CombineSmem<G, kWavesPerGroup>));
  static_assert(!kStaged || sizeof(CombineSmem<G, kWavesPerGroup>) <= kStageBytes, "combine fits the stage");
  __shared__ __align__(16) unsigned char smem[kSmemBytes];
  // the probabilities' LDS buffer is its own variable, so that its stores do
  // not wait for the staging loads in flight into smem
  __shared__ __align__(16) float pbuf_s[kStaged ? kWavesPerGroup * kPbufFloats : 1];

  int start, end, step;
  bool owns_last;  // this workgroup's range holds the list's last position
  if (p.chunk_pages > 0) {
    // a fixed number of pages per workgroup, whatever the list length, so
    // long and short lists cost by their length; the last workgroup takes
    // any remainder, workgroups past the end leave an empty record
    const int first = z * p.chunk_pages;
    end = z == p.splits - 1 ? L.total
                            : static_cast<int>(min<int64_t>(L.total, static_cast<int64_t>(first) + p.chunk_pages));
    start = first + wave;
    step = kWavesPerGroup;
    owns_last = first < L.total && end == L.total;
  } else {
    start = z * kWavesPerGroup + wave;
    end = L.total;
    step = p.splits * kWavesPerGroup;
    owns_last = L.total > 0 && ((L.total - 1) / kWavesPerGroup) % p.splits == z;
  }
  if constexpr (kStaged) {
    // the list's last page, when it is a partial tail page, is spread over
    // all waves of the workgroup that owns it (row groups, register loads)
    const bool split_last = L.total > L.n_sel && L.len % kPageTokens != 0;
    const int walk_end = split_last ? min(end, L.total - 1) : end;
    st.reset();
    float* pbuf = pbuf_s + wave * kPbufFloats;
    st.attend_staged_mfma(p.v, b, L, start, walk_end, step, lg, lane, g,
                          reinterpret_cast<uint4*>(smem) + wave * kStageVecs, pbuf, q_group, p.qscale);
    if (split_last && owns_last) {
      const PageRef pr = resolve_page(p.v, b, L.total - 1, L);
      if (pr.valid > 0) {
        st.load_q(q_group, p.qscale, lg.col);
        st.template attend_rows<kWavesPerGroup>(p.v, pr, lg, wave);
      }
    }
    __syncthreads();  // every wave is done with its slot before the combine reuses the area
  } else {
    st.init(q_group, p.qscale, lg.col);
    for (int i = start; i < end; i += step) {
      const PageRef pr = resolve_page(p.v, b, i, L);
      if (pr.valid <= 0) continue;
      st.attend(p.v, pr, lg);
    }
  }

  // ---- combine the waves of the workgroup through LDS ----------------------
  st.reduce_rows();
  CombineSmem<G, kWavesPerGroup>& cs = *reinterpret_cast<CombineSmem<G, kWavesPerGroup>*>(smem);
  publish_wave<G, kWavesPerGroup>(st, cs, wave, lane, lg.row, lg.col);
  __syncthreads();

  for (int o = threadIdx.x; o < G * D; o += kThreads) {
    const int h = o / D;
    const int d = o % D;
    float mx, lw, aw;
    combine_element<G, kWavesPerGroup>(cs, h, d, mx, lw, aw);
    const int qh = g * G + h;
    if (p.direct) {
      p.out[(static_cast<int64_t>(b) * p.query_heads + qh) * D + d] = lw > 0.0f ? aw / lw : 0.0f;
    } else {
      float* rec = p.part + (((static_cast<int64_t>(b) * p.v.kv_heads + g) * p.part_total + p.part_base + z) * G +
                             h) * part_stride(D);
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
      p.part + ((static_cast<int64_t>(b) * p.v.kv_heads + g) * p.part_total) * G * part_stride(D);
  // chunked: only the chunks that exist wrote records (chunk 0 always does)
  int records = p.part_total;
  if (p.chunk_pages > 0) {
    const int64_t total = page_list(p, b, g).total;
    records = static_cast<int>(min<int64_t>(p.part_total, max<int64_t>(1, (total + p.chunk_pages - 1) / p.chunk_pages)));
  }
  // The records' loads are issued kMergeBatch at a time (indices past the
  // last record read the last one and are not used); the maximum over all
  // records comes first, then the weighted sums are added in chunk order.
  constexpr int kMergeBatch = 8;
  for (int o = threadIdx.x; o < G * D; o += kThreads) {
    const int h = o / D;
    const int d = o % D;
    const float* rh = base + h * part_stride(D);
    const int64_t rstride = static_cast<int64_t>(G) * part_stride(D);
    float mx = kNegInf;
    for (int z0 = 0; z0 < records; z0 += kMergeBatch) {
      float m[kMergeBatch];
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j) m[j] = rh[min(z0 + j, records - 1) * rstride];
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j) mx = fmaxf(mx, m[j]);
    }
    float lw = 0.0f, aw = 0.0f;
    if (mx != kNegInf) {
      for (int z0 = 0; z0 < records; z0 += kMergeBatch) {
        float m[kMergeBatch], l[kMergeBatch], a[kMergeBatch];
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) {
          const float* rec = rh + min(z0 + j, records - 1) * rstride;
          m[j] = rec[0];
          l[j] = rec[1];
          a[j] = rec[kPartPad + d];
        }
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) {
          if (z0 + j >= records || m[j] == kNegInf) continue;
          const float f = __builtin_amdgcn_exp2f(m[j] - mx);
          lw = __builtin_fmaf(l[j], f, lw);
          aw = __builtin_fmaf(a[j], f, aw);
        }
      }
    }
    p.out[(static_cast<int64_t>(b) * p.query_heads + g * G + h) * D + d] = lw > 0.0f ? aw / lw : 0.0f;
  }
}

// mode 0: attention (+ merge when split); 1: partial records only; 2: merge only.
// ---- chunked attention: lists longest first ---------------------------------
// The chunks of a mixed-length batch run as independent workgroups; in grid
// order (chunk index slowest) the last ones dispatched are the late chunks of
// the longest lists, which leave most compute units idle at the end.  This
// kernel orders the workgroups by list length, longest first, with a list's
// chunks consecutive (a counting sort on the page total, one workgroup):
// short lists fill the end.  Results do not depend on the order: each chunk
// attends the same pages and the merge adds the chunks in chunk order.
__global__ __launch_bounds__(kSchedThreads) void chunk_schedule_kernel(const Params p, int batch, int32_t* sched) {
  const int n = batch * p.v.kv_heads;  // <= kSchedMaxLists
  build_list_schedule(n, static_cast<int64_t>(n) * p.splits, sched, [&](int l, int& key, int& chunks) {
    // each list's page total and chunk count (chunk 0 always runs: it writes
    // the record the merge reads; the last chunk takes any remainder)
    const PageList L = page_list(p, l / p.v.kv_heads, l % p.v.kv_heads);
    const int64_t total = L.total;
    chunks = total <= 0 ? 1 : static_cast<int>(min<int64_t>(p.splits, (total + p.chunk_pages - 1) / p.chunk_pages));
    key = static_cast<int>(total < 0 ? 0 : (total > kSchedBins - 1 ? kSchedBins - 1 : total));
  });
}

template <int G>
hipError_t launch_g(const Params& p, int batch, int mode, hipStream_t stream) {
  if (p.sched) {
    hipLaunchKernelGGL(chunk_schedule_kernel, dim3(1), dim3(kSchedThreads), 0, stream, p, batch,
                       const_cast<int32_t*>(p.sched));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (mode != 2) {
    const dim3 grid(p.v.kv_heads, batch, p.splits);
    hipLaunchKernelGGL(sparse_decode_attention_kernel<G>, grid, dim3(waves_per_group<G>() * kWave), 0, stream, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || mode == 1 || p.direct) return e;
  }
  hipLaunchKernelGGL(merge_partials_kernel<G>, dim3(p.v.kv_heads, batch), dim3(kMergeThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_sparse_decode_attention(const AttnLaunch& a, hipStream_t stream) {
  Params p{};
  p.v.pool = a.pool;
  p.v.table = a.table;
  p.v.status = a.status;
  p.v.num_pages = a.num_pages;
  p.v.contig_tokens = a.contig_tokens;
  p.v.token_elems = 2 * a.kv_heads * D;
  p.v.page_elems = static_cast<int64_t>(kPageTokens) * p.v.token_elems;
  p.v.table_stride = a.table_stride;
  p.v.kv_heads = a.kv_heads;
  p.seq_len = a.seq_len;
  p.sealed = a.sealed;
  p.selected = a.selected;
  p.counts = a.counts;
  p.query = a.query;
  p.out = a.out;
  p.part = a.part;
  p.sel_stride = a.sel_stride;
  p.select_groups = a.select_groups > 0 ? a.select_groups : 1;
  p.kv_per_sel = a.kv_heads / p.select_groups;
  p.query_heads = a.query_heads;
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
  p.chunk_pages = a.chunk_pages;
  p.qscale = a.scale * kLog2e;
  // chunked with room for the schedule: lists longest first
  p.sched = a.mode == 0 && a.chunk_pages > 0 && a.sched &&
                    static_cast<int64_t>(a.batch) * a.kv_heads <= kSchedMaxLists
                ? a.sched
                : nullptr;
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
