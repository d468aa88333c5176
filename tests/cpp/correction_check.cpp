// correction_check.cpp — self-checking driver of the long-context miss
// correction on the GPU, in the manner of the reference's P1 history-
// correction driver (cpp/src/pipeline_main.cpp:752-924, 1090-1123).  TEST
// INFRASTRUCTURE: the oracle is linked as the checker.  Prints one JSON line;
// exits 0 when every check holds, 2 on a parity failure, 1 on an error.
//
// Workload (defaults): Qwen3-8B attention shape (32 query heads, 8 KV heads,
// head_dim 128), batch 8, context 131072 tokens (4096 sealed blocks per
// sequence), budget 128 blocks = 4 init + 8 local + 116 dynamic, one block
// set per sequence over every query head (the reference's shared selection,
// selection_main.cpp:178-181).  The whole KV of a layer (4 GiB) sits in
// pinned host memory, standing in for the SSD tier; HBM holds every block
// representative plus 130 page slots per sequence.
//
// Planted blocks: each KV head has 16 planted blocks, 4 runs of 4 adjacent
// blocks, and every run moves one block position per step.  The query of
// query head 4g + i at step t is Hadamard row 32 i + t (entries +-1; rows
// are mutually orthogonal), and every key of block start + j of a run of KV
// head g is 0.5 x the sum of the rows of the steps whose run covers it
// (t = j - 3 .. j) over the four query heads, plus noise.  So at step t the
// run's blocks start + t .. start + t + 3 score 64 per query head of g and
// every other block scores noise: the selection is init + local + the runs'
// current blocks, known in closed form.  Three of the 32 runs of a sequence
// share their blocks with another KV head's run, so the 29 distinct runs
// fill the 116 dynamic slots exactly; each step brings 29 new blocks (each
// run's leading block), and the previous step's selection covers
// (128 - 29) / 128 = 0.7734 of it.
//
// Schedules, each replayed from the same state over the same steps (so each
// sees the same selections and misses), per step and layer:
//   append + seal, GPU score + select (split form), ids to the host,
//   compare_prediction against the resident set (pipeline_main.cpp:686-717),
//   block table and hit / miss lists to the device, fills of the misses into
//   the replaced slots on a copy stream, then
//   serial        host barrier on the fills, one attention over the selection
//                 (the reference's correct_and_wait, pipeline_main.cpp:305-331)
//   serial_split  host barrier, then the split arithmetic: hits (+ tail),
//                 misses, merge
//   overlapped    hits attended while the fills run, the compute stream waits
//                 on the fill event (no host barrier), misses, merge; fills by
//                 one hipMemcpyAsync per page, or
//   overlapped_gather  the same with the fills as one kernel reading the
//                 pinned store through its device mapping.
// Reported per schedule: host wall time per layer (the whole loop, host leg
// included), the host leg alone, the selection, the device critical path
// (first fill issued to attention output), the fill bandwidth.
//
// Checks: every schedule sees the same misses; every step's selection is the
// closed-form planted set; overlapped and overlapped_gather outputs equal
// serial_split's bit for bit at every step and layer (the reference's
// exact serial-vs-pipelined bar, pipeline_main.cpp:1123); serial (one pass)
// is within 2e-3 of serial_split; and after the last step, for every
// sequence of every layer: the selection equals the oracle's (bit-exact ids),
// the resident set equals the selection, every slot's bytes equal its store
// block, and the attention matches the oracle on the resident pages within
// 2e-3.
#include "solidattention/hip_kv.hpp"

extern "C" {
#include "sa_oracle.h"
}

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace hk = solidattention::hip;
using Clock = std::chrono::steady_clock;

namespace {

constexpr int HQ = 32, HKV = 8, G = HQ / HKV, D = 128, PAGE = 32;
constexpr int BUDGET = 128, INIT = 4, LOCAL = 8;
constexpr int RUNS_PER_HEAD = 4, RUN_LEN = 4, SHARED_RUNS = 3;
constexpr int RUNS = HKV * RUNS_PER_HEAD;        // 32 (KV head, run) pairs per sequence
constexpr int SLOTS_RUN = RUNS - SHARED_RUNS;    // 29 distinct runs
constexpr int SLOTS = BUDGET + 2;                // resident pages per sequence (+ tail, + spare)
static_assert(SLOTS_RUN * RUN_LEN == BUDGET - INIT - LOCAL, "the runs fill the dynamic budget");

struct Args {
  int layers = 2, steps = 5, warmup = 2, batch = 8, context = 131072;
  uint64_t seed = 20261201;
  bool cpu_plan = false;
};

void hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

uint64_t mix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// N(0,1) by Box-Muller over two splitmix64 uniforms (host only).
double host_normal(uint64_t seed, uint64_t i) {
  const double u1 = (static_cast<double>(mix64(seed ^ (2 * i)) >> 11) + 1.0) * 0x1.0p-53;
  const double u2 = static_cast<double>(mix64(seed ^ (2 * i + 1)) >> 11) * 0x1.0p-53;
  return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

// FP16 bits of a value that FP16 represents exactly (|x| < 16, a multiple of
// 1/128): sign, exponent and the significand shifted into place.
uint16_t exact_half(float x) {
  if (x == 0.0f) return 0;
  uint32_t u;
  std::memcpy(&u, &x, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const int exp = static_cast<int>((u >> 23) & 0xff) - 127 + 15;
  if (exp <= 0 || exp >= 31 || (u & 0x1fffu)) throw std::runtime_error("exact_half: value not exact in FP16");
  return static_cast<uint16_t>(sign | (exp << 10) | ((u >> 13) & 0x3ffu));
}

int hadamard(int row, int d) { return (__builtin_popcount(static_cast<unsigned>(row & d)) & 1) ? -1 : 1; }
// Hadamard row of query head 4g + i at step t (t < 32).
int q_row(int i, int t) { return 32 * i + t; }

// Planted runs of one layer: start block of run slot u of sequence b (the
// run of (KV head g, run r) is slot g * 4 + r, the last three sharing slots
// 0, 1, 2).
struct Plan {
  int nblk = 0, steps = 0;
  std::vector<int> start;  // [batch][SLOTS_RUN]
  static int slot_of(int g, int r) {
    const int idx = g * RUNS_PER_HEAD + r;
    return idx < SLOTS_RUN ? idx : idx - SLOTS_RUN;
  }
  // the closed-form selection at step t: init, the runs' current blocks, local
  std::vector<int32_t> expected(int b, int t) const {
    std::vector<int32_t> ids;
    for (int i = 0; i < INIT; ++i) ids.push_back(i);
    for (int u = 0; u < SLOTS_RUN; ++u)
      for (int j = 0; j < RUN_LEN; ++j) ids.push_back(start[b * SLOTS_RUN + u] + t + j);
    for (int i = nblk - LOCAL; i < nblk; ++i) ids.push_back(i);
    std::sort(ids.begin(), ids.end());
    return ids;
  }
};

Plan make_plan(int batch, int nblk, int steps, uint64_t seed) {
  Plan p;
  p.nblk = nblk;
  p.steps = steps;
  // each run's blocks over the steps 0 .. steps: start .. start + steps + 3,
  // one block of gap, in disjoint windows between init and local
  const int span = RUN_LEN + steps + 1;
  const int width = (nblk - INIT - LOCAL) / SLOTS_RUN;
  if (width < span) throw std::runtime_error("context too short for the planted runs over these steps");
  p.start.resize(static_cast<size_t>(batch) * SLOTS_RUN);
  for (int b = 0; b < batch; ++b)
    for (int u = 0; u < SLOTS_RUN; ++u) {
      const int slack = width - span;
      const int off = slack > 0 ? static_cast<int>(mix64(seed ^ (1000003ull * b + u)) % (slack + 1)) : 0;
      p.start[b * SLOTS_RUN + u] = INIT + u * width + off;
    }
  return p;
}

// The K rows (token-major, 128 FP16 values each) of KV head g in the blocks
// of run r of sequence b over steps 0 .. steps: block start + j carries the
// Hadamard rows of the steps t = j - 3 .. j of the four query heads of g,
// times 0.5, plus noise rounded to 1/128 (every value exact in FP16).
// Returns the row count, (4 + steps) x 32.
int plant_keys(const Plan& plan, int b, int g, int r, int steps, uint64_t seed, std::vector<uint16_t>& keys) {
  (void)plan;
  const int blocks = RUN_LEN + steps;
  keys.assign(static_cast<size_t>(blocks) * PAGE * D, 0);
  std::vector<float> sig(D);
  for (int j = 0; j < blocks; ++j) {
    std::fill(sig.begin(), sig.end(), 0.0f);
    for (int t = std::max(0, j - RUN_LEN + 1); t <= std::min(j, steps); ++t)
      for (int i = 0; i < G; ++i)
        for (int d = 0; d < D; ++d) sig[d] += 0.5f * static_cast<float>(hadamard(q_row(i, t), d));
    for (int tok = 0; tok < PAGE; ++tok)
      for (int d = 0; d < D; ++d) {
        const uint64_t idx =
            ((((static_cast<uint64_t>(b) * HKV + g) * RUNS_PER_HEAD + r) * 64 + j) * PAGE + tok) * D + d;
        double n = std::round(0.5 * host_normal(seed + 77, idx) * 128.0) / 128.0;
        n = std::max(-4.0, std::min(4.0, n));
        keys[(static_cast<size_t>(j) * PAGE + tok) * D + d] = exact_half(sig[d] + static_cast<float>(n));
      }
  }
  return blocks * PAGE;
}

// query rows of step t: [batch][HQ][D]
void queries(int batch, int t, float* q) {
  for (int b = 0; b < batch; ++b)
    for (int h = 0; h < HQ; ++h)
      for (int d = 0; d < D; ++d)
        q[(static_cast<size_t>(b) * HQ + h) * D + d] = static_cast<float>(hadamard(q_row(h % G, t), d));
}

template <class T>
struct Pinned {
  T* p = nullptr;
  size_t n = 0;
  Pinned() = default;
  explicit Pinned(size_t count) : n(count) {
    hip_ok(hipHostMalloc(reinterpret_cast<void**>(&p), std::max<size_t>(count, 1) * sizeof(T), hipHostMallocDefault),
           "hipHostMalloc");
  }
  ~Pinned() {
    if (p) (void)hipHostFree(p);
  }
  Pinned(const Pinned&) = delete;
  Pinned& operator=(const Pinned&) = delete;
  Pinned(Pinned&& o) noexcept : p(std::exchange(o.p, nullptr)), n(std::exchange(o.n, 0)) {}
  Pinned& operator=(Pinned&& o) noexcept {
    std::swap(p, o.p);
    std::swap(n, o.n);
    return *this;
  }
};

struct Layer {
  std::unique_ptr<hk::PagedKvPool> kv;  // resident slots + every representative
  Pinned<uint16_t> store;               // [batch * ts] pages: the layer's whole KV
  hk::DeviceArray<float> q, knew, vnew; // [steps + 1][batch][heads][D]
  std::vector<std::vector<int32_t>> resident0;  // per sequence: block of each slot after step 0
  Plan plan;
  hk::DeviceArray<int32_t> sel, cnt, hit, miss, hitc, missc, dst32;
  hk::DeviceArray<int64_t> srcblk;
  hk::DeviceArray<float> scores;
  Pinned<int32_t> h_table, h_sel, h_lists, h_counts, h_dst32;
  Pinned<int64_t> h_src;
};

enum Schedule { kSerial = 0, kSerialSplit, kOverlapped, kOverlappedGather, kSchedules };
const char* const kNames[kSchedules] = {"serial", "serial_split", "overlapped", "overlapped_gather"};

struct ScheduleStats {
  double wall_us = 0, host_us = 0, select_us = 0, crit_us = 0, h2d_us = 0, pages = 0, misses = 0, selected = 0;
  std::vector<int32_t> miss_log;  // misses of every (step, layer, sequence), in order
  long plan_mismatch = 0;
};

class Driver {
 public:
  explicit Driver(const Args& a) : a_(a) {
    if (a_.context % PAGE != 0) throw std::runtime_error("context must be a multiple of 32");
    nblk_ = a_.context / PAGE;
    ts_ = nblk_ + 2;
    total_steps_ = a_.warmup + a_.steps;
    if (total_steps_ < 1 || total_steps_ > PAGE - 1) throw std::runtime_error("warmup + steps must lie in [1, 31]");
    if (a_.batch < 1 || a_.layers < 1) throw std::runtime_error("batch and layers must be positive");
    page_elems_ = static_cast<size_t>(PAGE) * 2 * HKV * D;
    page_bytes_ = page_elems_ * 2;
    scale_ = 1.0f / std::sqrt(static_cast<float>(D));
    hip_ok(hipStreamCreateWithFlags(&compute_, hipStreamNonBlocking), "hipStreamCreate");
    params_ = sa_select_params{1, BUDGET, INIT, LOCAL, BUDGET, 0, nullptr};
    status_ = hk::DeviceArray<int32_t>(1);
  }
  ~Driver() {
    if (compute_) (void)hipStreamDestroy(compute_);
  }

  void setup();
  ScheduleStats run(Schedule s);
  void checks(std::vector<ScheduleStats>& st);
  void print(const std::vector<ScheduleStats>& st) const;
  bool ok() const { return ok_; }

 private:
  void reset(Layer& L);
  void record(const std::string& key, const std::string& value, bool pass) {
    json_ << (first_ ? "" : ", ") << '"' << key << "\": " << value;
    first_ = false;
    if (!pass) {
      ok_ = false;
      std::cerr << "FAIL " << key << " = " << value << '\n';
    }
  }
  float* out_slot(int sched, int step, int layer) {
    return outs_.get() + ((static_cast<size_t>(sched) * (total_steps_ + 1) + step) * a_.layers + layer) *
                             static_cast<size_t>(a_.batch) * HQ * D;
  }

  Args a_;
  int nblk_ = 0, ts_ = 0, total_steps_ = 0;
  size_t page_elems_ = 0, page_bytes_ = 0;
  float scale_ = 0;
  hipStream_t compute_{};
  sa_select_params params_{};
  hk::DeviceArray<int32_t> status_;
  std::vector<Layer> layers_;
  hk::MissCorrector corrector_;
  std::unique_ptr<hk::SplitAttention> split_;
  hk::DeviceArray<float> ws_single_;
  size_t ws_single_bytes_ = 0;
  hk::DeviceArray<float> outs_;  // [schedule][step][layer][batch][HQ][D]
  std::ostringstream json_;
  bool first_ = true, ok_ = true;
  double setup_s_ = 0;
};

void Driver::setup() {
  const auto t0 = Clock::now();
  const int B = a_.batch;
  const size_t q_elems = static_cast<size_t>(total_steps_ + 1) * B * HQ * D;
  const size_t kv_elems = static_cast<size_t>(total_steps_ + 1) * B * HKV * D;
  layers_.resize(a_.layers);
  for (int li = 0; li < a_.layers; ++li) {
    Layer& L = layers_[li];
    const uint64_t seed = a_.seed + 104729ull * li;
    L.plan = make_plan(B, nblk_, total_steps_, seed);
    {
      // the whole KV on the device once: synthetic FP16, planted keys, bulk
      // seal (every representative), then to the pinned store
      hk::PagedKvPool full(B, HQ, HKV, ts_, static_cast<size_t>(B) * ts_);
      std::vector<int32_t> table(static_cast<size_t>(B) * ts_);
      for (size_t i = 0; i < table.size(); ++i) table[i] = static_cast<int32_t>(i);
      full.block_table().upload(table);
      hk::check(sa_hip_fill_synthetic_f16(full.pool().get(), static_cast<int64_t>(full.pool().size()), seed, 0,
                                          compute_),
                "fill_synthetic_f16");
      std::vector<uint16_t> keys;
      for (int b = 0; b < B; ++b)
        for (int g = 0; g < HKV; ++g)
          for (int r = 0; r < RUNS_PER_HEAD; ++r) {
            const int rows = plant_keys(L.plan, b, g, r, total_steps_, seed, keys);
            const int start = L.plan.start[b * SLOTS_RUN + Plan::slot_of(g, r)];
            // the run's blocks are consecutive pages of the full pool: one
            // strided copy of the K rows of head g
            uint16_t* dst = full.pool().get() + (static_cast<size_t>(b) * ts_ + start) * page_elems_ + g * D;
            hip_ok(hipMemcpy2DAsync(dst, 2 * HKV * D * 2, keys.data(), D * 2, D * 2, rows, hipMemcpyHostToDevice,
                                    compute_),
                   "hipMemcpy2DAsync planted keys");
            hip_ok(hipStreamSynchronize(compute_), "planted keys");
          }
      std::vector<int32_t> len(B, a_.context);
      full.seq_len().upload(len);
      full.seal(0, compute_, status_.get());
      L.store = Pinned<uint16_t>(static_cast<size_t>(B) * ts_ * page_elems_);
      hip_ok(hipMemcpyAsync(L.store.p, full.pool().get(), L.store.n * 2, hipMemcpyDeviceToHost, compute_),
             "store D2H");
      L.kv = std::make_unique<hk::PagedKvPool>(B, HQ, HKV, ts_, static_cast<size_t>(B) * SLOTS, 0, full.rep_stride());
      hip_ok(hipMemcpyAsync(L.kv->reps().get(), full.reps().get(), full.reps().size() * 4, hipMemcpyDeviceToDevice,
                            compute_),
             "reps D2D");
      hip_ok(hipStreamSynchronize(compute_), "setup");
    }
    // queries: Hadamard rows; new K/V per step: synthetic
    std::vector<float> q(q_elems);
    for (int t = 0; t <= total_steps_; ++t) queries(B, t, q.data() + static_cast<size_t>(t) * B * HQ * D);
    L.q = hk::DeviceArray<float>(q_elems);
    L.q.upload(q);
    L.knew = hk::DeviceArray<float>(kv_elems);
    L.vnew = hk::DeviceArray<float>(kv_elems);
    hk::check(sa_hip_fill_synthetic_f32(L.knew.get(), static_cast<int64_t>(kv_elems), seed + 3, 0, compute_), "k");
    hk::check(sa_hip_fill_synthetic_f32(L.vnew.get(), static_cast<int64_t>(kv_elems), seed + 4, 0, compute_), "v");
    L.sel = hk::DeviceArray<int32_t>(static_cast<size_t>(B) * BUDGET);
    L.cnt = hk::DeviceArray<int32_t>(B);
    L.hit = hk::DeviceArray<int32_t>(static_cast<size_t>(B) * BUDGET);
    L.miss = hk::DeviceArray<int32_t>(static_cast<size_t>(B) * BUDGET);
    L.hitc = hk::DeviceArray<int32_t>(B);
    L.missc = hk::DeviceArray<int32_t>(B);
    L.dst32 = hk::DeviceArray<int32_t>(static_cast<size_t>(B) * BUDGET);
    L.srcblk = hk::DeviceArray<int64_t>(static_cast<size_t>(B) * BUDGET);
    L.scores = hk::DeviceArray<float>(static_cast<size_t>(B) * L.kv->rep_stride());
    L.h_table = Pinned<int32_t>(static_cast<size_t>(B) * ts_);
    L.h_sel = Pinned<int32_t>(static_cast<size_t>(B) * BUDGET);
    L.h_lists = Pinned<int32_t>(2 * static_cast<size_t>(B) * BUDGET);
    L.h_counts = Pinned<int32_t>(2 * static_cast<size_t>(B));
    L.h_dst32 = Pinned<int32_t>(static_cast<size_t>(B) * BUDGET);
    L.h_src = Pinned<int64_t>(static_cast<size_t>(B) * BUDGET);
    // step 0: the initial residency is the selection of the first query
    std::vector<int32_t> len(B, a_.context), sealed(B, nblk_);
    L.kv->seq_len().upload(len);
    L.kv->sealed().upload(sealed);
    const sa_paged_kv v = L.kv->view();
    hk::check(sa_hip_score_select_split(&v, L.q.get(), &params_, L.sel.get(), L.cnt.get(), L.scores.get(),
                                        status_.get(), compute_),
              "score_select_split (step 0)");
    // the compute stream does not synchronise with the null stream of the
    // blocking copies: wait for it before reading the ids
    hip_ok(hipStreamSynchronize(compute_), "step-0 selection");
    const std::vector<int32_t> ids = L.sel.download();
    L.resident0.assign(B, {});
    long mismatch = 0;
    for (int b = 0; b < B; ++b) {
      L.resident0[b].assign(ids.begin() + static_cast<long>(b) * BUDGET, ids.begin() + static_cast<long>(b + 1) * BUDGET);
      mismatch += L.resident0[b] != L.plan.expected(b, 0);
    }
    if (mismatch) throw std::runtime_error("step-0 selection differs from the planted set");
  }
  split_ = std::make_unique<hk::SplitAttention>(*layers_[0].kv, 4);
  ws_single_bytes_ = sa_hip_attention_workspace_bytes(a_.batch, HQ, HKV, D, 2);
  ws_single_ = hk::DeviceArray<float>((ws_single_bytes_ + 3) / 4);
  outs_ = hk::DeviceArray<float>(static_cast<size_t>(kSchedules) * (total_steps_ + 1) * a_.layers * a_.batch * HQ * D);
  hip_ok(hipDeviceSynchronize(), "setup");
  setup_s_ = std::chrono::duration<double>(Clock::now() - t0).count();
}

// The state after step 0: the lengths, the resident set of each sequence in
// its slots (bytes from the store), the tail page, the block table.
void Driver::reset(Layer& L) {
  const int B = a_.batch;
  std::vector<int32_t> len(B, a_.context), sealed(B, nblk_), gen(B, 0);
  L.kv->seq_len().upload(len);
  L.kv->sealed().upload(sealed);
  L.kv->generation().upload(gen);
  std::vector<int32_t> dst;
  std::vector<int64_t> src;
  std::fill(L.h_table.p, L.h_table.p + L.h_table.n, -1);
  for (int b = 0; b < B; ++b) {
    for (int slot = 0; slot < BUDGET; ++slot) {
      const int blk = L.resident0[b][slot];
      L.h_table.p[static_cast<size_t>(b) * ts_ + blk] = b * SLOTS + slot;
      dst.push_back(b * SLOTS + slot);
      src.push_back(static_cast<int64_t>(b) * ts_ + blk);
    }
    L.h_table.p[static_cast<size_t>(b) * ts_ + nblk_] = b * SLOTS + BUDGET;  // tail page
    dst.push_back(b * SLOTS + BUDGET);
    src.push_back(static_cast<int64_t>(b) * ts_ + nblk_);
  }
  hk::check(sa_hip_fill_pages_async(L.kv->pool().get(), static_cast<int64_t>(page_bytes_), dst.data(), L.store.p,
                                    src.data(), static_cast<int32_t>(dst.size()), compute_, nullptr),
            "reset fills");
  hip_ok(hipMemcpyAsync(L.kv->block_table().get(), L.h_table.p, L.h_table.n * 4, hipMemcpyHostToDevice, compute_),
         "reset table");
  hip_ok(hipStreamSynchronize(compute_), "reset");
}

ScheduleStats Driver::run(Schedule sch) {
  const int B = a_.batch;
  ScheduleStats st;
  for (Layer& L : layers_) reset(L);
  std::vector<std::vector<std::vector<int32_t>>> resident(a_.layers);
  for (int li = 0; li < a_.layers; ++li) resident[li] = layers_[li].resident0;
  struct Ev {
    hipEvent_t s0, s1, c0, c1, end;
    int pages;
  };
  std::vector<Ev> evs;
  auto make_ev = []() {
    hipEvent_t e;
    hip_ok(hipEventCreate(&e), "hipEventCreate");
    return e;
  };
  hipStream_t copy = corrector_.copy_stream();
  Clock::time_point wall0;
  double host_s = 0;
  for (int t = 1; t <= total_steps_; ++t) {
    const bool timed = t > a_.warmup;
    if (t == a_.warmup + 1) {
      hip_ok(hipDeviceSynchronize(), "before the timed steps");
      wall0 = Clock::now();
    }
    for (int li = 0; li < a_.layers; ++li) {
      Layer& L = layers_[li];
      hk::PagedKvPool& kv = *L.kv;
      const sa_paged_kv v = kv.view();
      const float* q = L.q.get() + static_cast<size_t>(t) * B * HQ * D;
      const size_t kvo = static_cast<size_t>(t) * B * HKV * D;
      Ev e{};
      if (timed) {
        e.s0 = make_ev();
        e.s1 = make_ev();
        e.c0 = make_ev();
        e.c1 = make_ev();
        e.end = make_ev();
      }
      kv.append_seal(L.knew.get() + kvo, L.vnew.get() + kvo, 0, compute_, status_.get());
      if (timed) hip_ok(hipEventRecord(e.s0, compute_), "record");
      hk::check(sa_hip_score_select_split(&v, q, &params_, L.sel.get(), L.cnt.get(), L.scores.get(), status_.get(),
                                          compute_),
                "score_select_split");
      if (timed) hip_ok(hipEventRecord(e.s1, compute_), "record");
      hip_ok(hipMemcpyAsync(L.h_sel.p, L.sel.get(), L.h_sel.n * 4, hipMemcpyDeviceToHost, compute_), "ids D2H");
      hip_ok(hipStreamSynchronize(compute_), "ids");
      // the host leg: compare_prediction, the table, the hit / miss lists
      const auto th = Clock::now();
      int n_fill = 0;
      int32_t* hits = L.h_lists.p;
      int32_t* misses = L.h_lists.p + static_cast<size_t>(B) * BUDGET;
      for (int b = 0; b < B; ++b) {
        const std::vector<int32_t> cur(L.h_sel.p + static_cast<size_t>(b) * BUDGET,
                                       L.h_sel.p + static_cast<size_t>(b + 1) * BUDGET);
        if (cur != L.plan.expected(b, t)) ++st.plan_mismatch;
        std::vector<int32_t>& res = resident[li][b];
        const hk::Correction c = hk::compare_prediction(res, cur);
        for (size_t m = 0; m < c.misses.size(); ++m) {
          const int slot = c.replacement_slots[m];
          L.h_table.p[static_cast<size_t>(b) * ts_ + res[slot]] = -1;
          L.h_table.p[static_cast<size_t>(b) * ts_ + c.misses[m]] = b * SLOTS + slot;
          res[slot] = c.misses[m];
          L.h_dst32.p[n_fill] = b * SLOTS + slot;
          L.h_src.p[n_fill] = static_cast<int64_t>(b) * ts_ + c.misses[m];
          ++n_fill;
        }
        std::vector<int32_t> ms(c.misses.begin(), c.misses.end());
        std::sort(ms.begin(), ms.end());
        int nh = 0;
        for (int32_t id : cur)
          if (!std::binary_search(ms.begin(), ms.end(), id)) hits[static_cast<size_t>(b) * BUDGET + nh++] = id;
        std::copy(ms.begin(), ms.end(), misses + static_cast<size_t>(b) * BUDGET);
        L.h_counts.p[b] = nh;
        L.h_counts.p[B + b] = static_cast<int32_t>(ms.size());
        if (timed) {
          st.misses += static_cast<double>(ms.size());
          st.selected += static_cast<double>(cur.size());
        }
        st.miss_log.push_back(static_cast<int32_t>(ms.size()));
      }
      hip_ok(hipMemcpyAsync(kv.block_table().get(), L.h_table.p, L.h_table.n * 4, hipMemcpyHostToDevice, compute_),
             "table H2D");
      hip_ok(hipMemcpyAsync(L.hit.get(), hits, static_cast<size_t>(B) * BUDGET * 4, hipMemcpyHostToDevice, compute_),
             "hits H2D");
      hip_ok(hipMemcpyAsync(L.miss.get(), misses, static_cast<size_t>(B) * BUDGET * 4, hipMemcpyHostToDevice,
                            compute_),
             "misses H2D");
      hip_ok(hipMemcpyAsync(L.hitc.get(), L.h_counts.p, B * 4, hipMemcpyHostToDevice, compute_), "hit counts H2D");
      hip_ok(hipMemcpyAsync(L.missc.get(), L.h_counts.p + B, B * 4, hipMemcpyHostToDevice, compute_),
             "miss counts H2D");
      const auto th1 = Clock::now();
      if (timed) host_s += std::chrono::duration<double>(th1 - th).count();
      // fills: the replaced slots were last read by this layer's previous
      // step, which completed before the ids came back
      if (timed) hip_ok(hipEventRecord(e.c0, copy), "record");
      if (sch == kOverlappedGather) {
        hip_ok(hipMemcpyAsync(L.dst32.get(), L.h_dst32.p, static_cast<size_t>(n_fill) * 4, hipMemcpyHostToDevice, copy),
               "fill lists H2D");
        hip_ok(hipMemcpyAsync(L.srcblk.get(), L.h_src.p, static_cast<size_t>(n_fill) * 8, hipMemcpyHostToDevice, copy),
               "fill lists H2D");
        corrector_.fill_gather(kv.pool().get(), page_bytes_, static_cast<int64_t>(B) * SLOTS, L.dst32.get(), L.store.p,
                               static_cast<int64_t>(B) * ts_, L.srcblk.get(), n_fill, status_.get());
      } else {
        corrector_.fill(kv.pool().get(), page_bytes_, std::vector<int32_t>(L.h_dst32.p, L.h_dst32.p + n_fill),
                        L.store.p, std::vector<int64_t>(L.h_src.p, L.h_src.p + n_fill));
      }
      if (timed) hip_ok(hipEventRecord(e.c1, copy), "record");
      float* out = out_slot(sch, t, li);
      switch (sch) {
        case kSerial:
          corrector_.wait();
          hk::check(sa_hip_sparse_decode_attention(&v, q, L.sel.get(), L.cnt.get(), 1, BUDGET, scale_, out,
                                                   ws_single_.get(), ws_single_bytes_, 2, status_.get(), compute_),
                    "sparse_decode_attention");
          break;
        case kSerialSplit:
          corrector_.wait();
          split_->partial(kv, q, L.hit.get(), L.hitc.get(), 1, BUDGET, scale_, true, 0, 2, compute_, status_.get());
          split_->partial(kv, q, L.miss.get(), L.missc.get(), 1, BUDGET, scale_, false, 2, 2, compute_, status_.get());
          split_->merge(kv, out, compute_);
          break;
        default:
          split_->partial(kv, q, L.hit.get(), L.hitc.get(), 1, BUDGET, scale_, true, 0, 2, compute_, status_.get());
          corrector_.order(compute_);
          split_->partial(kv, q, L.miss.get(), L.missc.get(), 1, BUDGET, scale_, false, 2, 2, compute_, status_.get());
          split_->merge(kv, out, compute_);
          break;
      }
      if (timed) {
        hip_ok(hipEventRecord(e.end, compute_), "record");
        e.pages = n_fill;
        evs.push_back(e);
      }
    }
  }
  hip_ok(hipDeviceSynchronize(), "after the timed steps");
  const double wall_s = std::chrono::duration<double>(Clock::now() - wall0).count();
  const double per = static_cast<double>(a_.steps) * a_.layers;
  st.wall_us = wall_s * 1e6 / per;
  st.host_us = host_s * 1e6 / per;
  for (const Ev& e : evs) {
    float ms = 0;
    hip_ok(hipEventElapsedTime(&ms, e.s0, e.s1), "elapsed");
    st.select_us += ms * 1000.0 / per;
    hip_ok(hipEventElapsedTime(&ms, e.c0, e.end), "elapsed");
    st.crit_us += ms * 1000.0 / per;
    hip_ok(hipEventElapsedTime(&ms, e.c0, e.c1), "elapsed");
    st.h2d_us += ms * 1000.0 / per;
    st.pages += e.pages;
    for (hipEvent_t x : {e.s0, e.s1, e.c0, e.c1, e.end}) (void)hipEventDestroy(x);
  }
  return st;
}

std::string num(double v) {
  std::ostringstream s;
  s.precision(7);
  s << v;
  return s.str();
}

void Driver::checks(std::vector<ScheduleStats>& st) {
  const int B = a_.batch;
  const size_t out_elems = static_cast<size_t>(B) * HQ * D;
  // 1. the same misses in every schedule; the closed-form selection
  bool same_misses = true;
  long plan_mismatch = 0;
  for (const ScheduleStats& s : st) {
    same_misses &= s.miss_log == st[0].miss_log;
    plan_mismatch += s.plan_mismatch;
  }
  record("same_misses_every_schedule", same_misses ? "true" : "false", same_misses);
  record("selection_equals_planted_set", plan_mismatch == 0 ? "true" : "false", plan_mismatch == 0);
  // 2. overlapped == serial_split bit for bit; serial within 2e-3
  std::vector<float> ref(out_elems), got(out_elems);
  bool exact = true, exact_gather = true, near = true;
  double max_err = 0;
  for (int t = 1; t <= total_steps_; ++t)
    for (int li = 0; li < a_.layers; ++li) {
      hip_ok(hipMemcpy(ref.data(), out_slot(kSerialSplit, t, li), out_elems * 4, hipMemcpyDeviceToHost), "D2H");
      hip_ok(hipMemcpy(got.data(), out_slot(kOverlapped, t, li), out_elems * 4, hipMemcpyDeviceToHost), "D2H");
      exact &= std::memcmp(ref.data(), got.data(), out_elems * 4) == 0;
      hip_ok(hipMemcpy(got.data(), out_slot(kOverlappedGather, t, li), out_elems * 4, hipMemcpyDeviceToHost), "D2H");
      exact_gather &= std::memcmp(ref.data(), got.data(), out_elems * 4) == 0;
      hip_ok(hipMemcpy(got.data(), out_slot(kSerial, t, li), out_elems * 4, hipMemcpyDeviceToHost), "D2H");
      for (size_t i = 0; i < out_elems; ++i) {
        const double err = std::fabs(static_cast<double>(got[i]) - ref[i]);
        max_err = std::max(max_err, err);
        near &= err <= 2e-3 || err <= 2e-3 * std::fabs(static_cast<double>(ref[i]));
      }
    }
  record("overlapped_equals_serial_split_bitwise", exact ? "true" : "false", exact);
  record("overlapped_gather_equals_serial_split_bitwise", exact_gather ? "true" : "false", exact_gather);
  record("serial_single_pass_within_2e-3_of_split", near ? "true" : "false", near);
  record("serial_single_pass_max_abs_err", num(max_err), true);
  // 3. the final state of the last schedule against the oracle
  bool sel_ok = true, sets_ok = true, bytes_ok = true, att_ok = true;
  double att_err = 0;
  for (int li = 0; li < a_.layers; ++li) {
    Layer& L = layers_[li];
    hk::PagedKvPool& kv = *L.kv;
    const int t = total_steps_;
    std::vector<float> q(static_cast<size_t>(B) * HQ * D);
    hip_ok(hipMemcpy(q.data(), L.q.get() + static_cast<size_t>(t) * B * HQ * D, q.size() * 4, hipMemcpyDeviceToHost),
           "q");
    const std::vector<float> reps = kv.reps().download();
    const std::vector<int32_t> sealed = kv.sealed().download(), seq_len = kv.seq_len().download();
    const std::vector<int32_t> sel = L.sel.download(), cnt = L.cnt.download(), table = kv.block_table().download();
    std::vector<int32_t> esel(static_cast<size_t>(B) * BUDGET, -1), ecnt(B, 0);
    if (sao_paged_score_select(q.data(), reps.data(), sealed.data(), B, HQ, HKV, D, kv.rep_heads(), kv.rep_stride(), 1,
                               BUDGET, INIT, LOCAL, esel.data(), ecnt.data(), BUDGET, nullptr) != 0)
      throw std::runtime_error("oracle selection failed");
    sel_ok &= sel == esel && cnt == ecnt;
    // resident set and slot bytes (the run of the last schedule)
    const std::vector<uint16_t> pool = kv.pool().download();
    for (int b = 0; b < B; ++b) {
      std::vector<int32_t> res;
      for (int blk = 0; blk < nblk_; ++blk) {
        const int32_t page = table[static_cast<size_t>(b) * ts_ + blk];
        if (page < 0) continue;
        res.push_back(blk);
        bytes_ok &= std::memcmp(pool.data() + static_cast<size_t>(page) * page_elems_,
                                L.store.p + (static_cast<size_t>(b) * ts_ + blk) * page_elems_, page_bytes_) == 0;
      }
      sets_ok &= res == std::vector<int32_t>(sel.begin() + static_cast<long>(b) * BUDGET,
                                             sel.begin() + static_cast<long>(b + 1) * BUDGET);
    }
    std::vector<float> expect(out_elems), out(out_elems);
    if (sao_paged_sparse_attention(pool.data(), PAGE, table.data(), ts_, seq_len.data(), sealed.data(), sel.data(),
                                   cnt.data(), BUDGET, 1, q.data(), B, HQ, HKV, D, scale_, expect.data()) != 0)
      throw std::runtime_error("oracle attention failed");
    hip_ok(hipMemcpy(out.data(), out_slot(kOverlappedGather, t, li), out_elems * 4, hipMemcpyDeviceToHost), "out");
    for (size_t i = 0; i < out_elems; ++i) {
      const double err = std::fabs(static_cast<double>(out[i]) - expect[i]);
      att_err = std::max(att_err, err);
      att_ok &= err <= 2e-3 || err <= 2e-3 * std::fabs(static_cast<double>(expect[i]));
    }
  }
  record("sequences", std::to_string(B * a_.layers), true);
  record("selection_equals_oracle", sel_ok ? "true" : "false", sel_ok);
  record("resident_set_equals_selection", sets_ok ? "true" : "false", sets_ok);
  record("slot_bytes_equal_store", bytes_ok ? "true" : "false", bytes_ok);
  record("attention_within_2e-3_of_oracle", att_ok ? "true" : "false", att_ok);
  record("attention_max_abs_err", num(att_err), true);
  std::vector<int32_t> status = status_.download();
  record("device_status", std::to_string(status[0]), status[0] == 0);
}

void Driver::print(const std::vector<ScheduleStats>& st) const {
  std::ostringstream o;
  const double coverage = 1.0 - st[0].misses / std::max(st[0].selected, 1.0);
  o << "{\"workload\": \"long-context miss correction, Qwen3-8B shape, B=" << a_.batch << ", " << a_.context
    << " tokens, budget 128 blocks, shared selection\", \"driver\": \"tests/cpp/correction_check (C++)\""
    << ", \"layers\": " << a_.layers << ", \"steps\": " << a_.steps << ", \"warmup\": " << a_.warmup
    << ", \"batch\": " << a_.batch << ", \"context\": " << a_.context << ", \"page_bytes\": " << page_bytes_
    << ", \"data\": \"synthetic FP16 KV (Irwin-Hall(4) generator), 16 planted blocks per KV head as 4 runs of 4 "
       "drifting one block per step (Hadamard-row keys and queries)\""
    << ", \"history_coverage\": " << num(coverage) << ", \"designed_coverage\": "
    << num(static_cast<double>(BUDGET - SLOTS_RUN) / BUDGET) << ", \"setup_s\": " << num(setup_s_)
    << ", \"schedules\": {";
  for (int s = 0; s < kSchedules; ++s) {
    const ScheduleStats& x = st[s];
    const double per = static_cast<double>(a_.steps) * a_.layers;
    o << (s ? ", " : "") << '"' << kNames[s] << "\": {\"wall_us_per_layer\": " << num(x.wall_us)
      << ", \"host_leg_us_per_layer\": " << num(x.host_us) << ", \"selection_us_per_layer\": " << num(x.select_us)
      << ", \"device_critical_us_per_layer\": " << num(x.crit_us)
      << ", \"misses_per_layer\": " << num(x.misses / per) << ", \"fill_us_per_layer\": " << num(x.h2d_us)
      << ", \"fill_gbps\": " << num(x.pages * static_cast<double>(page_bytes_) / (x.h2d_us * per * 1e-6) / 1e9) << "}";
  }
  o << "}, \"checks\": {" << json_.str() << "}, \"ok\": " << (ok_ ? "true" : "false") << "}";
  std::cout << o.str() << std::endl;
}

// CPU only (no GPU): the workload's store built on the host with the
// oracle's generator (the same bits as the device fill), the planted keys,
// the oracle's seal and, for every step, the oracle's selection against the
// closed-form planted set; the history coverage over the steps follows from
// compare_prediction (host set logic).  Pins the workload design.
int cpu_plan_check(const Args& a) {
  const int B = a.batch, nblk = a.context / PAGE, ts = nblk + 2, steps = a.warmup + a.steps;
  if (a.context % PAGE || steps < 1 || steps > PAGE - 1) throw std::runtime_error("bad shape");
  const size_t page_elems = static_cast<size_t>(PAGE) * 2 * HKV * D;
  const uint64_t seed = a.seed;
  const Plan plan = make_plan(B, nblk, steps, seed);
  std::vector<uint16_t> pool(static_cast<size_t>(B) * ts * page_elems);
  sao_synth_fill_half(seed, 0, pool.size(), pool.data());
  std::vector<uint16_t> keys;
  for (int b = 0; b < B; ++b)
    for (int g = 0; g < HKV; ++g)
      for (int r = 0; r < RUNS_PER_HEAD; ++r) {
        const int rows = plant_keys(plan, b, g, r, steps, seed, keys);
        const int start = plan.start[b * SLOTS_RUN + Plan::slot_of(g, r)];
        for (int row = 0; row < rows; ++row)
          std::memcpy(pool.data() + (static_cast<size_t>(b) * ts + start) * page_elems +
                          static_cast<size_t>(row) * 2 * HKV * D + g * D,
                      keys.data() + static_cast<size_t>(row) * D, D * 2);
      }
  std::vector<int32_t> table(static_cast<size_t>(B) * ts), seq_len(B, a.context), sealed(B, 0), gen(B, 0);
  for (size_t i = 0; i < table.size(); ++i) table[i] = static_cast<int32_t>(i);
  const size_t rep_stride = (ts + 31) / 32 * 32;
  std::vector<float> reps(static_cast<size_t>(B) * HKV * D * rep_stride, 0.0f);
  if (sao_paged_seal(pool.data(), PAGE, table.data(), ts, seq_len.data(), sealed.data(), gen.data(), reps.data(), HKV,
                     rep_stride, B, HQ, HKV, D, 0) != 0)
    throw std::runtime_error("oracle seal failed");
  std::vector<float> q(static_cast<size_t>(B) * HQ * D);
  std::vector<int32_t> sel(static_cast<size_t>(B) * BUDGET), cnt(B);
  std::vector<std::vector<int32_t>> resident(B);
  long mismatch = 0;
  double misses = 0, selected = 0;
  for (int t = 0; t <= steps; ++t) {
    queries(B, t, q.data());
    if (sao_paged_score_select(q.data(), reps.data(), sealed.data(), B, HQ, HKV, D, HKV, rep_stride, 1, BUDGET, INIT,
                               LOCAL, sel.data(), cnt.data(), BUDGET, nullptr) != 0)
      throw std::runtime_error("oracle selection failed");
    for (int b = 0; b < B; ++b) {
      const std::vector<int32_t> cur(sel.begin() + static_cast<long>(b) * BUDGET,
                                     sel.begin() + static_cast<long>(b + 1) * BUDGET);
      mismatch += cnt[b] != BUDGET || cur != plan.expected(b, t);
      if (t > 0) {
        const hk::Correction c = hk::compare_prediction(resident[b], cur);
        misses += static_cast<double>(c.misses.size());
        selected += static_cast<double>(cur.size());
        for (size_t m = 0; m < c.misses.size(); ++m) resident[b][c.replacement_slots[m]] = c.misses[m];
      } else {
        resident[b] = cur;
      }
    }
  }
  const double coverage = 1.0 - misses / std::max(selected, 1.0);
  const bool ok = mismatch == 0 && std::fabs(coverage - static_cast<double>(BUDGET - SLOTS_RUN) / BUDGET) < 1e-12;
  std::cout << "{\"cpu_plan_check\": true, \"batch\": " << B << ", \"context\": " << a.context
            << ", \"steps\": " << steps << ", \"selection_mismatches\": " << mismatch
            << ", \"history_coverage\": " << num(coverage) << ", \"ok\": " << (ok ? "true" : "false") << "}"
            << std::endl;
  return ok ? 0 : 2;
}

Args parse(int argc, char** argv) {
  Args a;
  for (int i = 1; i < argc; ++i) {
    const std::string k = argv[i];
    auto next = [&]() -> long long {
      if (i + 1 >= argc) throw std::runtime_error("missing value for " + k);
      return std::stoll(argv[++i]);
    };
    if (k == "--layers") a.layers = static_cast<int>(next());
    else if (k == "--steps") a.steps = static_cast<int>(next());
    else if (k == "--warmup") a.warmup = static_cast<int>(next());
    else if (k == "--batch") a.batch = static_cast<int>(next());
    else if (k == "--context") a.context = static_cast<int>(next());
    else if (k == "--seed") a.seed = static_cast<uint64_t>(next());
    else if (k == "--cpu-plan") a.cpu_plan = true;
    else throw std::runtime_error("unknown argument " + k);
  }
  return a;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    const Args a = parse(argc, argv);
    if (a.cpu_plan) return cpu_plan_check(a);
    if (hipSetDevice(0) != hipSuccess) throw std::runtime_error("no GPU");
    Driver d(a);
    std::cerr << "[correction] setup: " << a.layers << " layers, batch " << a.batch << ", context " << a.context
              << std::endl;
    d.setup();
    std::vector<ScheduleStats> st;
    for (int s = 0; s < kSchedules; ++s) {
      st.push_back(d.run(static_cast<Schedule>(s)));
      std::cerr << "[correction] schedule " << kNames[s] << ": " << st.back().wall_us << " us per layer" << std::endl;
    }
    d.checks(st);
    d.print(st);
    return d.ok() ? 0 : 2;
  } catch (const std::exception& e) {
    std::cerr << "fatal: " << e.what() << '\n';
    return 1;
  }
}
