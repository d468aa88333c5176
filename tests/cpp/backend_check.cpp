// backend_check.cpp — self-checking integration driver for the C++ boundary
// (make_hip_backend() and solidattention/hip_kv.hpp), in the manner of the
// reference's C0/C1/C2 and lifecycle drivers (cpp/src/main.cpp,
// attention_main.cpp, selection_main.cpp, kv_lifecycle_main.cpp), without
// the SSD tier.  TEST INFRASTRUCTURE: links the CPU oracle as the checker.
// Prints one JSON object; exits 0 when every check holds, 2 on a parity
// failure, 1 on an error (the reference drivers' convention).
#include "solidattention/backend.hpp"
#include "solidattention/hip_backend.hpp"
#include "solidattention/hip_kv.hpp"

extern "C" {
#include "sa_oracle.h"
}

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <iostream>
#include <memory>
#include <numeric>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace sa = solidattention;

namespace {

bool g_ok = true;
std::ostringstream g_json;
bool g_first = true;

void record(const std::string& key, const std::string& value, bool pass) {
  g_json << (g_first ? "" : ",\n") << "  \"" << key << "\": " << value;
  g_first = false;
  if (!pass) {
    g_ok = false;
    std::cerr << "FAILED: " << key << " = " << value << '\n';
  }
}

std::string num(double v) {
  char b[64];
  std::snprintf(b, sizeof b, "%.9g", v);
  return b;
}

struct Compare {
  double max_abs{};
  double cosine{};
};

Compare compare(const std::vector<float>& ref, const std::vector<float>& got) {
  Compare c;
  double dot = 0, rn = 0, gn = 0;
  for (std::size_t i = 0; i < ref.size(); ++i) {
    c.max_abs = std::max(c.max_abs, std::abs(static_cast<double>(ref[i]) - got[i]));
    dot += static_cast<double>(ref[i]) * got[i];
    rn += static_cast<double>(ref[i]) * ref[i];
    gn += static_cast<double>(got[i]) * got[i];
  }
  c.cosine = dot / std::sqrt(rn * gn);
  return c;
}

// C0: H2D, xor transform, D2H, checksum (reference cpp/src/main.cpp:79-116).
void check_c0(sa::AcceleratorBackend& backend) {
  const std::size_t bytes = 128 * 1024 + 5;
  auto* pinned = static_cast<std::uint8_t*>(backend.allocate_host(bytes));
  for (std::size_t i = 0; i < bytes; ++i) pinned[i] = static_cast<std::uint8_t>((i * 131 + 7) & 0xff);
  const std::uint8_t mask = 0x5a;
  std::uint64_t expect = 0;
  for (std::size_t i = 0; i < bytes; ++i) expect += static_cast<std::uint8_t>(pinned[i] ^ mask);
  const auto r = backend.execute(pinned, bytes, mask);
  backend.free_host(pinned);
  record("c0_checksum", std::to_string(r.checksum), r.checksum == expect);
}

// C1: 128-token fixture through every attention variant with the
// reference's acceptance bars (attention_main.cpp:265-270).
void check_c1(sa::AcceleratorBackend& backend, std::size_t tokens, const char* tag, std::size_t d = 128) {
  const std::size_t hq = 16, hkv = 8;
  std::vector<std::uint16_t> kv(tokens * 2 * hkv * d);
  std::vector<float> q(hq * d);
  sao_fixture_c1(tokens, hq, hkv, d, kv.data(), q.data());
  const float scale = 1.0f / std::sqrt(static_cast<float>(d));
  std::vector<float> ref(hq * d);
  if (sao_attention_reference(kv.data(), q.data(), tokens, hq, hkv, d, scale, ref.data()) != 0)
    throw std::runtime_error("oracle attention failed");
  float consumer_ref = 0.0f;
  for (std::size_t i = 0; i < ref.size(); ++i) consumer_ref += ref[i] * (1.0f + static_cast<float>(i % 17) * 0.001f);
  auto* pinned = static_cast<std::uint16_t*>(backend.allocate_host(kv.size() * 2));
  std::memcpy(pinned, kv.data(), kv.size() * 2);
  sa::AttentionProblem problem{pinned, q.data(), tokens, hq, hkv, d, scale};
  const char* modes[] = {"attention", "optimized", "persistent", "resident", "consumed"};
  for (int m = 0; m < 5; ++m) {
    for (int op = 0; op < 3; ++op) {
      sa::AttentionResult r;
      switch (m) {
        case 0: r = backend.attention(problem); break;
        case 1: r = backend.attention_optimized(problem); break;
        case 2: r = backend.attention_persistent(problem); break;
        case 3: r = backend.attention_resident(problem, op == 2); break;
        default: r = backend.attention_consumed(problem, op == 2); break;
      }
      if (m == 3 && op < 2 && !r.output.empty()) record(std::string(tag) + "_resident_unaudited_output", "1", false);
      if (op != 2) continue;
      if (m == 4) {
        const double err = std::abs(static_cast<double>(consumer_ref) - r.output.at(0));
        record(std::string(tag) + "_consumed_abs_error", num(err), err <= 1e-4);
      } else {
        const Compare c = compare(ref, r.output);
        record(std::string(tag) + "_" + modes[m] + "_max_abs_error", num(c.max_abs), c.max_abs <= 2e-5);
        record(std::string(tag) + "_" + modes[m] + "_cosine", num(c.cosine), c.cosine >= 0.999999);
      }
      record(std::string(tag) + "_" + modes[m] + "_kernel_ms", num(r.kernel_ms), r.kernel_ms >= 0.0);
    }
  }
  backend.free_host(pinned);
}

// C2.1: InfLLM representatives (host numerics, as in the reference driver),
// GPU selection over them, GPU gather of the selected blocks, attention over
// the packed blocks (selection_main.cpp:113-255).
void check_c2(sa::AcceleratorBackend& backend) {
  const std::size_t tokens = 512, blocks = 16, hq = 16, hkv = 8, d = 128, budget = 4;
  std::vector<std::uint16_t> kv(tokens * 2 * hkv * d);
  std::vector<float> pq(hq * tokens * d);
  sao_fixture_c2(tokens, hq, hkv, d, kv.data(), pq.data());
  std::vector<float> reps(hq * blocks * d);
  std::vector<std::size_t> offsets(hq * blocks * 4);
  sao_build_local_causal_representatives(pq.data(), kv.data(), tokens, hq, hkv, d, 32, 32, 4, reps.data(),
                                         offsets.data());
  std::vector<float> query(hq * d);
  for (std::size_t h = 0; h < hq; ++h)
    std::copy_n(pq.data() + (h * tokens + tokens - 1) * d, d, query.data() + h * d);

  // one sequence; 16 pages holding the fixture in order; per-query-head reps
  sa::hip::PagedKvPool pool(1, hq, hkv, blocks, blocks, hq, blocks);
  std::vector<std::uint16_t> pages(kv);  // block b = page b
  pool.pool().upload(pages);
  std::vector<int32_t> table(blocks);
  std::iota(table.begin(), table.end(), 0);
  pool.block_table().upload(table);
  pool.seq_len().upload({static_cast<int32_t>(tokens)});
  pool.sealed().upload({static_cast<int32_t>(blocks)});
  std::vector<float> dmajor(hq * d * blocks);
  for (std::size_t h = 0; h < hq; ++h)
    for (std::size_t b = 0; b < blocks; ++b)
      for (std::size_t i = 0; i < d; ++i) dmajor[(h * d + i) * blocks + b] = reps[(h * blocks + b) * d + i];
  pool.reps().upload(dmajor);
  sa::hip::DeviceArray<float> dq(hq * d);
  dq.upload(query);
  sa::hip::SparseDecoder dec(pool, sa_select_params{1, static_cast<int32_t>(budget), 1, 1, static_cast<int32_t>(budget)});
  dec.select(pool, dq.get());
  sa::hip::hip_check(hipDeviceSynchronize(), "select");
  const auto ids = dec.selected().download();
  const auto cnt = dec.counts().download();
  std::ostringstream s;
  s << "[";
  for (int i = 0; i < cnt[0]; ++i) s << (i ? "," : "") << ids[i];
  s << "]";
  record("c2_selected_block_ids", s.str(), s.str() == "[0,8,13,15]");

  // gather (pack) the selected pages and check the bytes
  const std::size_t page_elems = pool.page_elems();
  sa::hip::DeviceArray<std::uint16_t> packed(budget * page_elems);
  sa::hip::check(sa_hip_gather_pages(pool.pool().get(), static_cast<int64_t>(pool.page_bytes()), 16,
                                     dec.selected().get(), static_cast<int32_t>(budget), packed.get(), nullptr,
                                     nullptr),
                 "gather_pages");
  const auto host_packed = packed.download();
  bool exact = true;
  for (std::size_t i = 0; i < budget; ++i)
    exact &= std::memcmp(host_packed.data() + i * page_elems, kv.data() + ids[i] * page_elems, page_elems * 2) == 0;
  record("c2_packed_kv_exact", exact ? "true" : "false", exact);

  // attention over the packed blocks vs the oracle (reference bar 2e-5)
  const float scale = 1.0f / std::sqrt(static_cast<float>(d));
  std::vector<float> ref(hq * d), dense(hq * d);
  sao_attention_reference(host_packed.data(), query.data(), budget * 32, hq, hkv, d, scale, ref.data());
  sao_attention_reference(kv.data(), query.data(), tokens, hq, hkv, d, scale, dense.data());
  sa::AttentionProblem sparse{host_packed.data(), query.data(), budget * 32, hq, hkv, d, scale};
  backend.attention_persistent(sparse);  // warmup, as the reference driver does
  const auto r = backend.attention_persistent(sparse);
  const Compare c = compare(ref, r.output);
  record("c2_max_error_vs_sparse_cpu", num(c.max_abs), c.max_abs <= 2e-5 && c.cosine >= 0.999999);
  const Compare sd = compare(dense, ref);
  char cos6[32];
  std::snprintf(cos6, sizeof cos6, "%.6f", sd.cosine);
  record("c2_selected_vs_dense_cosine", cos6, std::string(cos6) == "0.987693");
}

// Lifecycle: local window 32, 32 + 512 appends per layer of the reference's
// synthetic byte formula (kv_lifecycle_main.cpp:31-45, 83-115): 16 seals per
// layer, tail 32, generation 16, sealed pages byte-exact.
void check_lifecycle() {
  const std::size_t layers = 28, hq = 16, hkv = 8, d = 128, local = 32, decode = 512;
  const std::size_t width = hkv * d, blocks = (local + decode) / 32 + 1;
  std::size_t sealed_total = 0;
  bool bytes_ok = true, tail_ok = true;
  // all 28 layers as 28 "sequences" of one pool: same kernels, one launch per step
  sa::hip::PagedKvPool pool(layers, hq, hkv, blocks, layers * blocks);
  std::vector<int32_t> table(layers * blocks);
  std::iota(table.begin(), table.end(), 0);
  pool.block_table().upload(table);
  sa::hip::DeviceArray<std::uint16_t> dk(layers * width), dv(layers * width);
  std::vector<std::uint16_t> k(layers * width), v(layers * width);
  for (std::size_t token = 0; token < local + decode; ++token) {
    for (std::size_t l = 0; l < layers; ++l)
      for (std::size_t i = 0; i < width; ++i) {
        k[l * width + i] = static_cast<std::uint16_t>((l * 1009 + token * 37 + i * 13) & 0xffff);
        v[l * width + i] = static_cast<std::uint16_t>((l * 1009 + token * 37 + (width + i) * 13) & 0xffff);
      }
    dk.upload(k);
    dv.upload(v);
    pool.append_seal_f16(dk.get(), dv.get(), static_cast<int>(local));
  }
  sa::hip::hip_check(hipDeviceSynchronize(), "lifecycle");
  const auto sealed = pool.sealed().download();
  const auto gen = pool.generation().download();
  const auto len = pool.seq_len().download();
  const auto bytes = pool.pool().download();
  const std::size_t token_values = 2 * width;
  for (std::size_t l = 0; l < layers; ++l) {
    sealed_total += static_cast<std::size_t>(sealed[l]);
    const std::size_t tail = static_cast<std::size_t>(len[l]) - static_cast<std::size_t>(sealed[l]) * 32;
    tail_ok &= tail >= local && tail < local + 32 && gen[l] == sealed[l];
    for (int b = 0; b < sealed[l]; ++b)
      for (std::size_t t = 0; t < 32; ++t)
        for (std::size_t i = 0; i < token_values; ++i) {
          const std::size_t token = static_cast<std::size_t>(b) * 32 + t;
          const auto expect = static_cast<std::uint16_t>((l * 1009 + token * 37 + i * 13) & 0xffff);
          bytes_ok &= bytes[(l * blocks + static_cast<std::size_t>(b)) * 32 * token_values + t * token_values + i] ==
                      expect;
        }
  }
  record("lifecycle_sealed_blocks", std::to_string(sealed_total), sealed_total == 448);
  record("lifecycle_resident_tail_tokens", std::to_string(len[0] - sealed[0] * 32), tail_ok && len[0] - sealed[0] * 32 == 32);
  record("lifecycle_generation", std::to_string(gen[0]), gen[0] == 16);
  record("lifecycle_sealed_bytes_exact", bytes_ok ? "true" : "false", bytes_ok);
}

// Decode steps through SparseDecoder::decode_step (one fused launch per
// step at G=2: the tuned kernel at head_dim 128, the token-row kernel at 64
// and 256): 4 sequences, 34 steps across seal boundaries, against the
// oracle's append, seal, select and attention (qwen_chain_main.cpp:390-395,
// kv_lifecycle_main.cpp:92-113, selection.cpp:96-147).  groups: selection
// groups (8: one block set per KV group; 1: the shared selection of the C2/P1
// drivers, also one launch at head_dim 128).  Record names carry `tag`.
void check_decode_step(std::size_t d = 128, const std::string& tag = "", std::size_t groups = 8) {
  const std::size_t batch = 4, hq = 16, hkv = 8, stride = 24, pages = batch * stride;
  const std::size_t budget = 8, steps = 34;
  sa::hip::PagedKvPool pool(batch, hq, hkv, stride, pages, 0, 0, d);
  const std::size_t page_elems = pool.page_elems();
  std::vector<std::uint16_t> host_pool(pages * page_elems);
  sao_synth_fill_half(31, 0, host_pool.size(), host_pool.data());
  std::vector<int32_t> table(batch * stride);
  for (std::size_t i = 0; i < table.size(); ++i) table[i] = static_cast<int32_t>((i * 37 + 11) % pages);
  std::vector<int32_t> seq_len = {32 * 9 + 30, 32 * 12, 32 * 5 + 7, 32 * 16 + 1};
  std::vector<int32_t> sealed(batch, 0), gen(batch, 0);
  const std::size_t rep_stride = pool.rep_stride();  // rows padded to whole 128-byte lines
  std::vector<float> reps(batch * hkv * d * rep_stride, 0.0f);
  sao_paged_seal(host_pool.data(), 32, table.data(), stride, seq_len.data(), sealed.data(), gen.data(),
                 reps.data(), hkv, rep_stride, batch, hq, hkv, d, 0);
  pool.pool().upload(host_pool);
  pool.block_table().upload(table);
  pool.seq_len().upload(seq_len);
  pool.sealed().upload(sealed);
  pool.generation().upload(gen);
  pool.reps().upload(reps);
  sa::hip::SparseDecoder dec(pool, sa_select_params{static_cast<int32_t>(groups), static_cast<int32_t>(budget), 1, 2,
                                                    static_cast<int32_t>(budget), 0, nullptr});
  // one launch at every head_dim up to 256 (the token-row kernel away from 128)
  record("decode_step_fused" + tag, dec.fused(pool) ? "true" : "false", dec.fused(pool) == (d <= 256));
  sa::hip::DeviceArray<float> dk(batch * hkv * d), dv(batch * hkv * d), dq(batch * hq * d), dout(batch * hq * d);
  std::vector<float> k(batch * hkv * d), v(batch * hkv * d), q(batch * hq * d), out(batch * hq * d);
  std::vector<int32_t> sel(batch * groups * budget), cnt(batch * groups);
  const float scale = 1.0f / std::sqrt(static_cast<float>(d));
  bool ids_ok = true;
  double max_err = 0.0;
  for (std::size_t step = 0; step < steps; ++step) {
    sao_synth_fill_float(1000 + step, 0, k.size(), k.data());
    sao_synth_fill_float(2000 + step, 0, v.size(), v.data());
    sao_synth_fill_float(3000 + step, 0, q.size(), q.data());
    dk.upload(k);
    dv.upload(v);
    dq.upload(q);
    dec.decode_step(pool, dk.get(), dv.get(), 0, dq.get(), scale, dout.get());
    sao_paged_append(host_pool.data(), 32, table.data(), stride, seq_len.data(), k.data(), v.data(), nullptr, nullptr,
                     batch, hkv, d);
    sao_paged_seal(host_pool.data(), 32, table.data(), stride, seq_len.data(), sealed.data(), gen.data(),
                   reps.data(), hkv, rep_stride, batch, hq, hkv, d, 0);
    sao_paged_score_select(q.data(), reps.data(), sealed.data(), batch, hq, hkv, d, hkv, rep_stride,
                           static_cast<int>(groups), budget, 1, 2, sel.data(), cnt.data(), budget, nullptr);
    sao_paged_sparse_attention(host_pool.data(), 32, table.data(), stride, seq_len.data(), sealed.data(), sel.data(),
                               cnt.data(), budget, static_cast<int>(groups), q.data(), batch, hq, hkv, d, scale,
                               out.data());
    const auto gsel = dec.selected().download();
    const auto gcnt = dec.counts().download();
    const auto gout = dout.download();
    for (std::size_t r = 0; r < batch * groups; ++r) {
      ids_ok &= gcnt[r] == cnt[r];
      for (int i = 0; i < cnt[r] && ids_ok; ++i) ids_ok &= gsel[r * budget + i] == sel[r * budget + i];
    }
    for (std::size_t i = 0; i < out.size(); ++i)
      max_err = std::max(max_err, std::abs(static_cast<double>(out[i]) - gout[i]) /
                                      std::max(1.0, std::abs(static_cast<double>(out[i]))));
  }
  const bool state_ok = pool.seq_len().download() == seq_len && pool.sealed().download() == sealed &&
                        pool.generation().download() == gen && pool.pool().download() == host_pool;
  const auto greps = pool.reps().download();
  const bool reps_ok = std::memcmp(greps.data(), reps.data(), reps.size() * sizeof(float)) == 0;
  record("decode_step_selected_ids_exact" + tag, ids_ok ? "true" : "false", ids_ok);
  record("decode_step_state_bytes_exact" + tag, state_ok && reps_ok ? "true" : "false", state_ok && reps_ok);
  record("decode_step_max_rel_error" + tag, num(max_err), max_err <= 2e-3);
  if (d != 128) {
    // select() + attend() over the last step's query (the general scoring
    // hands its scores over through the decoder's own buffer)
    dec.select(pool, dq.get());
    dec.attend(pool, dq.get(), scale, dout.get());
    const auto gout = dout.download();
    double err = 0.0;
    for (std::size_t i = 0; i < out.size(); ++i)
      err = std::max(err, std::abs(static_cast<double>(out[i]) - gout[i]) /
                              std::max(1.0, std::abs(static_cast<double>(out[i]))));
    record("select_attend_max_rel_error" + tag, num(err), err <= 2e-3);
    return;
  }
  if (groups != hkv) return;

  // the chunked schedule over the last step's selection: 3-page chunks of
  // lists of up to 9 pages, against the oracle's attention of that step
  sa::hip::SparseDecoder chunked(pool, sa_select_params{static_cast<int32_t>(hkv), static_cast<int32_t>(budget), 1, 2,
                                                        static_cast<int32_t>(budget), 0, nullptr},
                                 0, 3);
  chunked.select(pool, dq.get());
  chunked.attend_chunked(pool, dq.get(), scale, dout.get());
  const auto cout_ = dout.download();
  double chunk_err = 0.0;
  for (std::size_t i = 0; i < out.size(); ++i)
    chunk_err = std::max(chunk_err, std::abs(static_cast<double>(out[i]) - cout_[i]) /
                                        std::max(1.0, std::abs(static_cast<double>(out[i]))));
  record("attend_chunked_max_rel_error", num(chunk_err), chunk_err <= 2e-3);
}

// SparseDecoder::decode_step_qkv (the q/k/v projection's partials feeding
// the one-launch step, which runs the reduce's epilogue for its own heads)
// against the two calls it replaces, sa_hip_qkv_project_rms then
// SparseDecoder::decode_step, on two copies of the same pool over 34 steps
// across seals: q/k/v, ids, outputs and state equal bit for bit.
void check_decode_step_qkv() {
  const std::size_t batch = 4, hq = 16, hkv = 8, d = 128, stride = 24, pages = batch * stride, hidden = 1024;
  const std::size_t budget = 8, steps = 34;
  std::vector<std::uint16_t> host_pool(pages * 32 * 2 * hkv * d);
  sao_synth_fill_half(41, 0, host_pool.size(), host_pool.data());
  std::vector<int32_t> table(batch * stride);
  for (std::size_t i = 0; i < table.size(); ++i) table[i] = static_cast<int32_t>((i * 29 + 5) % pages);
  std::vector<int32_t> seq_len = {32 * 9 + 30, 32 * 12, 32 * 5 + 7, 32 * 16 + 1};
  sa::hip::PagedKvPool pa(batch, hq, hkv, stride, pages), pb(batch, hq, hkv, stride, pages);
  for (auto* pool : {&pa, &pb}) {
    pool->pool().upload(host_pool);
    pool->block_table().upload(table);
    pool->seq_len().upload(seq_len);
    pool->seal(0);
  }
  const sa_select_params params{static_cast<int32_t>(hkv), static_cast<int32_t>(budget), 1, 2,
                                static_cast<int32_t>(budget), 0, nullptr};
  sa::hip::SparseDecoder da(pa, params), db(pb, params);
  auto weights = [](std::size_t n, std::uint64_t seed, float scale, float offset) {
    std::vector<float> w(n);
    sao_synth_fill_float(seed, 0, n, w.data());
    for (auto& x : w) x = offset + scale * x;
    sa::hip::DeviceArray<float> dw(n);
    dw.upload(w);
    return dw;
  };
  const float ws = 1.0f / std::sqrt(static_cast<float>(hidden));
  auto wq = weights(hq * d * hidden, 51, ws, 0.0f), wk = weights(hkv * d * hidden, 52, ws, 0.0f),
       wv = weights(hkv * d * hidden, 53, ws, 0.0f), qn = weights(d, 54, 0.1f, 1.0f), kn = weights(d, 55, 0.1f, 1.0f),
       in_norm = weights(hidden, 56, 0.1f, 1.0f);
  const std::size_t qkv_bytes = sa_hip_qkv_workspace_bytes(static_cast<int32_t>(batch), static_cast<int32_t>(hidden),
                                                           static_cast<int32_t>(hq), static_cast<int32_t>(hkv));
  sa::hip::DeviceArray<float> qkv_ws((qkv_bytes + 3) / 4), x(batch * hidden);
  sa::hip::DeviceArray<float> qa(batch * hq * d), ka(batch * hkv * d), va(batch * hkv * d), oa(batch * hq * d);
  sa::hip::DeviceArray<float> qb(batch * hq * d), kb(batch * hkv * d), vb(batch * hkv * d), ob(batch * hq * d);
  std::vector<float> hx(batch * hidden);
  const float scale = 1.0f / std::sqrt(static_cast<float>(d));
  bool same = true;
  for (std::size_t step = 0; step < steps; ++step) {
    sao_synth_fill_float(4000 + step, 0, hx.size(), hx.data());
    x.upload(hx);
    int rc = sa_hip_qkv_project_rms(x.get(), in_norm.get(), 1e-6f, wq.get(), wk.get(), wv.get(), qn.get(), kn.get(),
                                    pa.seq_len().get(), static_cast<int32_t>(batch), static_cast<int32_t>(hidden),
                                    static_cast<int32_t>(hq), static_cast<int32_t>(hkv), 1e6f, 1e-6f, qa.get(),
                                    ka.get(), va.get(), qkv_ws.get(), qkv_bytes, nullptr);
    if (rc != 0) throw std::runtime_error(std::string("qkv_project_rms: ") + sa_hip_last_error());
    da.decode_step(pa, ka.get(), va.get(), 0, qa.get(), scale, oa.get());
    const sa_qkv_producer pr{x.get(), in_norm.get(), 1e-6f, wq.get(), wk.get(), wv.get(), qn.get(), kn.get(),
                             pb.seq_len().get(), static_cast<int32_t>(hidden), 1e6f, 1e-6f, qb.get(), kb.get(),
                             vb.get(), qkv_ws.get(), qkv_bytes};
    db.decode_step_qkv(pb, pr, 0, scale, ob.get());
    same &= qa.download() == qb.download() && ka.download() == kb.download() && va.download() == vb.download();
    same &= da.selected().download() == db.selected().download() && da.counts().download() == db.counts().download();
    const auto ga = oa.download(), gb = ob.download();
    same &= std::memcmp(ga.data(), gb.data(), ga.size() * sizeof(float)) == 0;
  }
  const auto ra = pa.reps().download(), rb = pb.reps().download();
  same &= pa.pool().download() == pb.pool().download() && pa.seq_len().download() == pb.seq_len().download() &&
          pa.sealed().download() == pb.sealed().download() &&
          std::memcmp(ra.data(), rb.data(), ra.size() * sizeof(float)) == 0;
  record("decode_step_qkv_equals_two_calls", same ? "true" : "false", same);
}

}  // namespace

int main() {
  try {
    auto backend = sa::make_hip_backend();
    g_json << "{\n";
    record("backend", "\"" + backend->name() + "\"", backend->name() == "hip-gfx950");
    check_c0(*backend);
    check_c1(*backend, 128, "c1");
    check_c1(*backend, 4096, "c1_4096_tokens");
    // the reference's attention takes any head_dim (attention_reference.cpp:55-96)
    check_c1(*backend, 1000, "c1_head_dim_64", 64);
    check_c1(*backend, 3000, "c1_head_dim_256", 256);
    check_c2(*backend);
    check_lifecycle();
    check_decode_step();
    check_decode_step(64, "_head_dim_64");
    check_decode_step(256, "_head_dim_256");
    check_decode_step(128, "_shared", 1);
    check_decode_step_qkv();
    g_json << "\n}\n";
    std::cout << g_json.str();
    return g_ok ? 0 : 2;
  } catch (const std::exception& e) {
    std::cerr << "fatal: " << e.what() << '\n';
    return 1;
  }
}
