// store_check.cpp — self-checking driver of the host store tier
// (solidattention/hip_store.hpp) on the GPU, in the manner of the
// reference's lifecycle and pipeline drivers (cpp/src/kv_lifecycle_main.cpp,
// cpp/src/pipeline_main.cpp), with the reference's own closed forms as the
// bar.  TEST INFRASTRUCTURE.  Prints one JSON object; exits 0 when every
// check holds, 2 on a parity failure, 1 on an error.
//
//   lifecycle_store: 28 layers, 32 local + 512 decode tokens of the
//     reference's synthetic bytes, appended and sealed on the GPU (local 32),
//     each sealed page written back to the main store at block
//     16 + sealed index of its layer (kv_lifecycle_main.cpp:58-112), then
//     every block read back and compared with the formula: P1.3b.0's 448
//     sealed / 448 verified, tail 32, generation 16, 121,110,528 store bytes.
//   store_prefetch: the P1.0 history-correction loop (pipeline_main.cpp
//     :752-850) over a deterministic store (uring_reader.cpp:124-140), 16
//     steps x 28 layers, 4-block sets in two pool slot sets; the next
//     layer's predicted blocks are prefetched store -> pinned -> pool with a
//     generation ticket, misses read and copied into the replaced slots: 346
//     misses, hit rate 0.80692, 448 verified tickets, a stale ticket
//     rejected, and every resident page equal to its store block.
#include "solidattention/hip_kv.hpp"
#include "solidattention/hip_store.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <array>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace hk = solidattention::hip;

namespace {

bool g_ok = true;
std::ostringstream g_json;
bool g_first = true;

void record(const std::string& key, const std::string& value, bool pass) {
  g_json << (g_first ? "" : ",\n") << "  \"" << key << "\": " << value;
  g_first = false;
  if (!pass) {
    g_ok = false;
    std::cerr << "FAIL " << key << " = " << value << '\n';
  }
}
std::string num(double v) {
  std::ostringstream s;
  s.precision(9);
  s << v;
  return s.str();
}
std::string boolean(bool b) { return b ? "true" : "false"; }

std::string make_temp_dir() {
  const char* base = std::getenv("TMPDIR");
  std::string templ = std::string(base && *base ? base : "/tmp") + "/sa_store_check_XXXXXX";
  std::vector<char> buf(templ.begin(), templ.end());
  buf.push_back('\0');
  if (!mkdtemp(buf.data())) throw std::runtime_error("mkdtemp failed");
  return std::string(buf.data());
}

double ms_since(std::chrono::steady_clock::time_point t0) {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

// ---- lifecycle store (P1.3b.0) ----------------------------------------------

void check_lifecycle_store(const std::string& dir) {
  constexpr std::size_t layers = 28, hq = 16, hkv = 8, d = 128;
  constexpr std::size_t local = 32, decode = 512, initial = 16, block_tokens = 32;
  constexpr std::size_t token_values = 2 * hkv * d;
  const std::size_t capacity = initial + (decode + 31) / 32 + 1;
  const std::size_t stride = (local + decode) / block_tokens + 2;
  const std::size_t pages = layers * stride;
  // sequence l of the pool holds layer l's tail
  hk::PagedKvPool pool(layers, hq, hkv, stride, pages);
  std::vector<int32_t> table(layers * stride);
  for (std::size_t i = 0; i < table.size(); ++i) table[i] = static_cast<int32_t>((i * 37 + 11) % pages);
  pool.block_table().upload(table);
  const std::size_t block_bytes = pool.page_bytes();
  hk::MainStore store(dir + "/main-kv-store.bin", layers, capacity, block_bytes, true);
  hk::SealWriteback writeback(store, 64);
  hipStream_t stream{};
  hk::hip_check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
  hk::PinnedBuffer hk16(layers * hkv * d * 2), hv16(layers * hkv * d * 2);
  hk::DeviceArray<std::uint16_t> dk(layers * hkv * d), dv(layers * hkv * d);
  auto* k = reinterpret_cast<std::uint16_t*>(hk16.data());
  auto* v = reinterpret_cast<std::uint16_t*>(hv16.data());
  std::vector<std::size_t> sealed(layers, 0), len(layers, 0);
  const auto t0 = std::chrono::steady_clock::now();
  for (std::size_t token = 0; token < local + decode; ++token) {
    // kv_lifecycle_main.cpp:33-35: value v of token t in layer l
    for (std::size_t l = 0; l < layers; ++l)
      for (std::size_t e = 0; e < hkv * d; ++e) {
        k[l * hkv * d + e] = static_cast<std::uint16_t>((l * 1009 + token * 37 + e * 13) & 0xffff);
        v[l * hkv * d + e] = static_cast<std::uint16_t>((l * 1009 + token * 37 + (hkv * d + e) * 13) & 0xffff);
      }
    hk::hip_check(hipMemcpyAsync(dk.get(), k, layers * hkv * d * 2, hipMemcpyHostToDevice, stream), "upload k");
    hk::hip_check(hipMemcpyAsync(dv.get(), v, layers * hkv * d * 2, hipMemcpyHostToDevice, stream), "upload v");
    pool.append_seal_f16(dk.get(), dv.get(), static_cast<int>(local), stream);
    for (std::size_t l = 0; l < layers; ++l) {
      len[l] += 1;
      std::vector<int32_t> pg;
      std::vector<int64_t> blocks;
      while (len[l] >= (sealed[l] + 1) * block_tokens + local) {
        pg.push_back(table[l * stride + sealed[l]]);
        blocks.push_back(static_cast<int64_t>(initial + sealed[l]));
        ++sealed[l];
      }
      if (!pg.empty()) writeback.submit(pool, stream, static_cast<int64_t>(l), pg, blocks);
    }
    // the pinned inputs are rewritten next token
    hk::hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
  }
  writeback.drain();
  const double wall_ms = ms_since(t0);
  hk::commit_marker(dir, "generation.json", "{\"generation\":16,\"layers\":28}\n");

  // read every sealed block back and compare with the formula
  hk::PinnedBuffer back(block_bytes);
  std::vector<std::uint16_t> expect(block_bytes / 2);
  std::size_t verified = 0, written = 0;
  for (std::size_t l = 0; l < layers; ++l) {
    for (std::size_t b = 0; b < sealed[l]; ++b, ++written) {
      store.read(static_cast<int64_t>(l), {static_cast<int64_t>(initial + b)}, back.data());
      for (std::size_t t = 0; t < block_tokens; ++t)
        for (std::size_t e = 0; e < token_values; ++e)
          expect[t * token_values + e] =
              static_cast<std::uint16_t>((l * 1009 + (b * block_tokens + t) * 37 + e * 13) & 0xffff);
      verified += std::memcmp(back.data(), expect.data(), block_bytes) == 0;
    }
  }
  const auto gsealed = pool.sealed().download();
  const auto glen = pool.seq_len().download();
  const auto ggen = pool.generation().download();
  bool counters = true;
  for (std::size_t l = 0; l < layers; ++l)
    counters &= gsealed[l] == 16 && glen[l] - 16 * 32 == 32 && ggen[l] == 16;
  FILE* f = std::fopen((dir + "/generation.json").c_str(), "r");
  char marker[64] = {0};
  if (f) {
    if (std::fread(marker, 1, sizeof marker - 1, f) == 0) marker[0] = 0;
    std::fclose(f);
  }
  record("lifecycle_store_sealed_blocks", std::to_string(written), written == 448);
  record("lifecycle_store_pages_written", std::to_string(writeback.pages_written()), writeback.pages_written() == 448);
  record("lifecycle_store_verified_reads", std::to_string(verified), verified == 448);
  record("lifecycle_store_bytes", std::to_string(store.bytes()), store.bytes() == 121110528);
  record("lifecycle_store_counters_tail32_generation16", boolean(counters), counters);
  record("lifecycle_store_commit_marker", boolean(std::strcmp(marker, "{\"generation\":16,\"layers\":28}\n") == 0),
         std::strcmp(marker, "{\"generation\":16,\"layers\":28}\n") == 0);
  record("lifecycle_store_o_direct", boolean(store.direct()), true);
  record("lifecycle_store_bounced_blocks", std::to_string(store.bounced()), true);
  record("lifecycle_store_wall_ms", num(wall_ms), true);
  (void)hipStreamDestroy(stream);
}

// ---- store -> pool prefetch with tickets (P1.0 / P1.3a) ----------------------

std::vector<int32_t> oracle_blocks(std::size_t step, std::size_t layer) {
  // pipeline_main.cpp:439-447
  const std::size_t phase = step / 2;
  std::size_t first = 1 + (layer * 3 + phase) % 13;
  std::size_t second = 1 + (layer * 7 + phase * 2 + 5) % 13;
  if (second == first) second = 1 + second % 13;
  std::vector<int32_t> b{0, static_cast<int32_t>(first), static_cast<int32_t>(second), 15};
  std::sort(b.begin(), b.end());
  return b;
}

void check_store_prefetch(const std::string& dir) {
  constexpr std::size_t layers = 28, blocks_per_layer = 16, steps = 16, set = 4;
  hk::PagedKvPool pool(1, 16, 8, blocks_per_layer, 2 * set);
  const std::size_t bb = pool.page_bytes();
  hk::MainStore store(dir + "/pipeline-store.bin", layers, blocks_per_layer, bb, true);
  {
    // uring_reader.cpp:130-140: byte i of global block g = (g * 17 + i * 13) & 0xff
    hk::PinnedBuffer layer_bytes(blocks_per_layer * bb);
    for (std::size_t l = 0; l < layers; ++l) {
      for (std::size_t b = 0; b < blocks_per_layer; ++b) {
        const std::size_t g = l * blocks_per_layer + b;
        for (std::size_t i = 0; i < bb; ++i) layer_bytes.data()[b * bb + i] = static_cast<std::uint8_t>((g * 17 + i * 13) & 0xff);
      }
      std::vector<int64_t> all(blocks_per_layer);
      for (std::size_t b = 0; b < blocks_per_layer; ++b) all[b] = static_cast<int64_t>(b);
      store.write(static_cast<int64_t>(l), all, layer_bytes.data());
    }
    store.sync();
  }
  hk::StorePrefetcher prefetcher(store, set);
  hk::MissCorrector corrector;
  hk::PinnedBuffer miss_staging(set * bb), check_pages(set * bb);
  hipStream_t compute{};
  hk::hip_check(hipStreamCreateWithFlags(&compute, hipStreamNonBlocking), "hipStreamCreate");
  auto slots = [&](std::size_t layer) {
    std::vector<int32_t> s(set);
    for (std::size_t i = 0; i < set; ++i) s[i] = static_cast<int32_t>((layer % 2) * set + i);
    return s;
  };
  std::vector<std::vector<int32_t>> history(layers);
  std::vector<int64_t> generation(layers, 0);
  for (std::size_t l = 0; l < layers; ++l) history[l] = oracle_blocks(0, l);
  std::size_t predicted_total = 0, hits = 0, misses = 0, pages_ok = 0, pages_checked = 0, sets_ok = 0;
  const auto t0 = std::chrono::steady_clock::now();
  double exposed_ms = 0.0;
  for (std::size_t step = 0; step < steps; ++step) {
    prefetcher.submit(hk::PrefetchTicket{static_cast<int64_t>(step), 0, generation[0], history[0]}, pool, slots(0),
                      compute);
    for (std::size_t layer = 0; layer < layers; ++layer) {
      const std::vector<int32_t> predicted = history[layer];
      const std::vector<int32_t> oracle = oracle_blocks(step, layer);
      const auto w0 = std::chrono::steady_clock::now();
      prefetcher.acquire(static_cast<int64_t>(step), static_cast<int64_t>(layer), generation[layer], predicted,
                         compute);
      exposed_ms += ms_since(w0);
      std::vector<int32_t> resident = predicted;
      const hk::Correction c = hk::compare_prediction(predicted, oracle);
      predicted_total += predicted.size();
      hits += c.hits;
      misses += c.misses.size();
      if (!c.misses.empty()) {
        const std::vector<int64_t> mb(c.misses.begin(), c.misses.end());
        store.read(static_cast<int64_t>(layer), mb, miss_staging.data());
        std::vector<int32_t> dst;
        std::vector<int64_t> src;
        for (std::size_t j = 0; j < c.misses.size(); ++j) {
          dst.push_back(slots(layer)[static_cast<std::size_t>(c.replacement_slots[j])]);
          src.push_back(static_cast<int64_t>(j));
          resident[static_cast<std::size_t>(c.replacement_slots[j])] = c.misses[j];
        }
        // the replaced slots were just written by the prefetch copies
        corrector.after(compute);
        corrector.fill(pool.pool().get(), bb, dst, miss_staging.data(), src);
        corrector.order(compute);
        // miss_staging is reused by the next layer's misses
        hk::hip_check(hipStreamSynchronize(corrector.copy_stream()), "hipStreamSynchronize copy");
      }
      history[layer] = oracle;
      ++generation[layer];
      if (layer + 1 < layers)
        prefetcher.submit(hk::PrefetchTicket{static_cast<int64_t>(step), static_cast<int64_t>(layer + 1),
                                             generation[layer + 1], history[layer + 1]},
                          pool, slots(layer + 1), compute);
      // the layer's "attention": its resident pages, read on the compute stream
      for (std::size_t i = 0; i < set; ++i)
        hk::hip_check(hipMemcpyAsync(check_pages.data() + i * bb,
                                     reinterpret_cast<std::uint8_t*>(pool.pool().get()) +
                                         static_cast<std::size_t>(slots(layer)[i]) * bb,
                                     bb, hipMemcpyDeviceToHost, compute),
                      "check copy");
      hk::hip_check(hipStreamSynchronize(compute), "hipStreamSynchronize compute");
      std::vector<int32_t> sorted_res = resident;
      std::sort(sorted_res.begin(), sorted_res.end());
      sets_ok += sorted_res == oracle;
      for (std::size_t i = 0; i < set; ++i) {
        const std::size_t g = layer * blocks_per_layer + static_cast<std::size_t>(resident[i]);
        bool same = true;
        for (std::size_t j = 0; j < bb && same; ++j)
          same = check_pages.data()[i * bb + j] == static_cast<std::uint8_t>((g * 17 + j * 13) & 0xff);
        pages_ok += same;
        ++pages_checked;
      }
    }
  }
  const double wall_ms = ms_since(t0);
  // a ticket issued for another selection generation is refused
  // (P1.3a's stale-ticket self test)
  bool stale_rejected = false;
  prefetcher.submit(hk::PrefetchTicket{0, 0, 7, history[0]}, pool, slots(0), compute);
  try {
    prefetcher.acquire(0, 0, 8, history[0], compute);
  } catch (const std::runtime_error&) {
    stale_rejected = true;
  }
  prefetcher.discard();
  const double hit_rate = static_cast<double>(hits) / static_cast<double>(predicted_total);
  record("store_prefetch_predicted_blocks", std::to_string(predicted_total), predicted_total == 1792);
  record("store_prefetch_miss_blocks", std::to_string(misses), misses == 346);
  record("store_prefetch_history_hit_rate", num(hit_rate), std::abs(hit_rate - 0.80692) < 5e-6);
  record("store_prefetch_verified_tickets", std::to_string(prefetcher.verified()), prefetcher.verified() == 448);
  record("store_prefetch_stale_ticket_rejected", boolean(stale_rejected && prefetcher.rejected() == 1),
         stale_rejected && prefetcher.rejected() == 1);
  record("store_prefetch_resident_equals_oracle", std::to_string(sets_ok), sets_ok == steps * layers);
  record("store_prefetch_pages_equal_store", "\"" + std::to_string(pages_ok) + "/" + std::to_string(pages_checked) + "\"",
         pages_ok == pages_checked && pages_checked == steps * layers * set);
  record("store_prefetch_wall_ms", num(wall_ms), true);
  record("store_prefetch_exposed_wait_ms", num(exposed_ms), true);
  (void)hipStreamDestroy(compute);
}

}  // namespace

int main() {
  try {
    const std::string dir = make_temp_dir();
    g_json << "{\n";
    check_lifecycle_store(dir);
    check_store_prefetch(dir);
    g_json << "\n}\n";
    std::cout << g_json.str();
    std::remove((dir + "/main-kv-store.bin").c_str());
    std::remove((dir + "/pipeline-store.bin").c_str());
    std::remove((dir + "/generation.json").c_str());
    std::remove(dir.c_str());
    return g_ok ? 0 : 2;
  } catch (const std::exception& e) {
    std::cerr << "fatal: " << e.what() << '\n';
    return 1;
  }
}
