// hip_store.hpp — the host store tier around the paged HBM pool (header-only;
// link libsa_hip.so): the main KV store file, seal writeback from the pool,
// and ticketed store-to-pool prefetch.
//
// The semantics carried over from the reference:
//   MainStore        the main store's per-layer reserved segments, O_DIRECT
//                    block I/O (kv_lifecycle_main.cpp:73-80, 105-108;
//                    pipeline_main.cpp:660-678)
//   commit_marker    crash-consistent generation marker
//                    (online_seal_main.cpp:59-70)
//   SealWriteback    a sealed block goes to its layer's segment at block
//                    initial_blocks + sealed index (kv_lifecycle_main.cpp
//                    :104-112); here it is copied out of the HBM pool on a
//                    copy stream and written by a host thread while decoding
//                    continues
//   PrefetchTicket,  the next layer's predicted blocks are read ahead and
//   StorePrefetcher  checked against (token, layer, generation, blocks) before
//                    the layer uses them (pipeline_main.cpp:425-437, 790-800,
//                    861-876); here the reads land in pinned staging and go
//                    to pool pages on a copy stream, and the compute stream
//                    waits on the device instead of the host
// The io_uring reader of the reference's SSD tier (uring_reader.cpp) stays
// host-side; MainStore is a plain pread/pwrite stand-in with the same block
// offsets, and any reader that fills pinned memory can feed
// sa_hip_fill_pages_async the same way.
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <condition_variable>
#include <cstdint>
#include <deque>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "sa_hip.h"
#include "sa_store.h"
#include "solidattention/hip_kv.hpp"

namespace solidattention::hip {

class MainStore {
 public:
  MainStore(const std::string& path, int64_t layers, int64_t blocks_per_layer, int64_t block_bytes, bool create,
            bool direct = true, int threads = 8)
      : block_bytes_(block_bytes) {
    s_ = sa_store_open(path.c_str(), layers, blocks_per_layer, block_bytes,
                       (create ? SA_STORE_CREATE : 0) | (direct ? SA_STORE_DIRECT : 0), threads);
    if (!s_) throw std::runtime_error(std::string("store_open: ") + sa_hip_last_error());
  }
  ~MainStore() { sa_store_close(s_); }
  MainStore(const MainStore&) = delete;
  MainStore& operator=(const MainStore&) = delete;

  void read(int64_t layer, const std::vector<int64_t>& blocks, void* dst) {
    check(sa_store_read_blocks(s_, layer, blocks.data(), static_cast<int32_t>(blocks.size()), dst), "store_read");
  }
  void write(int64_t layer, const std::vector<int64_t>& blocks, const void* src) {
    check(sa_store_write_blocks(s_, layer, blocks.data(), static_cast<int32_t>(blocks.size()), src), "store_write");
  }
  void sync() { check(sa_store_sync(s_), "store_sync"); }
  bool direct() const { return sa_store_is_direct(s_) != 0; }
  int64_t bytes() const { return sa_store_bytes(s_); }
  int64_t bounced() const { return sa_store_bounced(s_); }
  int64_t block_bytes() const { return block_bytes_; }
  sa_store* get_handle() const { return s_; }

 private:
  sa_store* s_{};
  int64_t block_bytes_{};
};

inline void commit_marker(const std::string& directory, const std::string& name, const std::string& body) {
  check(sa_store_commit_marker(directory.c_str(), name.c_str(), body.c_str()), "commit_marker");
}

// Page-aligned pinned host memory (hipHostMalloc).
class PinnedBuffer {
 public:
  explicit PinnedBuffer(std::size_t bytes) : bytes_(bytes) {
    hip_check(hipHostMalloc(&p_, bytes_, hipHostMallocDefault), "hipHostMalloc");
  }
  ~PinnedBuffer() {
    if (p_) (void)hipHostFree(p_);
  }
  PinnedBuffer(const PinnedBuffer&) = delete;
  PinnedBuffer& operator=(const PinnedBuffer&) = delete;
  std::uint8_t* data() const { return static_cast<std::uint8_t*>(p_); }
  std::size_t bytes() const { return bytes_; }

 private:
  void* p_{};
  std::size_t bytes_{};
};

// Writes sealed pool pages to the main store behind the decode steps: each
// submit() stages pages into a pinned ring on a copy stream (after the work
// already queued on the compute stream), and a host thread writes them to
// the store once the copies have landed.  drain() returns when every
// submitted page is on disk.
class SealWriteback {
 public:
  SealWriteback(MainStore& store, int staging_pages) : store_(store), cap_(staging_pages), used_(staging_pages, 0) {
    if (staging_pages < 1) throw std::runtime_error("SealWriteback: staging_pages must be positive");
    staging_ = std::make_unique<PinnedBuffer>(static_cast<std::size_t>(staging_pages) * store.block_bytes());
    hip_check(hipStreamCreateWithFlags(&copy_, hipStreamNonBlocking), "hipStreamCreate writeback");
    worker_ = std::thread([this] { run(); });
  }
  ~SealWriteback() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    worker_.join();
    if (copy_) (void)hipStreamDestroy(copy_);
  }
  SealWriteback(const SealWriteback&) = delete;
  SealWriteback& operator=(const SealWriteback&) = delete;

  // Stage pool pages `pages` (sealed by work already on `compute`) and write
  // them to blocks `store_blocks` of `layer`.  Blocks until ring space is free.
  void submit(const PagedKvPool& pool, hipStream_t compute, int64_t layer, const std::vector<int32_t>& pages,
              const std::vector<int64_t>& store_blocks) {
    if (pages.size() != store_blocks.size()) throw std::runtime_error("SealWriteback: page/block count mismatch");
    if (static_cast<int64_t>(pool.page_bytes()) != store_.block_bytes())
      throw std::runtime_error("SealWriteback: pool page and store block sizes differ");
    for (std::size_t off = 0; off < pages.size(); off += static_cast<std::size_t>(cap_)) {
      const int n = static_cast<int>(std::min<std::size_t>(static_cast<std::size_t>(cap_), pages.size() - off));
      const int first = reserve(n);
      Item it;
      it.layer = layer;
      it.first = first;
      it.blocks.assign(store_blocks.begin() + static_cast<std::ptrdiff_t>(off),
                       store_blocks.begin() + static_cast<std::ptrdiff_t>(off + static_cast<std::size_t>(n)));
      hip_check(hipEventCreateWithFlags(&it.after, hipEventDisableTiming), "hipEventCreate");
      hip_check(hipEventCreateWithFlags(&it.done, hipEventDisableTiming), "hipEventCreate");
      hip_check(hipEventRecord(it.after, compute), "hipEventRecord");
      const sa_paged_kv v = pool.view();
      check(sa_hip_pages_to_host_async(v.pool, static_cast<int64_t>(pool.page_bytes()), v.num_pages,
                                       pages.data() + off, n,
                                       staging_->data() + static_cast<std::size_t>(first) * pool.page_bytes(),
                                       copy_, it.after, it.done),
            "pages_to_host_async");
      {
        std::lock_guard<std::mutex> lk(mu_);
        queue_.push_back(std::move(it));
        ++outstanding_;
      }
      cv_.notify_all();
    }
  }

  // Every submitted page written; then the store is fsynced.
  void drain() {
    std::unique_lock<std::mutex> lk(mu_);
    cv_.wait(lk, [&] { return outstanding_ == 0; });
    const std::string err = error_;
    lk.unlock();
    if (!err.empty()) throw std::runtime_error("seal writeback: " + err);
    store_.sync();
  }
  int64_t pages_written() const {
    std::lock_guard<std::mutex> lk(mu_);
    return written_;
  }

 private:
  struct Item {
    int64_t layer{};
    int first{};
    std::vector<int64_t> blocks;
    hipEvent_t after{}, done{};
  };

  int reserve(int n) {
    std::unique_lock<std::mutex> lk(mu_);
    for (;;) {
      const int start = head_ + n <= cap_ ? head_ : 0;
      if (std::all_of(used_.begin() + start, used_.begin() + start + n, [](char u) { return u == 0; })) {
        std::fill(used_.begin() + start, used_.begin() + start + n, 1);
        head_ = start + n == cap_ ? 0 : start + n;
        return start;
      }
      cv_.wait(lk);
    }
  }

  void run() {
    for (;;) {
      Item it;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return stop_ || !queue_.empty(); });
        if (queue_.empty()) return;
        it = std::move(queue_.front());
        queue_.pop_front();
      }
      std::string err;
      if (hipEventSynchronize(it.done) != hipSuccess) {
        err = "staging copy failed";
      } else {
        const int rc = sa_store_write_blocks(store_.get_handle(), it.layer, it.blocks.data(),
                                             static_cast<int32_t>(it.blocks.size()),
                                             staging_->data() + static_cast<std::size_t>(it.first) *
                                                                    static_cast<std::size_t>(store_.block_bytes()));
        if (rc != SA_HIP_OK) err = sa_hip_last_error();
      }
      (void)hipEventDestroy(it.after);
      (void)hipEventDestroy(it.done);
      {
        std::lock_guard<std::mutex> lk(mu_);
        std::fill(used_.begin() + it.first, used_.begin() + it.first + static_cast<int>(it.blocks.size()), 0);
        if (err.empty()) written_ += static_cast<int64_t>(it.blocks.size());
        else if (error_.empty()) error_ = err;
        --outstanding_;
      }
      cv_.notify_all();
    }
  }

  MainStore& store_;
  int cap_;
  std::vector<char> used_;
  int head_ = 0;
  std::unique_ptr<PinnedBuffer> staging_;
  hipStream_t copy_{};
  mutable std::mutex mu_;
  std::condition_variable cv_;
  std::deque<Item> queue_;
  int64_t outstanding_ = 0, written_ = 0;
  std::string error_;
  bool stop_ = false;
  std::thread worker_;
};

// A prefetch is valid for exactly the (token, layer, selection generation,
// block set) it was issued for (pipeline_main.cpp:425-437).
struct PrefetchTicket {
  int64_t token{};
  int64_t layer{};
  int64_t generation{};
  std::vector<int32_t> blocks;
};

inline bool valid_ticket(const PrefetchTicket& t, int64_t token, int64_t layer, int64_t generation,
                         const std::vector<int32_t>& blocks) {
  return t.token == token && t.layer == layer && t.generation == generation && t.blocks == blocks;
}

// Reads a layer's predicted blocks from the store into pinned staging and
// copies them into pool pages on a copy stream, one prefetch outstanding at
// a time (the reference's one outstanding io_uring batch,
// uring_reader.cpp:97-99).  acquire() checks the ticket and orders the
// compute stream after the copies on the device.
class StorePrefetcher {
 public:
  StorePrefetcher(MainStore& store, int max_blocks) : store_(store), max_blocks_(max_blocks) {
    if (max_blocks < 1) throw std::runtime_error("StorePrefetcher: max_blocks must be positive");
    for (auto& b : staging_)
      b = std::make_unique<PinnedBuffer>(static_cast<std::size_t>(max_blocks) * store.block_bytes());
    hip_check(hipStreamCreateWithFlags(&copy_, hipStreamNonBlocking), "hipStreamCreate prefetch");
    for (auto& e : done_) hip_check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
    for (auto& e : after_) hip_check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
    worker_ = std::thread([this] { run(); });
  }
  ~StorePrefetcher() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    worker_.join();
    (void)hipStreamSynchronize(copy_);
    for (auto& e : done_) (void)hipEventDestroy(e);
    for (auto& e : after_) (void)hipEventDestroy(e);
    if (copy_) (void)hipStreamDestroy(copy_);
  }
  StorePrefetcher(const StorePrefetcher&) = delete;
  StorePrefetcher& operator=(const StorePrefetcher&) = delete;

  // Start reading ticket.blocks of ticket.layer; their bytes go to pool pages
  // dst_pages (same order) once the work queued so far on `after` (the last
  // readers of those pages) is done.  Returns at once.
  void submit(const PrefetchTicket& ticket, const PagedKvPool& pool, const std::vector<int32_t>& dst_pages,
              hipStream_t after) {
    if (ticket.blocks.size() != dst_pages.size() || ticket.blocks.empty() ||
        static_cast<int>(ticket.blocks.size()) > max_blocks_)
      throw std::runtime_error("StorePrefetcher: bad block list");
    if (static_cast<int64_t>(pool.page_bytes()) != store_.block_bytes())
      throw std::runtime_error("StorePrefetcher: pool page and store block sizes differ");
    std::lock_guard<std::mutex> lk(mu_);
    if (pending_) throw std::runtime_error("StorePrefetcher: a prefetch is already outstanding");
    slot_ ^= 1;
    hip_check(hipEventRecord(after_[slot_], after), "hipEventRecord");
    job_ = Job{ticket, dst_pages, pool.view().pool, static_cast<int64_t>(pool.page_bytes()), slot_};
    pending_ = true;
    ready_ = false;
    cv_.notify_all();
  }

  // The layer about to run uses `blocks` of `layer` at (token, generation):
  // throws unless the outstanding prefetch was issued for exactly that;
  // otherwise `compute` waits (on the device) for the copies.
  void acquire(int64_t token, int64_t layer, int64_t generation, const std::vector<int32_t>& blocks,
               hipStream_t compute) {
    std::unique_lock<std::mutex> lk(mu_);
    if (!pending_) {
      ++rejected_;
      throw std::runtime_error("stale or misrouted prefetch ticket: none outstanding");
    }
    cv_.wait(lk, [&] { return ready_; });
    if (!error_.empty()) {
      const std::string e = error_;
      error_.clear();
      pending_ = false;
      throw std::runtime_error("prefetch: " + e);
    }
    if (!valid_ticket(job_.ticket, token, layer, generation, blocks)) {
      ++rejected_;
      throw std::runtime_error("stale or misrouted prefetch ticket");
    }
    pending_ = false;
    ++verified_;
    check(sa_hip_stream_wait_event(compute, done_[job_.slot]), "stream_wait_event");
  }
  // Drop an outstanding prefetch without using it (after a rejected ticket).
  void discard() {
    std::unique_lock<std::mutex> lk(mu_);
    if (!pending_) return;
    cv_.wait(lk, [&] { return ready_; });
    pending_ = false;
    error_.clear();
  }
  int64_t verified() const {
    std::lock_guard<std::mutex> lk(mu_);
    return verified_;
  }
  int64_t rejected() const {
    std::lock_guard<std::mutex> lk(mu_);
    return rejected_;
  }

 private:
  struct Job {
    PrefetchTicket ticket;
    std::vector<int32_t> dst_pages;
    std::uint16_t* pool{};
    int64_t page_bytes{};
    int slot{};
  };

  void run() {
    for (;;) {
      Job job;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return stop_ || (pending_ && !ready_ && !taken_); });
        if (stop_) return;
        job = job_;
        taken_ = true;
      }
      std::string err;
      // the staging buffer's previous copies must have landed before reuse
      if (hipEventSynchronize(done_[job.slot]) != hipSuccess) err = "previous staging copy failed";
      const std::vector<int64_t> blocks(job.ticket.blocks.begin(), job.ticket.blocks.end());
      if (err.empty() && sa_store_read_blocks(store_.get_handle(), job.ticket.layer, blocks.data(),
                                              static_cast<int32_t>(blocks.size()), staging_[job.slot]->data()) !=
                             SA_HIP_OK)
        err = sa_hip_last_error();
      if (err.empty() && hipStreamWaitEvent(copy_, after_[job.slot], 0) != hipSuccess)
        err = "hipStreamWaitEvent before the page copies failed";
      if (err.empty()) {
        std::vector<int64_t> src(blocks.size());
        for (std::size_t i = 0; i < src.size(); ++i) src[i] = static_cast<int64_t>(i);
        if (sa_hip_fill_pages_async(job.pool, job.page_bytes, job.dst_pages.data(), staging_[job.slot]->data(),
                                    src.data(), static_cast<int32_t>(src.size()), copy_, done_[job.slot]) !=
            SA_HIP_OK)
          err = sa_hip_last_error();
      }
      {
        std::lock_guard<std::mutex> lk(mu_);
        error_ = err;
        ready_ = true;
        taken_ = false;
      }
      cv_.notify_all();
    }
  }

  MainStore& store_;
  int max_blocks_;
  std::unique_ptr<PinnedBuffer> staging_[2];
  hipEvent_t done_[2]{};
  hipEvent_t after_[2]{};
  hipStream_t copy_{};
  mutable std::mutex mu_;
  std::condition_variable cv_;
  Job job_;
  int slot_ = 1;
  bool pending_ = false, ready_ = false, taken_ = false, stop_ = false;
  std::string error_;
  int64_t verified_ = 0, rejected_ = 0;
  std::thread worker_;
};

}  // namespace solidattention::hip
