// store.cpp — the main KV store on local disk (include/sa_store.h): block
// reads and writes at the reference's per-layer segment offsets
// (cpp/src/kv_lifecycle_main.cpp:73-80, 105-108; cpp/src/pipeline_main.cpp
// :660-678), O_DIRECT where the file system allows it, a pool of worker
// threads so that a batch of blocks is in flight at once, and the
// crash-consistent commit marker of cpp/src/online_seal_main.cpp:59-70.
// Host code only.
#include "sa_store.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <atomic>
#include <cerrno>
#include <condition_variable>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "sa_hip.h"

namespace sa {
int report_error(int code, const char* message);
}

namespace {

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return sa::report_error(code, buf);
}

constexpr int64_t kDirectAlign = 4096;

// Full-length pread / pwrite (retries short transfers and EINTR).
int64_t transfer(int fd, bool write, char* ptr, int64_t bytes, int64_t offset) {
  int64_t done = 0;
  while (done < bytes) {
    const ssize_t r = write ? ::pwrite(fd, ptr + done, static_cast<size_t>(bytes - done), offset + done)
                            : ::pread(fd, ptr + done, static_cast<size_t>(bytes - done), offset + done);
    if (r < 0) {
      if (errno == EINTR) continue;
      return -errno;
    }
    if (r == 0) return done;  // end of file
    done += r;
  }
  return done;
}

struct Job {
  bool write;
  int64_t offset;
  char* ptr;
  int64_t batch;
};

struct Batch {
  int64_t pending = 0;
  int error = 0;
  std::string message;
};

}  // namespace

struct sa_store {
  int fd = -1;
  bool direct = false;
  int64_t layers = 0, blocks_per_layer = 0, block_bytes = 0;
  std::string path;

  std::mutex mu;
  std::condition_variable work_cv, done_cv;
  std::deque<Job> jobs;
  std::map<int64_t, Batch> batches;  // iterators stay valid while other batches come and go
  int64_t next_batch = 1;
  bool stop = false;
  std::atomic<int64_t> bounced{0};
  std::vector<std::thread> workers;

  void run() {
    for (;;) {
      Job job;
      {
        std::unique_lock<std::mutex> lk(mu);
        work_cv.wait(lk, [&] { return stop || !jobs.empty(); });
        if (jobs.empty()) return;
        job = jobs.front();
        jobs.pop_front();
      }
      int64_t r;
      if (direct && reinterpret_cast<uintptr_t>(job.ptr) % kDirectAlign != 0) {
        r = bounced_transfer(job);
      } else {
        r = transfer(fd, job.write, job.ptr, block_bytes, job.offset);
        if (r == -EFAULT && direct) r = bounced_transfer(job);
      }
      std::lock_guard<std::mutex> lk(mu);
      Batch& b = batches[job.batch];
      if (r != block_bytes && b.error == 0) {
        b.error = SA_HIP_EIO;
        char buf[256];
        if (r < 0)
          snprintf(buf, sizeof buf, "store %s at byte %lld: %s", job.write ? "write" : "read",
                   static_cast<long long>(job.offset), std::strerror(static_cast<int>(-r)));
        else
          snprintf(buf, sizeof buf, "store %s at byte %lld: short transfer (%lld of %lld bytes)",
                   job.write ? "write" : "read", static_cast<long long>(job.offset), static_cast<long long>(r),
                   static_cast<long long>(block_bytes));
        b.message = buf;
      }
      if (--b.pending == 0) done_cv.notify_all();
    }
  }

  // O_DIRECT needs 4096-byte aligned buffers and cannot pin memory that the
  // GPU driver mapped into the process (hipHostMalloc buffers: EFAULT); such
  // blocks go through a page-aligned bounce buffer of the worker thread.
  int64_t bounced_transfer(const Job& job) {
    thread_local std::unique_ptr<char, void (*)(void*)> bounce(nullptr, std::free);
    thread_local int64_t bounce_bytes = 0;
    if (bounce_bytes < block_bytes) {
      void* p = nullptr;
      if (posix_memalign(&p, kDirectAlign, static_cast<size_t>(block_bytes)) != 0) return -ENOMEM;
      bounce.reset(static_cast<char*>(p));
      bounce_bytes = block_bytes;
    }
    if (job.write) std::memcpy(bounce.get(), job.ptr, static_cast<size_t>(block_bytes));
    const int64_t r = transfer(fd, job.write, bounce.get(), block_bytes, job.offset);
    if (!job.write && r == block_bytes) std::memcpy(job.ptr, bounce.get(), static_cast<size_t>(block_bytes));
    bounced.fetch_add(1, std::memory_order_relaxed);
    return r;
  }

  int64_t submit(bool write, int64_t layer, const int64_t* blocks, int32_t count, char* base) {
    const char* op = write ? "store_submit_writes" : "store_submit_reads";
    if (count < 0 || (count > 0 && (!blocks || !base))) return fail(SA_HIP_EINVAL, "%s: bad arguments", op);
    if (layer < 0 || layer >= layers)
      return fail(SA_HIP_EINVAL, "%s: layer %lld outside [0, %lld)", op, static_cast<long long>(layer),
                  static_cast<long long>(layers));
    for (int32_t i = 0; i < count; ++i)
      if (blocks[i] < 0 || blocks[i] >= blocks_per_layer)
        return fail(SA_HIP_EINVAL, "%s: block %lld outside [0, %lld)", op, static_cast<long long>(blocks[i]),
                    static_cast<long long>(blocks_per_layer));
    std::lock_guard<std::mutex> lk(mu);
    const int64_t id = next_batch++;
    Batch& b = batches[id];
    b.pending = count;
    for (int32_t i = 0; i < count; ++i)
      jobs.push_back(Job{write, (layer * blocks_per_layer + blocks[i]) * block_bytes, base + i * block_bytes, id});
    work_cv.notify_all();
    return id;
  }

  int wait(int64_t id) {
    std::unique_lock<std::mutex> lk(mu);
    auto it = batches.find(id);
    if (it == batches.end()) return fail(SA_HIP_EINVAL, "store_wait: unknown batch %lld", static_cast<long long>(id));
    done_cv.wait(lk, [&] { return it->second.pending == 0; });
    const int err = it->second.error;
    const std::string msg = it->second.message;
    batches.erase(it);
    lk.unlock();
    if (err) return fail(err, "%s", msg.c_str());
    return SA_HIP_OK;
  }
};

extern "C" {

sa_store* sa_store_open(const char* path, int64_t layers, int64_t blocks_per_layer, int64_t block_bytes,
                        int32_t flags, int32_t threads) {
  if (!path || layers <= 0 || blocks_per_layer <= 0 || block_bytes <= 0 || threads < 1 || threads > 64) {
    fail(SA_HIP_EINVAL, "store_open: bad arguments");
    return nullptr;
  }
  const bool want_direct = (flags & SA_STORE_DIRECT) != 0;
  if (want_direct && block_bytes % kDirectAlign != 0) {
    fail(SA_HIP_EINVAL, "store_open: O_DIRECT needs block_bytes to be a multiple of 4096");
    return nullptr;
  }
  int oflags = O_RDWR;
  if (flags & SA_STORE_CREATE) oflags |= O_CREAT | O_TRUNC;
  int fd = -1;
  bool direct = false;
  if (want_direct) {
    fd = ::open(path, oflags | O_DIRECT, 0644);
    direct = fd >= 0;
    if (fd < 0 && errno != EINVAL) {
      fail(SA_HIP_EIO, "store_open %s: %s", path, std::strerror(errno));
      return nullptr;
    }
  }
  if (fd < 0) fd = ::open(path, oflags, 0644);  // file systems without O_DIRECT (tmpfs)
  if (fd < 0) {
    fail(SA_HIP_EIO, "store_open %s: %s", path, std::strerror(errno));
    return nullptr;
  }
  const int64_t total = layers * blocks_per_layer * block_bytes;
  if (flags & SA_STORE_CREATE) {
    const int r = ::posix_fallocate(fd, 0, total);
    if (r != 0 && ::ftruncate(fd, total) != 0) {
      fail(SA_HIP_EIO, "store_open %s: cannot reserve %lld bytes: %s", path, static_cast<long long>(total),
           std::strerror(r));
      ::close(fd);
      return nullptr;
    }
  }
  auto* s = new sa_store;
  s->fd = fd;
  s->direct = direct;
  s->layers = layers;
  s->blocks_per_layer = blocks_per_layer;
  s->block_bytes = block_bytes;
  s->path = path;
  for (int i = 0; i < threads; ++i) s->workers.emplace_back([s] { s->run(); });
  return s;
}

void sa_store_close(sa_store* s) {
  if (!s) return;
  {
    std::lock_guard<std::mutex> lk(s->mu);
    s->stop = true;
  }
  s->work_cv.notify_all();
  for (auto& t : s->workers) t.join();
  if (s->fd >= 0) ::close(s->fd);
  delete s;
}

int sa_store_is_direct(const sa_store* s) { return s && s->direct ? 1 : 0; }

int64_t sa_store_bytes(const sa_store* s) { return s ? s->layers * s->blocks_per_layer * s->block_bytes : 0; }

int64_t sa_store_bounced(const sa_store* s) { return s ? s->bounced.load() : 0; }

int64_t sa_store_submit_reads(sa_store* s, int64_t layer, const int64_t* blocks, int32_t count, void* dst) {
  if (!s) return fail(SA_HIP_EINVAL, "store_submit_reads: null store");
  return s->submit(false, layer, blocks, count, static_cast<char*>(dst));
}

int64_t sa_store_submit_writes(sa_store* s, int64_t layer, const int64_t* blocks, int32_t count, const void* src) {
  if (!s) return fail(SA_HIP_EINVAL, "store_submit_writes: null store");
  // the workers only read from src
  return s->submit(true, layer, blocks, count, const_cast<char*>(static_cast<const char*>(src)));
}

int sa_store_wait(sa_store* s, int64_t batch) {
  if (!s) return fail(SA_HIP_EINVAL, "store_wait: null store");
  return s->wait(batch);
}

int sa_store_read_blocks(sa_store* s, int64_t layer, const int64_t* blocks, int32_t count, void* dst) {
  const int64_t id = sa_store_submit_reads(s, layer, blocks, count, dst);
  return id < 0 ? static_cast<int>(id) : sa_store_wait(s, id);
}

int sa_store_write_blocks(sa_store* s, int64_t layer, const int64_t* blocks, int32_t count, const void* src) {
  const int64_t id = sa_store_submit_writes(s, layer, blocks, count, src);
  return id < 0 ? static_cast<int>(id) : sa_store_wait(s, id);
}

int sa_store_sync(sa_store* s) {
  if (!s) return fail(SA_HIP_EINVAL, "store_sync: null store");
  if (::fsync(s->fd) != 0) return fail(SA_HIP_EIO, "store_sync %s: %s", s->path.c_str(), std::strerror(errno));
  return SA_HIP_OK;
}

int sa_store_commit_marker(const char* directory, const char* name, const char* body) {
  if (!directory || !name || !body || !*name || std::strchr(name, '/'))
    return fail(SA_HIP_EINVAL, "store_commit_marker: bad arguments");
  const std::string dir = directory;
  const std::string final_path = dir + "/" + name;
  const std::string tmp_path = final_path + ".tmp";
  const int fd = ::open(tmp_path.c_str(), O_CREAT | O_TRUNC | O_WRONLY, 0644);
  if (fd < 0) return fail(SA_HIP_EIO, "commit marker %s: %s", tmp_path.c_str(), std::strerror(errno));
  const int64_t n = static_cast<int64_t>(std::strlen(body));
  const int64_t w = transfer(fd, true, const_cast<char*>(body), n, 0);
  if (w != n || ::fsync(fd) != 0) {
    const int e = errno;
    ::close(fd);
    return fail(SA_HIP_EIO, "commit marker %s: write/fsync failed: %s", tmp_path.c_str(), std::strerror(e));
  }
  ::close(fd);
  if (::rename(tmp_path.c_str(), final_path.c_str()) != 0)
    return fail(SA_HIP_EIO, "commit marker rename onto %s: %s", final_path.c_str(), std::strerror(errno));
  const int dfd = ::open(directory, O_RDONLY | O_DIRECTORY);
  if (dfd < 0) return fail(SA_HIP_EIO, "commit marker directory %s: %s", directory, std::strerror(errno));
  const int r = ::fsync(dfd);
  ::close(dfd);
  if (r != 0) return fail(SA_HIP_EIO, "commit marker directory fsync %s: %s", directory, std::strerror(errno));
  return SA_HIP_OK;
}

}  // extern "C"
