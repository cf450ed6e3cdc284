// Multi-threaded host memcpy for the pinned-staging weight store.
//
// The reference stages every transfer unit from the pageable arena into a
// page-locked slot with one tensor copy on a worker thread
// (layer_streaming/weight_store.py:258-268; vocab.py:143-147 on the main
// thread), which its own measurements put at ~14.8 GB/s single-threaded
// (IMPLEMENTATION_REPORT.md:61-67) -- below the H2D link it feeds.  Here one
// copy is split into 2 MiB pieces that several threads take from a shared
// counter; each piece is copied with 32-byte loads and non-temporal 32-byte
// stores (the staging slot is read next by the DMA engine, not by this CPU,
// so caching it only evicts the arena stream), and the call returns once
// every piece is written.
//
// The library keeps no thread or state of its own between calls:
// cascade_host_copy starts its helper threads for the one call, and a
// caller that copies often (the staging store, once per transfer unit)
// creates a pool with cascade_copy_pool_create, owns it, and destroys it.
// Pure host code; no HIP call is made.
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <mutex>
#include <system_error>
#include <thread>
#include <vector>

#include "../../include/cascade_hip.h"

namespace {

constexpr size_t kPiece = size_t{2} << 20;
constexpr int kMaxThreads = 64;

__attribute__((target("avx2"))) void stream_copy_avx2(char *dst,
                                                       const char *src,
                                                       size_t bytes) {
  // head: bring dst to a 32-byte boundary
  const size_t head =
      std::min(bytes, (32 - (reinterpret_cast<uintptr_t>(dst) & 31)) & 31);
  memcpy(dst, src, head);
  dst += head;
  src += head;
  bytes -= head;
  size_t i = 0;
  for (; i + 128 <= bytes; i += 128) {
    const __m256i a = _mm256_loadu_si256(reinterpret_cast<const __m256i *>(src + i));
    const __m256i b =
        _mm256_loadu_si256(reinterpret_cast<const __m256i *>(src + i + 32));
    const __m256i c =
        _mm256_loadu_si256(reinterpret_cast<const __m256i *>(src + i + 64));
    const __m256i d =
        _mm256_loadu_si256(reinterpret_cast<const __m256i *>(src + i + 96));
    _mm256_stream_si256(reinterpret_cast<__m256i *>(dst + i), a);
    _mm256_stream_si256(reinterpret_cast<__m256i *>(dst + i + 32), b);
    _mm256_stream_si256(reinterpret_cast<__m256i *>(dst + i + 64), c);
    _mm256_stream_si256(reinterpret_cast<__m256i *>(dst + i + 96), d);
  }
  memcpy(dst + i, src + i, bytes - i);
  _mm_sfence();
}

void copy_piece(char *dst, const char *src, size_t bytes, bool avx2) {
  if (avx2)
    stream_copy_avx2(dst, src, bytes);
  else
    memcpy(dst, src, bytes);
}

// One copy split into pieces that several threads take from a counter.
struct CopyJob {
  char *dst;
  const char *src;
  size_t bytes;
  size_t pieces;
  bool avx2;
  std::atomic<size_t> next{0};

  CopyJob(void *d, const void *s, size_t n, bool use_avx2)
      : dst(static_cast<char *>(d)),
        src(static_cast<const char *>(s)),
        bytes(n),
        pieces((n + kPiece - 1) / kPiece),
        avx2(use_avx2) {}

  void run() {
    for (;;) {
      const size_t p = next.fetch_add(1, std::memory_order_relaxed);
      if (p >= pieces) return;
      const size_t off = p * kPiece;
      copy_piece(dst + off, src + off, std::min(kPiece, bytes - off), avx2);
    }
  }
};

bool cpu_has_avx2() {
  static const bool avx2 = __builtin_cpu_supports("avx2");
  return avx2;
}

// CPUs of NUMA node `node` that this process may run on, from sysfs
// ("0-15,32-47").  Returns false when the node does not exist.
bool node_cpus(int node, std::vector<int> *cpus) {
  char path[96];
  snprintf(path, sizeof path, "/sys/devices/system/node/node%d/cpulist", node);
  FILE *f = fopen(path, "r");
  if (f == nullptr) return false;
  char line[4096] = {0};
  const bool read = fgets(line, sizeof line, f) != nullptr;
  fclose(f);
  if (!read) return false;
  cpu_set_t allowed;
  CPU_ZERO(&allowed);
  if (sched_getaffinity(0, sizeof allowed, &allowed) != 0) return false;
  // "a" or "a-b" ranges separated by commas, parsed with strtol over a
  // local cursor (no hidden parser state: pools may be created from
  // several threads at once)
  const char *p = line;
  while (*p != '\0' && *p != '\n') {
    char *end = nullptr;
    const long lo = strtol(p, &end, 10);
    if (end == p) break;  // not a number: malformed list, keep what we have
    long hi = lo;
    p = end;
    if (*p == '-') {
      hi = strtol(p + 1, &end, 10);
      if (end == p + 1) break;
      p = end;
    }
    for (long c = lo < 0 ? 0 : lo; c <= hi && c < CPU_SETSIZE; ++c)
      if (CPU_ISSET(static_cast<int>(c), &allowed)) cpus->push_back(static_cast<int>(c));
    if (*p == ',') ++p;
  }
  return true;
}

// A pool of helper threads owned by whoever created it (the staging store
// holds one for its lifetime).  A copy is split between the helpers and
// the calling thread; concurrent copies on one pool run one after another,
// since each already uses every helper.  Helpers may be bound to the CPUs
// of one NUMA node (the GPU's, so the copies read and write memory near
// the PCIe root the DMA engine reads the staging slots through).
class CopyPool {
 public:
  CopyPool(int helpers, const std::vector<int> &cpus) : bound_cpus_(0) {
    cpu_set_t set;
    CPU_ZERO(&set);
    for (int c : cpus) CPU_SET(c, &set);
    try {
      for (int id = 0; id < helpers; ++id) {
        workers_.emplace_back([this, id] { worker(id); });
        if (!cpus.empty() &&
            pthread_setaffinity_np(workers_.back().native_handle(), sizeof set,
                                   &set) == 0)
          bound_cpus_ = static_cast<int>(cpus.size());
      }
    } catch (...) {
      stop_workers();  // the threads already started end before the throw
      throw;
    }
  }

  ~CopyPool() { stop_workers(); }

  int copy(void *dst, const void *src, size_t bytes) {
    std::lock_guard<std::mutex> call(call_mutex_);
    CopyJob job(dst, src, bytes, cpu_has_avx2());
    const int helpers = static_cast<int>(std::min<size_t>(
        workers_.size(), job.pieces ? job.pieces - 1 : 0));
    {
      std::lock_guard<std::mutex> lock(mutex_);
      job_ = &job;
      active_ = helpers;
      pending_ = helpers;
      ++generation_;
    }
    wake_.notify_all();
    job.run();
    std::unique_lock<std::mutex> lock(mutex_);
    done_.wait(lock, [this] { return pending_ == 0; });
    job_ = nullptr;
    return 0;
  }

  int threads() const { return static_cast<int>(workers_.size()) + 1; }
  int bound_cpus() const { return bound_cpus_; }

 private:
  void stop_workers() {
    {
      std::lock_guard<std::mutex> lock(mutex_);
      stop_ = true;
    }
    wake_.notify_all();
    for (auto &t : workers_) t.join();
  }

  void worker(int id) {
    uint64_t seen = 0;
    for (;;) {
      CopyJob *job = nullptr;
      {
        std::unique_lock<std::mutex> lock(mutex_);
        wake_.wait(lock, [&] {
          return stop_ || (generation_ != seen && id < active_);
        });
        if (stop_) return;
        seen = generation_;
        job = job_;
      }
      job->run();
      std::lock_guard<std::mutex> lock(mutex_);
      if (--pending_ == 0) done_.notify_all();
    }
  }

  int bound_cpus_;
  std::mutex call_mutex_;
  std::mutex mutex_;
  std::condition_variable wake_;
  std::condition_variable done_;
  std::vector<std::thread> workers_;
  CopyJob *job_ = nullptr;
  uint64_t generation_ = 0;
  bool stop_ = false;
  int active_ = 0;
  int pending_ = 0;
};

int check_copy(const void *dst, const void *src, size_t bytes) {
  if (dst == nullptr || src == nullptr) return CASCADE_EINVAL;
  const char *d = static_cast<const char *>(dst);
  const char *s = static_cast<const char *>(src);
  if (d < s + bytes && s < d + bytes) return CASCADE_EINVAL;  // overlap
  return 0;
}

}  // namespace

extern "C" int cascade_host_copy(void *dst, const void *src, size_t bytes,
                                 int threads) {
  if (bytes == 0) return 0;
  if (threads < 1 || threads > kMaxThreads) return CASCADE_EINVAL;
  if (const int e = check_copy(dst, src, bytes)) return e;
  // helper threads live for this call only
  CopyJob job(dst, src, bytes, cpu_has_avx2());
  const size_t helpers =
      std::min<size_t>(static_cast<size_t>(threads) - 1, job.pieces - 1);
  std::vector<std::thread> workers;
  try {
    for (size_t i = 0; i < helpers; ++i) workers.emplace_back([&job] { job.run(); });
  } catch (const std::system_error &) {
    // fewer helpers than asked: the threads started so far and the caller
    // still finish every piece
  }
  job.run();
  for (auto &t : workers) t.join();
  return 0;
}

extern "C" int cascade_copy_pool_create(int threads, int numa_node,
                                        uint64_t *pool) {
  if (pool == nullptr) return CASCADE_EINVAL;
  *pool = 0;
  if (threads < 1 || threads > kMaxThreads || numa_node < -1)
    return CASCADE_EINVAL;
  std::vector<int> cpus;
  if (numa_node >= 0 && !node_cpus(numa_node, &cpus)) return CASCADE_EINVAL;
  try {
    *pool = reinterpret_cast<uint64_t>(new CopyPool(threads - 1, cpus));
  } catch (const std::exception &) {
    return CASCADE_EINVAL;
  }
  return 0;
}

extern "C" int cascade_copy_pool_copy(uint64_t pool, void *dst,
                                      const void *src, size_t bytes) {
  if (pool == 0) return CASCADE_EINVAL;
  if (bytes == 0) return 0;
  if (const int e = check_copy(dst, src, bytes)) return e;
  return reinterpret_cast<CopyPool *>(pool)->copy(dst, src, bytes);
}

extern "C" int cascade_copy_pool_info(uint64_t pool, int *threads,
                                      int *bound_cpus) {
  if (pool == 0 || threads == nullptr || bound_cpus == nullptr)
    return CASCADE_EINVAL;
  const CopyPool *p = reinterpret_cast<CopyPool *>(pool);
  *threads = p->threads();
  *bound_cpus = p->bound_cpus();
  return 0;
}

extern "C" int cascade_copy_pool_destroy(uint64_t pool) {
  if (pool == 0) return CASCADE_EINVAL;
  delete reinterpret_cast<CopyPool *>(pool);
  return 0;
}
