// Multi-threaded host memcpy for the pinned-staging weight store.
//
// The reference stages every transfer unit from the pageable arena into a
// page-locked slot with one tensor copy on a worker thread
// (layer_streaming/weight_store.py:258-268; vocab.py:143-147 on the main
// thread), which its own measurements put at ~14.8 GB/s single-threaded
// (IMPLEMENTATION_REPORT.md:61-67) -- below the H2D link it feeds.  Here one
// call splits the copy into 2 MiB pieces that a persistent pool of threads
// and the caller take from a shared counter; each piece is copied with
// 32-byte loads and non-temporal 32-byte stores (the staging slot is read
// next by the DMA engine, not by this CPU, so caching it only evicts the
// arena stream), then the call returns once every piece is written.
//
// Concurrent callers are serialised: each call already uses every pool
// thread.  Pure host code; no HIP call is made.
#include <immintrin.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <mutex>
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

class CopyPool {
 public:
  static CopyPool &instance() {
    static CopyPool pool;
    return pool;
  }

  int copy(void *dst, const void *src, size_t bytes, int threads) {
    std::lock_guard<std::mutex> call(call_mutex_);
    const size_t pieces = (bytes + kPiece - 1) / kPiece;
    const int helpers = static_cast<int>(
        std::min<size_t>(std::max(threads, 1) - 1, pieces ? pieces - 1 : 0));
    ensure_threads(helpers);
    {
      std::lock_guard<std::mutex> lock(mutex_);
      dst_ = static_cast<char *>(dst);
      src_ = static_cast<const char *>(src);
      bytes_ = bytes;
      pieces_ = pieces;
      next_.store(0, std::memory_order_relaxed);
      active_ = helpers;
      pending_ = helpers;
      ++generation_;
    }
    wake_.notify_all();
    run_pieces();
    std::unique_lock<std::mutex> lock(mutex_);
    done_.wait(lock, [this] { return pending_ == 0; });
    return 0;
  }

  int thread_count() {
    std::lock_guard<std::mutex> lock(mutex_);
    return static_cast<int>(workers_.size());
  }

 private:
  CopyPool() : avx2_(__builtin_cpu_supports("avx2")) {}

  ~CopyPool() {
    {
      std::lock_guard<std::mutex> lock(mutex_);
      stop_ = true;
    }
    wake_.notify_all();
    for (auto &t : workers_) t.join();
  }

  void ensure_threads(int n) {
    std::lock_guard<std::mutex> lock(mutex_);
    while (static_cast<int>(workers_.size()) < n) {
      const int id = static_cast<int>(workers_.size());
      workers_.emplace_back([this, id] { worker(id); });
    }
  }

  void run_pieces() {
    for (;;) {
      const size_t p = next_.fetch_add(1, std::memory_order_relaxed);
      if (p >= pieces_) return;
      const size_t off = p * kPiece;
      copy_piece(dst_ + off, src_ + off, std::min(kPiece, bytes_ - off), avx2_);
    }
  }

  void worker(int id) {
    uint64_t seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> lock(mutex_);
        wake_.wait(lock, [&] { return stop_ || (generation_ != seen && id < active_); });
        if (stop_) return;
        seen = generation_;
      }
      run_pieces();
      std::lock_guard<std::mutex> lock(mutex_);
      if (--pending_ == 0) done_.notify_all();
    }
  }

  const bool avx2_;
  std::mutex call_mutex_;
  std::mutex mutex_;
  std::condition_variable wake_;
  std::condition_variable done_;
  std::vector<std::thread> workers_;
  uint64_t generation_ = 0;
  bool stop_ = false;
  int active_ = 0;
  int pending_ = 0;
  char *dst_ = nullptr;
  const char *src_ = nullptr;
  size_t bytes_ = 0;
  size_t pieces_ = 0;
  std::atomic<size_t> next_{0};
};

}  // namespace

extern "C" int cascade_host_copy(void *dst, const void *src, size_t bytes,
                                 int threads) {
  if (bytes == 0) return 0;
  if (dst == nullptr || src == nullptr) return CASCADE_EINVAL;
  if (threads < 1 || threads > kMaxThreads) return CASCADE_EINVAL;
  const char *d = static_cast<const char *>(dst);
  const char *s = static_cast<const char *>(src);
  if (d < s + bytes && s < d + bytes) return CASCADE_EINVAL;  // overlap
  return CopyPool::instance().copy(dst, src, bytes, threads);
}
