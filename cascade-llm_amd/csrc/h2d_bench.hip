// h2d_bench: host->device copy bandwidth on one GPU (MI355X).
//
// The HIP counterpart of the reference's CUDA driver-API microbenchmark
// (h2d_driver_bench.c:720-958): it defines "achievable H2D", the
// denominator of the streamed-decode roofline.
//   * page-locked (hipHostMalloc) vs pageable (malloc) sources,
//     async (hipMemcpyAsync on a stream) vs sync (hipMemcpy);
//   * sizes from 4 KiB to --max-mib, plus the transfer units of the 8B plan
//     (48 / 32 / 224 / 112 MiB matrix groups, 128 MiB vocab chunk);
//   * pinned async copies also split over 2 and 4 streams (several DMA
//     engines at once);
//   * per size: --repeats event-timed copies after one warm-up,
//     p10 / median / p90 GB/s (1 GB = 1e9 bytes);
//   * host enqueue cost: least-squares slope of host time over batches of
//     1..1024 small async copies (h2d_driver_bench.c:472-648).
// Output: one JSON object on stdout.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#define CHECK(x)                                                          \
  do {                                                                    \
    hipError_t e_ = (x);                                                  \
    if (e_ != hipSuccess) {                                               \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x,      \
                   hipGetErrorString(e_));                                \
      std::exit(2);                                                       \
    }                                                                     \
  } while (0)

namespace {

struct Stats {
  double p10, median, p90;
};

Stats percentiles(std::vector<double> v) {
  std::sort(v.begin(), v.end());
  auto at = [&](double q) {
    const double pos = q * (v.size() - 1);
    const size_t lo = static_cast<size_t>(pos);
    const size_t hi = std::min(lo + 1, v.size() - 1);
    return v[lo] + (v[hi] - v[lo]) * (pos - lo);
  };
  return {at(0.1), at(0.5), at(0.9)};
}

double now_s() {
  using clock = std::chrono::steady_clock;
  return std::chrono::duration<double>(clock::now().time_since_epoch()).count();
}

// GB/s samples of `repeats` copies of `bytes`.
std::vector<double> time_copies(void *dst, void *src, size_t bytes, bool async,
                                int repeats, hipStream_t stream) {
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  std::vector<double> out;
  for (int r = -1; r < repeats; ++r) {
    float ms = 0.0f;
    if (async) {
      CHECK(hipEventRecord(a, stream));
      CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream));
      CHECK(hipEventRecord(b, stream));
      CHECK(hipEventSynchronize(b));
      CHECK(hipEventElapsedTime(&ms, a, b));
    } else {
      const double t0 = now_s();
      CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
      ms = static_cast<float>((now_s() - t0) * 1e3);
    }
    if (r >= 0) out.push_back(bytes / 1e9 / (ms / 1e3));
  }
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  return out;
}

// GB/s samples of `repeats` copies of `bytes`, each split into equal
// pieces on the `streams` given (one piece per stream; pieces 4 KiB
// aligned): stream 0 records the start, the others wait for it, and stream
// 0 waits for every piece before recording the end.
std::vector<double> time_split_copies(char *dst, const char *src, size_t bytes,
                                      int repeats,
                                      const std::vector<hipStream_t> &streams) {
  const size_t n = streams.size();
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  std::vector<hipEvent_t> done(n);
  for (auto &e : done) CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  const size_t piece = (bytes / n + 4095) / 4096 * 4096;
  std::vector<double> out;
  for (int r = -1; r < repeats; ++r) {
    CHECK(hipEventRecord(a, streams[0]));
    for (size_t i = 0; i < n; ++i) {
      const size_t off = std::min(bytes, i * piece);
      const size_t len = std::min(bytes - off, piece);
      if (i) CHECK(hipStreamWaitEvent(streams[i], a, 0));
      if (len)
        CHECK(hipMemcpyAsync(dst + off, src + off, len, hipMemcpyHostToDevice,
                             streams[i]));
      CHECK(hipEventRecord(done[i], streams[i]));
    }
    for (size_t i = 1; i < n; ++i) CHECK(hipStreamWaitEvent(streams[0], done[i], 0));
    CHECK(hipEventRecord(b, streams[0]));
    CHECK(hipEventSynchronize(b));
    float ms = 0.0f;
    CHECK(hipEventElapsedTime(&ms, a, b));
    if (r >= 0) out.push_back(bytes / 1e9 / (ms / 1e3));
  }
  for (auto &e : done) CHECK(hipEventDestroy(e));
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  return out;
}

}  // namespace

int main(int argc, char **argv) {
  int repeats = 7;
  size_t max_mib = 512;
  bool pageable = true;
  for (int i = 1; i < argc; ++i) {
    if (!std::strcmp(argv[i], "--repeats") && i + 1 < argc)
      repeats = std::atoi(argv[++i]);
    else if (!std::strcmp(argv[i], "--max-mib") && i + 1 < argc)
      max_mib = std::strtoull(argv[++i], nullptr, 10);
    else if (!std::strcmp(argv[i], "--no-pageable"))
      pageable = false;
    else {
      std::fprintf(stderr,
                   "usage: h2d_bench [--repeats N] [--max-mib M] "
                   "[--no-pageable]\n");
      return 1;
    }
  }
  if (repeats < 1 || max_mib < 1 || max_mib > 4096) {
    std::fprintf(stderr, "bad arguments\n");
    return 1;
  }
  const size_t mib = 1u << 20;
  const size_t max_bytes = max_mib * mib;
  std::vector<size_t> sizes;
  for (size_t s = 4096; s <= max_bytes; s *= 4) sizes.push_back(s);
  for (size_t m : {32, 48, 112, 128, 224}) {
    if (m * mib <= max_bytes) sizes.push_back(m * mib);
  }
  std::sort(sizes.begin(), sizes.end());
  sizes.erase(std::unique(sizes.begin(), sizes.end()), sizes.end());

  CHECK(hipSetDevice(0));
  hipDeviceProp_t prop;
  CHECK(hipGetDeviceProperties(&prop, 0));
  void *dev = nullptr;
  void *pinned = nullptr;
  CHECK(hipMalloc(&dev, max_bytes));
  CHECK(hipHostMalloc(&pinned, max_bytes, hipHostMallocDefault));
  std::memset(pinned, 1, max_bytes);
  void *pageable_buf = nullptr;
  if (pageable) {
    pageable_buf = std::malloc(max_bytes);
    if (pageable_buf == nullptr) return 3;
    std::memset(pageable_buf, 1, max_bytes);
  }
  hipStream_t stream;
  CHECK(hipStreamCreate(&stream));

  std::string json = "{\"device\": \"";
  json += prop.name;
  json += "\", \"gcn_arch\": \"";
  json += prop.gcnArchName;
  json += "\", \"repeats\": " + std::to_string(repeats) + ", \"copies\": [";
  bool first = true;
  double plateau = 0.0;
  struct Mode {
    const char *name;
    bool pinned;
    bool async;
  } modes[] = {{"pinned_async", true, true},
               {"pinned_sync", true, false},
               {"pageable_async", false, true},
               {"pageable_sync", false, false}};
  for (const Mode &mode : modes) {
    if (!mode.pinned && !pageable) continue;
    void *src = mode.pinned ? pinned : pageable_buf;
    for (size_t bytes : sizes) {
      if (!mode.pinned && bytes > 256 * mib) continue;
      const Stats s =
          percentiles(time_copies(dev, src, bytes, mode.async, repeats, stream));
      if (mode.pinned && mode.async) plateau = std::max(plateau, s.median);
      char buf[256];
      std::snprintf(buf, sizeof buf,
                    "%s{\"mode\": \"%s\", \"bytes\": %zu, \"gbps_p10\": %.3f, "
                    "\"gbps_median\": %.3f, \"gbps_p90\": %.3f}",
                    first ? "" : ", ", mode.name, bytes, s.p10, s.median,
                    s.p90);
      json += buf;
      first = false;
      std::fprintf(stderr, "h2d_bench: %s %zu B median %.2f GB/s\n", mode.name,
                   bytes, s.median);
    }
  }
  // The same pinned copies split over 2 and 4 streams (several DMA engines
  // at once), sizes of 1 MiB and up.
  std::vector<hipStream_t> extra(4);
  extra[0] = stream;
  for (int i = 1; i < 4; ++i) CHECK(hipStreamCreate(&extra[i]));
  for (int n : {2, 4}) {
    std::vector<hipStream_t> use(extra.begin(), extra.begin() + n);
    for (size_t bytes : sizes) {
      if (bytes < mib) continue;
      const Stats s = percentiles(time_split_copies(
          static_cast<char *>(dev), static_cast<const char *>(pinned), bytes,
          repeats, use));
      char buf[256];
      std::snprintf(buf, sizeof buf,
                    ", {\"mode\": \"pinned_async_%d_streams\", \"bytes\": %zu, "
                    "\"gbps_p10\": %.3f, \"gbps_median\": %.3f, \"gbps_p90\": %.3f}",
                    n, bytes, s.p10, s.median, s.p90);
      json += buf;
      std::fprintf(stderr, "h2d_bench: pinned_async_%d_streams %zu B median %.2f GB/s\n",
                   n, bytes, s.median);
    }
  }
  for (int i = 1; i < 4; ++i) CHECK(hipStreamDestroy(extra[i]));
  json += "]";

  // Host enqueue cost of async copies (4 KiB each).
  std::vector<double> xs, ys;
  for (int n = 1; n <= 1024; n *= 2) {
    CHECK(hipStreamSynchronize(stream));
    const double t0 = now_s();
    for (int i = 0; i < n; ++i)
      CHECK(hipMemcpyAsync(dev, pinned, 4096, hipMemcpyHostToDevice, stream));
    const double t1 = now_s();
    CHECK(hipStreamSynchronize(stream));
    xs.push_back(n);
    ys.push_back((t1 - t0) * 1e6);
  }
  double mx = 0, my = 0;
  for (size_t i = 0; i < xs.size(); ++i) {
    mx += xs[i];
    my += ys[i];
  }
  mx /= xs.size();
  my /= ys.size();
  double sxy = 0, sxx = 0;
  for (size_t i = 0; i < xs.size(); ++i) {
    sxy += (xs[i] - mx) * (ys[i] - my);
    sxx += (xs[i] - mx) * (xs[i] - mx);
  }
  const double slope = sxy / sxx;
  char tail[256];
  std::snprintf(tail, sizeof tail,
                ", \"enqueue_us_per_copy\": %.3f, \"pinned_async_plateau_gbps\": "
                "%.3f}",
                slope, plateau);
  json += tail;
  std::printf("%s\n", json.c_str());

  CHECK(hipStreamDestroy(stream));
  CHECK(hipHostFree(pinned));
  CHECK(hipFree(dev));
  std::free(pageable_buf);
  return 0;
}
