// Host-side checks of ferrite-tpu_amd/csrc/device_select.h with stand-in HIP
// lookups: which device a stream resolves to, and that per-device set-up runs
// exactly once per (kernel, device) however many threads race for it.
#include "../../ferrite-tpu_amd/csrc/device_select.h"

#include <atomic>
#include <cstdio>
#include <thread>
#include <vector>

using ferrite::device_of_stream;
using ferrite::OncePerDevice;

static int failures = 0;
#define CHECK(c)                                                \
  do {                                                          \
    if (!(c)) {                                                 \
      std::fprintf(stderr, "%s:%d: %s\n", __FILE__, __LINE__, #c); \
      ++failures;                                               \
    }                                                           \
  } while (0)

int main() {
  // Stand-ins: the thread's current device is 0; stream s7 lives on device 7,
  // stream s3 on device 3; an unknown stream fails its lookup.
  int s7, s3, bad;
  const void* kS7 = &s7;
  const void* kS3 = &s3;
  const void* kBad = &bad;
  int current = 0;
  int stream_calls = 0, current_calls = 0;
  auto stream_dev = [&](const void* s, int* d) {
    ++stream_calls;
    if (s == kS7) { *d = 7; return 0; }
    if (s == kS3) { *d = 3; return 0; }
    return 1;
  };
  auto current_dev = [&](int* d) {
    ++current_calls;
    *d = current;
    return 0;
  };
  CHECK(device_of_stream(kS7, stream_dev, current_dev) == 7);
  CHECK(device_of_stream(kS3, stream_dev, current_dev) == 3);
  CHECK(current_calls == 0);  // a real stream never consults the current device
  CHECK(device_of_stream(nullptr, stream_dev, current_dev) == 0);
  current = 5;
  CHECK(device_of_stream(nullptr, stream_dev, current_dev) == 5);
  CHECK(device_of_stream(reinterpret_cast<const void*>(ferrite::kPerThreadStream), stream_dev, current_dev) == 5);
  CHECK(stream_calls == 2);  // null and per-thread streams never ask the stream
  CHECK(device_of_stream(kBad, stream_dev, current_dev) == -1);
  auto current_fails = [](int* d) { *d = 0; return 1; };
  CHECK(device_of_stream(nullptr, stream_dev, current_fails) == -1);
  auto negative = [](const void*, int* d) { *d = -3; return 0; };
  CHECK(device_of_stream(kS7, negative, current_dev) == -1);

  // Once per (kernel, device): 16 threads x 3 kernels x 4 devices, each step
  // counted; every caller sees the step's own result.
  OncePerDevice once;
  std::atomic<int> runs[3][4];
  for (auto& r : runs)
    for (auto& x : r) x = 0;
  int kern[3];
  std::atomic<int> wrong{0};
  std::vector<std::thread> pool;
  for (int t = 0; t < 16; ++t)
    pool.emplace_back([&, t] {
      for (int i = 0; i < 200; ++i) {
        const int k = (i + t) % 3, dev = (i * 7 + t) % 4;
        const int rc = once.run(&kern[k], dev, [&] {
          runs[k][dev].fetch_add(1);
          std::this_thread::yield();
          return 10 * k + dev;
        });
        if (rc != 10 * k + dev) wrong.fetch_add(1);
      }
    });
  for (auto& th : pool) th.join();
  for (int k = 0; k < 3; ++k)
    for (int dev = 0; dev < 4; ++dev) CHECK(runs[k][dev].load() == 1);
  CHECK(wrong.load() == 0);
  // A failed step is remembered too: later callers get its error without rerunning it.
  int calls = 0;
  CHECK(once.run(&kern[0], 9, [&] { ++calls; return 98; }) == 98);
  CHECK(once.run(&kern[0], 9, [&] { ++calls; return 0; }) == 98);
  CHECK(calls == 1);

  if (failures) {
    std::fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  std::printf("device_select: all checks passed\n");
  return 0;
}
