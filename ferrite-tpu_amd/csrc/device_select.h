// Which GPU a C ABI call works on, and once-per-device set-up.
//
// An entry point receives a stream and no device. Its launches go to the stream's
// device, so every per-device quantity it looks up (the CU count that shapes a
// grid, a kernel's dynamic-LDS limit, the device address of a file-scope array)
// must come from that device, not from whichever device happens to be current on
// the calling thread (an XLA handler thread or a multi-GPU process may call with
// another device current).
//
// Plain C++ with no HIP dependency: the lookups are passed in, so the host-side
// logic is exercised on the CPU (tests/cpp/device_select_test.cpp) with stand-in
// lookups.
#pragma once

#include <stdint.h>

#include <map>
#include <memory>
#include <mutex>
#include <utility>

namespace ferrite {

// HIP's per-thread default stream handle (hipStreamPerThread).
constexpr uintptr_t kPerThreadStream = 2;

// Device of `stream`: for the null stream and the per-thread default stream, the
// device current on this thread (`current_dev`); otherwise the stream's own
// (`stream_dev`). Each lookup returns 0 on success. -1 if the lookup fails.
template <class StreamDev, class CurrentDev>
int device_of_stream(const void* stream, StreamDev&& stream_dev, CurrentDev&& current_dev) {
  int dev = -1;
  const uintptr_t v = reinterpret_cast<uintptr_t>(stream);
  const int rc = (v == 0 || v == kPerThreadStream) ? current_dev(&dev) : stream_dev(stream, &dev);
  return rc == 0 && dev >= 0 ? dev : -1;
}

// Runs a set-up step once per (key, device), e.g. raising one kernel's LDS limit
// on one GPU, and hands every later caller the step's result. Callers on other
// threads wait for a step in progress (std::call_once). The registry only
// grows: one entry per kernel and device used.
class OncePerDevice {
 public:
  template <class Fn>
  int run(const void* key, int dev, Fn&& fn) {
    Slot* slot;
    {
      std::lock_guard<std::mutex> lock(mu_);
      std::unique_ptr<Slot>& p = slots_[std::make_pair(key, dev)];
      if (!p) p.reset(new Slot);
      slot = p.get();
    }
    std::call_once(slot->once, [&] { slot->result = fn(); });
    return slot->result;
  }

 private:
  struct Slot {
    std::once_flag once;
    int result = 0;
  };
  std::mutex mu_;
  std::map<std::pair<const void*, int>, std::unique_ptr<Slot>> slots_;
};

}  // namespace ferrite
