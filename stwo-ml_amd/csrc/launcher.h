// Kernel launches issued by a host thread of their own.
//
// A launch through the HIP runtime (hipLaunchKernel) costs the calling
// thread 5-10 us on MI355X under ROCm 7.  The prover's host thread computes
// the Fiat-Shamir transcript between device results, so every launch it
// makes itself delays the transcript, and a launch queued behind kernels the
// device has already finished delays the device too.  With a Launcher the
// host thread instead copies the launch (kernel, shape, stream and the
// argument values, converted to the kernel's parameter types at that point)
// into a ring slot, about 0.1 us, and goes on; the launcher thread issues the
// slots in ring order, so the stream sees the launches in program order.
//
// Ordering rule: every other HIP call of the library that touches memory or
// a stream (copies, fills, frees, synchronisations, stream queries, event
// records outside the ring) first drains the ring of the context it works
// on, so it never overtakes a launch queued before it on that context.
// Launch errors are recorded by the launcher thread and reported, for that
// context only, by check_launch(c) and by the waits.
//
// One producer per ring: the thread that calls the library on the context.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <memory>
#include <mutex>
#include <new>
#include <thread>
#include <tuple>
#include <type_traits>
#include <utility>

#include <immintrin.h>

namespace gkr {

class Launcher {
 public:
  static constexpr size_t kSlotBytes = 4096 - 64;  // largest launch closure (two PointArg = 2 KiB) fits
  static constexpr uint64_t kSlots = 256;
  // The launcher thread spins this long for the next slot before it sleeps
  // (a sleeping thread takes a futex wake-up, several us, to resume).
  static constexpr double kSpinSeconds = 0.005;

  // device < 0: the thread makes no HIP call of its own (the host-only tests)
  explicit Launcher(int device) : ring_(new Slot[kSlots]) {
    th_ = std::thread([this, device] { loop(device); });
  }
  ~Launcher() {
    drain();
    {
      std::lock_guard<std::mutex> lk(m_);
      stop_.store(true, std::memory_order_seq_cst);
    }
    cv_.notify_one();
    th_.join();
  }
  Launcher(const Launcher&) = delete;
  Launcher& operator=(const Launcher&) = delete;

  // Queues f (a callable returning hipError_t) behind every earlier slot.
  template <class F>
  void submit(F&& f) {
    using T = std::decay_t<F>;
    static_assert(sizeof(T) <= kSlotBytes && alignof(T) <= 64, "launch closure too large for a ring slot");
    const uint64_t h = head_.load(std::memory_order_relaxed);
    while (h - tail_.load(std::memory_order_acquire) >= kSlots) _mm_pause();  // ring full
    Slot& s = ring_[h % kSlots];
    new (s.buf) T(std::forward<F>(f));
    s.run = [](void* p) -> hipError_t {
      T* t = static_cast<T*>(p);
      const hipError_t e = (*t)();
      t->~T();
      return e;
    };
    head_.store(h + 1, std::memory_order_seq_cst);
    if (sleeping_.load(std::memory_order_seq_cst)) {
      std::lock_guard<std::mutex> lk(m_);
      cv_.notify_one();
    }
  }
  // Returns once every submitted slot has been issued.
  void drain() const {
    const uint64_t h = head_.load(std::memory_order_relaxed);
    while (tail_.load(std::memory_order_acquire) != h) _mm_pause();
  }
  bool idle() const { return tail_.load(std::memory_order_acquire) == head_.load(std::memory_order_relaxed); }
  // First error a queued call returned (hipSuccess if none); cleared by take_error.
  hipError_t error() const { return (hipError_t)err_.load(std::memory_order_acquire); }
  hipError_t take_error() { return (hipError_t)err_.exchange(0, std::memory_order_acq_rel); }

 private:
  struct alignas(64) Slot {
    hipError_t (*run)(void*);
    alignas(64) unsigned char buf[kSlotBytes];
  };
  std::unique_ptr<Slot[]> ring_;
  alignas(64) std::atomic<uint64_t> head_{0};  // slots submitted (producer)
  alignas(64) std::atomic<uint64_t> tail_{0};  // slots issued (launcher thread)
  std::atomic<bool> sleeping_{false}, stop_{false};
  std::atomic<int> err_{0};
  std::mutex m_;
  std::condition_variable cv_;
  std::thread th_;

  void loop(int device) {
    if (device >= 0) (void)hipSetDevice(device);
    uint64_t t = 0;
    for (;;) {
      if (head_.load(std::memory_order_acquire) == t) {
        const auto t0 = std::chrono::steady_clock::now();
        bool more = false;
        for (uint32_t i = 1;; i++) {
          _mm_pause();
          if (head_.load(std::memory_order_acquire) != t) {
            more = true;
            break;
          }
          if ((i & 1023) == 0 &&
              std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() > kSpinSeconds)
            break;
        }
        if (!more) {
          std::unique_lock<std::mutex> lk(m_);
          sleeping_.store(true, std::memory_order_seq_cst);
          cv_.wait(lk, [&] {
            return head_.load(std::memory_order_seq_cst) != t || stop_.load(std::memory_order_seq_cst);
          });
          sleeping_.store(false, std::memory_order_seq_cst);
          if (head_.load(std::memory_order_seq_cst) == t) return;  // stopped with nothing queued
        }
      }
      Slot& s = ring_[t % kSlots];
      const hipError_t e = s.run(s.buf);
      if (e != hipSuccess) {
        int none = 0;
        err_.compare_exchange_strong(none, (int)e, std::memory_order_acq_rel);
      }
      tail_.store(++t, std::memory_order_release);
    }
  }
};

// Start and stop events taken from the kernel's own dispatch
// (hipExtLaunchKernel): timing without event-record packets between kernels.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
// A kernel launch with its arguments converted to the kernel's parameter
// types now, issued through l (or at once when l is null); with ev set, the
// kernel's start and end times go to those events.
template <class... KArgs, class... Args>
inline hipError_t launch_kernel(Launcher* l, LaunchEvents ev, void (*kernel)(KArgs...), dim3 grid, dim3 block,
                                uint32_t shmem, hipStream_t stream, Args&&... args) {
  static_assert(sizeof...(KArgs) == sizeof...(Args), "kernel argument count");
  auto issue = [kernel, grid, block, shmem, stream, ev,
                tup = std::tuple<std::decay_t<KArgs>...>(std::forward<Args>(args)...)]() mutable -> hipError_t {
    return std::apply(
        [&](auto&... a) -> hipError_t {
          void* argv[] = {(void*)&a..., nullptr};
          if (ev.start || ev.stop)
            return hipExtLaunchKernel((const void*)kernel, grid, block, argv, shmem, stream, ev.start, ev.stop, 0);
          return hipLaunchKernel((const void*)kernel, grid, block, argv, shmem, stream);
        },
        tup);
  };
  if (!l) return issue();
  l->submit(std::move(issue));
  return hipSuccess;
}

}  // namespace gkr
