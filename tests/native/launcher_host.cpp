// Host-only checks of the launch ring (stwo-ml_amd/csrc/launcher.h): order,
// wrap-around, error reporting, sleep and wake-up, draining on destruction.
// The closures do host work instead of HIP calls, so no GPU is needed.
#include <chrono>
#include <memory>
#include <thread>
#include <vector>

#include "../../stwo-ml_amd/csrc/launcher.h"


extern "C" int lt_order(int n) {
  std::vector<int> seen;
  seen.reserve(n);
  {
    gkr::Launcher l(-1);
    for (int i = 0; i < n; i++)
      l.submit([&seen, i]() -> hipError_t {
        seen.push_back(i);
        return hipSuccess;
      });
    l.drain();
    if ((int)seen.size() != n) return 1;
    for (int i = 0; i < n; i++)
      if (seen[i] != i) return 2;
  }
  return 0;
}

extern "C" int lt_error() {
  gkr::Launcher l(-1);
  int ran = 0;
  for (int i = 0; i < 10; i++)
    l.submit([&ran, i]() -> hipError_t {
      ran++;
      return i == 4 ? hipErrorInvalidValue : (i == 7 ? hipErrorOutOfMemory : hipSuccess);
    });
  l.drain();
  if (ran != 10) return 1;
  if (l.error() != hipErrorInvalidValue) return 2;  // the first error is kept
  if (l.take_error() != hipErrorInvalidValue) return 3;
  if (l.error() != hipSuccess) return 4;
  return 0;
}

extern "C" int lt_sleep_wake() {
  gkr::Launcher l(-1);
  std::atomic<int> ran{0};
  for (int round = 0; round < 3; round++) {
    l.submit([&ran]() -> hipError_t {
      ran++;
      return hipSuccess;
    });
    l.drain();
    if (ran.load() != round + 1) return 1 + round;
    // longer than the spin period: the thread goes to sleep and must wake up
    std::this_thread::sleep_for(std::chrono::milliseconds(20));
  }
  return l.idle() ? 0 : 9;
}

extern "C" int lt_destroy_pending(int n) {
  std::atomic<int> ran{0};
  {
    gkr::Launcher l(-1);
    for (int i = 0; i < n; i++)
      l.submit([&ran]() -> hipError_t {
        std::this_thread::sleep_for(std::chrono::microseconds(50));
        ran++;
        return hipSuccess;
      });
  }  // the destructor drains before it stops the thread
  return ran.load() == n ? 0 : 1;
}

extern "C" int lt_big_closure() {
  // a closure near the slot size keeps its bytes
  struct Big {
    unsigned char b[gkr::Launcher::kSlotBytes - 64];
  };
  Big big;
  for (size_t i = 0; i < sizeof big.b; i++) big.b[i] = (unsigned char)(i * 7 + 3);
  int bad = -1;
  {
    gkr::Launcher l(-1);
    l.submit([big, &bad]() -> hipError_t {
      bad = 0;
      for (size_t i = 0; i < sizeof big.b; i++)
        if (big.b[i] != (unsigned char)(i * 7 + 3)) bad++;
      return hipSuccess;
    });
    l.drain();
  }
  return bad;
}

// Two rings: an error on one is taken from that ring only; the other's stays clear.
extern "C" int lt_errors_per_ring() {
  gkr::Launcher a(-1), b(-1);
  a.submit([]() -> hipError_t { return hipErrorInvalidValue; });
  b.submit([]() -> hipError_t { return hipSuccess; });
  a.drain();
  b.drain();
  if (b.take_error() != hipSuccess) return 1;
  if (a.take_error() != hipErrorInvalidValue) return 2;
  if (a.take_error() != hipSuccess) return 3;
  return 0;
}
