// worker_pool.hpp -- the fixed host thread pool of the CPU paths (host
// engine, hybrid host executor).  run(n, f) calls f(i) for every i < n on the
// calling thread and on the pool's workers, handing indices out dynamically,
// and returns when all calls are done.  One run at a time per pool.  If a
// call throws, no further indices are handed out, the run is closed and
// drained as usual, and run() rethrows the first exception on the calling
// thread; the pool stays usable.
//
// A call of the host paths is a few short phases back to back (tens of
// microseconds each), so the hand-offs are built for latency:
//  * one futex word (the run generation) wakes up to n - 1 sleeping workers
//    with one system call, and a worker that finished a run in the last
//    spin_us microseconds is still polling it and joins without one;
//  * a run is "open" until the caller finds the index range exhausted; it
//    then closes it and waits only for the workers that are inside it.  A
//    worker that arrives after the close leaves without touching the run,
//    so a late wake-up never delays the caller.
// Linux only (futex).
#pragma once
#include <linux/futex.h>
#include <stdint.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <climits>
#include <exception>
#include <functional>
#include <mutex>
#include <memory>
#include <thread>
#include <vector>

#ifndef MIMOE_POOL_SPIN_US
#define MIMOE_POOL_SPIN_US 50
#endif

namespace mimoe_pool {

inline void cpu_relax() {
#if defined(__x86_64__) || defined(__i386__)
  __builtin_ia32_pause();
#endif
}

class WorkerPool {
 public:
  // nthreads counts the calling thread; on_start(i) runs first on worker i
  // (1 <= i < nthreads), e.g. to pin it to a CPU.  A worker polls for the
  // next run for spin_us microseconds after each run before it sleeps.
  explicit WorkerPool(int nthreads, std::function<void(int)> on_start = nullptr,
                      int spin_us = MIMOE_POOL_SPIN_US)
      : spin_(std::chrono::microseconds(spin_us < 0 ? 0 : spin_us)) {
    if (nthreads < 1) nthreads = 1;
    for (int i = 1; i < nthreads; ++i)
      th_.emplace_back([this, i, on_start] {
        if (on_start) on_start(i);
        work();
      });
  }
  ~WorkerPool() {
    stop_.store(true);
    gen_.fetch_add(1);
    futex_wake(INT_MAX);
    for (auto& t : th_) t.join();
  }
  WorkerPool(const WorkerPool&) = delete;
  WorkerPool& operator=(const WorkerPool&) = delete;
  int size() const { return (int)th_.size() + 1; }

  void run(int64_t n, const std::function<void(int64_t)>& f) {
    if (n <= 0) return;
    if (th_.empty() || n == 1) {
      for (int64_t i = 0; i < n; ++i) f(i);
      return;
    }
    fn_ = &f;
    n_ = n;
    err_ = nullptr;
    next_.store(0, std::memory_order_relaxed);
    // open the run: clears the closed bit, keeps the count of any worker
    // that is passing through on its way out of the previous run
    state_.fetch_and(~kClosed);
    gen_.fetch_add(1);
    if (sleepers_.load() > 0) futex_wake((int)std::min<int64_t>(n - 1, (int64_t)th_.size()));
    call_all(f, n);
    state_.fetch_or(kClosed);
    // the workers still inside finish their current index at most
    for (unsigned spins = 0; (state_.load(std::memory_order_acquire) & ~kClosed) != 0; ++spins) {
      if (spins < 4096) cpu_relax();
      else std::this_thread::yield();
    }
    fn_ = nullptr;
    if (err_) {
      std::exception_ptr e = err_;
      err_ = nullptr;
      std::rethrow_exception(e);
    }
  }

 private:
  static constexpr uint32_t kClosed = 1u << 31;

  // f(i) for the indices this thread takes; the first exception of the run is
  // kept and the remaining indices are skipped
  void call_all(const std::function<void(int64_t)>& f, int64_t n) {
    for (int64_t i; (i = next_.fetch_add(1, std::memory_order_relaxed)) < n;) {
      try {
        f(i);
      } catch (...) {
        std::lock_guard<std::mutex> lk(err_mu_);
        if (!err_) err_ = std::current_exception();
        next_.store(n, std::memory_order_relaxed);
      }
    }
  }

  void futex_wake(int count) {
    syscall(SYS_futex, reinterpret_cast<uint32_t*>(&gen_), FUTEX_WAKE_PRIVATE, count, nullptr, nullptr, 0);
  }
  void futex_wait(uint32_t seen) {
    syscall(SYS_futex, reinterpret_cast<uint32_t*>(&gen_), FUTEX_WAIT_PRIVATE, seen, nullptr, nullptr, 0);
  }

  void work() {
    uint32_t seen = 0;   // gen_'s initial value: a worker that starts late still sees every bump
    for (;;) {
      uint32_t g = gen_.load(std::memory_order_acquire);
      if (g == seen && spin_.count() > 0) {   // poll for a run that follows closely
        const auto until = std::chrono::steady_clock::now() + spin_;
        for (unsigned k = 1; (g = gen_.load(std::memory_order_acquire)) == seen; ++k) {
          cpu_relax();
          if ((k & 63) == 0 && std::chrono::steady_clock::now() >= until) break;
        }
      }
      if (g == seen) {   // sleep; the caller wakes sleepers after bumping gen_
        sleepers_.fetch_add(1);
        while ((g = gen_.load()) == seen) futex_wait(seen);
        sleepers_.fetch_sub(1);
      }
      seen = g;
      if (stop_.load()) return;
      const uint32_t s = state_.fetch_add(1);
      if (!(s & kClosed)) {   // inside an open run: its fn_ / n_ are set
        call_all(*fn_, n_);
      }
      state_.fetch_sub(1, std::memory_order_release);
    }
  }

  const std::chrono::microseconds spin_;
  std::vector<std::thread> th_;
  std::atomic<uint32_t> gen_{0};             // futex word, bumped once per run and at shutdown
  std::atomic<uint32_t> state_{kClosed};     // closed bit | workers inside the run
  std::atomic<int> sleepers_{0};
  std::atomic<bool> stop_{false};
  std::atomic<int64_t> next_{0};
  const std::function<void(int64_t)>* fn_ = nullptr;
  int64_t n_ = 0;
  std::mutex err_mu_;
  std::exception_ptr err_;   // first exception of the current run
};

}  // namespace mimoe_pool
