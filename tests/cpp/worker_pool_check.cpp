// Exception handling of the host thread pool (worker_pool.hpp): a task that
// throws on the calling thread or on a worker makes run() rethrow it on the
// calling thread after the run is closed and drained, and the pool keeps
// working.  Built and run by tests/test_worker_pool.py; prints "ok".
#include <atomic>
#include <cstdio>
#include <stdexcept>

#include "worker_pool.hpp"

int main() {
  mimoe_pool::WorkerPool pool(6);
  for (int round = 0; round < 50; ++round) {
    const int64_t bad = round % 2 ? 0 : 997 + round;   // index 0 runs on the caller first; others anywhere
    std::atomic<int64_t> done{0};
    bool caught = false;
    try {
      pool.run(2000, [&](int64_t i) {
        if (i == bad) throw std::runtime_error("task failed");
        done.fetch_add(1);
      });
    } catch (const std::runtime_error& e) {
      caught = std::string(e.what()) == "task failed";
    }
    if (!caught || done.load() >= 2000) {
      std::printf("round %d: exception not propagated (caught=%d, done=%lld)\n", round, (int)caught,
                  (long long)done.load());
      return 1;
    }
    // the pool still runs every index of the next run
    std::atomic<int64_t> sum{0};
    pool.run(1000, [&](int64_t i) { sum.fetch_add(i); });
    if (sum.load() != 999 * 1000 / 2) {
      std::printf("round %d: pool broken after an exception (sum %lld)\n", round, (long long)sum.load());
      return 1;
    }
  }
  std::printf("ok\n");
  return 0;
}
