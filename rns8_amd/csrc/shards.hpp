// Host-side fan-out over a few threads that never fails: a shard whose thread
// cannot be started (thread creation or its allocation fails) runs on the
// calling thread instead, so no exception leaves with threads still joinable.
#pragma once

#include <thread>
#include <vector>

namespace rns8x {

// work(t) for t in [0, n); work must not throw.
template <typename F>
void run_shards(unsigned n, F&& work) {
  std::vector<std::thread> pool;
  unsigned started = 1;  // shards 1 .. started - 1 have threads
  try {
    pool.reserve(n > 1 ? n - 1 : 0);
    for (unsigned t = 1; t < n; ++t) {
      pool.emplace_back(work, t);
      started = t + 1;
    }
  } catch (...) {
    // the remaining shards run below, on this thread
  }
  work(0u);
  for (auto& th : pool) th.join();
  for (unsigned t = started; t < n; ++t) work(t);
}

}  // namespace rns8x
