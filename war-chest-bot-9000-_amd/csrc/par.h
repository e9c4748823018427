// A small host-side parallel loop for wave packing (independent per-job and
// per-player work).
#pragma once

#include <algorithm>
#include <atomic>
#include <cstddef>
#include <thread>
#include <vector>

namespace wc {

// Runs fn(i) for every i in [0, n) on up to max_threads host threads (at most
// the hardware's), taking indices from a shared counter. fn must not throw.
template <class F>
void parallel_for(size_t n, F fn, unsigned max_threads = 16) {
    if (n == 0) return;
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const size_t nt = std::min<size_t>(std::min(hw, std::max(1u, max_threads)), n);
    std::atomic<size_t> next{0};
    auto work = [&]() {
        for (size_t i = next.fetch_add(1); i < n; i = next.fetch_add(1)) fn(i);
    };
    std::vector<std::thread> pool;
    for (size_t t = 1; t < nt; t++) pool.emplace_back(work);
    work();
    for (auto& th : pool) th.join();
}

}  // namespace wc
