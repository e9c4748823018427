// A small host-side parallel loop for wave packing (independent per-job and
// per-player work).
#pragma once

#include <algorithm>
#include <atomic>
#include <cstddef>
#include <exception>
#include <mutex>
#include <thread>
#include <vector>

namespace wc {

// The calling thread's budget of host threads for parallel loops. Callers
// that run side by side (a service's lanes packing at once) each take a share
// of the cores, so that together they do not oversubscribe the host.
inline unsigned& par_budget() {
    static thread_local unsigned budget = 16;
    return budget;
}
struct ParBudget {  // sets the calling thread's budget for its lifetime
    unsigned old;
    explicit ParBudget(unsigned n) : old(par_budget()) { par_budget() = std::max(1u, n); }
    ~ParBudget() { par_budget() = old; }
    ParBudget(const ParBudget&) = delete;
    ParBudget& operator=(const ParBudget&) = delete;
};

// Runs fn(i) for every i in [0, n) on up to max_threads host threads (at most
// the hardware's and the caller's budget), taking indices from a shared
// counter; loops nested inside fn share the caller's budget. The first
// exception fn throws (std::bad_alloc on a huge wave) ends the loop and is
// rethrown on the calling thread.
template <class F>
void parallel_for(size_t n, F fn, unsigned max_threads = 16) {
    if (n == 0) return;
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const unsigned budget = par_budget();
    const size_t nt = std::min<size_t>(std::min({hw, std::max(1u, max_threads), budget}), n);
    const unsigned inner = std::max<unsigned>(1u, budget / (unsigned)nt);
    std::atomic<size_t> next{0};
    std::exception_ptr failure;
    std::mutex failure_lock;
    auto work = [&]() {
        ParBudget share(inner);
        try {
            for (size_t i = next.fetch_add(1); i < n; i = next.fetch_add(1)) fn(i);
        } catch (...) {
            std::lock_guard<std::mutex> hold(failure_lock);
            if (!failure) failure = std::current_exception();
            next.store(n);  // the other threads take no further index
        }
    };
    std::vector<std::thread> pool;
    for (size_t t = 1; t < nt; t++) pool.emplace_back(work);
    work();
    for (auto& th : pool) th.join();
    if (failure) std::rethrow_exception(failure);
}

}  // namespace wc
