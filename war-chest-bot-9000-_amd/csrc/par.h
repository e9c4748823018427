// A small host-side parallel loop for wave packing (independent per-job and
// per-player work), over one pool of worker threads shared by every caller in
// the process.
//
// A service's lanes pack waves side by side. With a fixed share of the cores
// per lane, a lane packing a large wave kept its share while the other lanes'
// threads sat idle waiting on the device; the shared pool lets every idle
// worker join whichever loop still has indices left, so one large wave is
// packed on all the cores the others are not using.
#pragma once

#include <pthread.h>
#include <sched.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstddef>
#include <exception>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace wc {

// Host cores this process may run on (its affinity mask), at least 1.
inline unsigned host_cores() {
    cpu_set_t set;
    CPU_ZERO(&set);
    if (sched_getaffinity(0, sizeof(set), &set) == 0) {
        const int n = CPU_COUNT(&set);
        if (n > 0) return (unsigned)n;
    }
    return std::max(1u, std::thread::hardware_concurrency());
}

// The calling thread's cap on the threads one parallel loop may use (itself
// included); loops nested inside a loop's body inherit it.
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

class HostPool {
  public:
    // The process's pool: host_cores() - 1 workers (callers work too). Never
    // destroyed, so a thread still packing while the process exits does not
    // meet a pool that is being torn down.
    static HostPool& get() {
        static HostPool* pool = new HostPool(host_cores() > 1 ? host_cores() - 1 : 0);
        return *pool;
    }

    // Runs body(i) for every i in [0, n): the caller takes indices from a
    // shared counter, and up to `helpers` idle workers join while indices
    // remain. Returns when every index has run; the first exception a body
    // throws ends the loop (no further index is taken) and is rethrown here.
    void run(size_t n, unsigned helpers, unsigned budget, const std::function<void(size_t)>& body) {
        Loop L;
        L.n = n;
        L.max_helpers = std::min<size_t>(helpers, n > 0 ? n - 1 : 0);
        L.budget = budget;
        L.body = &body;
        if (L.max_helpers && !workers_.empty()) {
            {
                std::lock_guard<std::mutex> lk(mu_);
                loops_.push_back(&L);
            }
            for (unsigned k = 0; k < L.max_helpers && k < workers_.size(); k++) work_cv_.notify_one();
        }
        drain(L);
        {
            std::unique_lock<std::mutex> lk(mu_);
            auto it = std::find(loops_.begin(), loops_.end(), &L);
            if (it != loops_.end()) loops_.erase(it);  // no helper joins from here on
            done_cv_.wait(lk, [&] { return L.active == 0; });
        }
        if (L.failure) std::rethrow_exception(L.failure);
    }

  private:
    struct Loop {
        size_t n = 0;
        std::atomic<size_t> next{0};
        unsigned max_helpers = 0, budget = 1;
        unsigned helpers = 0, active = 0;  // under mu_
        const std::function<void(size_t)>* body = nullptr;
        std::exception_ptr failure;
        std::mutex failure_lock;
    };

    explicit HostPool(unsigned workers) {
        // A fork copies only the forking thread: the pool's lock is taken
        // across the fork so that no worker holds it in the child, whose pool
        // then has no workers (its loops run on their callers).
        pthread_atfork([] { get().mu_.lock(); }, [] { get().mu_.unlock(); },
                       [] {
                           HostPool& p = get();
                           p.workers_.clear();
                           p.loops_.clear();
                           p.mu_.unlock();
                       });
        for (unsigned w = 0; w < workers; w++) workers_.emplace_back([this] { worker(); });
        for (auto& th : workers_) th.detach();
    }

    static void drain(Loop& L) {
        ParBudget share(L.budget);
        try {
            for (size_t i = L.next.fetch_add(1); i < L.n; i = L.next.fetch_add(1)) (*L.body)(i);
        } catch (...) {
            std::lock_guard<std::mutex> hold(L.failure_lock);
            if (!L.failure) L.failure = std::current_exception();
            L.next.store(L.n);  // no thread takes a further index
        }
    }

    void worker() {
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            Loop* pick = nullptr;
            work_cv_.wait(lk, [&] {
                for (Loop* L : loops_)
                    if (L->helpers < L->max_helpers && L->next.load(std::memory_order_relaxed) < L->n) {
                        pick = L;
                        return true;
                    }
                return false;
            });
            pick->helpers++;
            pick->active++;
            lk.unlock();
            drain(*pick);
            lk.lock();
            if (--pick->active == 0) done_cv_.notify_all();
        }
    }

    std::mutex mu_;
    std::condition_variable work_cv_, done_cv_;
    std::vector<Loop*> loops_;  // loops that helpers may still join
    std::vector<std::thread> workers_;
};

// Runs fn(i) for every i in [0, n) on the calling thread and up to
// min(max_threads, the caller's budget) - 1 pool workers; see HostPool::run.
template <class F>
void parallel_for(size_t n, F fn, unsigned max_threads = 16) {
    if (n == 0) return;
    const unsigned budget = par_budget();
    const unsigned threads = std::max(1u, std::min(max_threads, budget));
    if (threads == 1 || n == 1) {
        for (size_t i = 0; i < n; i++) fn(i);
        return;
    }
    const std::function<void(size_t)> body = [&fn](size_t i) { fn(i); };
    HostPool::get().run(n, threads - 1, budget, body);
}

}  // namespace wc
