// Stress check of the process-wide host thread pool (csrc/par.h), built with
// a thread sanitizer by tests/test_host_pool.py: eight threads own parallel
// loops at once, loop bodies open nested loops, bodies throw, a budget of one
// runs a loop on its caller alone. Every result is checked; the exit status
// is the number of wrong results (the sanitizer adds its own failure).
#include <atomic>
#include <cstdio>
#include <stdexcept>
#include <thread>
#include <vector>

#include "par.h"

using namespace wc;

int main() {
    std::atomic<long> bad{0}, threw{0};
    std::vector<std::thread> owners;
    for (int o = 0; o < 8; o++)
        owners.emplace_back([&, o] {
            for (int rep = 0; rep < 60; rep++) {
                // nested loops: each outer index sums an inner loop
                std::vector<long> out(700, -1);
                parallel_for(out.size(), [&](size_t i) {
                    std::vector<long> inner(9, 0);
                    parallel_for(inner.size(), [&](size_t j) { inner[j] = (long)(i * j + o); });
                    long s = 0;
                    for (long v : inner) s += v;
                    out[i] = s;
                });
                for (size_t i = 0; i < out.size(); i++)
                    if (out[i] != (long)(36 * i + 9 * o)) bad++;
                // the first exception ends the loop and reaches the owner
                try {
                    parallel_for(500, [&](size_t i) {
                        if (i % 97 == 13) throw std::runtime_error("planted");
                    });
                    bad++;
                } catch (const std::runtime_error&) {
                    threw++;
                }
                // a budget of one: the caller alone, in index order
                ParBudget one(1);
                std::vector<size_t> order;
                parallel_for(50, [&](size_t i) { order.push_back(i); });
                for (size_t i = 0; i < order.size(); i++)
                    if (order[i] != i) bad++;
                if (order.size() != 50) bad++;
            }
        });
    for (auto& t : owners) t.join();
    if (threw != 8 * 60) bad++;
    std::printf("host pool: %ld wrong results, %ld exceptions delivered\n", bad.load(), threw.load());
    return (int)bad.load();
}
