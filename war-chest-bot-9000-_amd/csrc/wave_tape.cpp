// wc_tape: the service's throughput through the C ABI, from a native caller
// (the counterpart of the reference's throughput tape, engine/examples/
// wave_tape.rs:80-99: jobs prepared once, then submitted wave after wave by
// several threads, results waited on). Built beside libwcwave.so; uses only
// include/wc_wave.h.
//
//   wc_tape TAPE_FILE WAVES LANES SUBMIT_THREADS PRECISION
//
// TAPE_FILE: "WCTP", u32 njobs, then per job u64 length + WCJ8 bytes, then
// the network: u32 ndims + dims, u64 nw + w, u64 nb + b, u64 nln + ln
// (little-endian, floats as IEEE single). One "wave" is one copy of the file's
// jobs. The service takes waves of up to njobs jobs, the reference's 48k-row
// target and 800 us fill window (engine/src/gpu/service.rs:554-556).
//
// After warm-up streams of LANES waves of each kind, prepared jobs
// (wc_prepare once, wc_submit_prepared per wave) and WCJ8 bytes per
// submission (wc_submit) are timed alternately, twice each; each submitted
// job's result is waited on and its strategy read. Prints one JSON line.
#include <atomic>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/wc_wave.h"

namespace {

struct Tape {
    std::vector<std::vector<uint8_t>> jobs;
    std::vector<uint32_t> dims;
    std::vector<float> w, b, ln;
};

template <class T>
bool take(FILE* f, T* v, size_t n = 1) {
    return n == 0 || std::fread(v, sizeof(T), n, f) == n;
}

bool read_tape(const char* path, Tape* t, std::string* err) {
    FILE* f = std::fopen(path, "rb");
    if (!f) {
        *err = std::string("cannot open ") + path;
        return false;
    }
    char magic[4];
    uint32_t njobs = 0;
    bool ok = take(f, magic, 4) && std::memcmp(magic, "WCTP", 4) == 0 && take(f, &njobs);
    for (uint32_t k = 0; ok && k < njobs; k++) {
        uint64_t len = 0;
        ok = take(f, &len) && len > 0 && len < (uint64_t(1) << 34);
        if (ok) {
            t->jobs.emplace_back(len);
            ok = take(f, t->jobs.back().data(), len);
        }
    }
    uint32_t ndims = 0;
    ok = ok && take(f, &ndims) && ndims > 0 && ndims < 64;
    if (ok) {
        t->dims.resize(ndims);
        ok = take(f, t->dims.data(), ndims);
    }
    for (std::vector<float>* v : {&t->w, &t->b, &t->ln}) {
        uint64_t n = 0;
        ok = ok && take(f, &n) && n < (uint64_t(1) << 32);
        if (ok) {
            v->resize(n);
            ok = take(f, v->data(), n);
        }
    }
    std::fclose(f);
    if (!ok || t->jobs.empty()) *err = std::string("malformed tape file ") + path;
    return ok && !t->jobs.empty();
}

double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// One stream: `waves` copies of the jobs, job j of wave i submitted by thread
// (i * njobs + j) % threads in that order; then every result waited on in
// submission order. Returns the seconds from the first submission to the last
// result, or a negative value on failure.
template <class Submit>
double stream(size_t njobs, uint32_t waves, uint32_t threads, Submit submit, std::string* err) {
    const size_t n = njobs * waves;
    std::vector<wc_ticket*> tickets(n, nullptr);
    std::atomic<bool> failed{false};
    std::mutex err_lock;  // wc_last_error is per thread: the failing thread records it
    const double t0 = now_s();
    std::vector<std::thread> pool;
    for (uint32_t t = 0; t < threads; t++)
        pool.emplace_back([&, t] {
            for (size_t i = t; i < n && !failed; i += threads)
                if (submit(i % njobs, (uint64_t)i, &tickets[i]) != WC_OK) {
                    std::lock_guard<std::mutex> hold(err_lock);
                    if (!failed) *err = std::string("a submission failed: ") + wc_last_error();
                    failed = true;
                }
        });
    for (auto& th : pool) th.join();
    double strategy_sum = 0.0;
    for (size_t i = 0; i < n; i++) {
        if (!tickets[i]) continue;
        wc_result* r = nullptr;
        if (wc_wait(tickets[i], &r) != WC_OK) {
            if (!failed) *err = std::string("a wait failed: ") + wc_last_error();
            failed = true;
            continue;
        }
        size_t m = 0;
        const float* s = wc_result_strategy(r, &m);
        if (s && m) strategy_sum += s[0] + s[m - 1];  // the caller reads its result
        wc_result_free(r);
    }
    const double dt = now_s() - t0;
    if (failed) return -1.0;
    if (strategy_sum != strategy_sum) {
        *err = "a result's strategy holds NaN";
        return -1.0;
    }
    return dt;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 6) {
        std::fprintf(stderr, "usage: %s TAPE_FILE WAVES LANES SUBMIT_THREADS PRECISION\n", argv[0]);
        return 2;
    }
    const uint32_t waves = (uint32_t)std::strtoul(argv[2], nullptr, 10);
    const uint32_t lanes = (uint32_t)std::strtoul(argv[3], nullptr, 10);
    const uint32_t threads = (uint32_t)std::strtoul(argv[4], nullptr, 10);
    const int precision = (int)std::strtol(argv[5], nullptr, 10);
    if (waves == 0 || lanes == 0 || threads == 0) {
        std::fprintf(stderr, "WAVES, LANES and SUBMIT_THREADS must be positive\n");
        return 2;
    }
    Tape tape;
    std::string err;
    if (!read_tape(argv[1], &tape, &err)) {
        std::fprintf(stderr, "%s\n", err.c_str());
        return 1;
    }
    const size_t njobs = tape.jobs.size();
    wc_net_desc net{tape.dims.data(), (uint32_t)tape.dims.size(), tape.w.data(), tape.w.size(), tape.b.data(),
                    tape.b.size(), tape.ln.empty() ? nullptr : tape.ln.data(), tape.ln.size()};
    wc_service_opts opts{lanes, (uint32_t)njobs, 48 * 1024, 800, 1, 0, 0};
    wc_service* svc = nullptr;
    if (wc_service_create(0, &net, precision, &opts, &svc) != WC_OK) {
        std::fprintf(stderr, "wc_service_create: %s\n", wc_last_error());
        return 1;
    }
    int rc = 0;
    std::vector<wc_prepared*> prepared(njobs, nullptr);
    const double tp = now_s();
    for (size_t j = 0; j < njobs && rc == 0; j++)
        if (wc_prepare(tape.jobs[j].data(), tape.jobs[j].size(), precision, &prepared[j]) != WC_OK) {
            std::fprintf(stderr, "wc_prepare job %zu: %s\n", j, wc_last_error());
            rc = 1;
        }
    const double prep_ms = (now_s() - tp) * 1e3;
    auto by_prep = [&](size_t j, uint64_t tag, wc_ticket** out) {
        return wc_submit_prepared(svc, prepared[j], tag, out);
    };
    auto by_bytes = [&](size_t j, uint64_t tag, wc_ticket** out) {
        return wc_submit(svc, tape.jobs[j].data(), tape.jobs[j].size(), tag, out);
    };
    uint64_t w0 = 0, w1 = 0, g = 0;
    double dp = 0.0, db = 0.0;
    uint64_t waves_prep = 0, waves_bytes = 0;
    if (rc == 0) {
        // warm-up: full-size waves of both kinds on every lane
        if (stream(njobs, lanes, threads, by_prep, &err) < 0 || stream(njobs, lanes, threads, by_bytes, &err) < 0)
            rc = 1;
        for (int rep = 0; rep < 2 && rc == 0; rep++) {
            wc_service_stats(svc, &w0, &g);
            const double a = stream(njobs, waves, threads, by_prep, &err);
            wc_service_stats(svc, &w1, &g);
            waves_prep += w1 - w0;
            const double b2 = a < 0 ? -1.0 : stream(njobs, waves, threads, by_bytes, &err);
            wc_service_stats(svc, &w0, &g);
            waves_bytes += w0 - w1;
            if (a < 0 || b2 < 0) rc = 1;
            dp += a;
            db += b2;
        }
        if (rc) std::fprintf(stderr, "%s\n", err.c_str());
    }
    for (wc_prepared* p : prepared)
        if (p) wc_prepared_free(p);
    wc_service_destroy(svc);
    if (rc) return rc;
    dp /= 2;
    db /= 2;
    std::printf("{\"waves\": %u, \"jobs_per_wave\": %zu, \"lanes\": %u, \"submit_threads\": %u, "
                "\"ms_per_wave\": %.3f, \"bytes_ms_per_wave\": %.3f, \"prepare_ms_once\": %.1f, "
                "\"device_waves\": %.1f, \"bytes_device_waves\": %.1f}\n",
                waves, njobs, lanes, threads, dp / waves * 1e3, db / waves * 1e3, prep_ms, waves_prep / 2.0,
                waves_bytes / 2.0);
    return 0;
}
