// The solve service: thread-safe submission, lanes that bucket compatible jobs
// into waves, weight versions, backpressure, cost classes and guarded routes
// for very large jobs. Counterpart of the reference's dispatcher, lanes, route
// worker and client (engine/src/gpu/service.rs:55-991,
// engine/src/gpu/client.rs:165-313).
#pragma once

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdint>
#include <deque>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "executor.h"
#include "job.h"

namespace wc {

// `WorkVector` (engine/src/serialize.rs:159-201,394-431): the admission and
// scheduling cost of one job, in work units and bytes.
struct WorkVector {
    uint64_t network_rows = 0, legal_cells = 0, reach_slots = 0, reverse_nonzeros = 0;
    uint64_t table_bytes = 0;          // the job's owned tables, roots and carried roots
    uint64_t mutable_bytes = 0;        // this executor's one-job device arena, power-of-two reserved
    uint64_t carried_output_bytes = 0; // strategy, root values and f16 carries
    uint64_t levels = 0;
    // The device reservation: the arena plus the tables rounded up to a power of two.
    uint64_t reserved_bytes() const;
    // Route thresholds are in units of `unit` bytes (1 GiB in the reference;
    // tests lower it to route small jobs).
    // A job that needs a one-job wave on a whale lane (reservation >= 4 units).
    bool requires_exclusive_route(uint64_t unit = ROUTE_UNIT) const;
    // A four-unit arena: runs alone after the other lanes have drained and trimmed.
    bool requires_arena_guard_route(uint64_t unit = ROUTE_UNIT) const;
    // A reservation >= 6 units: drains and trims the whole device around it.
    bool requires_card_exclusive_route(uint64_t unit = ROUTE_UNIT) const;
    static constexpr uint64_t ROUTE_UNIT = uint64_t(1) << 30;
};

// `PackedJob::work` for a job run by an executor of `precision`.
WorkVector work_vector(const Job& j, int precision);
// `job_cost` (engine/src/gpu/client.rs:282-291): a monotone work estimate with
// saturating arithmetic.
uint64_t job_cost(const WorkVector& w, uint32_t iters);
// `cost_class` (engine/src/gpu/service.rs:967-991): only jobs of one class
// share a wave; class 31 runs alone. `shift` (WARCHEST_WAVE_CLASS_SHIFT,
// 0..2) coarsens the ordinary classes.
uint8_t cost_class(const WorkVector& w, uint32_t shift, uint64_t unit = WorkVector::ROUTE_UNIT);

// PreparedJob (engine/src/gpu/client.rs:165-181): an immutable job with its
// admission vector and cost computed once for an executor precision; cheap
// to share between submissions.
struct Prepared {
    std::shared_ptr<const Job> job;
    WorkVector work;
    uint64_t cost = 0;
    int precision = 0;
};
// Parse, validate and cost one WCJ8 job for `precision`.
bool prepare(const uint8_t* bytes, size_t len, int precision, std::shared_ptr<const Prepared>* out, std::string* err);

struct Ticket {
    std::mutex mu;
    std::condition_variable cv;
    bool done = false;
    int rc = 0;
    std::string err;
    Result result;
    uint64_t tag = 0;
    uint64_t cost = 0;
    bool oversize = false, card = false;  // the job's routes, reported in its result
};

struct ServiceOpts {
    uint32_t lanes = 2, wave_jobs = 64, wave_rows = 49152, window_us = 800;
    uint32_t whale_lanes = 1;  // lanes that take exclusive-route jobs (WARCHEST_WAVE_WHALE_LANES)
    uint32_t class_shift = 0;  // WARCHEST_WAVE_CLASS_SHIFT
    uint64_t route_unit = WorkVector::ROUTE_UNIT;
};

struct NetCopy {
    uint64_t version = 0;
    NetShape ns;
    std::vector<uint32_t> dims;
    std::vector<float> w, b, ln;
};

class Service {
  public:
    Service(int device, int precision, const ServiceOpts& opts);
    ~Service();
    // Starts the lanes and publishes `net` as version 0; blocks until every lane is ready.
    bool start(const NetCopy& net, std::string* err);
    uint64_t set_weights(NetCopy net, std::string* err);
    uint64_t queued_work() const { return queued_.load(std::memory_order_relaxed); }
    bool submit(const uint8_t* bytes, size_t len, uint64_t tag, std::shared_ptr<Ticket>* out, std::string* err);
    // GpuClient::submit_prepared (engine/src/gpu/client.rs:212-221): a job
    // parsed, validated and costed once (Prepared), shared, not copied.
    bool submit_prepared(const std::shared_ptr<const struct Prepared>& job, uint64_t tag, std::shared_ptr<Ticket>* out,
                         std::string* err);
    int precision() const { return precision_; }
    void shutdown();
    // Waves launched so far and guarded routes taken (for tests and tooling).
    uint64_t waves() const { return waves_.load(std::memory_order_relaxed); }
    uint64_t guarded_routes() const { return guarded_.load(std::memory_order_relaxed); }

  private:
    struct Pending {
        std::shared_ptr<Ticket> ticket;
        std::shared_ptr<const Job> job;
        WorkVector work;
        uint8_t cls = 0;
        size_t rows = 0;
        std::shared_ptr<const NetCopy> net;  // the weights current when the job was submitted
        uint64_t seq = 0;                    // arrival order: the queue is sorted by it
        std::chrono::steady_clock::time_point queued;
    };
    // One launched wave of a lane: its tickets, weight version and executor record.
    struct Flight {
        InFlight f;
        std::vector<std::shared_ptr<Ticket>> tickets;
        uint64_t version = 0;
        // for the per-wave profile line
        uint8_t cls = 0;
        size_t rows = 0;
        double oldest_ms = 0, pack_ms = 0, launch_ms = 0;
        std::chrono::steady_clock::time_point launched;
    };
    bool enqueue(Pending&& p, uint64_t tag, uint64_t cost, std::shared_ptr<Ticket>* out, std::string* err);
    void lane_main(uint32_t lane);
    // Under mu_: the index of the first queued job this lane may seed a wave
    // with, or -1.
    long first_for(uint32_t lane) const;
    void fill_wave(std::unique_lock<std::mutex>& lk, uint32_t lane, long seed, std::vector<Pending>* wave);
    // Completes every ticket of a landed (or failed) wave.
    void answer(Flight& fl, bool ok, std::vector<Result>* results, std::string err);

    int device_, precision_;
    ServiceOpts opts_;
    bool profile_ = false;  // WC_SERVICE_PROFILE: one line per landed wave on stderr
    std::vector<std::thread> lanes_;
    std::mutex mu_;
    std::condition_variable cv_;
    std::deque<Pending> queue_;
    uint64_t next_seq_ = 0;
    bool stop_ = false;
    // Guarded routes (engine/src/gpu/service.rs:452-532): one at a time; the
    // other lanes land their waves, trim their executors once per epoch and
    // wait until it is over.
    bool guard_ = false;
    uint32_t guard_lane_ = 0;
    uint64_t trim_epoch_ = 0;
    uint32_t trimmed_ = 0;
    std::atomic<uint64_t> queued_{0};
    std::atomic<uint64_t> waves_{0}, guarded_{0};
    std::shared_ptr<const NetCopy> current_;  // newest published weights
    uint64_t next_version_ = 0;
    // lane start-up handshake
    std::mutex ready_mu_;
    std::condition_variable ready_cv_;
    uint32_t ready_ = 0, failed_ = 0;
    std::string start_err_;
};

}  // namespace wc
