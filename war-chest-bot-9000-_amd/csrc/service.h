// The solve service: thread-safe submission, lanes that bucket compatible jobs
// into waves, weight versions, backpressure. Counterpart of the reference's
// dispatcher/lanes and client (engine/src/gpu/service.rs:55-742,
// engine/src/gpu/client.rs:196-313).
#pragma once

#include <atomic>
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

struct Ticket {
    std::mutex mu;
    std::condition_variable cv;
    bool done = false;
    int rc = 0;
    std::string err;
    Result result;
    uint64_t tag = 0;
    uint64_t cost = 0;
};

struct ServiceOpts {
    uint32_t lanes = 2, wave_jobs = 64, wave_rows = 49152, window_us = 800;
};

struct NetCopy {
    uint64_t version = 0;
    NetShape ns;
    std::vector<uint32_t> dims;
    std::vector<float> w, b;
};

// `job_cost` (engine/src/gpu/client.rs:282-291): a monotone work estimate.
uint64_t job_cost(const Job& j, size_t bytes);

class Service {
  public:
    Service(int device, int precision, const ServiceOpts& opts);
    ~Service();
    // Starts the lanes and publishes `net` as version 0; blocks until every lane is ready.
    bool start(const NetCopy& net, std::string* err);
    uint64_t set_weights(NetCopy net, std::string* err);
    uint64_t queued_work() const { return queued_.load(std::memory_order_relaxed); }
    bool submit(const uint8_t* bytes, size_t len, uint64_t tag, std::shared_ptr<Ticket>* out, std::string* err);
    void shutdown();

  private:
    struct Pending {
        std::shared_ptr<Ticket> ticket;
        Job job;
        size_t rows = 0;
        std::shared_ptr<const NetCopy> net;  // the weights current when the job was submitted
    };
    void lane_main(uint32_t lane);
    bool take_wave(std::vector<Pending>* wave);

    int device_, precision_;
    ServiceOpts opts_;
    std::vector<std::thread> lanes_;
    std::mutex mu_;
    std::condition_variable cv_;
    std::deque<Pending> queue_;
    bool stop_ = false;
    std::atomic<uint64_t> queued_{0};
    std::shared_ptr<const NetCopy> current_;  // newest published weights
    uint64_t next_version_ = 0;
    // lane start-up handshake
    std::mutex ready_mu_;
    std::condition_variable ready_cv_;
    uint32_t ready_ = 0, failed_ = 0;
    std::string start_err_;
};

}  // namespace wc
