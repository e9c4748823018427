// Solve service: submission queue, lanes, wave formation, weight versions.
#include "service.h"

#include <algorithm>
#include <chrono>
#include <cstring>
#include <iterator>

namespace wc {

uint64_t job_cost(const Job& j, size_t bytes) {
    const Tables& t = j.t;
    uint64_t iters = std::max<uint32_t>(j.meta.iters, 1);
    // Reach slots the device keeps (engine/src/serialize.rs:431-443).
    uint64_t slots = t.nodes ? uint64_t(t.nc(0, 0)) + t.nc(0, 1) : 0;
    for (uint32_t i = 1; i < t.nodes; i++) slots += t.nc(i, t.node_player[t.node_parent[i]]);
    uint64_t c = uint64_t(t.rows) * iters * 16 + uint64_t(t.ncells) * iters + slots * iters + bytes / 16;
    return std::max<uint64_t>(c, 1);
}

Service::Service(int device, int precision, const ServiceOpts& opts)
    : device_(device), precision_(precision), opts_(opts) {
    if (opts_.lanes == 0) opts_.lanes = 1;
    if (opts_.lanes > 12) opts_.lanes = 12;  // the reference clamps lanes to 1..12
    if (opts_.wave_jobs == 0) opts_.wave_jobs = 1;
}

Service::~Service() { shutdown(); }

bool Service::start(const NetCopy& net, std::string* err) {
    auto first = std::make_shared<NetCopy>(net);
    first->version = next_version_++;
    current_ = first;
    for (uint32_t l = 0; l < opts_.lanes; l++) lanes_.emplace_back(&Service::lane_main, this, l);
    std::unique_lock<std::mutex> lk(ready_mu_);
    ready_cv_.wait(lk, [&] { return ready_ + failed_ == opts_.lanes; });
    if (failed_) {
        *err = start_err_;
        lk.unlock();
        shutdown();
        return false;
    }
    return true;
}

uint64_t Service::set_weights(NetCopy net, std::string* err) {
    std::lock_guard<std::mutex> lk(mu_);
    if (stop_) {
        *err = "GPU wave executor is gone";
        return 0;
    }
    auto copy = std::make_shared<NetCopy>(std::move(net));
    copy->version = next_version_++;
    // Jobs already queued keep the version they were submitted under
    // (engine/src/gpu/service.rs:233); each holds its own reference to it.
    current_ = copy;
    return copy->version;
}

bool Service::submit(const uint8_t* bytes, size_t len, uint64_t tag, std::shared_ptr<Ticket>* out,
                     std::string* err) {
    Pending p;
    if (!from_bytes(bytes, len, &p.job, err)) return false;
    if (!validate(p.job, err)) return false;
    NetShape ns;
    if (!ns.parse(p.job.meta.net_dims, err)) return false;
    p.rows = p.job.t.rows;
    p.ticket = std::make_shared<Ticket>();
    p.ticket->tag = tag;
    p.ticket->cost = job_cost(p.job, len);
    std::shared_ptr<Ticket> t = p.ticket;
    {
        std::lock_guard<std::mutex> lk(mu_);
        if (stop_) {
            *err = "GPU wave executor is gone";
            return false;
        }
        p.net = current_;
        queued_.fetch_add(t->cost, std::memory_order_relaxed);
        queue_.push_back(std::move(p));
    }
    cv_.notify_one();
    *out = t;
    return true;
}

// Bucket the queue head with compatible followers: same schedule metadata, at
// most wave_jobs jobs and wave_rows network rows, filling for up to window_us
// (engine/src/gpu/service.rs:554-637).
bool Service::take_wave(std::vector<Pending>* wave) {
    std::unique_lock<std::mutex> lk(mu_);
    cv_.wait(lk, [&] { return stop_ || !queue_.empty(); });
    if (stop_) return false;
    auto deadline = std::chrono::steady_clock::now() + std::chrono::microseconds(opts_.window_us);
    size_t rows = 0;
    const Meta head = queue_.front().job.meta;
    const uint64_t head_version = queue_.front().net->version;
    // One wave runs one schedule under one weight version (service.rs:626).
    auto compatible = [&](const Pending& q) {
        const Meta& m = q.job.meta;
        return q.net->version == head_version && m.iters == head.iters && m.snapshots == head.snapshots &&
               m.snap_iters == head.snap_iters && m.net_dims == head.net_dims && m.depth == head.depth &&
               std::memcmp(&m.cfr, &head.cfr, sizeof(Cfr)) == 0;
    };
    for (;;) {
        for (auto it = queue_.begin(); it != queue_.end() && wave->size() < opts_.wave_jobs;) {
            if (compatible(*it) && (wave->empty() || rows + it->rows <= opts_.wave_rows)) {
                rows += it->rows;
                wave->push_back(std::move(*it));
                it = queue_.erase(it);
            } else {
                ++it;
            }
        }
        if (wave->size() >= opts_.wave_jobs || stop_) break;
        if (cv_.wait_until(lk, deadline) == std::cv_status::timeout) {
            for (auto it = queue_.begin(); it != queue_.end() && wave->size() < opts_.wave_jobs;) {
                if (compatible(*it) && rows + it->rows <= opts_.wave_rows) {
                    rows += it->rows;
                    wave->push_back(std::move(*it));
                    it = queue_.erase(it);
                } else {
                    ++it;
                }
            }
            break;
        }
    }
    return true;
}

void Service::lane_main(uint32_t lane) {
    (void)lane;
    std::unique_ptr<Executor> ex(new Executor(device_, precision_));
    std::map<uint64_t, uint64_t> bank_of;  // service version -> executor version
    {
        std::string err;
        bool ok = ex->ok();
        if (!ok) err = ex->error();
        std::shared_ptr<const NetCopy> net;
        {
            std::lock_guard<std::mutex> lk(mu_);
            net = current_;
        }
        if (ok && net) {
            uint64_t v = ex->publish(net->ns, net->dims, net->w.data(), net->w.size(), net->b.data(), net->b.size(), &err);
            ok = v != 0;
            if (ok) bank_of[net->version] = v;
        }
        std::lock_guard<std::mutex> lk(ready_mu_);
        if (ok)
            ready_++;
        else {
            failed_++;
            start_err_ = "lane start-up failed: " + err;
        }
        ready_cv_.notify_all();
        if (!ok) return;
    }
    WaveHost wh;  // reused wave to wave: its lists keep their buffers
    for (;;) {
        std::vector<Pending> wave;
        if (!take_wave(&wave)) break;
        if (wave.empty()) continue;
        std::shared_ptr<const NetCopy> net = wave.front().net;
        std::string err;
        bool ok = true;
        uint64_t exv = 0;
        auto found = bank_of.find(net->version);
        if (found == bank_of.end()) {
            exv = ex->publish(net->ns, net->dims, net->w.data(), net->w.size(), net->b.data(), net->b.size(), &err);
            ok = exv != 0;
            if (ok) {
                bank_of[net->version] = exv;
                // keep the three newest banks on this lane; an older version
                // still queued is published again when its wave comes
                while (bank_of.size() > 3) {
                    ex->retain_from(std::next(bank_of.begin())->second);
                    bank_of.erase(bank_of.begin());
                }
            }
        } else {
            exv = found->second;
        }
        std::vector<Result> results;
        std::vector<std::shared_ptr<Ticket>> tickets;
        std::vector<Job> jobs;
        for (auto& p : wave) {
            tickets.push_back(p.ticket);
            jobs.push_back(std::move(p.job));
        }
        if (ok) ok = pack_wave(std::move(jobs), &wh, &err, UNIT_SLOTS, true);  // validated at submit
        if (ok) ok = ex->solve(wh, exv, &results, &err);
        for (size_t k = 0; k < tickets.size(); k++) {
            auto& t = tickets[k];
            {
                std::lock_guard<std::mutex> lk(t->mu);
                if (ok) {
                    t->result = std::move(results[k]);
                    t->result.tag = t->tag;
                    t->result.weight_version = net->version;
                    t->rc = 0;
                } else {
                    t->rc = -2;
                    t->err = err;
                }
                t->done = true;
            }
            t->cv.notify_all();
            queued_.fetch_sub(t->cost, std::memory_order_relaxed);
        }
    }
}

void Service::shutdown() {
    {
        std::lock_guard<std::mutex> lk(mu_);
        if (stop_ && lanes_.empty()) return;
        stop_ = true;
    }
    cv_.notify_all();
    for (auto& th : lanes_)
        if (th.joinable()) th.join();
    lanes_.clear();
    std::deque<Pending> left;
    {
        std::lock_guard<std::mutex> lk(mu_);
        left.swap(queue_);
    }
    for (auto& p : left) {
        {
            std::lock_guard<std::mutex> lk(p.ticket->mu);
            p.ticket->rc = -3;
            p.ticket->err = "GPU wave executor is gone";
            p.ticket->done = true;
        }
        p.ticket->cv.notify_all();
        queued_.fetch_sub(p.ticket->cost, std::memory_order_relaxed);
    }
}

}  // namespace wc
