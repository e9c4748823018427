// Solve service: submission queue, lanes, wave formation, weight versions,
// cost classes and guarded routes.
#include "service.h"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iterator>
#include <limits>
#include <thread>

#include "../../include/wc_wave.h"
#include "kernels.h"
#include "par.h"

namespace wc {

namespace {

constexpr uint64_t U64_MAX = std::numeric_limits<uint64_t>::max();

uint64_t sat_add(uint64_t a, uint64_t b) { return a > U64_MAX - b ? U64_MAX : a + b; }
uint64_t sat_mul(uint64_t a, uint64_t b) { return a && b > U64_MAX / a ? U64_MAX : a * b; }
uint64_t sat_sub(uint64_t a, uint64_t b) { return a > b ? a - b : 0; }
// usize::checked_next_power_of_two().unwrap_or(x)
uint64_t next_pow2_or_self(uint64_t x) {
    if (x <= 1) return 1;
    uint64_t p = 1;
    while (p < x) {
        if (p > U64_MAX / 2) return x;
        p <<= 1;
    }
    return p;
}
uint64_t align256(uint64_t x) { return (x + 255) & ~uint64_t(255); }

// `PackedTables::owned_bytes` (engine/src/serialize.rs:642-686): the bytes of
// every array the job owns.
uint64_t owned_bytes(const Tables& t) {
    const uint64_t u8s = t.node_kind.size() + t.node_player.size() + t.leaf_raw.size() + t.cplayer.size();
    const uint64_t u32s = t.node_child_start.size() + t.node_child.size() + t.obs_off.size() + t.obs_start.size() +
                          t.obs_act.size() + t.obs_child.size() + t.legal_row_of.size() + t.legal_off.size() +
                          t.legal_action.size() + t.legal_child.size() + t.legal_trans.size() + t.cell_row.size() +
                          t.draw_off.size() + t.draw_to.size() + t.draw_row_off.size() + t.draw_row_start.size() +
                          t.cfg_off.size() + t.reach_off.size() + t.soff.size() + t.node_parent.size() +
                          t.rev_row_of.size() + t.rev_start.size() + t.rev_src.size() + t.rev_cell.size() +
                          t.rvd_row_of.size() + t.rvd_start.size() + t.rvd_src.size() + t.leaf_rows.size() +
                          t.term_leaves.size() + t.leaf_coff.size() + t.leaf_cidx.size() + t.snap_coff.size() +
                          t.bfs_order.size() + t.level_start.size();
    const uint64_t f32s = t.draw_p.size() + t.rvd_p.size() + t.terminal_utility.size() + t.card_feat.size() +
                          t.cphi.size();
    return u8s + 4 * (u32s + f32s);
}

// `device_reach_slots` (engine/src/serialize.rs:432-445): the root's configs of
// both players, then per node the configs of the player who acted at its parent.
uint64_t reach_slots(const Tables& t) {
    if (t.nodes == 0) return 0;
    uint64_t slots = sat_add(t.nc(0, 0), t.nc(0, 1));
    for (uint32_t i = 1; i < t.nodes; i++) slots = sat_add(slots, t.nc(i, t.node_player[t.node_parent[i]]));
    return slots;
}

// The value span: per player, every node but the chance nodes the player does
// not draw at (they alias their child, engine/src/serialize.rs:447-480); the
// two players share the longer span.
uint64_t value_slots(const Tables& t) {
    uint64_t len[2] = {0, 0};
    for (int p = 0; p < 2; p++)
        for (uint32_t i = 0; i < t.nodes; i++)
            if (!(t.node_kind[i] == 1 && t.node_player[i] != p)) len[p] += t.nc(i, p);
    return std::max(len[0], len[1]);
}

// This executor's device memory for the job as a one-job wave: the mutable
// arena (CFR state, reach, values, masses, outputs) and the leaf-net buffers,
// each reserved at a power of two as Executor::ensure reserves them. The
// two-tower readout block is bounded by rows x interned configs.
uint64_t device_arena_bytes(const Job& j, int precision) {
    const Tables& t = j.t;
    NetShape ns;
    std::string err;
    if (!ns.parse(j.meta.net_dims, &err)) return U64_MAX;
    const uint64_t cells = std::max<uint64_t>(t.ncells, 1), reach = std::max<uint64_t>(reach_slots(t), 1),
                   vals = std::max<uint64_t>(value_slots(t), 1), rows = t.rows;
    const uint64_t roots = uint64_t(j.nroots()) * (j.root[0].size() + j.root[1].size());
    const uint64_t snaps = j.meta.snapshots && !j.meta.snap_iters.empty() ? j.meta.snap_iters.size() - 1 : 0;
    uint64_t arena = 0;
    auto take = [](uint64_t* at, uint64_t bytes) { *at = sat_add(align256(*at), std::max<uint64_t>(bytes, 4)); };
    for (int k = 0; k < 4; k++) take(&arena, sat_mul(cells, 4));
    take(&arena, sat_mul(reach, 4));
    take(&arena, sat_mul(reach, 4));
    take(&arena, sat_mul(vals, 4));
    take(&arena, sat_mul(rows, 8));
    take(&arena, sat_mul(roots, 4));
    take(&arena, sat_mul(sat_mul(snaps, t.snapshot_configs()), 2));
    const bool tower = ns.kind == MODEL_TWO_TOWER;
    const uint64_t esz = precision == WC_PRECISE || precision == WC_F16X ? 4 : 2;
    const uint64_t prow = precision == WC_PRECISE ? rows : (rows + GEMM_ROWS - 1) / GEMM_ROWS * GEMM_ROWS;
    const uint64_t ncfg = t.ncfg, pcfg = precision == WC_PRECISE ? ncfg : (ncfg + GEMM_ROWS - 1) / GEMM_ROWS * GEMM_ROWS;
    uint64_t mlp = 0;
    const bool v5net = ns.kind == MODEL_V5;
    const uint64_t xin = v5net && precision != WC_PRECISE ? v5::JOIN_IN_PAD : ns.in;
    take(&mlp, sat_mul(sat_mul(prow, xin), esz));
    take(&mlp, sat_mul(sat_mul(prow, xin), esz));
    take(&mlp, sat_mul(sat_mul(prow, ns.hidden), esz));
    take(&mlp, sat_mul(sat_mul(prow, ns.hidden), esz));
    take(&mlp, readout_net(ns.kind) ? sat_mul(sat_mul(rows, ncfg), 4) : sat_mul(sat_mul(rows, ns.heads), 4));
    const bool split = ns.kind == MODEL_MLP && (precision == WC_F16 || precision == WC_BF16) &&
                       chain_fits(ns.in, ns.hidden, ns.layers) && ns.pool > 0 && ns.in > 2 * ns.pool &&
                       (2 * ns.pool) % 32 == 0;
    if (split) {
        take(&mlp, sat_mul(sat_mul(prow, ns.hidden), 4));
        take(&mlp, sat_mul(sat_mul(prow, ns.hidden), 4));
    }
    if (tower) {
        take(&mlp, precision == WC_PRECISE ? 0 : sat_mul(sat_mul(pcfg, ns.priv_in), esz));
        take(&mlp, sat_mul(sat_mul(pcfg, ns.hidden), esz));
        take(&mlp, sat_mul(sat_mul(pcfg, ns.hidden), esz));
        take(&mlp, sat_mul(sat_mul(ncfg, ns.hidden), esz));
    }
    if (v5net) {  // cards and bag rows, P and Jp, g and f, the join's input scratch
        take(&mlp, 2ull * v5::NTYPE * v5::TYPE * 4);
        take(&mlp, 2ull * v5::NTYPE * 3 * v5::POOL * 4);
        take(&mlp, sat_mul(rows, v5::D * 4));
        take(&mlp, sat_mul(rows, v5::JW * 4));
        take(&mlp, sat_mul(ncfg, v5::POOL * 4));
        take(&mlp, sat_mul(ncfg, v5::D * esz));
        take(&mlp, precision == WC_PRECISE ? 0 : sat_mul(rows, v5::JOIN_IN * 4));
    }
    return sat_add(next_pow2_or_self(arena), next_pow2_or_self(mlp));
}

}  // namespace

uint64_t WorkVector::reserved_bytes() const { return sat_add(mutable_bytes, next_pow2_or_self(table_bytes)); }
bool WorkVector::requires_exclusive_route(uint64_t unit) const { return reserved_bytes() >= sat_mul(4, unit); }
bool WorkVector::requires_arena_guard_route(uint64_t unit) const {
    return mutable_bytes >= sat_mul(4, unit) && !requires_card_exclusive_route(unit);
}
bool WorkVector::requires_card_exclusive_route(uint64_t unit) const { return reserved_bytes() >= sat_mul(6, unit); }

// PackedJob::work (engine/src/serialize.rs:394-431).
WorkVector work_vector(const Job& j, int precision) {
    const Tables& t = j.t;
    WorkVector w;
    w.network_rows = t.rows;
    w.legal_cells = t.ncells;
    w.reach_slots = reach_slots(t);
    w.reverse_nonzeros = t.rev_src.size() + t.rvd_src.size();
    const uint64_t root_configs = t.cfg_off.size() > 2 ? uint64_t(t.cfg_off[2]) - t.cfg_off[0] : 0;
    // owned tables, the reach offsets' second player (2 nodes - len(reach_off)
    // words), the root beliefs and the carried roots
    w.table_bytes = sat_add(sat_add(owned_bytes(t), sat_mul(sat_sub(sat_mul(2, t.nodes), t.reach_off.size()), 4)),
                            4 * (j.root[0].size() + j.root[1].size()) + 4 * uint64_t(j.nroots()) * root_configs);
    w.mutable_bytes = device_arena_bytes(j, precision);
    const uint64_t fp32_output = sat_mul(sat_add(t.ncells, sat_mul(j.nroots(), root_configs)), 4);
    const uint64_t fp16_carry = sat_mul(sat_mul(sat_sub(j.meta.snap_iters.size(), 1), t.snapshot_configs()), 2);
    w.carried_output_bytes = sat_add(fp32_output, fp16_carry);
    w.levels = t.nlevels();
    return w;
}

uint64_t job_cost(const WorkVector& w, uint32_t iters) {
    const uint64_t it = std::max<uint32_t>(iters, 1);
    uint64_t c = sat_mul(sat_mul(w.network_rows, it), 16);
    c = sat_add(c, sat_mul(w.legal_cells, it));
    c = sat_add(c, sat_mul(w.reach_slots, it));
    c = sat_add(c, w.table_bytes / 16);
    return std::max<uint64_t>(c, 1);
}

uint8_t cost_class(const WorkVector& w, uint32_t shift, uint64_t unit) {
    const uint64_t bytes = sat_add(sat_add(w.table_bytes, w.mutable_bytes), w.carried_output_bytes);
    if (w.requires_exclusive_route(unit) || w.legal_cells >= 8000000) return 31;
    const uint64_t work = std::max({w.network_rows, w.legal_cells / 8, w.reach_slots / 16, w.reverse_nonzeros / 16,
                                    uint64_t(1)});
    uint8_t c;
    if (bytes >= (uint64_t(512) << 20) || work >= 4000000)
        c = 3;
    else if (bytes >= (uint64_t(64) << 20) || work >= 500000)
        c = 2;
    else if (bytes >= (uint64_t(16) << 20) || work >= 125000)
        c = 1;
    else
        c = 0;
    return (uint8_t)(c >> std::min<uint32_t>(shift, 2));
}

Service::Service(int device, int precision, const ServiceOpts& opts)
    : device_(device), precision_(precision), opts_(opts) {
    if (opts_.lanes == 0) opts_.lanes = 1;
    if (opts_.lanes > 12) opts_.lanes = 12;  // the reference clamps lanes to 1..12
    if (opts_.wave_jobs == 0) opts_.wave_jobs = 1;
    opts_.whale_lanes = std::min(std::max<uint32_t>(opts_.whale_lanes, 1), opts_.lanes);
    opts_.class_shift = std::min<uint32_t>(opts_.class_shift, 2);
    if (opts_.route_unit == 0) opts_.route_unit = WorkVector::ROUTE_UNIT;
    if (const char* env = std::getenv("WC_SERVICE_PROFILE")) profile_ = std::strcmp(env, "0") != 0;
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

bool prepare(const uint8_t* bytes, size_t len, int precision, std::shared_ptr<const Prepared>* out, std::string* err) {
    auto job = std::make_shared<Job>();
    if (!from_bytes(bytes, len, job.get(), err)) return false;
    if (!validate(*job, err)) return false;
    NetShape ns;
    if (!ns.parse(job->meta.net_dims, err)) return false;
    auto p = std::make_shared<Prepared>();
    p->work = work_vector(*job, precision);
    p->cost = job_cost(p->work, job->meta.iters);
    p->precision = precision;
    p->job = std::move(job);
    *out = std::move(p);
    return true;
}

bool Service::submit(const uint8_t* bytes, size_t len, uint64_t tag, std::shared_ptr<Ticket>* out,
                     std::string* err) {
    std::shared_ptr<const Prepared> prep;
    if (!prepare(bytes, len, precision_, &prep, err)) return false;
    return submit_prepared(prep, tag, out, err);
}

bool Service::submit_prepared(const std::shared_ptr<const Prepared>& prep, uint64_t tag,
                              std::shared_ptr<Ticket>* out, std::string* err) {
    if (!prep || !prep->job) {
        *err = "no prepared job";
        return false;
    }
    if (prep->precision != precision_) {
        *err = "the job was prepared for precision " + std::to_string(prep->precision) + ", the service runs " +
               std::to_string(precision_);
        return false;
    }
    Pending p;
    p.job = prep->job;
    p.rows = p.job->t.rows;
    p.work = prep->work;
    return enqueue(std::move(p), tag, prep->cost, out, err);
}

bool Service::enqueue(Pending&& p, uint64_t tag, uint64_t cost, std::shared_ptr<Ticket>* out, std::string* err) {
    p.cls = cost_class(p.work, opts_.class_shift, opts_.route_unit);
    p.ticket = std::make_shared<Ticket>();
    p.ticket->tag = tag;
    p.ticket->cost = cost;
    p.ticket->oversize = p.work.requires_exclusive_route(opts_.route_unit);
    p.ticket->card = p.work.requires_card_exclusive_route(opts_.route_unit);
    std::shared_ptr<Ticket> t = p.ticket;
    {
        std::lock_guard<std::mutex> lk(mu_);
        if (stop_) {
            *err = "GPU wave executor is gone";
            return false;
        }
        p.net = current_;
        p.seq = ++next_seq_;
        p.queued = std::chrono::steady_clock::now();
        queued_.fetch_add(t->cost, std::memory_order_relaxed);
        queue_.push_back(std::move(p));
    }
    cv_.notify_all();  // lanes differ in which jobs they may take
    *out = t;
    return true;
}

// Exclusive-route jobs go to the whale lanes only (engine/src/gpu/service.rs:354-372).
long Service::first_for(uint32_t lane) const {
    for (size_t i = 0; i < queue_.size(); i++)
        if (lane < opts_.whale_lanes || !queue_[i].work.requires_exclusive_route(opts_.route_unit)) return (long)i;
    return -1;
}

// Bucket a seed with compatible followers: the same weight version, cost
// class and schedule metadata, at most wave_jobs jobs and wave_rows network
// rows, filling until window_us after the seed was queued; a class-31 seed runs alone
// (engine/src/gpu/service.rs:554-637).
void Service::fill_wave(std::unique_lock<std::mutex>& lk, uint32_t lane, long seed, std::vector<Pending>* wave) {
    wave->push_back(std::move(queue_[(size_t)seed]));
    queue_.erase(queue_.begin() + seed);
    const Pending& head = wave->front();
    const auto seed_queued = head.queued;
    if (head.cls == 31) return;
    const Meta hm = head.job->meta;
    const uint64_t hv = head.net->version;
    const uint8_t hc = head.cls;
    size_t rows = head.rows;
    auto compatible = [&](const Pending& q) {
        const Meta& m = q.job->meta;
        return q.net->version == hv && q.cls == hc && m.iters == hm.iters && m.snapshots == hm.snapshots &&
               m.snap_iters == hm.snap_iters && m.net_dims == hm.net_dims && m.depth == hm.depth &&
               std::memcmp(&m.cfr, &hm.cfr, sizeof(Cfr)) == 0;
    };
    // A job once passed over stays passed over (compatibility is fixed and the
    // wave's rows only grow), so each sweep examines only jobs that arrived
    // since the last one, and closes the gaps it leaves in one pass: a burst
    // of thousands of queued jobs costs each filling lane linear work, not a
    // rescan per wake-up and a deque shift per job taken.
    uint64_t seen = 0;
    auto sweep = [&]() {
        const size_t from = (size_t)(std::partition_point(queue_.begin(), queue_.end(),
                                                          [&](const Pending& q) { return q.seq <= seen; }) -
                                     queue_.begin());
        size_t keep = from;
        for (size_t i = from; i < queue_.size(); i++) {
            Pending& q = queue_[i];
            if (wave->size() < opts_.wave_jobs) {
                seen = q.seq;
                if (compatible(q) && rows + q.rows <= opts_.wave_rows) {
                    rows += q.rows;
                    wave->push_back(std::move(q));
                    continue;
                }
            }
            if (keep != i) queue_[keep] = std::move(q);
            keep++;
        }
        queue_.erase(queue_.begin() + (long)keep, queue_.end());
    };
    // The fill window runs from the seed's arrival, not from now: a seed that
    // has already waited that long in the queue (a burst of submissions)
    // starts its wave with what is there (engine/src/gpu/service.rs:587-593).
    const auto deadline = seed_queued + std::chrono::microseconds(opts_.window_us);
    for (;;) {
        sweep();
        if (wave->size() >= opts_.wave_jobs || stop_ || (guard_ && guard_lane_ != lane)) break;
        if (cv_.wait_until(lk, deadline) == std::cv_status::timeout) {
            sweep();
            break;
        }
    }
}

void Service::answer(Flight& fl, bool ok, std::vector<Result>* results, std::string err) {
    if (ok && results->size() != fl.tickets.size()) {
        ok = false;
        err = "GPU wave returned " + std::to_string(results->size()) + " results for " +
              std::to_string(fl.tickets.size()) + " jobs";
    }
    for (size_t k = 0; k < fl.tickets.size(); k++) {
        auto& t = fl.tickets[k];
        {
            std::lock_guard<std::mutex> lk(t->mu);
            if (ok) {
                t->result = std::move((*results)[k]);
                t->result.tag = t->tag;
                t->result.weight_version = fl.version;
                t->result.oversize_route = t->oversize;
                t->result.card_exclusive_route = t->card;
                t->rc = 0;
            } else {
                t->rc = WC_ERR_DEVICE;
                t->err = err;
            }
            t->done = true;
        }
        t->cv.notify_all();
        queued_.fetch_sub(t->cost, std::memory_order_relaxed);
    }
    fl.tickets.clear();
}

void Service::lane_main(uint32_t lane) {
    // packing and staging copies draw on the process's shared host pool: a
    // lane packing a large wave gets the cores the other lanes leave idle
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
            uint64_t v = ex->publish(net->ns, net->dims, net->w.data(), net->w.size(), net->b.data(), net->b.size(), &err,
                                     net->ln.data(), net->ln.size());
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
    // Two waves may fly at once: the lane packs and launches wave N + 1 while
    // wave N runs, then answers wave N (the reference's launch / land split,
    // engine/src/gpu/service.rs:546-742). The packed wave is reused: launch
    // keeps what the unpack needs.
    WaveHost wh;
    Flight fl[2];
    uint32_t last = 1;  // the flight launched most recently
    auto land = [&](Flight& F) {
        if (!F.f.live) return;
        std::vector<Result> res;
        std::string err;
        const auto t_collect = std::chrono::steady_clock::now();
        const bool ok = ex->collect(&F.f, &res, &err);
        if (profile_) {
            // the reference's per-wave line (engine/src/gpu/service.rs:795-806):
            // launch_ms is the launch call (staging copy, upload and schedule
            // enqueued), flight_ms runs from the launch to the results on the
            // host, collect_ms is the collection (waiting for the device, then
            // the results unpacked)
            const auto now = std::chrono::steady_clock::now();
            const double flight_ms = std::chrono::duration<double, std::milli>(now - F.launched).count();
            const double collect_ms = std::chrono::duration<double, std::milli>(now - t_collect).count();
            std::fprintf(stderr,
                         "wc_service device=%d lane=%u class=%u jobs=%zu rows=%zu oldest_ms=%.2f pack_ms=%.2f "
                         "launch_ms=%.2f flight_ms=%.2f collect_ms=%.2f\n",
                         device_, lane, (unsigned)F.cls, F.tickets.size(), F.rows, F.oldest_ms, F.pack_ms,
                         F.launch_ms, flight_ms, collect_ms);
        }
        answer(F, ok, &res, err);
    };
    auto land_all = [&]() {
        land(fl[last ^ 1]);  // the older flight first
        land(fl[last]);
    };
    uint64_t my_epoch = 0;
    for (;;) {
        std::vector<Pending> wave;
        bool guarded = false;
        {
            std::unique_lock<std::mutex> lk(mu_);
            long seed = -1;
            for (;;) {
                if (stop_) break;
                if (guard_ && guard_lane_ != lane) {
                    // Another lane's guarded route holds the device: land, trim once, wait.
                    if (my_epoch != trim_epoch_) {
                        lk.unlock();
                        land_all();
                        std::string e;
                        ex->trim(&e);
                        lk.lock();
                        my_epoch = trim_epoch_;
                        trimmed_++;
                        cv_.notify_all();
                        continue;
                    }
                    cv_.wait(lk);
                    continue;
                }
                seed = first_for(lane);
                if (seed >= 0) break;
                if (fl[0].f.live || fl[1].f.live) {  // nothing to start: answer what is flying
                    lk.unlock();
                    land_all();
                    lk.lock();
                    continue;
                }
                cv_.wait(lk);
            }
            if (stop_) {
                lk.unlock();
                land_all();
                break;
            }
            fill_wave(lk, lane, seed, &wave);
            const WorkVector& w0 = wave.front().work;
            guarded = w0.requires_arena_guard_route(opts_.route_unit) || w0.requires_card_exclusive_route(opts_.route_unit);
            if (guarded) {
                guard_ = true;
                guard_lane_ = lane;
                trimmed_ = 0;
                my_epoch = ++trim_epoch_;
                cv_.notify_all();
            }
        }
        if (guarded) {  // engine/src/gpu/service.rs:452-532: drain and trim every lane first
            land_all();
            std::string e;
            ex->trim(&e);
            std::unique_lock<std::mutex> lk(mu_);
            cv_.wait(lk, [&] { return stop_ || trimmed_ + 1 >= opts_.lanes; });
            guarded_.fetch_add(1, std::memory_order_relaxed);
        }
        std::shared_ptr<const NetCopy> net = wave.front().net;
        std::string err;
        bool ok = true;
        uint64_t exv = 0;
        auto found = bank_of.find(net->version);
        if (found == bank_of.end()) {
            exv = ex->publish(net->ns, net->dims, net->w.data(), net->w.size(), net->b.data(), net->b.size(), &err,
                                     net->ln.data(), net->ln.size());
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
        const uint32_t k = last ^ 1;
        land(fl[k]);  // its slot is needed (normally landed already)
        Flight& F = fl[k];
        std::vector<std::shared_ptr<const Job>> jobs;
        const auto t_pack = std::chrono::steady_clock::now();
        F.cls = wave.front().cls;
        F.rows = 0;
        F.oldest_ms = 0;
        for (auto& p : wave) {
            F.tickets.push_back(p.ticket);
            F.rows += p.rows;
            F.oldest_ms = std::max(F.oldest_ms, std::chrono::duration<double, std::milli>(t_pack - p.queued).count());
            jobs.push_back(std::move(p.job));
        }
        F.version = net->version;
        if (ok) {
            // Validated at submit; a wave too large for host memory fails its
            // tickets. The lanes pack without fused top-depth launches: the
            // service is bound by the host, and their planning costs the lane
            // more host time than the launches save on the device.
            try {
                ok = pack_wave(std::move(jobs), &wh, &err, UNIT_SLOTS, true, false);
            } catch (const std::exception& e) {
                ok = false;
                err = std::string("packing the wave failed: ") + e.what();
            }
        }
        F.launched = std::chrono::steady_clock::now();
        F.pack_ms = std::chrono::duration<double, std::milli>(F.launched - t_pack).count();
        // the previous wave is answered while this one's upload is checked on the device
        if (ok) ok = ex->launch(wh, exv, &F.f, &err, [&] { land(fl[k ^ 1]); });
        F.launch_ms =
            std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - F.launched).count();
        if (!ok) {
            std::vector<Result> none;
            answer(F, false, &none, err);
        } else {
            waves_.fetch_add(1, std::memory_order_relaxed);
            last = k;
            if (guarded) land(F);  // the guarded wave runs alone (no other flight is live)
        }
        if (guarded) {
            {
                std::lock_guard<std::mutex> lk(mu_);
                guard_ = false;
            }
            cv_.notify_all();
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
            p.ticket->rc = WC_ERR_GONE;
            p.ticket->err = "GPU wave executor is gone";
            p.ticket->done = true;
        }
        p.ticket->cv.notify_all();
        queued_.fetch_sub(p.ticket->cost, std::memory_order_relaxed);
    }
}

}  // namespace wc
