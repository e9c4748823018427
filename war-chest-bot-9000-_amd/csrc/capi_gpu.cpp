// Device-facing entry points of the C ABI: executor, wave, service, results.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <memory>
#include <string>
#include <type_traits>

#include "../../include/wc_wave.h"
#include "common.h"
#include "par.h"
#include "executor.h"
#include "service.h"
#include "wave.h"

using namespace wc;

struct wc_executor {
    std::unique_ptr<Executor> ex;
};
struct wc_wave {
    WaveHost host;
    bool packed = false;  // false after a failed wc_wave_repack: the lists are partial
};
struct wc_result {
    Result r;
};
struct wc_service {
    std::unique_ptr<Service> svc;
};
struct wc_ticket {
    std::shared_ptr<Ticket> t;
};
struct wc_inflight {
    InFlight f;
};
struct wc_prepared {
    std::shared_ptr<const Prepared> p;
};

namespace {

// Runs an entry point's body, turning a C++ exception (std::bad_alloc from a
// result or job buffer, above all) into a status instead of letting it cross
// the C boundary.
template <class F>
int shielded(const char* what, F&& body) {
    try {
        return body();
    } catch (const std::bad_alloc&) {
        return fail(WC_ERR_DEVICE, std::string(what) + ": out of host memory");
    } catch (const std::exception& e) {
        return fail(WC_ERR_DEVICE, std::string(what) + ": " + e.what());
    } catch (...) {
        return fail(WC_ERR_DEVICE, std::string(what) + ": unknown exception");
    }
}

void hand_out(std::vector<Result>& out, wc_result** results) {
    size_t k = 0;
    try {
        for (; k < out.size(); k++) {
            results[k] = new wc_result;
            results[k]->r = std::move(out[k]);
        }
    } catch (...) {
        for (size_t j = 0; j < k; j++) delete results[j];
        throw;
    }
}

bool read_net(const wc_net_desc* net, NetCopy* out, std::string* err) {
    if (!net || !net->dims || net->ndims == 0 || (!net->w && net->nw) || (!net->b && net->nb)) {
        *err = "network description is incomplete";
        return false;
    }
    out->dims.assign(net->dims, net->dims + net->ndims);
    if (!out->ns.parse(out->dims, err)) return false;
    out->w.assign(net->w, net->w + net->nw);
    out->b.assign(net->b, net->b + net->nb);
    if (net->nln && !net->ln) {
        *err = "network description is incomplete";
        return false;
    }
    out->ln.assign(net->ln, net->ln + net->nln);
    return true;
}

}  // namespace

extern "C" {

int wc_executor_create(int device, int precision, wc_executor** out) {
    if (!out) return fail(WC_ERR_INVALID, "wc_executor_create: null output");
    try {
        auto* e = new wc_executor;
        e->ex.reset(new Executor(device, precision));
        if (!e->ex->ok()) {
            std::string m = e->ex->error();
            delete e;
            return fail(WC_ERR_DEVICE, m);
        }
        *out = e;
    } catch (const std::exception& e) {
        return fail(WC_ERR_DEVICE, e.what());
    }
    return WC_OK;
}

void wc_executor_destroy(wc_executor* ex) { delete ex; }

uint64_t wc_executor_publish(wc_executor* ex, const wc_net_desc* net) {
    if (!ex) {
        fail(WC_ERR_INVALID, "wc_executor_publish: null executor");
        return 0;
    }
    uint64_t v = 0;
    shielded("wc_executor_publish", [&] {
        NetCopy n;
        std::string err;
        if (!read_net(net, &n, &err)) return fail(WC_ERR_INVALID, err);
        v = ex->ex->publish(n.ns, n.dims, n.w.data(), n.w.size(), n.b.data(), n.b.size(), &err, n.ln.data(),
                            n.ln.size());
        return v ? WC_OK : fail(WC_ERR_INVALID, err);
    });
    return v;
}

namespace {

// The jobs of a wave parsed (in parallel), and the subtree-unit budget
// (WC_UNIT_SLOTS tunes it: value slots per unit).
int parse_wave(const char* fn, const uint8_t* const* jobs, const size_t* lens, uint32_t njobs, std::vector<Job>* parsed,
               uint32_t* slots) {
    parsed->assign(njobs, Job{});
    std::vector<std::string> errs(njobs);
    std::vector<uint8_t> bad(njobs, 0);
    parallel_for(njobs, [&](size_t k) {  // jobs parse independently
        if (!jobs[k]) {
            errs[k] = "null job";
            bad[k] = 1;
        } else if (!from_bytes(jobs[k], lens[k], &(*parsed)[k], &errs[k])) {
            bad[k] = 1;
        }
    });
    for (uint32_t k = 0; k < njobs; k++)
        if (bad[k]) return fail(WC_ERR_INVALID, std::string(fn) + ": job " + std::to_string(k) + ": " + errs[k]);
    *slots = UNIT_SLOTS;
    if (const char* env = std::getenv("WC_UNIT_SLOTS")) {
        long v = std::strtol(env, nullptr, 10);
        if (v < 64 || v > (1L << 24)) return fail(WC_ERR_INVALID, "WC_UNIT_SLOTS out of range [64, 2^24]");
        *slots = (uint32_t)v;
    }
    return WC_OK;
}

// A wave whose last repack failed holds partial lists: nothing may read them.
bool unpacked(const wc_wave* w, const char* fn) {
    if (w->packed) return false;
    fail(WC_ERR_INVALID, std::string(fn) + ": the wave holds no packed jobs (its last repack failed)");
    return true;
}

}  // namespace

int wc_wave_pack(const uint8_t* const* jobs, const size_t* lens, uint32_t njobs, wc_wave** out) {
    if (!jobs || !lens || !out || njobs == 0) return fail(WC_ERR_INVALID, "wc_wave_pack: empty wave");
    return shielded("wc_wave_pack", [&] {
        std::vector<Job> parsed;
        uint32_t slots = 0;
        const int rc = parse_wave("wc_wave_pack", jobs, lens, njobs, &parsed, &slots);
        if (rc != WC_OK) return rc;
        std::string err;
        std::unique_ptr<wc_wave> w(new wc_wave);
        if (!pack_wave(std::move(parsed), &w->host, &err, slots)) return fail(WC_ERR_INVALID, err);
        w->packed = true;
        *out = w.release();
        return WC_OK;
    });
}

int wc_wave_repack(wc_wave* w, const uint8_t* const* jobs, const size_t* lens, uint32_t njobs) {
    if (!w || !jobs || !lens || njobs == 0) return fail(WC_ERR_INVALID, "wc_wave_repack: null argument or empty wave");
    return shielded("wc_wave_repack", [&] {
        std::vector<Job> parsed;
        uint32_t slots = 0;
        const int rc = parse_wave("wc_wave_repack", jobs, lens, njobs, &parsed, &slots);
        if (rc != WC_OK) return rc;  // the wave keeps its jobs
        w->packed = false;
        std::string err;
        if (!pack_wave(std::move(parsed), &w->host, &err, slots)) return fail(WC_ERR_INVALID, err);
        w->packed = true;
        return WC_OK;
    });
}

int wc_wave_digest(const wc_wave* w, uint64_t* out) {
    if (!w || !out) return fail(WC_ERR_INVALID, "wc_wave_digest: null argument");
    if (unpacked(w, "wc_wave_digest")) return WC_ERR_INVALID;
    *out = digest(w->host);
    return WC_OK;
}

void wc_wave_free(wc_wave* w) { delete w; }

int wc_wave_stats_get(const wc_wave* w, wc_wave_stats* s) {
    if (!w || !s) return fail(WC_ERR_INVALID, "wc_wave_stats_get: null argument");
    if (unpacked(w, "wc_wave_stats_get")) return WC_ERR_INVALID;
    const WaveHost& h = w->host;
    std::memset(s, 0, sizeof *s);
    s->jobs = (uint32_t)h.jobs.size();
    s->nodes = h.nodes();
    for (uint32_t i = 0; i < h.nodes(); i++) {
        uint32_t kind = h.node_meta[i] & 3u;
        if (kind == 0) s->decision_nodes++;
        if (kind == 1) s->chance_nodes++;
        if (kind == 2) s->leaves++;
    }
    s->rows = h.rows();
    s->terminals = (uint32_t)h.term_node.size();
    s->levels = h.max_levels;
    s->units = (uint32_t)h.units.size();
    s->top_levels = h.top_levels;
    s->max_window = h.max_vwin;
    s->iters = h.meta.iters;
    s->nroots_max = h.nroots_max;
    s->carry_slots = h.carry_slots;
    s->cells = h.ncells;
    s->reach_slots = h.reach_task[0].size() + h.reach_task[1].size();
    s->reach_len = h.reach_len;
    s->vals_len = h.vals_len;
    s->rev_nnz = h.rev_src.size();
    s->rvd_nnz = h.rvd_src.size();
    s->draw_nnz = h.draw_to.size();
    s->snapshot_configs = h.snapshot_configs;
    // The immutable tables the executor uploads (without alignment padding).
    auto bytes = [](const auto& v) { return uint64_t(v.size()) * sizeof(v[0]); };
    uint64_t tb = bytes(h.node_meta) + bytes(h.node_nc) + bytes(h.legal_value) + bytes(h.draw_to) + bytes(h.draw_p) +
                  bytes(h.reach_base) + bytes(h.vals_base) + bytes(h.rev_src) + bytes(h.rev_cell) + bytes(h.rvd_src) +
                  bytes(h.rvd_p) + bytes(h.row_node) + bytes(h.row_cfg_off) + bytes(h.row_cfg) + bytes(h.cfg_emb) +
                  bytes(h.cfg_priv) + bytes(h.pub_raw) + bytes(h.term_node) + bytes(h.term_util) + bytes(h.roots) +
                  bytes(h.carried) + bytes(h.exit_node) + bytes(h.exit_coff) + bytes(h.trees) + bytes(h.units) +
                  bytes(h.unit_term) + bytes(h.head_tile_n);
    for (int p = 0; p < 2; p++)
        tb += bytes(h.back_rec[p]) + bytes(h.reach_rec[p]) + bytes(h.acc_rec[p]) + bytes(h.top_back_rec[p]) +
              bytes(h.top_reach_rec[p]) + bytes(h.leaf_rec[p]) + bytes(h.back_lvl[p]) + bytes(h.reach_lvl[p]) +
              bytes(h.child_vb[p]) + bytes(h.pool_grp[p]) + bytes(h.tower_blk[p]) + bytes(h.tower_unit[p]) +
              bytes(h.top_back_lvl[p]) + bytes(h.top_reach_lvl[p]);
    s->table_bytes = tb;
    s->arena_bytes = 4 * (4ull * h.ncells + 2ull * h.reach_len + h.vals_len + 2ull * h.rows() * (h.net.pool + 1) +
                          h.root_values_len) +
                     2ull * h.carry_slots * h.snapshot_configs;
    for (int p = 0; p < 2; p++) {
        CfrBytes cb = cfr_bytes_per_iter(h, p);
        s->cfr_bytes_per_iter[p] = cb.total();
        for (int k = 0; k < 4; k++) s->cfr_bytes_by_kernel[p][k] = cb.part[k];
        s->leaf_input_bytes[p] = leaf_input_bytes(h, p, 2);
    }
    const NetShape& ns = h.net;
    if (ns.kind == MODEL_V5) {
        // Per pass: the join over every row (net.rs:801-841), plus one 256-long
        // readout per (row, config) of the traverser (averaged over both).
        const uint64_t join = 2ull * (uint64_t(v5::JOIN_IN) * v5::JW + uint64_t(v5::JBLOCKS) * v5::JW * v5::JW +
                                      uint64_t(v5::JW) * v5::D);
        s->mlp_flops_per_query = join + 2ull * v5::D;
        const uint64_t slots = h.row_cfg.size();
        const uint64_t tiles = h.tower_unit[0].size() + h.tower_unit[1].size();
        s->mlp_flops_algorithmic = h.rows() * join + uint64_t(v5::D) * slots;
        s->mlp_flops_executed = h.rows() * join + tiles * TOWER_TILE * TOWER_TILE * v5::D;
        return WC_OK;
    }
    if (ns.kind == MODEL_TWO_TOWER) {
        // Per pass: the public tower over every row, plus one width-long
        // readout per (row, config) of the traverser (averaged over both).
        const uint64_t tower = 2ull * (uint64_t(ns.in) * ns.hidden + uint64_t(ns.layers - 1) * ns.hidden * ns.hidden);
        s->mlp_flops_per_query = tower + 2ull * ns.hidden;
        const uint64_t slots = h.row_cfg.size();
        const uint64_t tiles = h.tower_unit[0].size() + h.tower_unit[1].size();  // 64 x 64 readout tiles
        s->mlp_flops_algorithmic = h.rows() * tower + ns.hidden * slots;
        s->mlp_flops_executed = h.rows() * tower + tiles * TOWER_TILE * TOWER_TILE * ns.hidden;
        return WC_OK;
    }
    s->mlp_flops_per_query = 2ull * (uint64_t(ns.in) * ns.hidden + uint64_t(ns.layers - 1) * ns.hidden * ns.hidden +
                                     uint64_t(ns.hidden) * ns.heads);
    // Executed per wave query: the trunk, plus the head columns of its 128-row tile
    // rounded up to whole 128-column tiles; algorithmic: the trunk plus one head row
    // per config of the traverser (averaged over the two traversers).
    uint64_t head_exec = 0, head_alg = 0;
    for (uint32_t r = 0; r < h.rows(); r++) {
        uint64_t tn = h.head_tile_n[r / 128];
        head_exec += std::min<uint64_t>((tn + 127) / 128 * 128, ns.heads);
        head_alg += h.row_cfg_off[2 * r + 2] - h.row_cfg_off[2 * r];
    }
    const uint64_t trunk = 2ull * (uint64_t(ns.in) * ns.hidden + uint64_t(ns.layers - 1) * ns.hidden * ns.hidden);
    s->mlp_flops_executed = h.rows() * trunk + 2ull * ns.hidden * head_exec;
    s->mlp_flops_algorithmic = h.rows() * trunk + ns.hidden * head_alg;
    return WC_OK;
}

extern "C++" {
namespace {

// One packed table of a wave as uint32 words, by name: index lists, and the
// record and unit lists (structs of uint32 fields, field-major within each
// entry). Null for an unknown name; an empty table is a valid pointer to no
// words.
template <class W>
auto u32_table(W& h, const std::string& k, size_t* n) -> decltype(h.row_node.data()) {
    using P = decltype(h.row_node.data());
    static uint32_t none[1] = {0};
    auto list = [&](auto& v) -> P {
        using E = typename std::remove_reference_t<decltype(v)>::value_type;
        static_assert(sizeof(E) % 4 == 0, "a table of uint32 words");
        *n = v.size() * (sizeof(E) / 4);
        return v.empty() ? none : reinterpret_cast<P>(v.data());  // (the entries are structs of uint32 fields)
    };
    if (k == "row_node") return list(h.row_node);
    if (k == "reach_base") return list(h.reach_base);
    if (k == "vals_base") return list(h.vals_base);
    if (k == "exit_node") return list(h.exit_node);
    if (k == "exit_coff") return list(h.exit_coff);
    if (k == "legal_value") return list(h.legal_value);
    if (k == "child_start") return list(h.child_start);
    if (k == "child") return list(h.child);
    if (k == "legal_off") return list(h.legal_off);
    if (k == "node_meta") return list(h.node_meta);
    if (k == "node_nc") return list(h.node_nc);
    if (k == "row_cfg") return list(h.row_cfg);
    if (k == "row_cfg_off") return list(h.row_cfg_off);
    if (k == "draw_to") return list(h.draw_to);
    if (k == "rev_src") return list(h.rev_src);
    if (k == "rvd_src") return list(h.rvd_src);
    if (k == "term_node") return list(h.term_node);
    if (k == "unit_term") return list(h.unit_term);
    if (k == "units") return list(h.units);
    if (k == "trees") return list(h.trees);
    for (int p = 0; p < 2; p++) {
        const std::string s = std::to_string(p);
        if (k == "back_rec" + s) return list(h.back_rec[p]);
        if (k == "top_back_rec" + s) return list(h.top_back_rec[p]);
        if (k == "reach_rec" + s) return list(h.reach_rec[p]);
        if (k == "top_reach_rec" + s) return list(h.top_reach_rec[p]);
        if (k == "acc_rec" + s) return list(h.acc_rec[p]);
        if (k == "leaf_rec" + s) return list(h.leaf_rec[p]);
        if (k == "pool_grp" + s) return list(h.pool_grp[p]);
        if (k == "child_vb" + s) return list(h.child_vb[p]);
        if (k == "back_lvl" + s) return list(h.back_lvl[p]);
        if (k == "reach_lvl" + s) return list(h.reach_lvl[p]);
        if (k == "top_back" + s) return list(h.top_back[p]);
        if (k == "top_reach" + s) return list(h.top_reach[p]);
        if (k == "top_back_lvl" + s) return list(h.top_back_lvl[p]);
        if (k == "top_reach_lvl" + s) return list(h.top_reach_lvl[p]);
        if (k == "top_back_run" + s) return list(h.top_back_run[p]);
        if (k == "top_back_chunk" + s) return list(h.top_back_chunk[p]);
        if (k == "top_reach_run" + s) return list(h.top_reach_run[p]);
        if (k == "top_reach_chunk" + s) return list(h.top_reach_chunk[p]);
        if (k == "top_reach_par" + s) return list(h.top_reach_par[p]);
        if (k == "head_rb_n" + s) return list(h.head_rb_n[p]);
    }
    return nullptr;
}

}  // namespace
}  // extern "C++"

const uint32_t* wc_wave_array(const wc_wave* w, const char* name, size_t* n) {
    if (n) *n = 0;
    if (!w || !name) {
        fail(WC_ERR_INVALID, "wc_wave_array: null argument");
        return nullptr;
    }
    if (unpacked(w, "wc_wave_array")) return nullptr;
    size_t len = 0;
    const uint32_t* v = u32_table(w->host, name, &len);
    if (!v) {
        fail(WC_ERR_INVALID, std::string("wc_wave_array: unknown array ") + name);
        return nullptr;
    }
    if (n) *n = len;
    return v;
}

int wc_wave_poke(wc_wave* w, const char* name, size_t index, uint32_t value) {
    if (!w || !name) return fail(WC_ERR_INVALID, "wc_wave_poke: null argument");
    if (unpacked(w, "wc_wave_poke")) return WC_ERR_INVALID;
    size_t len = 0;
    uint32_t* v = u32_table(w->host, name, &len);
    if (!v) return fail(WC_ERR_INVALID, std::string("wc_wave_poke: unknown array ") + name);
    if (index >= len) return fail(WC_ERR_INVALID, std::string("wc_wave_poke: index beyond ") + name);
    v[index] = value;
    w->host.checked = false;  // what the packer checked is no longer what the wave holds
    return WC_OK;
}

int wc_wave_check(const wc_wave* w, wc_executor* ex, uint64_t version) {
    if (!w) return fail(WC_ERR_INVALID, "wc_wave_check: null argument");
    if (unpacked(w, "wc_wave_check")) return WC_ERR_INVALID;
    return shielded("wc_wave_check", [&] {
        std::string err;
        if (!ex) return validate_deep(w->host, &err) ? WC_OK : fail(WC_ERR_INVALID, err);
        if (ex->ex->check(w->host, version, &err)) return WC_OK;
        return fail(err.rfind("wave bounds: ", 0) == 0 ? WC_ERR_INVALID : WC_ERR_DEVICE, err);
    });
}

static_assert(CHAIN_PASS_BLOCKS == 8, "wc_value_net_plan rows are 2 + 8 words");
int wc_value_net_plan(const uint32_t* cols, uint32_t nrb, uint32_t heads, uint32_t cus, uint32_t* out, size_t cap,
                      size_t* npass) {
    if (npass) *npass = 0;
    if (!npass || (cap && !out)) return fail(WC_ERR_INVALID, "wc_value_net_plan: null argument");
    try {
        const std::vector<ChainPass> plan = plan_chain(cols, nrb, heads, cus);
        std::string err;
        if (!check_chain_plan(plan, cols, nrb, heads, &err)) return fail(WC_ERR_INVALID, err);
        *npass = plan.size();
        for (size_t i = 0; i < plan.size() && i < cap; i++) {
            uint32_t* row = out + i * (2 + CHAIN_PASS_BLOCKS);
            row[0] = plan[i].n;
            row[1] = plan[i].cols;
            for (uint32_t j = 0; j < CHAIN_PASS_BLOCKS; j++) row[2 + j] = j < plan[i].n ? plan[i].rb[j] : 0;
        }
        return WC_OK;
    } catch (const std::exception& e) {
        return fail(WC_ERR_INVALID, e.what());
    }
}

int wc_solve_wave(wc_executor* ex, wc_wave* w, uint64_t version, wc_result** results) {
    if (!ex || !w || !results) return fail(WC_ERR_INVALID, "wc_solve_wave: null argument");
    if (unpacked(w, "wc_solve_wave")) return WC_ERR_INVALID;
    return shielded("wc_solve_wave", [&] {
        std::vector<Result> out;
        std::string err;
        if (!ex->ex->solve(w->host, version, &out, &err)) return fail(WC_ERR_DEVICE, err);
        hand_out(out, results);
        return WC_OK;
    });
}

int wc_launch(wc_executor* ex, wc_wave* w, uint64_t version, wc_inflight** out) {
    if (!ex || !w || !out) return fail(WC_ERR_INVALID, "wc_launch: null argument");
    if (unpacked(w, "wc_launch")) return WC_ERR_INVALID;
    return shielded("wc_launch", [&] {
        std::unique_ptr<wc_inflight> f(new wc_inflight);
        std::string err;
        if (!ex->ex->launch(w->host, version, &f->f, &err)) return fail(WC_ERR_DEVICE, err);
        *out = f.release();
        return WC_OK;
    });
}

int wc_inflight_ready(const wc_executor* ex, const wc_inflight* f) { return ex && f && ex->ex->ready(f->f) ? 1 : 0; }

int wc_collect(wc_executor* ex, wc_inflight* f, wc_result** results) {
    if (!ex || !f || !results) return fail(WC_ERR_INVALID, "wc_collect: null argument");
    std::unique_ptr<wc_inflight> own(f);
    return shielded("wc_collect", [&] {
        std::vector<Result> out;
        std::string err;
        if (!ex->ex->collect(&own->f, &out, &err)) return fail(WC_ERR_DEVICE, err);
        hand_out(out, results);
        return WC_OK;
    });
}

int wc_wave_leaf_probe(wc_executor* ex, wc_wave* w, uint64_t version, int traverser, float* values, size_t cap,
                       size_t* count, float* mass) {
    if (!ex || !w || !count || (cap && !values)) return fail(WC_ERR_INVALID, "wc_wave_leaf_probe: null argument");
    if (unpacked(w, "wc_wave_leaf_probe")) return WC_ERR_INVALID;
    return shielded("wc_wave_leaf_probe", [&] {
        std::vector<float> v, m;
        std::string err;
        if (!ex->ex->leaf_probe(w->host, version, traverser, &v, &m, &err)) return fail(WC_ERR_DEVICE, err);
        *count = v.size();
        if (v.size() <= cap) std::copy(v.begin(), v.end(), values);
        if (mass) std::copy(m.begin(), m.end(), mass);
        return WC_OK;
    });
}

int wc_wave_leaf_trace(wc_executor* ex, wc_wave* w, uint64_t version, const int32_t* points, size_t npoints,
                       float* values, size_t values_cap, float* mass, size_t mass_cap, float* reach, size_t reach_cap,
                       size_t* counts) {
    if (!ex || !w || !counts || (npoints && !points)) return fail(WC_ERR_INVALID, "wc_wave_leaf_trace: null argument");
    if (unpacked(w, "wc_wave_leaf_trace")) return WC_ERR_INVALID;
    return shielded("wc_wave_leaf_trace", [&] {
        const WaveHost& h = w->host;
        size_t c[4] = {0, 0, h.rows(), 0};
        for (uint32_t r = 0; r < h.rows(); r++) {
            c[0] += h.nc(h.row_node[r], 0);
            c[1] += h.nc(h.row_node[r], 1);
        }
        c[3] = c[0] + c[1];
        std::copy(c, c + 4, counts);
        size_t nv = 0;
        for (size_t k = 0; k < npoints; k++) nv += c[points[k] >= 0 ? (points[k] & 1) : ((-points[k] - 1) & 1)];
        if (!values || !mass || values_cap < nv || mass_cap < npoints * 2 * c[2] ||
            (reach && reach_cap < npoints * c[3]))
            return WC_OK;
        LeafTrace t;
        std::string err;
        if (!ex->ex->leaf_trace(h, version, std::vector<int32_t>(points, points + npoints), reach != nullptr, &t,
                                &err))
            return fail(WC_ERR_DEVICE, err);
        std::copy(t.values.begin(), t.values.end(), values);
        std::copy(t.mass.begin(), t.mass.end(), mass);
        if (reach) std::copy(t.reach.begin(), t.reach.end(), reach);
        return WC_OK;
    });
}

int wc_time_wave(wc_executor* ex, wc_wave* w, uint64_t version, uint32_t warmup, uint32_t reps, double* wave_ms,
                 double* kernel_ms) {
    if (!ex || !w || !wave_ms) return fail(WC_ERR_INVALID, "wc_time_wave: null argument");
    if (unpacked(w, "wc_time_wave")) return WC_ERR_INVALID;
    ScheduleTimes prof;
    std::string err;
    const int rc = shielded("wc_time_wave", [&] {
        return ex->ex->time_wave(w->host, version, warmup, reps, wave_ms, kernel_ms ? &prof : nullptr, &err)
                   ? WC_OK
                   : fail(WC_ERR_DEVICE, err);
    });
    if (rc != WC_OK) return rc;
    if (kernel_ms) {
        kernel_ms[0] = prof.cfr;
        kernel_ms[1] = prof.mlp;
        kernel_ms[2] = prof.leaf_input;
        kernel_ms[3] = prof.other;
        kernel_ms[4] = prof.cfr_launch_mean;
        kernel_ms[5] = prof.back_mean;
        kernel_ms[6] = prof.top_mean;
        kernel_ms[7] = prof.reach_mean;
        kernel_ms[8] = prof.graph_build_ms;
        kernel_ms[9] = prof.net_build;
        kernel_ms[10] = prof.v5_join;
    }
    return WC_OK;
}

int wc_mlp_forward(wc_executor* ex, uint64_t version, uint32_t rows, const float* x, float* out) {
    if (!ex || !x || !out) return fail(WC_ERR_INVALID, "wc_mlp_forward: null argument");
    return shielded("wc_mlp_forward", [&] {
        std::string err;
        return ex->ex->mlp_forward(version, rows, x, out, &err) ? WC_OK : fail(WC_ERR_DEVICE, err);
    });
}

int wc_mlp_forward_noalloc(wc_executor* ex, uint64_t version, uint32_t rows, const float* x, float* out,
                           void* stream) {
    if (!ex || (rows && (!x || !out))) return fail(WC_ERR_INVALID, "wc_mlp_forward_noalloc: null argument");
    return shielded("wc_mlp_forward_noalloc", [&] {
        std::string err;
        if (ex->ex->mlp_forward_noalloc(version, rows, x, out, (hipStream_t)stream, &err)) return WC_OK;
        return fail(err.find("scratch") != std::string::npos || err.find("version") != std::string::npos ||
                            err.find("takes the MLP") != std::string::npos
                        ? WC_ERR_INVALID
                        : WC_ERR_DEVICE,
                    err);
    });
}

int wc_time_mlp(wc_executor* ex, uint64_t version, uint32_t rows, const float* x, uint32_t reps, double* chain_ms,
                double* layer_ms) {
    if (!ex || !x || !chain_ms) return fail(WC_ERR_INVALID, "wc_time_mlp: null argument");
    std::string err;
    std::vector<double> layers;
    const int rc = shielded("wc_time_mlp", [&] {
        return ex->ex->time_mlp(version, rows, x, reps, chain_ms, layer_ms ? &layers : nullptr, &err)
                   ? WC_OK
                   : fail(WC_ERR_DEVICE, err);
    });
    if (rc != WC_OK) return rc;
    if (layer_ms)
        for (size_t k = 0; k < layers.size() && k < 8; k++) layer_ms[k] = layers[k];
    return WC_OK;
}

// ------------------------------------------------------------------ service

int wc_service_create(int device, const wc_net_desc* net, int precision, const wc_service_opts* opts,
                      wc_service** out) {
    if (!out) return fail(WC_ERR_INVALID, "wc_service_create: null output");
    NetCopy n;
    std::string err;
    if (!read_net(net, &n, &err)) return fail(WC_ERR_INVALID, err);
    ServiceOpts o;
    if (opts) {
        if (opts->lanes) o.lanes = opts->lanes;
        if (opts->wave_jobs) o.wave_jobs = opts->wave_jobs;
        if (opts->wave_rows) o.wave_rows = opts->wave_rows;
        o.window_us = opts->window_us;
        if (opts->whale_lanes) o.whale_lanes = opts->whale_lanes;
        o.class_shift = opts->class_shift;
        if (opts->route_unit) o.route_unit = opts->route_unit;
    }
    try {
        auto* s = new wc_service;
        s->svc.reset(new Service(device, precision, o));
        if (!s->svc->start(n, &err)) {
            delete s;
            return fail(WC_ERR_DEVICE, err);
        }
        *out = s;
    } catch (const std::exception& e) {
        return fail(WC_ERR_DEVICE, e.what());
    }
    return WC_OK;
}

void wc_service_destroy(wc_service* svc) { delete svc; }

uint64_t wc_set_weights(wc_service* svc, const wc_net_desc* net) {
    if (!svc) {
        fail(WC_ERR_INVALID, "wc_set_weights: null service");
        return 0;
    }
    uint64_t v = 0;
    shielded("wc_set_weights", [&] {
        NetCopy n;
        std::string err;
        if (!read_net(net, &n, &err)) return fail(WC_ERR_INVALID, err);
        v = svc->svc->set_weights(std::move(n), &err);
        return v ? WC_OK : fail(WC_ERR_GONE, err);
    });
    return v;
}

uint64_t wc_queued_work(wc_service* svc) { return svc ? svc->svc->queued_work() : 0; }

int wc_submit(wc_service* svc, const uint8_t* job, size_t len, uint64_t tag, wc_ticket** out) {
    if (!svc || !job || !out) return fail(WC_ERR_INVALID, "wc_submit: null argument");
    return shielded("wc_submit", [&] {
        std::shared_ptr<Ticket> t;
        std::string err;
        if (!svc->svc->submit(job, len, tag, &t, &err))
            return fail(err == "GPU wave executor is gone" ? WC_ERR_GONE : WC_ERR_INVALID, err);
        *out = new wc_ticket{t};
        return WC_OK;
    });
}

int wc_prepare(const uint8_t* job, size_t len, int precision, wc_prepared** out) {
    if (!job || !out) return fail(WC_ERR_INVALID, "wc_prepare: null argument");
    if (precision < WC_PRECISE || precision > WC_F16X) return fail(WC_ERR_INVALID, "wc_prepare: unknown precision");
    return shielded("wc_prepare", [&] {
        std::shared_ptr<const Prepared> p;
        std::string err;
        if (!prepare(job, len, precision, &p, &err)) return fail(WC_ERR_INVALID, err);
        *out = new wc_prepared{std::move(p)};
        return WC_OK;
    });
}

uint64_t wc_prepared_cost(const wc_prepared* p) { return p && p->p ? p->p->cost : 0; }

void wc_prepared_free(wc_prepared* p) { delete p; }

int wc_submit_prepared(wc_service* svc, const wc_prepared* job, uint64_t tag, wc_ticket** out) {
    if (!svc || !job || !out) return fail(WC_ERR_INVALID, "wc_submit_prepared: null argument");
    return shielded("wc_submit_prepared", [&] {
        std::shared_ptr<Ticket> t;
        std::string err;
        if (!svc->svc->submit_prepared(job->p, tag, &t, &err))
            return fail(err == "GPU wave executor is gone" ? WC_ERR_GONE : WC_ERR_INVALID, err);
        *out = new wc_ticket{t};
        return WC_OK;
    });
}

int wc_wait(wc_ticket* t, wc_result** out) {
    if (!t || !out) return fail(WC_ERR_INVALID, "wc_wait: null argument");
    std::shared_ptr<Ticket> tk = t->t;
    delete t;
    return shielded("wc_wait", [&] {
        std::unique_lock<std::mutex> lk(tk->mu);
        tk->cv.wait(lk, [&] { return tk->done; });
        if (tk->rc != 0) return fail(tk->rc, tk->err);
        std::unique_ptr<wc_result> r(new wc_result);
        r->r = std::move(tk->result);
        *out = r.release();
        return WC_OK;
    });
}

int wc_poll(const wc_ticket* t) {
    if (!t) return 0;
    std::lock_guard<std::mutex> lk(t->t->mu);
    return t->t->done ? 1 : 0;
}

void wc_ticket_free(wc_ticket* t) { delete t; }

int wc_service_stats(wc_service* svc, uint64_t* waves, uint64_t* guarded_routes) {
    if (!svc) return fail(WC_ERR_INVALID, "wc_service_stats: null service");
    if (waves) *waves = svc->svc->waves();
    if (guarded_routes) *guarded_routes = svc->svc->guarded_routes();
    return WC_OK;
}

int wc_job_work(const uint8_t* job, size_t len, int precision, uint64_t route_unit, uint32_t class_shift,
                wc_work_vector* out, uint64_t* cost, uint32_t* cls) {
    if (!job || !out) return fail(WC_ERR_INVALID, "wc_job_work: null argument");
    if (precision < WC_PRECISE || precision > WC_F16X) return fail(WC_ERR_INVALID, "wc_job_work: unknown precision");
    return shielded("wc_job_work", [&] {
        Job j;
        std::string err;
        if (!from_bytes(job, len, &j, &err)) return fail(WC_ERR_INVALID, err);
        const uint64_t unit = route_unit ? route_unit : WorkVector::ROUTE_UNIT;
        const WorkVector w = work_vector(j, precision);
        std::memset(out, 0, sizeof *out);
        out->network_rows = w.network_rows;
        out->legal_cells = w.legal_cells;
        out->reach_slots = w.reach_slots;
        out->reverse_nonzeros = w.reverse_nonzeros;
        out->table_bytes = w.table_bytes;
        out->mutable_bytes = w.mutable_bytes;
        out->carried_output_bytes = w.carried_output_bytes;
        out->levels = w.levels;
        out->reserved_bytes = w.reserved_bytes();
        out->exclusive_route = w.requires_exclusive_route(unit);
        out->arena_guard_route = w.requires_arena_guard_route(unit);
        out->card_exclusive_route = w.requires_card_exclusive_route(unit);
        if (cost) *cost = job_cost(w, j.meta.iters);
        if (cls) *cls = cost_class(w, class_shift, unit);
        return WC_OK;
    });
}

uint64_t wc_result_tag(const wc_result* r) { return r ? r->r.tag : 0; }
uint64_t wc_result_weight_version(const wc_result* r) { return r ? r->r.weight_version : 0; }

const float* wc_result_strategy(const wc_result* r, size_t* n) {
    if (!r) {
        if (n) *n = 0;
        return nullptr;
    }
    if (n) *n = r->r.strategy.size();
    return r->r.strategy.data();
}

const float* wc_result_root_values(const wc_result* r, uint32_t* nroots, uint32_t* n0, uint32_t* n1) {
    if (!r) return nullptr;
    if (nroots) *nroots = r->r.nroots;
    if (n0) *n0 = r->r.n0;
    if (n1) *n1 = r->r.n1;
    return r->r.root_values.data();
}

const uint16_t* wc_result_carries(const wc_result* r, uint32_t* slots, uint32_t* snapshot_configs) {
    if (!r) return nullptr;
    if (slots) *slots = r->r.slots;
    if (snapshot_configs) *snapshot_configs = r->r.snapshot_configs;
    return r->r.carries.data();
}

int wc_result_routes(const wc_result* r, int* oversize_route, int* card_exclusive_route) {
    if (!r) return fail(WC_ERR_INVALID, "wc_result_routes: null result");
    if (oversize_route) *oversize_route = r->r.oversize_route ? 1 : 0;
    if (card_exclusive_route) *card_exclusive_route = r->r.card_exclusive_route ? 1 : 0;
    return WC_OK;
}

void wc_result_free(wc_result* r) { delete r; }

}  // extern "C"
