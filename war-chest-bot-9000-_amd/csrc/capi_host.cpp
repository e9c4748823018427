// Host-only entry points of the C ABI: errors, the job codec, synthetic workloads.
#include <cstring>
#include <exception>
#include <string>

#include "../../include/wc_wave.h"
#include "common.h"
#include "job.h"
#include "synth.h"
#include "v5.h"

namespace wc {
thread_local std::string g_last_error;
int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}
}  // namespace wc

using namespace wc;

extern "C" {

const char* wc_last_error(void) { return g_last_error.c_str(); }

int wc_net_sizes(const uint32_t* dims, uint32_t ndims, size_t* nw, size_t* nb) {
    if (!dims || !nw || !nb) return fail(WC_ERR_INVALID, "wc_net_sizes: null argument");
    NetShape ns;
    std::string err;
    if (!ns.parse(std::vector<uint32_t>(dims, dims + ndims), &err)) return fail(WC_ERR_INVALID, err);
    if (ns.kind == MODEL_MLP) {
        *nw = size_t(ns.in) * ns.hidden + size_t(ns.layers - 1) * ns.hidden * ns.hidden + size_t(ns.heads) * ns.hidden;
        *nb = size_t(ns.layers) * ns.hidden + ns.heads;
        return WC_OK;
    }
    if (ns.kind == MODEL_TWO_TOWER) {
        *nw = size_t(ns.in) * ns.hidden + size_t(ns.layers - 1) * ns.hidden * ns.hidden +
              size_t(ns.priv_in) * ns.hidden + size_t(ns.priv_layers - 1) * ns.hidden * ns.hidden + ns.hidden;
        *nb = size_t(ns.layers) * ns.hidden + size_t(ns.priv_layers) * ns.hidden + 1;
        return WC_OK;
    }
    const v5::Layout L = v5::layout();  // net.rs:272-316
    *nw = L.w_len;
    *nb = L.b_len;
    return WC_OK;
}

int wc_net_norms(const uint32_t* dims, uint32_t ndims, size_t* nln) {
    if (!dims || !nln) return fail(WC_ERR_INVALID, "wc_net_norms: null argument");
    NetShape ns;
    std::string err;
    if (!ns.parse(std::vector<uint32_t>(dims, dims + ndims), &err)) return fail(WC_ERR_INVALID, err);
    *nln = ns.kind == MODEL_V5 ? v5::layout().ln_len : 0;
    return WC_OK;
}

int wc_job_roundtrip(const uint8_t* job, size_t len, uint8_t* out, size_t cap, size_t* out_len) {
    if (!job || !out_len) return fail(WC_ERR_INVALID, "wc_job_roundtrip: null argument");
    Job j;
    std::string err;
    if (!from_bytes(job, len, &j, &err)) return fail(WC_ERR_INVALID, err);
    std::vector<uint8_t> b = to_bytes(j);
    *out_len = b.size();
    if (out) std::memcpy(out, b.data(), std::min(cap, b.size()));
    return WC_OK;
}

int wc_job_validate(const uint8_t* job, size_t len) {
    if (!job) return fail(WC_ERR_INVALID, "wc_job_validate: null job");
    Job j;
    std::string err;
    if (!from_bytes(job, len, &j, &err)) return fail(WC_ERR_INVALID, err);
    if (!validate(j, &err)) return fail(WC_ERR_INVALID, err);
    return WC_OK;
}

void wc_synth_spec_default(wc_synth_spec* s) {
    if (!s) return;
    SynthSpec d;
    std::memset(s, 0, sizeof *s);
    s->seed = d.seed;
    s->trees = d.trees;
    s->nodes_lo = d.nodes_lo;
    s->nodes_hi = d.nodes_hi;
    s->exact_decisions = d.exact_decisions;
    s->exact_leaves = d.exact_leaves;
    s->act_lo = d.act_lo;
    s->act_hi = d.act_hi;
    s->collapse = d.collapse;
    s->chance = d.chance;
    s->draw_lo = d.draw_lo;
    s->draw_hi = d.draw_hi;
    s->info_fixed = d.info_fixed;
    s->info_median = d.info_median;
    s->info_p99 = d.info_p99;
    s->info_cap = d.info_cap;
    s->legal_p = d.legal_p;
    s->shift_p = d.shift_p;
    s->notrans_p = d.notrans_p;
    s->terminal_p = d.terminal_p;
    s->dirichlet = d.dirichlet;
    s->nroots = d.nroots;
    s->whale_frac = d.whale_frac;
    s->whale_nodes = d.whale_nodes;
    s->whale_info = d.whale_info;
    s->depth = d.depth;
    s->iters = d.iters;
    s->snapshots = d.snapshots;
    s->alpha = d.cfr.alpha;
    s->beta = d.cfr.beta;
    s->gamma = d.cfr.gamma;
    s->predict = d.cfr.predict;
}

struct wc_jobset {
    std::vector<std::vector<uint8_t>> jobs;
};

int wc_synth(const wc_synth_spec* in, wc_jobset** out) {
    if (!in || !out) return fail(WC_ERR_INVALID, "wc_synth: null argument");
    if (!in->net_dims || in->n_net_dims == 0) return fail(WC_ERR_INVALID, "wc_synth: net_dims required");
    if (in->act_lo == 0 || in->act_hi < in->act_lo || in->draw_lo == 0 || in->draw_hi < in->draw_lo ||
        in->nodes_hi < in->nodes_lo || in->nodes_lo == 0)
        return fail(WC_ERR_INVALID, "wc_synth: empty range in the spec");
    SynthSpec s;
    s.seed = in->seed;
    s.trees = in->trees;
    s.nodes_lo = in->nodes_lo;
    s.nodes_hi = in->nodes_hi;
    s.exact_decisions = in->exact_decisions;
    s.exact_leaves = in->exact_leaves;
    s.act_lo = in->act_lo;
    s.act_hi = in->act_hi;
    s.collapse = in->collapse;
    s.chance = in->chance;
    s.draw_lo = in->draw_lo;
    s.draw_hi = in->draw_hi;
    s.info_fixed = in->info_fixed;
    s.info_median = in->info_median;
    s.info_p99 = in->info_p99;
    s.info_cap = in->info_cap;
    s.legal_p = in->legal_p;
    s.shift_p = in->shift_p;
    s.notrans_p = in->notrans_p;
    s.terminal_p = in->terminal_p;
    s.dirichlet = in->dirichlet;
    s.nroots = in->nroots;
    s.whale_frac = in->whale_frac;
    s.whale_nodes = in->whale_nodes;
    s.whale_info = in->whale_info;
    s.depth = in->depth;
    s.iters = in->iters;
    s.snapshots = in->snapshots;
    s.cfr = Cfr{in->alpha, in->beta, in->gamma, in->predict};
    s.net_dims.assign(in->net_dims, in->net_dims + in->n_net_dims);
    try {
        std::vector<Job> jobs = synth_jobs(s);
        auto* set = new wc_jobset;
        set->jobs.reserve(jobs.size());
        for (const Job& j : jobs) set->jobs.push_back(to_bytes(j));
        *out = set;
    } catch (const std::exception& e) {
        return fail(WC_ERR_INVALID, std::string("wc_synth: ") + e.what());
    }
    return WC_OK;
}

uint32_t wc_jobset_count(const wc_jobset* s) { return s ? (uint32_t)s->jobs.size() : 0; }

const uint8_t* wc_jobset_job(const wc_jobset* s, uint32_t k, size_t* len) {
    if (!s || k >= s->jobs.size()) {
        if (len) *len = 0;
        return nullptr;
    }
    if (len) *len = s->jobs[k].size();
    return s->jobs[k].data();
}

void wc_jobset_free(wc_jobset* s) { delete s; }

int wc_synth_weights(const uint32_t* dims, uint32_t ndims, uint64_t seed, float* w, size_t nw, float* b,
                     size_t nb) {
    size_t need_w, need_b;
    int rc = wc_net_sizes(dims, ndims, &need_w, &need_b);
    if (rc) return rc;
    if (nw != need_w || nb != need_b || !w || !b) return fail(WC_ERR_INVALID, "wc_synth_weights: buffer sizes");
    std::vector<float> vw, vb;
    try {
        synth_weights(std::vector<uint32_t>(dims, dims + ndims), seed, &vw, &vb);
    } catch (const std::exception& e) {
        return fail(WC_ERR_INVALID, e.what());
    }
    std::memcpy(w, vw.data(), nw * sizeof(float));
    std::memcpy(b, vb.data(), nb * sizeof(float));
    return WC_OK;
}

int wc_synth_norms(const uint32_t* dims, uint32_t ndims, uint64_t seed, float* ln, size_t nln) {
    size_t need = 0;
    int rc = wc_net_norms(dims, ndims, &need);
    if (rc) return rc;
    if (nln != need || (need && !ln)) return fail(WC_ERR_INVALID, "wc_synth_norms: buffer size");
    std::vector<float> v;
    try {
        synth_norms(std::vector<uint32_t>(dims, dims + ndims), seed, &v);
    } catch (const std::exception& e) {
        return fail(WC_ERR_INVALID, e.what());
    }
    if (need) std::memcpy(ln, v.data(), need * sizeof(float));
    return WC_OK;
}

int wc_synth_features(uint32_t rows, uint32_t width, uint64_t seed, float* x) {
    if (!x) return fail(WC_ERR_INVALID, "wc_synth_features: null output");
    std::vector<float> v;
    synth_features(rows, width, seed, &v);
    std::memcpy(x, v.data(), v.size() * sizeof(float));
    return WC_OK;
}

}  // extern "C"
