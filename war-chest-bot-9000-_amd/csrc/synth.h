// Seeded synthetic subgames in the job contract's layout.
//
// The reference builds its trees from War Chest states (engine/src/search.rs:942-1253)
// and packs them with `PackedTables::from_solver` (engine/src/serialize.rs:689-956).
// This generator produces trees of the same form without a rules engine:
// decision nodes with config-dependent legal cells, actions grouped into public
// observations, config transitions into each child's support, collapsed chance
// nodes with per-config outcome rows, and network or terminal leaves. The
// tables (reverse gathers in the CPU accumulation order, BFS levels, support
// offsets) are built exactly the way `from_solver` builds them.
#pragma once

#include <cstdint>
#include <vector>

#include "job.h"

namespace wc {

// xorshift64* (Vigna 2016), seeded as engine/src/rng.rs:8-12 does.
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) {
        uint64_t x = seed ^ 0x9E3779B97F4A7C15ull;
        s = x ? x : 0xDEADBEEFCAFEF00Dull;
    }
    uint64_t next() {
        uint64_t x = s;
        x ^= x >> 12;
        x ^= x << 25;
        x ^= x >> 27;
        s = x;
        return x * 0x2545F4914F6CDD1Dull;
    }
    uint32_t below(uint32_t n) { return (uint32_t)(next() % n); }
    double unit() { return double(next() >> 11) * (1.0 / 9007199254740992.0); }
    uint32_t range(uint32_t lo, uint32_t hi) { return lo + below(hi - lo + 1); }  // U{lo..hi}
    double normal();  // Box-Muller
};

struct SynthSpec {
    uint64_t seed = 0;
    uint32_t trees = 1;
    // Public tree shape. Growth is breadth-first to a node budget drawn from
    // U{nodes_lo..nodes_hi}; with exact_decisions > 0 the tree instead has exactly
    // that many decision nodes and exact_leaves leaves (no chance nodes).
    uint32_t nodes_lo = 32, nodes_hi = 128;
    uint32_t exact_decisions = 0, exact_leaves = 0;
    uint32_t act_lo = 3, act_hi = 12;  // private actions per decision node
    float collapse = 0.25f;            // P(an action shares an earlier action's observation)
    uint32_t chance = 0;               // 1: a chance node follows every decision ply
    uint32_t draw_lo = 2, draw_hi = 6; // outcomes per source config at a chance node
    // Infostates (configs) per player at the root.
    uint32_t info_fixed = 0;           // > 0: exactly this many
    float info_median = 22.0f, info_p99 = 567.0f;
    uint32_t info_cap = 567;
    float legal_p = 0.75f;             // P(a (config, action) cell is legal)
    float shift_p = 0.15f;             // P(a cell's successor is the next config key)
    float notrans_p = 0.02f;           // P(a legal cell has no successor config)
    float terminal_p = 0.0f;           // P(a leaf is terminal rather than a network leaf)
    uint32_t dirichlet = 0;            // root beliefs Dirichlet(1); else uniform
    uint32_t nroots = 1;               // carried roots; the first is the root belief itself
    // Heavy tail: this fraction of trees uses whale_nodes / whale_info instead.
    float whale_frac = 0.0f;
    uint32_t whale_nodes = 2000, whale_info = 567;
    // Runtime metadata.
    uint32_t depth = 1, iters = 16, snapshots = 1;
    Cfr cfr;
    std::vector<uint32_t> net_dims;  // must be an MLP or two-tower tag
};

// One job per tree. Tree k uses the k-th draw of a master stream seeded by `seed`,
// so a tree does not depend on how many others are generated after it.
std::vector<Job> synth_jobs(const SynthSpec& spec);

// Value-net weights in the flat `set_weights(dims, w, b, ln)` layout:
// Kaiming-normal N(0, 2/fan_in) matrices, biases U[-0.1, 0.1].
// MLP: w = W_1 [in x hidden], W_2..W_L [hidden x hidden], W_head [heads x hidden];
//      b = b_1..b_L [hidden], b_head [heads].
// Two-tower: w = public tower (in x width, width x width ...), private tower
//      (priv_in x width, width x width ...), readout weight [width]; b = matching biases
//      and one readout bias.
// v5: w, b in the flat blob order of net.rs:272-316 (Kaiming-normal matrices,
//      N(0, 0.25) embeddings, U[-0.1, 0.1] biases).
void synth_weights(const std::vector<uint32_t>& dims, uint64_t seed, std::vector<float>* w,
                   std::vector<float>* b);
// LayerNorm pairs of a family (v5: gains 1 + N(0, 0.01), shifts N(0, 0.01);
// empty for the synthetic families).
void synth_norms(const std::vector<uint32_t>& dims, uint64_t seed, std::vector<float>* ln);

// Dense leaf-query features (U[0,1) with 30% of dims in one-hot blocks of width 8).
void synth_features(uint32_t rows, uint32_t width, uint64_t seed, std::vector<float>* x);

}  // namespace wc
