// The CPU-to-GPU job contract: one solve = one immutable sparse subgame tree,
// its root beliefs and the carried root beliefs Phase 2 must value.
//
// Field names, meanings and the WCJ8 byte order follow the reference contract
// (docs/TREE.md; engine/src/serialize.rs:36-148 for the structs,
// serialize.rs:1052-1261 for the byte layout). The network-row payload
// (`leaf_raw`, `card_feat`, `cphi`) is interpreted through `meta.net_dims`,
// which names the leaf network: the reference's v5 tag `[5]` or one of the
// synthetic value-net tags defined in `NetShape` below.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace wc {

constexpr uint32_t NONE = 0xffffffffu;
constexpr uint32_t JOB_MAGIC = 0x57434A38u;  // "WCJ8"
constexpr uint32_t JOB_VERSION = 8;

// Leaf-network families named by `net_dims[0]`.
enum ModelKind : uint32_t {
    MODEL_V5 = 5,          // the reference's v5 network (engine/src/net.rs:41)
    MODEL_MLP = 101,       // [101, in, hidden, layers, heads, pool]
    MODEL_TWO_TOWER = 102, // [102, in, width, pub_layers, priv_in, priv_layers, pool]
};

// v5 payload widths (engine/src/rebel.rs:61-71,891,985-986; units.rs:46,71).
constexpr uint32_t V5_CFEAT = 15;
constexpr uint32_t V5_CARD_FEAT = 10 * (10 + 12 + 2 + 1);
constexpr uint32_t V5_ROW_BYTES = 201;  // GPU_ROW_BYTES (rebel.rs:986)

// The families whose leaf value is a readout <f(c), h(row)> + bias per
// (row, config): the two-tower net and the v5 network (net.rs:844-853).
inline bool readout_net(uint32_t kind) { return kind == MODEL_TWO_TOWER || kind == MODEL_V5; }

struct Cfr {
    float alpha = 1.5f, beta = 0.0f, gamma = 2.0f, predict = 0.0f;
};

struct Meta {
    uint32_t depth = 1;
    uint32_t iters = 0;
    bool snapshots = true;
    Cfr cfr;
    std::vector<uint32_t> snap_iters;
    std::vector<uint32_t> net_dims;
};

// What a job's network payload looks like, derived from `net_dims`.
struct NetShape {
    uint32_t kind = 0;
    uint32_t in = 0;         // value-net input width per query
    uint32_t hidden = 0;     // trunk width
    uint32_t layers = 0;     // trunk depth (ReLU layers)
    uint32_t heads = 0;      // rows of the per-infostate head (MLP)
    uint32_t pool = 0;       // pooled-belief width per player
    uint32_t priv_in = 0;    // private-tower input width (two-tower)
    uint32_t priv_layers = 0;
    uint32_t row_bytes = 0;  // leaf_raw bytes per network row
    uint32_t cfeat = 0;      // cphi floats per interned config
    uint32_t card_feat = 0;  // card_feat floats per job
    bool parse(const std::vector<uint32_t>& dims, std::string* err);
};

// Every uploaded array of the contract (serialize.rs:52-148).
struct Tables {
    uint32_t nodes = 0, ncfg = 0, rows = 0, ncells = 0;
    std::vector<uint8_t> node_kind, node_player;
    std::vector<uint32_t> node_child_start, node_child;
    std::vector<uint32_t> obs_off, obs_start, obs_act, obs_child;
    std::vector<uint32_t> legal_row_of, legal_off, legal_action, legal_child, legal_trans, cell_row;
    std::vector<uint32_t> draw_off, draw_to;
    std::vector<float> draw_p;
    std::vector<uint32_t> draw_row_off, draw_row_start;
    std::vector<uint32_t> cfg_off, reach_off, soff, node_parent;
    std::vector<uint32_t> rev_row_of, rev_start, rev_src, rev_cell;
    std::vector<uint32_t> rvd_row_of, rvd_start, rvd_src;
    std::vector<float> rvd_p;
    std::vector<uint32_t> leaf_rows, term_leaves;
    std::vector<float> terminal_utility;
    std::vector<uint32_t> leaf_coff, leaf_cidx, snap_coff;
    std::vector<uint8_t> leaf_raw;
    std::vector<float> card_feat, cphi;
    std::vector<uint8_t> cplayer;
    std::vector<uint32_t> bfs_order, level_start;

    uint32_t nc(uint32_t node, int p) const { return cfg_off[2 * node + p + 1] - cfg_off[2 * node + p]; }
    uint32_t nlevels() const { return level_start.empty() ? 0 : (uint32_t)level_start.size() - 1; }
    uint32_t snapshot_configs() const { return snap_coff.empty() ? 0 : snap_coff.back(); }
};

struct Job {
    Meta meta;
    Tables t;
    std::vector<float> root[2];
    std::vector<std::vector<float>> carried[2];  // carried[p][r]
    uint32_t nroots() const { return (uint32_t)carried[0].size(); }
};

// `snapshot_iters` (engine/src/search.rs:102-110): 0, powers of two, and the final iteration.
std::vector<uint32_t> snapshot_iters(uint32_t iters);

// WCJ8 bytes (serialize.rs:1052-1129 writes, 1131-1261 reads).
std::vector<uint8_t> to_bytes(const Job& job);
bool from_bytes(const uint8_t* b, size_t n, Job* out, std::string* err);

// Structural checks beyond the reader's count checks: every index in range,
// every CSR monotone, parents before children, and (for the MLP nets) each
// config's head row below the net's heads. Returns false with a message.
bool validate(const Job& job, std::string* err);

// A config's head row: cphi[c][0] of the MLP nets holds it as a float. True
// (with the row in *row) when it is a whole number below `heads` (any whole
// number when heads is 0); the range is checked before the conversion.
inline bool head_row(float key, uint32_t heads, uint32_t* row) {
    if (!(key >= 0.0f && key < 4294967296.0f)) return false;
    const uint32_t r = (uint32_t)key;
    if ((float)r != key || (heads && r >= heads)) return false;
    *row = r;
    return true;
}

}  // namespace wc
