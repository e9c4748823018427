// Host packing of one immutable wave: jobs concatenated into one wave-global
// index space, offsets patched, value/reach aliasing laid out, and the
// unit schedules the device sweeps walk.
//
// Counterpart of the reference's `Wave::pack` (engine/src/gpu/wave.rs:132-644)
// and `device_value_layout` (engine/src/serialize.rs:447-480). The reach and
// value aliasing follow the reference; the schedules differ. Instead of
// wave-wide level task lists walked under grid-wide barriers, each tree is cut
// into units that one workgroup sweeps with block barriers: runs of sibling
// subtrees that fit a slot budget, swept independently and largest first so
// big and small trees balance across the CUs. The nodes above them (the top
// region of a tree that does not fit one unit) are swept one depth per launch
// across all trees: after the units for values, before them for reach. Value
// slots are allocated in reverse DFS preorder, so every unit's slots form one
// contiguous window.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "job.h"

namespace wc {

struct Task {
    uint32_t node, config;
};

// Row records the device sweeps read: everything a row needs is one load away
// (its output slot, its element range and what the elements index), so a
// level costs one record read, one element read and one gather.
enum : uint32_t { BACK_OWN = 0, BACK_DRAW = 1, BACK_OPP = 2 };
enum : uint32_t { REACH_REV = 0, REACH_RVD = 1 };
constexpr uint32_t REC_N = 0x1fffffffu;       // element count bits of `kn`
constexpr uint32_t REC_EXPORT = 1u << 29;     // BackRec: the row's value is read outside its unit
// unit_term entries: the terminal index, plus one bit per player whose values
// at that terminal are read outside the unit.
constexpr uint32_t TERM_INDEX = 0x3fffffffu;
constexpr uint32_t term_export(int p) { return 1u << (31 - p); }

// One value row of the traverser: out = its value slot; kn = kind << 30 |
// REC_EXPORT (when set) | n.
//   BACK_OWN  cells [start, start + n) of the traverser's decision row (arg unused)
//   BACK_DRAW draw entries [start, start + n) (wave-global), values at arg + draw_to
//   BACK_OPP  child value bases child_vb[p][start .. start + n), plus arg = the config
struct BackRec {
    uint32_t out, arg, start, kn;
};
// One reach row: out = its reach slot; pbase = the parent's reach slot of the
// same player; kn = kind << 31 | n over rev or rvd entries [start, start + n).
struct ReachRec {
    uint32_t out, pbase, start, kn;
};
// One decision row: its reach slot and its cells [lo, lo + n).
struct AccRec {
    uint32_t ridx, lo, n, pad;
};

// Per-tree record: root beliefs, carried roots, outputs.
struct TreeDev {
    uint32_t node0, nodes;        // wave-global node range
    uint32_t reach0, reach_len;   // reach span (zeroed by seed)
    uint32_t root0, n0, n1;       // root beliefs at roots[root0 ..], n0 + n1 floats
    uint32_t carried0, nroots;    // carried roots at carried[carried0 + k * (n0 + n1)]
    uint32_t root_value0;         // output offset of this tree's root values
    uint32_t exit0, nexit;
};
static_assert(sizeof(TreeDev) == 12 * 4, "TreeDev is 48 bytes");

// One subtree unit, swept by one workgroup: a run of sibling subtrees whose
// value slots fit the unit budget. Levels are unit-local depths; task and row
// lists live in the wave's flattened arrays at the offsets given here.
struct UnitDev {
    uint32_t nlevels, lvl0;     // level boundaries at back_lvl / reach_lvl [lvl0, lvl0 + nlevels]
    uint32_t dec0[2], dec1[2];  // decision rows of each player: decision[p][dec0 .. dec1)
    uint32_t row0, row1;        // network leaf rows: unit_row[row0 .. row1)
    uint32_t term0, term1;      // terminal leaves: unit_term[term0 .. term1)
    uint32_t slots;             // value slots (max over players, before aliasing)
    uint32_t tree;              // owning tree
    uint32_t vwin[2], vwin_n[2];  // the unit's value slots of each player: [vwin, vwin + vwin_n)
    uint32_t leaf0[2], leaf1[2];  // network-leaf value slots of each player: leaf_rec[p][leaf0 .. leaf1)
    uint32_t rwin[2], rwin_n[2];  // the unit's own reach slots of each player: [rwin, rwin + rwin_n)
};
static_assert(sizeof(UnitDev) == 24 * 4, "UnitDev is 96 bytes");

// One network-leaf value slot of the traverser: vals[out] = head_out[head] * mass[mass]
// (the net's value of the slot's config times the opponent's reach mass);
// exported = 1 when the slot is read outside its unit. head is row * heads +
// the config's head row for the MLP; for the two-tower net, whose readout
// gives one value per (row, config), it is the (row, config) entry of the
// tree's readout block for the player (TowerBlock).
struct LeafRec {
    uint32_t out, head, mass, exported;
};

// Two-tower readout, block-diagonal by tree: per (tree, player), the tree's
// network rows [r0, r1) times the configs [clo, chi) the player's rows name,
// computed densely into tower values at dbase + (row - r0) (chi - clo) +
// (config - clo). A unit is one 64 x 64 tile of a block: rows from `row`
// (16-aligned, so whole fragment blocks; rows outside the block are not
// stored), configs from `cfg`.
struct TowerBlock {
    uint32_t r0, r1, clo, chi, dbase, pad[3];
};
struct TowerUnit {
    uint32_t block, row, cfg, pad;
};
constexpr uint32_t TOWER_TILE = 64;

// Network rows whose configs for one player are the same list, pooled by one
// wavefront of the 16-bit nets: every config's embedding is read once for all
// of them (the f32 MFMA's 16 rows: up to 15 network rows and a ones row).
constexpr uint32_t POOL_GROUP = 15;
struct PoolGroup {
    uint32_t cfg, n, nrows;  // the shared list row_cfg[cfg .. cfg + n), rows row[0 .. nrows)
    uint32_t row[POOL_GROUP];
    // each row's reach slots of the group's player, reach_base[2 * node + p]
    // (entries past nrows repeat row 0's): the pooling reads the reach with
    // no lookup through the row's node
    uint32_t rbase[POOL_GROUP];
    uint32_t pad[3];
};
static_assert(sizeof(PoolGroup) == 36 * 4, "PoolGroup is 144 bytes");

// One pass of the fused value net: up to CHAIN_PASS_BLOCKS 16-row blocks of the
// network rows (any blocks, in any order; rb[0 .. n)) and the head columns
// they need (cols).
constexpr uint32_t CHAIN_PASS_BLOCKS = 8;
struct ChainPass {
    uint32_t rb[CHAIN_PASS_BLOCKS];
    uint32_t n, cols, pad[2];
};
static_assert(sizeof(ChainPass) == 12 * 4, "ChainPass is 48 bytes");

// Passes of the fused value net over nrb row blocks whose head widths are
// cols[rb] (cols null: every block needs `heads`), for a device of `cus`
// compute units that each run one pass at a time. Blocks are taken widest
// head first; consecutive blocks of that order are dealt to at most `cus`
// shares of about equal estimated cost (a per-pass overhead, a per-block
// trunk cost and a per-block head cost that grows with the width), each share
// is cut into passes of up to CHAIN_PASS_BLOCKS blocks and at most the cost of
// a full pass of 64-column blocks (wide-head passes hold fewer), and the passes are
// listed by estimated cost, longest first: run in list order on CUs that take
// the next pass as they free up (longest-processing-time-first list
// scheduling), the last passes end at about the same time. Every block is in
// exactly one pass.
std::vector<ChainPass> plan_chain(const uint32_t* cols, uint32_t nrb, uint32_t heads, uint32_t cus);
// What the fused kernel assumes of a plan: every block below nrb in exactly
// one pass, 1..CHAIN_PASS_BLOCKS blocks per pass, and each pass's cols at
// least every one of its blocks' widths.
bool check_chain_plan(const std::vector<ChainPass>& plan, const uint32_t* cols, uint32_t nrb, uint32_t heads,
                      std::string* err);

// Default unit budget in value slots (floats of one player's value vector).
constexpr uint32_t UNIT_SLOTS = 4096;
// Top-region value launches: words per run (WaveHost::top_back_run), the rows
// a fused chunk takes per depth before it closes (one per thread of a
// one-wavefront workgroup), and the largest group of dependent rows of two
// depths that still fuses them into one launch.
constexpr uint32_t TOP_RUN = 4, TOP_CHUNK_ROWS = 64, TOP_FUSE_MAX = 128;

struct WaveHost {
    Meta meta;
    NetShape net;
    std::vector<std::shared_ptr<const Job>> jobs;  // the wave's jobs (shared, immutable), kept for result unpacking
    std::vector<TreeDev> trees;

    // Tree and sparse-cell SoA, wave-global.
    std::vector<uint32_t> node_meta;  // kind | player << 2
    std::vector<uint32_t> node_nc;    // 2 * node + p
    std::vector<uint32_t> child_start, child;
    std::vector<uint32_t> legal_row_of, legal_off, legal_value;
    std::vector<uint32_t> draw_off, draw_row_off, draw_row_start, draw_to;
    std::vector<float> draw_p;
    std::vector<uint32_t> reach_base, vals_base;
    uint32_t reach_len = 0, vals_len = 0;
    std::vector<uint32_t> parent;
    std::vector<uint32_t> rev_row_of, rev_start, rev_src, rev_cell;
    std::vector<uint32_t> rvd_row_of, rvd_start, rvd_src;
    std::vector<float> rvd_p;
    uint32_t ncells = 0;

    // Leaf network rows.
    std::vector<uint32_t> row_node, row_cfg_off, row_cfg;
    std::vector<uint32_t> cfg_key;  // head row of each interned config
    std::vector<float> cfg_emb;     // [ncfg, pool]
    std::vector<float> cfg_priv;    // [ncfg, priv_in] private-tower features (two-tower); [ncfg, 15] counts (v5)
    std::vector<uint8_t> pub_raw;   // [rows, row_bytes]
    // v5 network: each config's job and owning seat, each row's job, each
    // job's card table ([jobs][NTYPE * CARD_FEATS], physical coin-type order).
    std::vector<uint32_t> cfg_job, row_job;
    std::vector<uint8_t> cfg_owner;
    std::vector<float> card_feat;
    // Head columns each 128-row tile of the network rows needs: 1 + the largest
    // head key among the tile's configs (the head GEMM skips the rest).
    std::vector<uint32_t> head_tile_n;
    // The same per 16-row block and player: the keys of that player's configs.
    std::vector<uint32_t> head_rb_n[2];
    std::vector<uint32_t> term_node;
    std::vector<float> term_util;
    std::vector<float> roots, carried;
    uint32_t root_values_len = 0;
    std::vector<uint32_t> exit_node, exit_coff;
    std::vector<uint32_t> exit_reach;  // reach slot of each (exit, player): reach_base[2 * exit_node[e] + p]
    uint32_t snapshot_configs = 0;

    // Subtree units in descending size; lists are unit-major and level l of
    // unit u spans [lvl[u.lvl0 + l], lvl[u.lvl0 + l + 1]).
    std::vector<UnitDev> units;
    uint32_t nsub = 0;
    std::vector<Task> back_task[2], reach_task[2], decision[2];
    std::vector<uint32_t> back_lvl[2], reach_lvl[2];
    std::vector<uint32_t> unit_row, unit_term;
    uint32_t lvl_len = 0;
    // Top regions (the nodes whose subtree does not fit a unit), all trees
    // together by depth: level l spans [top_*_lvl[p][l], top_*_lvl[p][l + 1]).
    // Their decision rows close each decision list: decision[p][top_dec0[p] ..).
    std::vector<Task> top_back[2], top_reach[2];
    uint32_t top_dec0[2] = {0, 0};
    std::vector<uint32_t> top_back_lvl[2], top_reach_lvl[2];
    uint32_t top_levels = 0;
    // The value pass's launches over the top depths, deepest first, TOP_RUN
    // words each: {depth, second depth or NONE, first chunk offset, chunks}.
    // A run of two depths (the next non-empty one above) is one launch of
    // `chunks` workgroups: workgroup k runs the deeper depth's rows
    // [off[k], off[k + 1]), then, after a barrier, the shallower depth's rows
    // [off[chunks + 1 + k], off[chunks + 2 + k]), off = top_back_chunk[p] +
    // first chunk offset. The deeper rows whose values a shallower row reads
    // sit in its chunk, so no other workgroup's results are needed. A run of
    // one depth is one launch over its rows.
    std::vector<uint32_t> top_back_run[2], top_back_chunk[2];
    // The reach pass's launches over the top depths, top-down, TOP_RUN words
    // each: {depth, second depth or NONE, first chunk offset, chunks}. A run
    // of two depths (the next non-empty one below) is one launch of `chunks`
    // workgroups: workgroup k computes the shallower depth's rows named by
    // top_reach_par[p][off[chunks + 1 + k] .. off[chunks + 2 + k]), then,
    // after a barrier, the deeper depth's rows [off[k], off[k + 1]), off =
    // top_reach_chunk[p] + first chunk offset. Each chunk names every
    // shallower row its deeper rows read (a shallower row read by several
    // chunks is computed by each: the same value, written again); shallower
    // rows that no deeper row reads fill chunks with no deeper rows.
    std::vector<uint32_t> top_reach_run[2], top_reach_chunk[2], top_reach_par[2];
    std::vector<uint8_t> node_top;  // 1 for a node of a top region

    uint32_t max_levels = 0, nroots_max = 0, carry_slots = 0;
    // The packed lists passed validate_deep on the host. When not (a service
    // wave of jobs validated at submit), an upload checks the element tables
    // on the device before the schedule may read them.
    bool checked = false;
    uint32_t max_vwin = 0;  // the widest unit value window (floats): the sweep's LDS size
    uint32_t max_rwin = 0;  // the widest unit reach window (floats): the reach pass's LDS size

    // Device row records, index-aligned with the task lists above.
    std::vector<BackRec> back_rec[2], top_back_rec[2];
    std::vector<ReachRec> reach_rec[2], top_reach_rec[2];
    std::vector<AccRec> acc_rec[2];
    std::vector<LeafRec> leaf_rec[2];  // unit-major network-leaf slots
    std::vector<PoolGroup> pool_grp[2];  // network rows grouped by config list, longest lists first
    // Readout blocks of the two-tower and v5 nets (<f(c), h(row)> per row and
    // config) and their tiles, per player; tower_len floats of values.
    std::vector<TowerBlock> tower_blk[2];
    std::vector<TowerUnit> tower_unit[2];
    uint64_t tower_len = 0;
    std::vector<uint32_t> child_vb[2];  // child value bases of the opponent rows

    uint32_t nodes() const { return (uint32_t)node_meta.size(); }
    uint32_t rows() const { return (uint32_t)row_node.size(); }
    // Empty every list, keeping its buffer, and zero every count: packing the
    // next wave into the same WaveHost then neither allocates nor faults in
    // fresh pages for lists that have grown before. (A member added to this
    // struct must be added to reset(): the size check next to it fails until
    // it is.)
    void reset();
    uint32_t nc(uint32_t node, int p) const { return node_nc[2 * node + p]; }
};

// Pack parsed jobs into one wave. Fails (with a message) on incompatible
// schedules, malformed tables or unsupported networks. `unit_slots` bounds the
// value slots of one subtree unit.
// `validated`: every job already passed validate() (the service checks each
// job when it is submitted), so the per-job checks are not repeated, nor the
// deep check of the packed wave (validate_deep) unless WC_DEEP_CHECK=1: the
// wave's `checked` stays false and its upload checks it on the device.
// `fuse_top`: plan fused launches over pairs of top depths (one launch fewer
// per pair, for some host work: WaveHost::top_back_run); WC_TOP_FUSE=0 or 1
// overrides it.
bool pack_wave(std::vector<std::shared_ptr<const Job>>&& jobs, WaveHost* w, std::string* err,
               uint32_t unit_slots = UNIT_SLOTS, bool validated = false, bool fuse_top = true);
// The same for jobs owned by the caller (moved into the wave).
// A 64-bit digest of every list and count of a packed wave (FNV-1a over
// 8-byte words), for tests that compare two packings of the same jobs.
uint64_t digest(const WaveHost& w);

bool pack_wave(std::vector<Job>&& jobs, WaveHost* w, std::string* err, uint32_t unit_slots = UNIT_SLOTS,
               bool validated = false, bool fuse_top = true);

// Bounds of every index the kernels dereference (run by pack_wave):
// validate_shape, then the element tables on host threads.
bool validate_deep(const WaveHost& w, std::string* err);
// The checks of validate_deep that read no element table: each list's size
// against the counts it must match, and the short per-config, per-unit,
// per-tree and per-exit lists. An upload of a wave that did not pass
// validate_deep runs these, then the element checks on the device (check.h).
bool validate_shape(const WaveHost& w, std::string* err);

// Algorithmic HBM bytes of one CFR iteration for traverser p (the counting
// rule is written next to the implementation), split by the launch that moves
// them: [0] the subtree value sweep, [1] the top-region launches, [2] the
// subtree reach, [3] the average-strategy accumulation (run in the leaf-input
// launch).
struct CfrBytes {
    uint64_t part[4] = {0, 0, 0, 0};
    uint64_t total() const { return part[0] + part[1] + part[2] + part[3]; }
};
CfrBytes cfr_bytes_per_iter(const WaveHost& w, int p);

// Algorithmic HBM bytes of one leaf-input pooling of player p's network rows
// (the pooled-belief half of a leaf-input launch): every row's reach over its
// configs and its outputs (two pooled blocks of `elem`-byte operands and the
// mass), every distinct config list's indices and every distinct config's
// embedding once.
uint64_t leaf_input_bytes(const WaveHost& w, int p, uint32_t elem);

}  // namespace wc
