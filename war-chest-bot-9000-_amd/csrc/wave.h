// Host packing of one immutable wave: jobs concatenated into one wave-global
// index space, offsets patched, value/reach aliasing laid out, and the
// per-tree level schedules the device sweeps walk.
//
// Counterpart of the reference's `Wave::pack` (engine/src/gpu/wave.rs:132-644)
// and `device_value_layout` (engine/src/serialize.rs:447-480). The reach and
// value aliasing follow the reference exactly; the schedules differ: instead
// of wave-wide level task lists walked under grid-wide barriers, every tree
// keeps its own level lists so one workgroup can sweep it with block barriers.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "job.h"

namespace wc {

struct Task {
    uint32_t node, config;
};

// Per-tree record the device kernels read (one workgroup per tree).
struct TreeDev {
    uint32_t node0, nodes, nlevels, lvl0;  // lvl0: base of this tree's (nlevels + 1) level boundaries
    uint32_t dec0[2], dec1[2];             // decision-row task ranges per player
    uint32_t row0, rows, term0, nterm;     // network rows and terminal leaves
    uint32_t reach0, reach_len;            // reach span (zeroed by seed)
    uint32_t root0, n0, n1;                // root beliefs at roots[root0 ..], n0 + n1 floats
    uint32_t carried0, nroots;             // carried roots at carried[carried0 + k * (n0 + n1)]
    uint32_t root_value0;                  // output offset of this tree's root values
    uint32_t exit0, nexit;
    uint32_t pad[2];
};
static_assert(sizeof(TreeDev) == 24 * 4, "TreeDev is 96 bytes");

struct WaveHost {
    Meta meta;
    NetShape net;
    std::vector<Job> jobs;  // parsed, kept for result unpacking
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
    std::vector<uint8_t> pub_raw;   // [rows, row_bytes]
    std::vector<uint32_t> term_node;
    std::vector<float> term_util;
    std::vector<float> roots, carried;
    uint32_t root_values_len = 0;
    std::vector<uint32_t> exit_node, exit_coff;
    uint32_t snapshot_configs = 0;

    // Schedules. Level boundaries: tree t, level l -> [lvl[lvl0 + l], lvl[lvl0 + l + 1]).
    std::vector<Task> back_task[2], reach_task[2], decision[2];
    std::vector<uint32_t> back_lvl[2], reach_lvl[2];
    uint32_t lvl_len = 0;

    uint32_t max_levels = 0, nroots_max = 0, carry_slots = 0;

    uint32_t nodes() const { return (uint32_t)node_meta.size(); }
    uint32_t rows() const { return (uint32_t)row_node.size(); }
    uint32_t nc(uint32_t node, int p) const { return node_nc[2 * node + p]; }
};

// Pack parsed jobs into one wave. Fails (with a message) on incompatible
// schedules, malformed tables or unsupported networks.
bool pack_wave(std::vector<Job>&& jobs, WaveHost* w, std::string* err);

// Bounds of every index the kernels dereference (run by pack_wave).
bool validate_deep(const WaveHost& w, std::string* err);

// Algorithmic HBM bytes of one CFR iteration for traverser p (the counting
// rule is written next to the implementation).
uint64_t cfr_bytes_per_iter(const WaveHost& w, int p);

}  // namespace wc
