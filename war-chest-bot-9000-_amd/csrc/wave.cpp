// Host wave packing (counterpart of engine/src/gpu/wave.rs:132-644).
#include "wave.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <memory>
#include <string>
#include <unordered_map>

#include "par.h"

namespace wc {

namespace {

bool same_meta(const Meta& a, const Meta& b) {
    auto bits = [](float x) {
        uint32_t u;
        std::memcpy(&u, &x, 4);
        return u;
    };
    return a.depth == b.depth && a.iters == b.iters && a.snapshots == b.snapshots &&
           bits(a.cfr.alpha) == bits(b.cfr.alpha) && bits(a.cfr.beta) == bits(b.cfr.beta) &&
           bits(a.cfr.gamma) == bits(b.cfr.gamma) && bits(a.cfr.predict) == bits(b.cfr.predict) &&
           a.snap_iters == b.snap_iters && a.net_dims == b.net_dims;
}

// DFS preorder of one tree, children in child order.
std::vector<uint32_t> preorder(const Tables& t) {
    std::vector<uint32_t> pre, stack{0};
    pre.reserve(t.nodes);
    while (!stack.empty()) {
        uint32_t i = stack.back();
        stack.pop_back();
        pre.push_back(i);
        for (uint32_t k = t.node_child_start[i + 1]; k-- > t.node_child_start[i];) stack.push_back(t.node_child[k]);
    }
    return pre;
}

// Per-player value slots: the two players share one span (values are built for
// one traverser at a time); across a chance edge the non-drawing player's
// vector is its sole child's and aliases it (engine/src/serialize.rs:447-480).
// Slots are allocated in reverse preorder, so a subtree (a preorder range) owns
// one contiguous run of slots.
bool value_layout(const Tables& t, const std::vector<uint32_t>& pre, std::vector<uint32_t> base[2], uint32_t* len,
                  std::string* err) {
    uint32_t lengths[2] = {0, 0};
    for (int p = 0; p < 2; p++) {
        base[p].assign(t.nodes, 0);
        std::vector<uint8_t> ready(t.nodes, 0);
        uint32_t at = 0;
        for (size_t k = pre.size(); k-- > 0;) {
            uint32_t node = pre[k];
            if (t.node_kind[node] == 1 && t.node_player[node] != p) {
                uint32_t lo = t.node_child_start[node], hi = t.node_child_start[node + 1];
                if (hi != lo + 1) {
                    *err = "chance node without exactly one child";
                    return false;
                }
                uint32_t child = t.node_child[lo];
                if (!ready[child]) {
                    *err = "value layout: child not ready";
                    return false;
                }
                base[p][node] = base[p][child];
            } else {
                base[p][node] = at;
                at += t.nc(node, p);
            }
            ready[node] = 1;
        }
        lengths[p] = at;
    }
    *len = std::max(lengths[0], lengths[1]);
    return true;
}

template <class T>
void append_shift(std::vector<T>& dst, const std::vector<T>& src, size_t skip, T add, bool keep_none) {
    for (size_t k = skip; k < src.size(); k++) {
        T x = src[k];
        dst.push_back(keep_none && x == (T)NONE ? x : (T)(x + add));
    }
}

// Runs fn(lo, hi) over [0, n) in chunks on the host threads.
template <class F>
void chunked(size_t n, F fn, size_t chunk = 16384) {
    parallel_for((n + chunk - 1) / chunk, [&](size_t c) { fn(c * chunk, std::min(n, (c + 1) * chunk)); });
}

// One job's layout inside its own tree, independent of every other job of
// the wave: preorder, value slots, reach length, depths, its subtree units
// and its top region, and how many entries it adds to each unit list.
struct JobLayout {
    std::vector<uint32_t> pre, vb[2], depth, row_of, term_of;
    uint32_t vlen = 0, reach_len = 0;
    std::vector<uint32_t> unit_nodes;      // every unit's nodes (preorder), unit after unit
    std::vector<uint32_t> unit_at{0};      // unit j: unit_nodes[unit_at[j] .. unit_at[j + 1])
    std::vector<uint32_t> unit_d0;         // unit j's top depth
    std::vector<uint32_t> top;             // the top region's nodes, preorder
    uint32_t top_depths = 0;               // 1 + the deepest top node's depth (0: no top region)
    uint32_t lvls = 0, max_levels = 0, nback[2] = {0, 0}, nreach[2] = {0, 0}, ndec[2] = {0, 0};
    uint32_t nrow = 0, nterm = 0;
    uint32_t max_vwin = 0, max_rwin = 0;   // filled with the unit records
    std::vector<Task> top_back[2], top_reach[2], top_dec[2];
    std::vector<uint32_t> top_back_d[2], top_reach_d[2];  // depth of each top task
    std::string err;

    uint32_t levels_of(uint32_t j) const {
        uint32_t L = 0;
        for (uint32_t x = unit_at[j]; x < unit_at[j + 1]; x++) L = std::max(L, depth[unit_nodes[x]] - unit_d0[j] + 1);
        return L;
    }

    void build(const Tables& t, const NetShape& net, bool v5, uint32_t unit_slots) {
        const uint32_t N = t.nodes;
        pre = preorder(t);
        if (pre.size() != N) {
            err = "tree is not connected from its root";
            return;
        }
        if (!value_layout(t, pre, vb, &vlen, &err)) return;
        for (uint32_t c = 0; c < t.ncfg && !v5; c++) {
            uint32_t row;
            if (!head_row(t.cphi[size_t(c) * net.cfeat], net.heads, &row)) {
                err = "config head index out of range";
                return;
            }
        }
        for (uint32_t local : t.bfs_order)
            for (int p = 0; p < 2; p++)
                if (local == 0 || t.node_player[t.node_parent[local]] == p) reach_len += t.nc(local, p);
        depth.assign(N, 0);
        for (uint32_t l = 0; l < t.nlevels(); l++)
            for (uint32_t k = t.level_start[l]; k < t.level_start[l + 1]; k++) depth[t.bfs_order[k]] = l;
        std::vector<uint64_t> sub(N, 0);
        for (size_t k = pre.size(); k-- > 0;) {
            uint32_t i = pre[k];
            sub[i] += std::max<uint32_t>(std::max(t.nc(i, 0), t.nc(i, 1)), 1);
            if (t.node_parent[i] != NONE) sub[t.node_parent[i]] += sub[i];
        }
        std::vector<uint32_t> pos(N);
        for (uint32_t k = 0; k < N; k++) pos[pre[k]] = k;
        row_of.assign(N, NONE);
        term_of.assign(N, NONE);
        for (uint32_t r = 0; r < t.rows; r++) row_of[t.leaf_rows[r]] = r;
        for (uint32_t k = 0; k < t.term_leaves.size(); k++) term_of[t.term_leaves[k]] = k;
        auto close_unit = [&](uint32_t d0) {
            unit_at.push_back((uint32_t)unit_nodes.size());
            unit_d0.push_back(d0);
        };
        // The nodes of the subtree rooted at r, in preorder.
        auto subtree = [&](uint32_t r) {
            uint32_t k = pos[r];
            uint32_t end = k + 1;
            while (end < N && depth[pre[end]] > depth[r]) end++;
            unit_nodes.insert(unit_nodes.end(), pre.begin() + k, pre.begin() + end);
        };
        if (sub[0] <= unit_slots) {
            unit_nodes = pre;
            close_unit(0);
        } else {
            for (uint32_t i : pre)
                if (sub[i] > unit_slots) top.push_back(i);
            // Runs of fitting sibling subtrees below each top node, in child order.
            // A top child ends the run: its subtree's value slots lie between
            // its siblings', and a unit's window must stay contiguous.
            for (uint32_t i : top) {
                uint64_t run_slots = 0;
                bool open = false;
                for (uint32_t k = t.node_child_start[i]; k < t.node_child_start[i + 1]; k++) {
                    uint32_t c = t.node_child[k];
                    const bool fits = sub[c] <= unit_slots;
                    if (open && (!fits || run_slots + sub[c] > unit_slots)) {
                        close_unit(depth[i] + 1);
                        open = false;
                        run_slots = 0;
                    }
                    if (!fits) continue;
                    subtree(c);
                    open = true;
                    run_slots += sub[c];
                }
                if (open) close_unit(depth[i] + 1);
            }
            for (uint32_t i : top) top_depths = std::max(top_depths, depth[i] + 1);
        }
        // What the units add to the wave's unit lists.
        for (uint32_t j = 0; j + 1 < unit_at.size(); j++) {
            const uint32_t L = levels_of(j);
            lvls += L + 1;
            max_levels = std::max(max_levels, L);
            for (uint32_t x = unit_at[j]; x < unit_at[j + 1]; x++) {
                const uint32_t local = unit_nodes[x];
                const uint8_t kind = t.node_kind[local];
                for (int p = 0; p < 2; p++) {
                    if (kind != 2 && !(kind == 1 && t.node_player[local] != p)) nback[p] += t.nc(local, p);
                    if (local != 0 && t.node_player[t.node_parent[local]] == p) nreach[p] += t.nc(local, p);
                    if (kind == 0 && t.node_player[local] == p) ndec[p] += t.nc(local, p);
                }
                nrow += row_of[local] != NONE;
                nterm += term_of[local] != NONE;
            }
        }
    }
};

// Where one job's entries start in each wave list.
struct JobAt {
    uint32_t node, child, lrow, cell, draw, drow, reach, vals, rrow, rev, vrow, rvd, row, coff, member, cfg, exit,
        ecoff, ecfg, term, rootv, unit, lvl, urow, uterm, back[2], rch[2], dec[2];
    size_t pub, card, priv, emb, roots, carried, rowjob;
};

// Row records from the task lists (see BackRec / ReachRec / AccRec). Every
// record is a function of its task alone, once the opponent rows' child
// value-base lists are laid out (first appearance among the value tasks, in
// task order), so the records are built in parallel chunks.
void build_records(WaveHost* wp) {
    WaveHost& w = *wp;
    // The child value-base lists: each opponent decision node's children's
    // value bases, nodes in the order of their first value task (the unit
    // tasks, then the top tasks). Built in three parallel passes over the
    // tasks: each node's first task (an atomic minimum), the list bytes each
    // chunk of tasks adds (a prefix over the chunks), then the writes.
    std::vector<uint32_t> cvb_at[2];
    for (int p = 0; p < 2; p++) {
        const std::vector<Task>& unit_tasks = w.back_task[p];
        const std::vector<Task>& top_tasks = w.top_back[p];
        const size_t nu = unit_tasks.size(), n = nu + top_tasks.size();
        auto node_of = [&](size_t i) { return i < nu ? unit_tasks[i].node : top_tasks[i - nu].node; };
        auto opp = [&](uint32_t node) {
            const uint32_t kind = w.node_meta[node] & 3u, actor = w.node_meta[node] >> 2;
            return kind != 1 && actor != (uint32_t)p;
        };
        std::vector<uint32_t> first(w.nodes(), NONE);  // each opponent node's first task
        chunked(n, [&](size_t lo, size_t hi) {
            for (size_t i = lo; i < hi; i++) {
                const uint32_t node = node_of(i);
                if (!opp(node)) continue;
                uint32_t cur = __atomic_load_n(&first[node], __ATOMIC_RELAXED);
                while ((uint32_t)i < cur &&
                       !__atomic_compare_exchange_n(&first[node], &cur, (uint32_t)i, true, __ATOMIC_RELAXED,
                                                    __ATOMIC_RELAXED)) {
                }
            }
        });
        constexpr size_t CHUNK = 16384;
        const size_t nch = (n + CHUNK - 1) / CHUNK;
        std::vector<size_t> at(nch + 1, 0);
        parallel_for(nch, [&](size_t c) {
            size_t len = 0;
            for (size_t i = c * CHUNK; i < std::min(n, (c + 1) * CHUNK); i++) {
                const uint32_t node = node_of(i);
                if (opp(node) && first[node] == (uint32_t)i) len += w.child_start[node + 1] - w.child_start[node];
            }
            at[c + 1] = len;
        });
        for (size_t c = 0; c < nch; c++) at[c + 1] += at[c];
        w.child_vb[p].resize(at[nch]);
        cvb_at[p].assign(w.nodes(), NONE);  // written by the chunk holding the node's first task only
        parallel_for(nch, [&](size_t c) {
            size_t o = at[c];
            for (size_t i = c * CHUNK; i < std::min(n, (c + 1) * CHUNK); i++) {
                const uint32_t node = node_of(i);
                if (!opp(node) || first[node] != (uint32_t)i) continue;
                cvb_at[p][node] = (uint32_t)o;
                for (uint32_t x = w.child_start[node]; x < w.child_start[node + 1]; x++)
                    w.child_vb[p][o++] = w.vals_base[2 * w.child[x] + p];
            }
        });
    }
    auto back = [&](int p, const Task& q) {
        const uint32_t node = q.node, c = q.config;
        const uint32_t kind = w.node_meta[node] & 3u, actor = w.node_meta[node] >> 2;
        BackRec r{};
        r.out = w.vals_base[2 * node + p] + c;
        if (kind == 1) {
            uint32_t child = w.child[w.child_start[node]];
            uint32_t d0 = w.draw_off[node], rb = w.draw_row_off[node];
            uint32_t lo = w.draw_row_start[rb + c], hi = w.draw_row_start[rb + c + 1];
            r.arg = w.vals_base[2 * child + p];
            r.start = d0 + lo;
            r.kn = BACK_DRAW << 30 | (hi - lo);
        } else if (actor != (uint32_t)p) {
            r.arg = c;
            r.start = cvb_at[p][node];
            r.kn = BACK_OPP << 30 | (w.child_start[node + 1] - w.child_start[node]);
        } else {
            uint32_t row = w.legal_row_of[node] + c;
            r.start = w.legal_off[row];
            r.kn = BACK_OWN << 30 | (w.legal_off[row + 1] - w.legal_off[row]);
        }
        return r;
    };
    auto reach = [&](int p, const Task& q) {
        const uint32_t node = q.node, c = q.config;
        ReachRec r{};
        r.out = w.reach_base[2 * node + p] + c;
        r.pbase = w.reach_base[2 * w.parent[node] + p];
        if (w.rev_row_of[node] != NONE) {
            uint32_t row = w.rev_row_of[node] + c;
            r.start = w.rev_start[row];
            r.kn = REACH_REV << 31 | (w.rev_start[row + 1] - w.rev_start[row]);
        } else {
            uint32_t row = w.rvd_row_of[node] + c;
            r.start = w.rvd_start[row];
            r.kn = REACH_RVD << 31 | (w.rvd_start[row + 1] - w.rvd_start[row]);
        }
        return r;
    };
    parallel_for(10, [&](size_t k) {  // the record lists side by side
        const int p = (int)(k & 1);
        switch (k >> 1) {
            case 0: w.back_rec[p].resize(w.back_task[p].size()); break;
            case 1: w.top_back_rec[p].resize(w.top_back[p].size()); break;
            case 2: w.reach_rec[p].resize(w.reach_task[p].size()); break;
            case 3: w.top_reach_rec[p].resize(w.top_reach[p].size()); break;
            default: w.acc_rec[p].resize(w.decision[p].size()); break;
        }
    });
    for (int p = 0; p < 2; p++) {
        chunked(w.back_task[p].size(), [&](size_t lo, size_t hi) {
            for (size_t k = lo; k < hi; k++) w.back_rec[p][k] = back(p, w.back_task[p][k]);
        });
        chunked(w.top_back[p].size(), [&](size_t lo, size_t hi) {
            for (size_t k = lo; k < hi; k++) w.top_back_rec[p][k] = back(p, w.top_back[p][k]);
        });
        chunked(w.reach_task[p].size(), [&](size_t lo, size_t hi) {
            for (size_t k = lo; k < hi; k++) w.reach_rec[p][k] = reach(p, w.reach_task[p][k]);
        });
        chunked(w.top_reach[p].size(), [&](size_t lo, size_t hi) {
            for (size_t k = lo; k < hi; k++) w.top_reach_rec[p][k] = reach(p, w.top_reach[p][k]);
        });
        chunked(w.decision[p].size(), [&](size_t lo, size_t hi) {
            for (size_t k = lo; k < hi; k++) {
                const Task& q = w.decision[p][k];
                const uint32_t row = w.legal_row_of[q.node] + q.config;
                w.acc_rec[p][k] = {w.reach_base[2 * q.node + p] + q.config, w.legal_off[row],
                                   w.legal_off[row + 1] - w.legal_off[row], 0};
            }
        });
    }
    // Each exit's reach slots, so the carry gather reads them in one load.
    w.exit_reach.resize(2 * w.exit_node.size());
    chunked(w.exit_node.size(), [&](size_t lo, size_t hi) {
        for (size_t e = lo; e < hi; e++)
            for (int p = 0; p < 2; p++) w.exit_reach[2 * e + p] = w.reach_base[2 * size_t(w.exit_node[e]) + p];
    });
    // Network-leaf slots, unit by unit (the value sweep writes them first):
    // each unit's first slot from a prefix sum, then the units in parallel.
    const uint32_t heads = w.net.heads;
    const bool tower = readout_net(w.net.kind);
    std::vector<uint32_t> unit_leaves(2 * w.units.size());
    parallel_for(w.units.size(), [&](size_t ui) {
        const UnitDev& u = w.units[ui];
        for (int p = 0; p < 2; p++) {
            uint32_t c = 0;
            for (uint32_t k = u.row0; k < u.row1; k++) c += w.nc(w.row_node[w.unit_row[k]], p);
            unit_leaves[2 * ui + p] = c;
        }
    });
    uint32_t nleaf[2] = {0, 0};
    for (size_t ui = 0; ui < w.units.size(); ui++)
        for (int p = 0; p < 2; p++) {
            w.units[ui].leaf0[p] = nleaf[p];
            nleaf[p] += unit_leaves[2 * ui + p];
            w.units[ui].leaf1[p] = nleaf[p];
        }
    parallel_for(2, [&](size_t p) { w.leaf_rec[p].resize(nleaf[p]); });
    for (int p = 0; p < 2; p++) {
        std::vector<uint32_t> row_blk;  // readout nets: each row's readout block for p
        if (tower) {
            row_blk.assign(w.rows(), NONE);
            for (uint32_t bi = 0; bi < w.tower_blk[p].size(); bi++)
                for (uint32_t r = w.tower_blk[p][bi].r0; r < w.tower_blk[p][bi].r1; r++) row_blk[r] = bi;
        }
        parallel_for(w.units.size(), [&](size_t ui) {
            const UnitDev& u = w.units[ui];
            uint32_t slot = u.leaf0[p];
            for (uint32_t k = u.row0; k < u.row1; k++) {
                const uint32_t r = w.unit_row[k], node = w.row_node[r];
                const uint32_t* cfgs = &w.row_cfg[w.row_cfg_off[2 * r + p]];
                for (uint32_t c = 0; c < w.nc(node, p); c++) {
                    uint32_t head;
                    if (tower) {
                        const TowerBlock& b = w.tower_blk[p][row_blk[r]];
                        head = b.dbase + (r - b.r0) * (b.chi - b.clo) + (cfgs[c] - b.clo);
                    } else {
                        head = r * heads + w.cfg_key[cfgs[c]];
                    }
                    w.leaf_rec[p][slot++] = {w.vals_base[2 * node + p] + c, head, 2 * r + (1 - p), 0};
                }
            }
        });
    }
    // Exported slots: the values read outside their unit, by the top
    // regions' rows or as a tree's root values. Only these leave an
    // LDS-staged unit sweep for HBM.
    // (flags set from several threads at once: relaxed atomic byte stores of
    // the same value)
    std::unique_ptr<uint8_t[]> ex[2];
    std::vector<uint8_t> term_ex[2];
    for (int p = 0; p < 2; p++) {
        ex[p].reset(new uint8_t[w.vals_len]);  // cleared in parallel below
        uint8_t* flag = ex[p].get();
        chunked(w.vals_len, [&](size_t lo, size_t hi) { std::fill(flag + lo, flag + hi, (uint8_t)0); });
        chunked(
            w.top_back_rec[p].size(),
            [&](size_t lo, size_t hi) {
                for (size_t i = lo; i < hi; i++) {
                    const BackRec& r = w.top_back_rec[p][i];
                    const uint32_t n = r.kn & REC_N, kind = r.kn >> 30;
                    for (uint32_t k = 0; k < n; k++) {
                        uint32_t slot;
                        if (kind == BACK_OWN)
                            slot = w.legal_value[r.start + k];
                        else if (kind == BACK_DRAW)
                            slot = r.arg + w.draw_to[r.start + k];
                        else
                            slot = w.child_vb[p][r.start + k] + r.arg;
                        if (slot < w.vals_len) __atomic_store_n(flag + slot, (uint8_t)1, __ATOMIC_RELAXED);
                    }
                }
            },
            4096);
        chunked(
            w.trees.size(),
            [&](size_t lo, size_t hi) {
                for (size_t t = lo; t < hi; t++) {
                    const uint32_t node0 = w.trees[t].node0;
                    for (uint32_t c = 0; c < w.nc(node0, p); c++)
                        __atomic_store_n(flag + w.vals_base[2 * node0 + p] + c, (uint8_t)1, __ATOMIC_RELAXED);
                }
            },
            64);
        term_ex[p].assign(w.unit_term.size(), 0);
        chunked(w.unit_term.size(), [&](size_t lo, size_t hi) {
            for (size_t k = lo; k < hi; k++) {
                const uint32_t node = w.term_node[w.unit_term[k] & TERM_INDEX];
                for (uint32_t c = 0; c < w.nc(node, p); c++)
                    if (ex[p][w.vals_base[2 * node + p] + c]) term_ex[p][k] = 1;
            }
        });
    }
    for (int p = 0; p < 2; p++) {
        chunked(w.back_rec[p].size(), [&](size_t lo, size_t hi) {
            for (size_t k = lo; k < hi; k++)
                if (ex[p][w.back_rec[p][k].out]) w.back_rec[p][k].kn |= REC_EXPORT;
        });
        chunked(w.leaf_rec[p].size(), [&](size_t lo, size_t hi) {
            for (size_t k = lo; k < hi; k++) w.leaf_rec[p][k].exported = ex[p][w.leaf_rec[p][k].out];
        });
    }
    for (size_t k = 0; k < w.unit_term.size(); k++)
        for (int p = 0; p < 2; p++)
            if (term_ex[p][k]) w.unit_term[k] |= term_export(p);
}

// The top regions' value launches (WaveHost::top_back_run). The non-empty
// depths are taken deepest first; each depth and the next one above fuse
// into one launch when every group of their dependent rows stays small (a
// group: a shallower row with the deeper rows whose values it reads, closed
// under sharing them; at most TOP_FUSE_MAX rows), else the depth runs alone
// and the next is tried with the one above it. A fused pair's rows are
// reordered within each depth so that each chunk (whole groups, at most
// TOP_CHUNK_ROWS rows of each depth unless one group holds more) is
// contiguous in both. The rows of two trees share no slot, so each tree's
// rows of a depth (a contiguous range: trees are in job order at every
// depth) are grouped on their own, in parallel. Without `fuse` every depth is
// its own launch.
void plan_top_back(WaveHost* wp, bool fuse) {
    WaveHost& w = *wp;
    const size_t J = w.trees.size();
    parallel_for(2, [&](size_t pi) {  // the players' rows are apart
        const int p = (int)pi;
        std::vector<uint32_t>& run = w.top_back_run[p];
        std::vector<uint32_t>& chunk = w.top_back_chunk[p];
        run.clear();
        chunk.clear();
        const std::vector<uint32_t>& lvl = w.top_back_lvl[p];
        std::vector<Task>& task = w.top_back[p];
        std::vector<BackRec>& rec = w.top_back_rec[p];
        std::vector<uint32_t> depths;  // the non-empty ones, deepest first
        for (uint32_t l = w.top_levels; l-- > 0;)
            if (lvl[l + 1] > lvl[l]) depths.push_back(l);
        // Tree k's rows at depth d: [cut(d, k), cut(d, k + 1)).
        auto cut = [&](uint32_t d, size_t k) -> uint32_t {
            if (k >= J) return lvl[d + 1];
            return (uint32_t)(std::lower_bound(task.begin() + lvl[d], task.begin() + lvl[d + 1], w.trees[k].node0,
                                               [](const Task& t, uint32_t n) { return t.node < n; }) -
                              task.begin());
        };
        // The slots a record reads (none for a record whose elements fall
        // outside their lists: validation refuses such a wave later).
        auto reads = [&](const BackRec& r, auto&& fn) {
            const uint32_t n = r.kn & REC_N, kind = r.kn >> 30;
            const size_t len = kind == BACK_OWN    ? w.legal_value.size()
                               : kind == BACK_DRAW ? w.draw_to.size()
                                                   : w.child_vb[p].size();
            if (uint64_t(r.start) + n > len) return;
            for (uint32_t k = 0; k < n; k++) {
                if (kind == BACK_OWN) {
                    if (w.legal_value[r.start + k] != NONE) fn(w.legal_value[r.start + k]);
                } else if (kind == BACK_DRAW) {
                    fn(r.arg + w.draw_to[r.start + k]);
                } else {
                    fn(w.child_vb[p][r.start + k] + r.arg);
                }
            }
        };
        // One tree's groups for the pair (deeper depth a, shallower b): a
        // group per row (a's rows, then b's), numbered in order of first
        // appearance over b's rows, then a's. False when a group outgrows
        // TOP_FUSE_MAX (or another tree's did: `stop`).
        struct Grouping {
            uint32_t a0 = 0, na = 0, b0 = 0, nb = 0;
            std::vector<uint32_t> label, size_a, size_b;
        };
        auto group = [&](uint32_t a, uint32_t b, size_t k, Grouping* g, const bool* stop) {
            g->a0 = cut(a, k);
            g->na = cut(a, k + 1) - g->a0;
            g->b0 = cut(b, k);
            g->nb = cut(b, k + 1) - g->b0;
            const uint32_t a0 = g->a0, na = g->na, b0 = g->b0, nb = g->nb;
            // a's rows by output slot: each node's rows are consecutive, its
            // configs in order from its value base, so a slot is found among
            // the nodes' slot ranges (few, sorted by base). Rows laid out
            // otherwise, or ranges that overlap, leave the pair apart.
            struct Range {
                uint32_t base, n, row;
            };
            std::vector<Range> ranges;
            for (uint32_t i = 0; i < na;) {
                const uint32_t base = rec[a0 + i].out;
                uint32_t j = i;
                for (; j < na && task[a0 + j].node == task[a0 + i].node; j++)
                    if (task[a0 + j].config != j - i || rec[a0 + j].out != base + (j - i)) return false;
                ranges.push_back({base, j - i, i});
                i = j;
            }
            std::sort(ranges.begin(), ranges.end(), [](const Range& x, const Range& y) { return x.base < y.base; });
            for (size_t r = 1; r < ranges.size(); r++)
                if (uint64_t(ranges[r - 1].base) + ranges[r - 1].n > ranges[r].base) return false;
            // The rows of one node of b read the same few children: the
            // ranges found for the current node are tried first.
            constexpr uint32_t RECENT = 16;
            const Range* recent[RECENT];
            uint32_t nrecent = 0;
            auto row_of = [&](uint32_t s) -> uint32_t {  // NONE: no row of a writes s
                for (uint32_t q = 0; q < nrecent; q++)
                    if (s - recent[q]->base < recent[q]->n) return recent[q]->row + (s - recent[q]->base);
                auto it = std::upper_bound(ranges.begin(), ranges.end(), s,
                                           [](uint32_t v, const Range& r) { return v < r.base; });
                if (it == ranges.begin()) return NONE;
                --it;
                if (s - it->base >= it->n) return NONE;
                if (nrecent < RECENT) recent[nrecent++] = &*it;
                return it->row + (s - it->base);
            };
            std::vector<uint32_t> up(na + nb), size(na + nb, 1);
            for (uint32_t i = 0; i < na + nb; i++) up[i] = i;
            auto find = [&](uint32_t x) {
                while (up[x] != x) x = up[x] = up[up[x]];
                return x;
            };
            bool fits = true;
            for (uint32_t j = 0; j < nb && fits; j++) {
                if ((j & 255) == 0 && __atomic_load_n(stop, __ATOMIC_RELAXED)) return false;
                if (j == 0 || task[b0 + j].node != task[b0 + j - 1].node) nrecent = 0;
                reads(rec[b0 + j], [&](uint32_t s) {
                    const uint32_t i = row_of(s);
                    if (i == NONE) return;
                    uint32_t x = find(i), y = find(na + j);
                    if (x == y) return;
                    if (size[x] > size[y]) std::swap(x, y);
                    up[x] = y;
                    size[y] += size[x];
                    if (size[y] > TOP_FUSE_MAX) fits = false;
                });
            }
            if (!fits) return false;
            std::vector<uint32_t>& id = size;  // reused: each root's group number
            std::fill(id.begin(), id.end(), NONE);
            g->label.assign(na + nb, 0);
            g->size_a.clear();
            g->size_b.clear();
            for (uint32_t v = 0; v < na + nb; v++) {
                const uint32_t x = v < nb ? na + v : v - nb;  // b's rows first
                const uint32_t r = find(x);
                if (id[r] == NONE) {
                    id[r] = (uint32_t)g->size_a.size();
                    g->size_a.push_back(0);
                    g->size_b.push_back(0);
                }
                g->label[x] = id[r];
                (x < na ? g->size_a : g->size_b)[id[r]]++;
            }
            return true;
        };
        // A fused pair: each tree's groups dealt into chunks in order, and
        // its rows of each depth reordered by (chunk, group).
        auto fuse_pair = [&](std::vector<Grouping>& gs, std::vector<std::vector<uint32_t>>& ca,
                             std::vector<std::vector<uint32_t>>& cb) {
            parallel_for(J, [&](size_t k) {
                Grouping& g = gs[k];
                const size_t ng = g.size_a.size();
                std::vector<uint32_t> gchunk(ng);
                for (size_t c = 0; c < ng; c++) {
                    const bool open = !ca[k].empty(), empty = open && ca[k].back() == 0 && cb[k].back() == 0;
                    if (!open || (!empty && (ca[k].back() + g.size_a[c] > TOP_CHUNK_ROWS ||
                                             cb[k].back() + g.size_b[c] > TOP_CHUNK_ROWS))) {
                        ca[k].push_back(0);
                        cb[k].push_back(0);
                    }
                    gchunk[c] = (uint32_t)ca[k].size() - 1;
                    ca[k].back() += g.size_a[c];
                    cb[k].back() += g.size_b[c];
                }
                auto reorder = [&](uint32_t base, uint32_t n, bool side_b, const std::vector<uint32_t>& per_chunk) {
                    const uint32_t lab0 = side_b ? g.na : 0;
                    std::vector<uint32_t> fill(per_chunk.size(), 0), gat(ng);
                    for (size_t c = 1; c < per_chunk.size(); c++) fill[c] = fill[c - 1] + per_chunk[c - 1];
                    for (size_t c = 0; c < ng; c++) {  // groups inside a chunk keep their order
                        gat[c] = fill[gchunk[c]];
                        fill[gchunk[c]] += side_b ? g.size_b[c] : g.size_a[c];
                    }
                    std::vector<Task> t(n);
                    std::vector<BackRec> r(n);
                    for (uint32_t i = 0; i < n; i++) {
                        const uint32_t to = gat[g.label[lab0 + i]]++;
                        t[to] = task[base + i];
                        r[to] = rec[base + i];
                    }
                    std::copy(t.begin(), t.end(), task.begin() + base);
                    std::copy(r.begin(), r.end(), rec.begin() + base);
                };
                reorder(g.a0, g.na, false, ca[k]);
                reorder(g.b0, g.nb, true, cb[k]);
            });
        };
        for (size_t i = 0; i < depths.size();) {
            const uint32_t a = depths[i];
            // A draw of the traverser sums outcomes that several of its
            // configs share: rows of b that draw join large groups, so such a
            // pair is not grouped at all.
            auto draws = [&](uint32_t d) {
                for (uint32_t r = lvl[d]; r < lvl[d + 1]; r++)
                    if ((rec[r].kn >> 30) == BACK_DRAW) return true;
                return false;
            };
            if (fuse && i + 1 < depths.size() && !draws(depths[i + 1])) {
                const uint32_t b = depths[i + 1];
                std::vector<Grouping> gs(J);
                bool stop = false;
                parallel_for(J, [&](size_t k) {
                    if (!group(a, b, k, &gs[k], &stop)) __atomic_store_n(&stop, true, __ATOMIC_RELAXED);
                });
                if (!stop) {
                    std::vector<std::vector<uint32_t>> ca(J), cb(J);  // rows of a and of b per chunk, per tree
                    fuse_pair(gs, ca, cb);
                    size_t nchunks = 0;
                    for (size_t k = 0; k < J; k++) nchunks += ca[k].size();
                    run.insert(run.end(), {a, b, (uint32_t)chunk.size(), (uint32_t)nchunks});
                    for (int side = 0; side < 2; side++) {
                        uint32_t at = lvl[side ? b : a];
                        chunk.push_back(at);
                        for (size_t k = 0; k < J; k++)
                            for (uint32_t n : side ? cb[k] : ca[k]) chunk.push_back(at += n);
                    }
                    i += 2;
                    continue;
                }
            }
            run.insert(run.end(), {a, NONE, (uint32_t)chunk.size(), 0u});
            i += 1;
        }
    });
}

// The reach pass's launches over the top depths (WaveHost::top_reach_run).
// The non-empty depths are taken top-down; each depth and the next one below
// fuse into one launch when chunks of the deeper depth's rows (TOP_CHUNK_ROWS
// consecutive rows of one tree) each read at most TOP_FUSE_MAX rows of the
// shallower depth (a reach row reads parent reach slots through its gather).
// Each chunk names those rows and computes them itself, so a shallower row
// read by two chunks is computed twice; the shallower rows no chunk reads
// fill chunks of their own. Reach rows keep no state, so computing one twice
// writes the same value twice. The rows keep their order. Without `fuse`
// every depth is its own launch.
void plan_top_reach(WaveHost* wp, bool fuse) {
    WaveHost& w = *wp;
    const size_t J = w.trees.size();
    parallel_for(2, [&](size_t pi) {
        const int p = (int)pi;
        std::vector<uint32_t>& run = w.top_reach_run[p];
        std::vector<uint32_t>& chunk = w.top_reach_chunk[p];
        std::vector<uint32_t>& par = w.top_reach_par[p];
        run.clear();
        chunk.clear();
        par.clear();
        const std::vector<uint32_t>& lvl = w.top_reach_lvl[p];
        const std::vector<Task>& task = w.top_reach[p];
        const std::vector<ReachRec>& rec = w.top_reach_rec[p];
        std::vector<uint32_t> depths;  // the non-empty ones, top-down
        for (uint32_t l = 0; l < w.top_levels; l++)
            if (lvl[l + 1] > lvl[l]) depths.push_back(l);
        auto cut = [&](uint32_t d, size_t k) -> uint32_t {
            if (k >= J) return lvl[d + 1];
            return (uint32_t)(std::lower_bound(task.begin() + lvl[d], task.begin() + lvl[d + 1], w.trees[k].node0,
                                               [](const Task& t, uint32_t n) { return t.node < n; }) -
                              task.begin());
        };
        // One tree's chunks for the pair (shallower d, deeper e): the deeper
        // rows per chunk and the shallower rows each chunk names (wave-global
        // row indices), then the chunks of unread shallower rows. False when
        // a chunk would name more than TOP_FUSE_MAX rows (or another tree's
        // did: `stop`), or the shallower rows are not laid out node by node.
        struct Chunks {
            std::vector<uint32_t> deep, npar, par;
        };
        auto plan = [&](uint32_t d, uint32_t e, size_t k, Chunks* c, const bool* stop) {
            const uint32_t a0 = cut(d, k), na = cut(d, k + 1) - a0, b0 = cut(e, k), nb = cut(e, k + 1) - b0;
            struct Range {
                uint32_t base, n, row;
            };
            std::vector<Range> ranges;
            for (uint32_t i = 0; i < na;) {
                const uint32_t base = rec[a0 + i].out;
                uint32_t j = i;
                for (; j < na && task[a0 + j].node == task[a0 + i].node; j++)
                    if (task[a0 + j].config != j - i || rec[a0 + j].out != base + (j - i)) return false;
                ranges.push_back({base, j - i, i});
                i = j;
            }
            std::sort(ranges.begin(), ranges.end(), [](const Range& x, const Range& y) { return x.base < y.base; });
            for (size_t r = 1; r < ranges.size(); r++)
                if (uint64_t(ranges[r - 1].base) + ranges[r - 1].n > ranges[r].base) return false;
            const Range* last = nullptr;  // a row's gather reads one parent's slots
            auto row_of = [&](uint32_t s) -> uint32_t {
                if (last && s - last->base < last->n) return last->row + (s - last->base);
                auto it = std::upper_bound(ranges.begin(), ranges.end(), s,
                                           [](uint32_t v, const Range& r) { return v < r.base; });
                if (it == ranges.begin()) return NONE;
                --it;
                if (s - it->base >= it->n) return NONE;
                last = &*it;
                return it->row + (s - it->base);
            };
            std::vector<uint8_t> read(na, 0);
            std::vector<uint32_t> mine;
            for (uint32_t c0 = 0; c0 < nb; c0 += TOP_CHUNK_ROWS) {
                if (__atomic_load_n(stop, __ATOMIC_RELAXED)) return false;
                const uint32_t c1 = std::min(nb, c0 + TOP_CHUNK_ROWS);
                mine.clear();
                for (uint32_t j = c0; j < c1; j++) {
                    const ReachRec& q = rec[b0 + j];
                    const uint32_t n = q.kn & REC_N;
                    const std::vector<uint32_t>& src = (q.kn >> 31) == REACH_REV ? w.rev_src : w.rvd_src;
                    if (uint64_t(q.start) + n > src.size()) continue;  // refused by validation later
                    for (uint32_t x = 0; x < n; x++) {
                        const uint32_t i = row_of(q.pbase + src[q.start + x]);
                        if (i != NONE) mine.push_back(i);
                    }
                }
                std::sort(mine.begin(), mine.end());
                mine.erase(std::unique(mine.begin(), mine.end()), mine.end());
                if (mine.size() > TOP_FUSE_MAX) return false;
                c->deep.push_back(c1 - c0);
                c->npar.push_back((uint32_t)mine.size());
                for (uint32_t i : mine) {
                    c->par.push_back(a0 + i);
                    read[i] = 1;
                }
            }
            uint32_t fill = 0;  // unread shallower rows, TOP_CHUNK_ROWS per chunk
            for (uint32_t i = 0; i < na; i++) {
                if (read[i]) continue;
                if (fill == 0) {
                    c->deep.push_back(0);
                    c->npar.push_back(0);
                }
                c->par.push_back(a0 + i);
                c->npar.back()++;
                fill = fill + 1 == TOP_CHUNK_ROWS ? 0 : fill + 1;
            }
            return true;
        };
        for (size_t i = 0; i < depths.size();) {
            const uint32_t d = depths[i];
            if (fuse && i + 1 < depths.size()) {
                const uint32_t e = depths[i + 1];
                std::vector<Chunks> cs(J);
                bool stop = false;
                parallel_for(J, [&](size_t k) {
                    if (!plan(d, e, k, &cs[k], &stop)) __atomic_store_n(&stop, true, __ATOMIC_RELAXED);
                });
                if (!stop) {
                    size_t nchunks = 0;
                    for (size_t k = 0; k < J; k++) nchunks += cs[k].deep.size();
                    run.insert(run.end(), {d, e, (uint32_t)chunk.size(), (uint32_t)nchunks});
                    uint32_t at = lvl[e];
                    chunk.push_back(at);
                    for (size_t k = 0; k < J; k++)
                        for (uint32_t n : cs[k].deep) chunk.push_back(at += n);
                    uint32_t pat = (uint32_t)par.size();
                    chunk.push_back(pat);
                    for (size_t k = 0; k < J; k++) {
                        for (uint32_t n : cs[k].npar) chunk.push_back(pat += n);
                        par.insert(par.end(), cs[k].par.begin(), cs[k].par.end());
                    }
                    i += 2;
                    continue;
                }
            }
            run.insert(run.end(), {d, NONE, (uint32_t)chunk.size(), 0u});
            i += 1;
        }
    });
}

}  // namespace

constexpr size_t WAVE_HOST_BYTES = 2576;  // sizeof(WaveHost) on x86-64 (libstdc++)
static_assert(sizeof(WaveHost) == WAVE_HOST_BYTES, "a WaveHost member was added or changed: update reset() and digest()");
// Lists the packer sizes with resize() and then overwrites whole keep their
// length (and contents) here: the next resize then clears only what the
// wave adds over the last one's length, instead of every entry of a few
// hundred MB again. Lists built by appending are emptied.
void WaveHost::reset() {
    const WaveHost blank;
    auto empty = [](auto& v) { v.clear(); };
    meta = blank.meta;
    net = blank.net;
    empty(jobs);
    empty(units);
    empty(node_top);
    empty(legal_value);
    empty(head_tile_n);
    for (int p = 0; p < 2; p++) {
        empty(head_rb_n[p]);
        empty(top_back[p]);
        empty(top_reach[p]);
        empty(top_back_lvl[p]);
        empty(top_reach_lvl[p]);
        empty(top_back_run[p]);
        empty(top_back_chunk[p]);
        empty(top_reach_run[p]);
        empty(top_reach_chunk[p]);
        empty(top_reach_par[p]);
        empty(pool_grp[p]);
        empty(tower_blk[p]);
        empty(tower_unit[p]);
        top_dec0[p] = blank.top_dec0[p];
    }
    reach_len = blank.reach_len;
    vals_len = blank.vals_len;
    ncells = blank.ncells;
    root_values_len = blank.root_values_len;
    snapshot_configs = blank.snapshot_configs;
    nsub = blank.nsub;
    lvl_len = blank.lvl_len;
    top_levels = blank.top_levels;
    max_levels = blank.max_levels;
    nroots_max = blank.nroots_max;
    carry_slots = blank.carry_slots;
    max_vwin = blank.max_vwin;
    max_rwin = blank.max_rwin;
    checked = blank.checked;
    tower_len = blank.tower_len;
}

bool pack_wave(std::vector<std::shared_ptr<const Job>>&& jobs, WaveHost* out, std::string* err, uint32_t unit_slots,
               bool validated, bool fuse_top) {
    if (jobs.empty()) {
        *err = "cannot pack an empty wave";
        return false;
    }
    WaveHost& w = *out;  // packed in place: a reused WaveHost keeps its buffers
    w.reset();
    w.meta = jobs[0]->meta;
    for (size_t k = 1; k < jobs.size(); k++)
        if (!same_meta(jobs[0]->meta, jobs[k]->meta)) {
            *err = "wave mixes different CFR schedules";
            return false;
        }
    if (!w.net.parse(w.meta.net_dims, err)) return false;
    if (!validated) {  // jobs validate independently; the first failure in job order is reported
        std::vector<std::string> errs(jobs.size());
        std::vector<uint8_t> bad(jobs.size(), 0);
        parallel_for(jobs.size(), [&](size_t k) { bad[k] = !validate(*jobs[k], &errs[k]); });
        for (size_t k = 0; k < jobs.size(); k++)
            if (bad[k]) {
                *err = errs[k];
                return false;
            }
    }
    for (uint32_t x : w.meta.snap_iters)
        if (x > w.meta.iters) {
            *err = "snap_iters beyond iters";
            return false;
        }

    if (unit_slots == 0) {
        *err = "unit budget must be positive";
        return false;
    }
    // Every leaf must fit a unit (tops carry no leaves): the budget is at least
    // the widest node of the wave.
    for (const auto& job : jobs)
        for (uint32_t i = 0; i < job->t.nodes; i++)
            unit_slots = std::max(unit_slots, std::max(job->t.nc(i, 0), job->t.nc(i, 1)));

    // The jobs are packed in three steps: each job's own layout (in parallel),
    // every job's offset into each wave list (a prefix over the jobs), then
    // each job's entries written at its offsets (in parallel). The lists are
    // exactly what appending the jobs one after another makes.
    const size_t J = jobs.size();
    const bool v5 = w.net.kind == MODEL_V5, tower = w.net.kind == MODEL_TWO_TOWER;
    std::vector<JobLayout> lay(J);
    parallel_for(J, [&](size_t k) { lay[k].build(jobs[k]->t, w.net, v5, unit_slots); });
    for (size_t k = 0; k < J; k++)  // the first failure in job order
        if (!lay[k].err.empty()) {
            *err = lay[k].err;
            return false;
        }
    std::vector<JobAt> at(J);
    JobAt n{};  // running totals: the next job's offsets
    uint32_t top_levels = 0;
    for (size_t k = 0; k < J; k++) {
        const Tables& t = jobs[k]->t;
        const JobLayout& L = lay[k];
        at[k] = n;
        n.node += t.nodes;
        n.child += (uint32_t)t.node_child.size();
        n.lrow += (uint32_t)t.legal_off.size() - 1;
        n.cell += t.ncells;
        n.draw += (uint32_t)t.draw_to.size();
        n.drow += (uint32_t)t.draw_row_start.size();
        n.reach += L.reach_len;
        n.vals += L.vlen;
        n.rrow += (uint32_t)t.rev_start.size() - 1;
        n.rev += (uint32_t)t.rev_src.size();
        n.vrow += (uint32_t)t.rvd_start.size() - 1;
        n.rvd += (uint32_t)t.rvd_src.size();
        n.row += (uint32_t)t.leaf_rows.size();
        n.coff += (uint32_t)t.leaf_coff.size() - 1;
        n.member += (uint32_t)t.leaf_cidx.size();
        n.cfg += t.ncfg;
        n.exit += (uint32_t)(t.leaf_rows.size() + t.term_leaves.size());
        n.ecoff += (uint32_t)t.snap_coff.size() - 1;
        n.ecfg += t.snapshot_configs();
        n.term += (uint32_t)t.term_leaves.size();
        n.rootv += jobs[k]->nroots() * (t.nc(0, 0) + t.nc(0, 1));
        n.unit += (uint32_t)L.unit_d0.size();
        n.lvl += L.lvls;
        n.urow += L.nrow;
        n.uterm += L.nterm;
        for (int p = 0; p < 2; p++) {
            n.back[p] += L.nback[p];
            n.rch[p] += L.nreach[p];
            n.dec[p] += L.ndec[p];
        }
        n.pub += t.leaf_raw.size();
        n.card += v5 ? t.card_feat.size() : 0;
        n.priv += v5 ? size_t(t.ncfg) * w.net.cfeat : tower ? size_t(t.ncfg) * w.net.priv_in : 0;
        n.emb += v5 ? 0 : size_t(t.ncfg) * w.net.pool;
        n.roots += jobs[k]->root[0].size() + jobs[k]->root[1].size();
        for (uint32_t r = 0; r < jobs[k]->nroots(); r++) n.carried += jobs[k]->carried[0][r].size() + jobs[k]->carried[1][r].size();
        n.rowjob += v5 ? t.rows : 0;
        w.max_levels = std::max(w.max_levels, L.max_levels);
        w.nroots_max = std::max(w.nroots_max, jobs[k]->nroots());
        top_levels = std::max(top_levels, L.top_depths);
    }
    // Every list at its final size, the larger ones side by side (a resize
    // clears its new entries: the fill below overwrites them all).
    std::vector<std::function<void()>> sizing = {
        [&] {
            for (auto* v : {&w.node_meta, &w.child_start, &w.legal_row_of, &w.draw_off, &w.draw_row_off, &w.parent,
                            &w.rev_row_of, &w.rvd_row_of})
                v->resize(n.node);
            w.node_nc.resize(2 * size_t(n.node));
            w.reach_base.resize(2 * size_t(n.node));
            w.vals_base.resize(2 * size_t(n.node));
            w.node_top.assign(n.node, 0);
            w.child.resize(n.child);
            w.legal_off.resize(1 + size_t(n.lrow));
            w.legal_off[0] = 0;
        },
        [&] { w.legal_value.assign(n.cell, NONE); },
        [&] { w.draw_to.resize(n.draw); },
        [&] { w.draw_p.resize(n.draw); },
        [&] { w.draw_row_start.resize(n.drow); },
        [&] {
            w.rev_start.resize(1 + size_t(n.rrow));
            w.rev_start[0] = 0;
            w.rvd_start.resize(1 + size_t(n.vrow));
            w.rvd_start[0] = 0;
        },
        [&] { w.rev_src.resize(n.rev); },
        [&] { w.rev_cell.resize(n.rev); },
        [&] { w.rvd_src.resize(n.rvd); },
        [&] { w.rvd_p.resize(n.rvd); },
        [&] {
            w.row_node.resize(n.row);
            w.row_cfg_off.resize(1 + size_t(n.coff));
            w.row_cfg_off[0] = 0;
            w.row_cfg.resize(n.member);
            w.cfg_key.resize(n.cfg);
            w.cfg_job.resize(v5 ? n.cfg : 0);
            w.cfg_owner.resize(v5 ? n.cfg : 0);
            w.row_job.resize(n.rowjob);
        },
        [&] {
            w.cfg_emb.resize(n.emb);
            w.cfg_priv.resize(n.priv);
            w.card_feat.resize(n.card);
        },
        [&] { w.pub_raw.resize(n.pub); },
        [&] {
            w.term_node.resize(n.term);
            w.term_util.resize(n.term);
            w.roots.resize(n.roots);
            w.carried.resize(n.carried);
            w.exit_node.resize(n.exit);
            w.exit_coff.resize(1 + size_t(n.ecoff));
            w.exit_coff[0] = 0;
            w.trees.resize(J);
            w.unit_row.resize(n.urow);
            w.unit_term.resize(n.uterm);
        },
    };
    for (int p = 0; p < 2; p++) {
        sizing.push_back([&, p] {
            w.back_lvl[p].resize(n.lvl);
            w.reach_lvl[p].resize(n.lvl);
            w.decision[p].resize(n.dec[p]);
        });
        sizing.push_back([&, p] { w.back_task[p].resize(n.back[p]); });
        sizing.push_back([&, p] { w.reach_task[p].resize(n.rch[p]); });
    }
    parallel_for(sizing.size(), [&](size_t k) { sizing[k](); });
    std::vector<UnitDev> sub_units(n.unit);
    std::vector<uint32_t> job_rows(J);  // first network row of each job
    w.ncells = n.cell;
    w.reach_len = n.reach;
    w.vals_len = n.vals;
    w.snapshot_configs = n.ecfg;
    w.root_values_len = n.rootv;
    w.lvl_len = n.lvl;

    parallel_for(J, [&](size_t k) {
        const Job& job = *jobs[k];
        const Tables& t = job.t;
        const JobAt& a = at[k];
        JobLayout& L = lay[k];
        const uint32_t N = t.nodes, node0 = a.node;
        for (uint32_t i = 0; i < N; i++) {
            const uint32_t g = node0 + i;
            w.node_meta[g] = uint32_t(t.node_kind[i]) | uint32_t(t.node_player[i]) << 2;
            w.node_nc[2 * size_t(g)] = t.nc(i, 0);
            w.node_nc[2 * size_t(g) + 1] = t.nc(i, 1);
            w.child_start[g] = a.child + t.node_child_start[i];
            w.legal_row_of[g] = t.legal_row_of[i] == NONE ? NONE : a.lrow + t.legal_row_of[i];
            w.draw_off[g] = a.draw + t.draw_off[i];
            w.draw_row_off[g] = a.drow + t.draw_row_off[i];
            w.parent[g] = t.node_parent[i] == NONE ? NONE : node0 + t.node_parent[i];
            w.rev_row_of[g] = t.rev_row_of[i] == NONE ? NONE : a.rrow + t.rev_row_of[i];
            w.rvd_row_of[g] = t.rvd_row_of[i] == NONE ? NONE : a.vrow + t.rvd_row_of[i];
        }
        for (size_t x = 0; x < t.node_child.size(); x++) w.child[a.child + x] = node0 + t.node_child[x];
        for (size_t x = 1; x < t.legal_off.size(); x++) w.legal_off[a.lrow + x] = t.legal_off[x] + a.cell;
        std::copy(t.draw_row_start.begin(), t.draw_row_start.end(), w.draw_row_start.begin() + a.drow);
        std::copy(t.draw_to.begin(), t.draw_to.end(), w.draw_to.begin() + a.draw);
        std::copy(t.draw_p.begin(), t.draw_p.end(), w.draw_p.begin() + a.draw);

        // Reach slots: a player who did not act at the parent keeps the
        // parent's vector, every other node gets its own (the slots of
        // engine/src/gpu/wave.rs:358-374). They are handed out to the top
        // region's nodes in BFS order, then unit by unit (below), each unit's
        // nodes level by level, player 0's before player 1's: every unit owns
        // one contiguous run of each player's slots, its reach window.
        uint32_t reach_at = a.reach;
        auto own_reach = [&](uint32_t local, int p) {
            const uint32_t node = node0 + local;
            if (local == 0 || t.node_player[t.node_parent[local]] == p) {
                w.reach_base[2 * size_t(node) + p] = reach_at;
                reach_at += t.nc(local, p);
            } else {
                w.reach_base[2 * size_t(node) + p] = w.reach_base[2 * size_t(node0 + t.node_parent[local]) + p];
            }
        };
        if (!L.top.empty()) {
            std::vector<uint8_t> is_top(N, 0);
            for (uint32_t i : L.top) is_top[i] = 1;
            for (uint32_t local : t.bfs_order)
                if (is_top[local])
                    for (int p = 0; p < 2; p++) own_reach(local, p);
        }
        for (uint32_t i = 0; i < N; i++)
            for (int p = 0; p < 2; p++) w.vals_base[2 * size_t(node0 + i) + p] = a.vals + L.vb[p][i];

        // Direct value index of each legal cell's successor (wave.rs:393-411).
        for (uint32_t i = 0; i < N; i++) {
            if (t.node_kind[i] != 0) continue;
            int p = t.node_player[i];
            uint32_t rowa = t.legal_row_of[i];
            for (uint32_t c = 0; c < t.nc(i, p); c++)
                for (uint32_t g = t.legal_off[rowa + c]; g < t.legal_off[rowa + c + 1]; g++)
                    if (t.legal_trans[g] != NONE)
                        w.legal_value[a.cell + g] = w.vals_base[2 * size_t(node0 + t.legal_child[g]) + p] + t.legal_trans[g];
        }

        for (size_t x = 1; x < t.rev_start.size(); x++) w.rev_start[a.rrow + x] = t.rev_start[x] + a.rev;
        std::copy(t.rev_src.begin(), t.rev_src.end(), w.rev_src.begin() + a.rev);
        for (size_t x = 0; x < t.rev_cell.size(); x++) w.rev_cell[a.rev + x] = t.rev_cell[x] + a.cell;
        for (size_t x = 1; x < t.rvd_start.size(); x++) w.rvd_start[a.vrow + x] = t.rvd_start[x] + a.rvd;
        std::copy(t.rvd_src.begin(), t.rvd_src.end(), w.rvd_src.begin() + a.rvd);
        std::copy(t.rvd_p.begin(), t.rvd_p.end(), w.rvd_p.begin() + a.rvd);

        // Network rows and interned configs.
        job_rows[k] = a.row;
        for (size_t r = 0; r < t.leaf_rows.size(); r++) w.row_node[a.row + r] = node0 + t.leaf_rows[r];
        for (size_t x = 1; x < t.leaf_coff.size(); x++) w.row_cfg_off[a.coff + x] = t.leaf_coff[x] + a.member;
        for (size_t x = 0; x < t.leaf_cidx.size(); x++) w.row_cfg[a.member + x] = t.leaf_cidx[x] + a.cfg;
        if (v5) {
            std::fill(w.row_job.begin() + a.rowjob, w.row_job.begin() + a.rowjob + t.rows, (uint32_t)k);
            std::copy(t.card_feat.begin(), t.card_feat.end(), w.card_feat.begin() + a.card);
            // the config encoder reads the counts, the owner's card view and its job's table
            for (uint32_t c = 0; c < t.ncfg; c++) {
                w.cfg_key[a.cfg + c] = 0;
                std::copy(&t.cphi[size_t(c) * w.net.cfeat], &t.cphi[size_t(c) * w.net.cfeat] + w.net.cfeat,
                          w.cfg_priv.begin() + a.priv + size_t(c) * w.net.cfeat);
                w.cfg_job[a.cfg + c] = (uint32_t)k;
                w.cfg_owner[a.cfg + c] = t.cplayer[c];
            }
        } else {
            for (uint32_t c = 0; c < t.ncfg; c++) {
                const float* phi = &t.cphi[size_t(c) * w.net.cfeat];
                w.cfg_key[a.cfg + c] = (uint32_t)phi[0];
                std::copy(phi + 1, phi + 1 + w.net.pool, w.cfg_emb.begin() + a.emb + size_t(c) * w.net.pool);
                if (tower)
                    std::copy(phi + 1 + w.net.pool, phi + 1 + w.net.pool + w.net.priv_in,
                              w.cfg_priv.begin() + a.priv + size_t(c) * w.net.priv_in);
            }
        }
        std::copy(t.leaf_raw.begin(), t.leaf_raw.end(), w.pub_raw.begin() + a.pub);
        for (size_t x = 0; x < t.term_leaves.size(); x++) {
            w.term_node[a.term + x] = node0 + t.term_leaves[x];
            w.term_util[a.term + x] = t.terminal_utility[x];
        }

        TreeDev td{};
        td.node0 = node0;
        td.nodes = N;
        td.reach0 = a.reach;
        td.reach_len = L.reach_len;
        td.root0 = (uint32_t)a.roots;
        td.n0 = t.nc(0, 0);
        td.n1 = t.nc(0, 1);
        std::copy(job.root[0].begin(), job.root[0].end(), w.roots.begin() + a.roots);
        std::copy(job.root[1].begin(), job.root[1].end(), w.roots.begin() + a.roots + job.root[0].size());
        td.carried0 = (uint32_t)a.carried;
        td.nroots = job.nroots();
        size_t ca = a.carried;
        for (uint32_t r = 0; r < job.nroots(); r++)
            for (int p = 0; p < 2; p++) {
                std::copy(job.carried[p][r].begin(), job.carried[p][r].end(), w.carried.begin() + ca);
                ca += job.carried[p][r].size();
            }
        td.root_value0 = a.rootv;
        td.exit0 = a.exit;
        td.nexit = (uint32_t)(t.leaf_rows.size() + t.term_leaves.size());
        for (size_t r = 0; r < t.leaf_rows.size(); r++) w.exit_node[a.exit + r] = node0 + t.leaf_rows[r];
        for (size_t r = 0; r < t.term_leaves.size(); r++)
            w.exit_node[a.exit + t.leaf_rows.size() + r] = node0 + t.term_leaves[r];
        for (size_t x = 1; x < t.snap_coff.size(); x++) w.exit_coff[a.ecoff + x] = t.snap_coff[x] + a.ecfg;
        w.trees[k] = td;

        // Sweep units of this tree: level l of unit u holds its nodes at depth
        // d0 + l; each list is unit-major, then player, then level.
        uint32_t lvl = a.lvl, urow = a.urow, uterm = a.uterm, back[2] = {a.back[0], a.back[1]},
                 rch[2] = {a.rch[0], a.rch[1]}, dec[2] = {a.dec[0], a.dec[1]};
        std::vector<std::vector<uint32_t>> by_level;
        for (uint32_t j = 0; j + 1 < L.unit_at.size(); j++) {
            const uint32_t b = L.unit_at[j], e = L.unit_at[j + 1], d0 = L.unit_d0[j];
            UnitDev u{};
            u.tree = (uint32_t)k;
            const uint32_t nl = L.levels_of(j);
            u.nlevels = nl;
            u.lvl0 = lvl;
            lvl += nl + 1;
            by_level.assign(nl, {});
            for (uint32_t x = b; x < e; x++) by_level[L.depth[L.unit_nodes[x]] - d0].push_back(L.unit_nodes[x]);
            for (int p = 0; p < 2; p++) {  // the unit's reach window of each player
                // The tree's root (seeded, written by no row) stays outside it.
                if (d0 == 0 && !by_level.empty() && by_level[0].size() == 1 && by_level[0][0] == 0) own_reach(0, p);
                u.rwin[p] = reach_at;
                for (uint32_t l = 0; l < nl; l++)
                    for (uint32_t local : by_level[l])
                        if (local != 0) own_reach(local, p);
                u.rwin_n[p] = reach_at - u.rwin[p];
                L.max_rwin = std::max(L.max_rwin, u.rwin_n[p]);
            }
            uint64_t slots = 0;
            for (uint32_t x = b; x < e; x++)
                slots += std::max(t.nc(L.unit_nodes[x], 0), t.nc(L.unit_nodes[x], 1));
            u.slots = (uint32_t)std::min<uint64_t>(slots, 0xffffffffu);
            // Value window of each player: the unit owns a contiguous run of slots.
            for (int p = 0; p < 2; p++) {
                uint32_t lo = NONE, hi = 0;
                for (uint32_t x = b; x < e; x++) {
                    const uint32_t i = L.unit_nodes[x];
                    if (t.nc(i, p) == 0) continue;
                    const uint32_t vb = a.vals + L.vb[p][i];
                    lo = std::min(lo, vb);
                    hi = std::max(hi, vb + t.nc(i, p));
                }
                u.vwin[p] = lo == NONE ? 0 : lo;
                u.vwin_n[p] = lo == NONE ? 0 : hi - lo;
                L.max_vwin = std::max(L.max_vwin, u.vwin_n[p]);
            }
            for (int p = 0; p < 2; p++) {
                for (uint32_t l = 0; l < nl; l++) {
                    w.back_lvl[p][u.lvl0 + l] = back[p];
                    w.reach_lvl[p][u.lvl0 + l] = rch[p];
                    for (uint32_t local : by_level[l]) {
                        const uint32_t node = node0 + local;
                        const uint8_t kind = t.node_kind[local];
                        if (kind != 2 && !(kind == 1 && t.node_player[local] != p))
                            for (uint32_t c = 0; c < t.nc(local, p); c++) w.back_task[p][back[p]++] = {node, c};
                        if (local != 0 && t.node_player[t.node_parent[local]] == p)
                            for (uint32_t c = 0; c < t.nc(local, p); c++) w.reach_task[p][rch[p]++] = {node, c};
                    }
                }
                w.back_lvl[p][u.lvl0 + nl] = back[p];
                w.reach_lvl[p][u.lvl0 + nl] = rch[p];
                u.dec0[p] = dec[p];
                for (uint32_t x = b; x < e; x++) {
                    const uint32_t local = L.unit_nodes[x];
                    if (t.node_kind[local] == 0 && t.node_player[local] == p)
                        for (uint32_t c = 0; c < t.nc(local, p); c++) w.decision[p][dec[p]++] = {node0 + local, c};
                }
                u.dec1[p] = dec[p];
            }
            u.row0 = urow;
            for (uint32_t x = b; x < e; x++)
                if (L.row_of[L.unit_nodes[x]] != NONE) w.unit_row[urow++] = a.row + L.row_of[L.unit_nodes[x]];
            u.row1 = urow;
            u.term0 = uterm;
            for (uint32_t x = b; x < e; x++)
                if (L.term_of[L.unit_nodes[x]] != NONE) w.unit_term[uterm++] = a.term + L.term_of[L.unit_nodes[x]];
            u.term1 = uterm;
            sub_units[a.unit + j] = u;
        }
        if (reach_at != a.reach + L.reach_len) L.err = "reach slots: the units and top region do not cover the tree";
        // This tree's top region, by depth (joined with the other trees' below).
        for (uint32_t local : L.top) {
            const uint32_t node = node0 + local, d = L.depth[local];
            w.node_top[node] = 1;
            for (int p = 0; p < 2; p++) {
                const uint8_t kind = t.node_kind[local];
                if (kind != 2 && !(kind == 1 && t.node_player[local] != p))
                    for (uint32_t c = 0; c < t.nc(local, p); c++) {
                        L.top_back[p].push_back({node, c});
                        L.top_back_d[p].push_back(d);
                    }
                if (local != 0 && t.node_player[t.node_parent[local]] == p)
                    for (uint32_t c = 0; c < t.nc(local, p); c++) {
                        L.top_reach[p].push_back({node, c});
                        L.top_reach_d[p].push_back(d);
                    }
                if (kind == 0 && t.node_player[local] == p)
                    for (uint32_t c = 0; c < t.nc(local, p); c++) L.top_dec[p].push_back({node, c});
            }
        }
    });
    for (size_t k = 0; k < J; k++)
        if (!lay[k].err.empty()) {
            *err = lay[k].err;
            return false;
        }
    // Top regions: every tree's rows at one depth together, trees in job order.
    std::vector<std::vector<Task>> top_back[2], top_reach[2];
    std::vector<Task> top_dec[2];
    for (int p = 0; p < 2; p++) {
        top_back[p].resize(top_levels);
        top_reach[p].resize(top_levels);
        for (size_t k = 0; k < J; k++) {
            const JobLayout& L = lay[k];
            for (size_t x = 0; x < L.top_back[p].size(); x++) top_back[p][L.top_back_d[p][x]].push_back(L.top_back[p][x]);
            for (size_t x = 0; x < L.top_reach[p].size(); x++)
                top_reach[p][L.top_reach_d[p][x]].push_back(L.top_reach[p][x]);
            top_dec[p].insert(top_dec[p].end(), L.top_dec[p].begin(), L.top_dec[p].end());
        }
    }
    for (size_t k = 0; k < J; k++) {
        w.max_vwin = std::max(w.max_vwin, lay[k].max_vwin);
        w.max_rwin = std::max(w.max_rwin, lay[k].max_rwin);
    }
    w.child_start.push_back((uint32_t)w.child.size());
    // Head width per 128-row tile of the network rows.
    const uint32_t nrows = w.rows();
    w.head_tile_n.assign((nrows + 127) / 128, 0);
    for (int p = 0; p < 2; p++) w.head_rb_n[p].assign((nrows + 15) / 16, 0);
    parallel_for(w.head_tile_n.size(), [&](size_t tile) {  // one 128-row tile (eight 16-row blocks) each
        const uint32_t r0 = (uint32_t)tile * 128, r1 = std::min<uint32_t>(nrows, r0 + 128);
        uint32_t rb[2][8] = {};  // the tile's blocks, kept local (neighbouring tiles share cache lines)
        for (uint32_t r = r0; r < r1; r++)
            for (int p = 0; p < 2; p++) {
                uint32_t& m = rb[p][(r - r0) / 16];
                for (uint32_t x = w.row_cfg_off[2 * r + p]; x < w.row_cfg_off[2 * r + p + 1]; x++)
                    m = std::max(m, w.cfg_key[w.row_cfg[x]] + 1);
            }
        uint32_t t = 0;
        for (uint32_t b = 0; r0 + 16 * b < r1; b++)
            for (int p = 0; p < 2; p++) {
                w.head_rb_n[p][r0 / 16 + b] = rb[p][b];
                t = std::max(t, rb[p][b]);
            }
        w.head_tile_n[tile] = t;
    });
    // Pool groups: rows with the same config list (same tree, same
    // infostates in the same order), at most POOL_GROUP per group, in row
    // order within a list; longest lists launch first. Config ids are
    // wave-global, so a list never spans two trees: each tree's lists are
    // found on their own, in parallel, and concatenated in tree order, which
    // keeps the lists in the order of their first rows.
    // (Rows with an empty list share one list across the wave: they are set
    // aside per tree and grouped once, in row order, after the others.)
    auto emit = [&](const std::vector<uint32_t>& rows_of, int p, std::vector<PoolGroup>* out) {
        for (size_t k = 0; k < rows_of.size(); k += POOL_GROUP) {
            PoolGroup g{};
            g.cfg = w.row_cfg_off[2 * rows_of[0] + p];
            g.n = w.row_cfg_off[2 * rows_of[0] + p + 1] - g.cfg;
            g.nrows = (uint32_t)std::min<size_t>(POOL_GROUP, rows_of.size() - k);
            for (uint32_t i = 0; i < g.nrows; i++) g.row[i] = rows_of[k + i];
            for (uint32_t i = 0; i < POOL_GROUP; i++)
                g.rbase[i] = w.reach_base[2 * w.row_node[g.row[i < g.nrows ? i : 0]] + p];
            out->push_back(g);
        }
    };
    std::vector<std::vector<PoolGroup>> tree_grp(2 * J);
    std::vector<std::vector<uint32_t>> tree_empty(2 * J);
    parallel_for(2 * J, [&](size_t i) {
        const int p = (int)(i & 1);
        const size_t k = i >> 1;
        const uint32_t ra = job_rows[k], rb = k + 1 < J ? job_rows[k + 1] : nrows;
        // lists keyed by a 64-bit hash of their contents; equal hashes are
        // confirmed element by element (a collision starts its own list)
        std::unordered_multimap<uint64_t, uint32_t> key_of;
        std::vector<std::vector<uint32_t>> lists;
        for (uint32_t r = ra; r < rb; r++) {
            const uint32_t a = w.row_cfg_off[2 * r + p], b = w.row_cfg_off[2 * r + p + 1];
            if (a == b) {
                tree_empty[i].push_back(r);
                continue;
            }
            uint64_t h = 0xcbf29ce484222325ull ^ (b - a);  // FNV-1a over the 32-bit entries
            for (uint32_t x = a; x < b; x++) h = (h ^ w.row_cfg[x]) * 0x100000001b3ull;
            uint32_t id = NONE;
            auto range = key_of.equal_range(h);
            for (auto it = range.first; it != range.second && id == NONE; ++it) {
                const uint32_t r0 = lists[it->second][0];
                const uint32_t a0 = w.row_cfg_off[2 * r0 + p], b0 = w.row_cfg_off[2 * r0 + p + 1];
                if (b0 - a0 == b - a && std::equal(w.row_cfg.begin() + a, w.row_cfg.begin() + b, w.row_cfg.begin() + a0))
                    id = it->second;
            }
            if (id == NONE) {
                id = (uint32_t)lists.size();
                key_of.emplace(h, id);
                lists.emplace_back();
            }
            lists[id].push_back(r);
        }
        for (const auto& rows_of : lists) emit(rows_of, p, &tree_grp[i]);
    });
    for (int p = 0; p < 2; p++) {
        auto& out = w.pool_grp[p];
        out.clear();
        std::vector<uint32_t> empty;
        for (size_t k = 0; k < J; k++) {
            out.insert(out.end(), tree_grp[2 * k + p].begin(), tree_grp[2 * k + p].end());
            empty.insert(empty.end(), tree_empty[2 * k + p].begin(), tree_empty[2 * k + p].end());
        }
        emit(empty, p, &out);  // n = 0: sorted after every other group
        std::stable_sort(out.begin(), out.end(), [](const PoolGroup& a, const PoolGroup& b) { return a.n > b.n; });
    }
    // Two-tower readout blocks: per tree and player, its rows times the
    // config range its rows name.
    if (readout_net(w.net.kind)) {
        job_rows.push_back(nrows);
        w.tower_len = 0;
        for (int p = 0; p < 2; p++) {
            for (size_t t = 0; t + 1 < job_rows.size(); t++) {
                TowerBlock b{};
                b.r0 = job_rows[t];
                b.r1 = job_rows[t + 1];
                b.clo = NONE;
                for (uint32_t r = b.r0; r < b.r1; r++)
                    for (uint32_t x = w.row_cfg_off[2 * r + p]; x < w.row_cfg_off[2 * r + p + 1]; x++) {
                        b.clo = std::min(b.clo, w.row_cfg[x]);
                        b.chi = std::max(b.chi, w.row_cfg[x] + 1);
                    }
                if (b.clo == NONE) continue;  // no configs named by this player's rows
                b.dbase = (uint32_t)w.tower_len;
                w.tower_len += uint64_t(b.r1 - b.r0) * (b.chi - b.clo);
                const uint32_t bi = (uint32_t)w.tower_blk[p].size();
                for (uint32_t r = b.r0 / 16 * 16; r < b.r1; r += TOWER_TILE)
                    for (uint32_t c = b.clo; c < b.chi; c += TOWER_TILE) w.tower_unit[p].push_back({bi, r, c, 0});
                w.tower_blk[p].push_back(b);
            }
        }
        if (w.tower_len >= (1ull << 32)) {
            *err = "wave too large for the two-tower readout";
            return false;
        }
    }
    // Subtree units largest first: the device takes them in launch order.
    std::stable_sort(sub_units.begin(), sub_units.end(),
                     [](const UnitDev& a, const UnitDev& b) { return a.slots > b.slots; });
    w.nsub = (uint32_t)sub_units.size();
    w.units = std::move(sub_units);
    w.top_levels = (uint32_t)std::max(top_back[0].size(), top_back[1].size());
    for (int p = 0; p < 2; p++) {
        top_back[p].resize(w.top_levels);
        top_reach[p].resize(w.top_levels);
        for (uint32_t l = 0; l < w.top_levels; l++) {
            w.top_back_lvl[p].push_back((uint32_t)w.top_back[p].size());
            w.top_reach_lvl[p].push_back((uint32_t)w.top_reach[p].size());
            w.top_back[p].insert(w.top_back[p].end(), top_back[p][l].begin(), top_back[p][l].end());
            w.top_reach[p].insert(w.top_reach[p].end(), top_reach[p][l].begin(), top_reach[p][l].end());
        }
        w.top_back_lvl[p].push_back((uint32_t)w.top_back[p].size());
        w.top_reach_lvl[p].push_back((uint32_t)w.top_reach[p].size());
        // Top decision rows follow every unit's rows, so whole-list kernels
        // (uniform start, seeded sums, the average) cover them too.
        w.top_dec0[p] = (uint32_t)w.decision[p].size();
        w.decision[p].insert(w.decision[p].end(), top_dec[p].begin(), top_dec[p].end());
    }
    w.carry_slots = (w.meta.snapshots && w.meta.snap_iters.size() > 1) ? (uint32_t)w.meta.snap_iters.size() - 1 : 0;
    if (uint64_t(w.rows()) * w.net.heads >= (1ull << 32)) {
        *err = "wave too large: network rows x heads exceeds 2^32";
        return false;
    }
    // Row records keep element counts in REC_N bits and terminal indices in TERM_INDEX bits.
    if (w.ncells > REC_N || w.draw_to.size() > REC_N || w.child.size() > REC_N || w.rev_src.size() > REC_N ||
        w.rvd_src.size() > REC_N || w.term_node.size() > TERM_INDEX) {
        *err = "wave too large for the row records";
        return false;
    }
    build_records(&w);
    // WC_TOP_FUSE=0 or 1 overrides the caller's choice.
    static const int top_fuse_env = [] {
        const char* e = std::getenv("WC_TOP_FUSE");
        return e && *e ? (*e == '0' ? 0 : 1) : -1;
    }();
    plan_top_back(&w, top_fuse_env < 0 ? fuse_top : top_fuse_env == 1);
    plan_top_reach(&w, top_fuse_env < 0 ? fuse_top : top_fuse_env == 1);
    w.jobs = std::move(jobs);
    // A wave packed from jobs that each passed validate() is this packer's own
    // output and is not checked again (about 40% of the packing's host work);
    // WC_DEEP_CHECK=1 checks it anyway. Every other wave is checked.
    static const bool force_deep = [] {
        const char* e = std::getenv("WC_DEEP_CHECK");
        return e && *e && *e != '0';
    }();
    w.checked = false;
    if ((!validated || force_deep) && !validate_deep(w, err)) return false;
    w.checked = !validated || force_deep;
    return true;
}

// (`checked` records how the wave was checked, not what it holds: it stays out.)
uint64_t digest(const WaveHost& w) {
    uint64_t h = 0xcbf29ce484222325ull;
    auto word = [&](uint64_t v) { h = (h ^ v) * 0x100000001b3ull; };
    auto list = [&](const auto& v) {
        const uint8_t* b = (const uint8_t*)v.data();
        const size_t n = v.size() * sizeof(v[0]);
        word(n);
        size_t i = 0;
        for (; i + 8 <= n; i += 8) {
            uint64_t x;
            std::memcpy(&x, b + i, 8);
            word(x);
        }
        uint64_t tail = 0;
        std::memcpy(&tail, b + i, n - i);
        word(tail);
    };
    for (const auto* v : {&w.node_meta, &w.node_nc, &w.child_start, &w.child, &w.legal_row_of, &w.legal_off,
                          &w.legal_value, &w.draw_off, &w.draw_row_off, &w.draw_row_start, &w.draw_to, &w.reach_base,
                          &w.vals_base, &w.parent, &w.rev_row_of, &w.rev_start, &w.rev_src, &w.rev_cell, &w.rvd_row_of,
                          &w.rvd_start, &w.rvd_src, &w.row_node, &w.row_cfg_off, &w.row_cfg, &w.cfg_key,
                          &w.head_tile_n, &w.term_node, &w.exit_node, &w.exit_coff, &w.exit_reach, &w.unit_row,
                          &w.unit_term, &w.cfg_job, &w.row_job})
        list(*v);
    for (const auto* v : {&w.draw_p, &w.rvd_p, &w.cfg_emb, &w.cfg_priv, &w.term_util, &w.roots, &w.carried, &w.card_feat})
        list(*v);
    list(w.pub_raw);
    list(w.cfg_owner);
    list(w.node_top);
    list(w.trees);
    list(w.units);
    for (int p = 0; p < 2; p++) {
        for (const auto* v : {&w.head_rb_n[p], &w.back_lvl[p], &w.reach_lvl[p], &w.top_back_lvl[p], &w.top_reach_lvl[p],
                              &w.top_back_run[p], &w.top_back_chunk[p], &w.top_reach_run[p],
                              &w.top_reach_chunk[p], &w.top_reach_par[p], &w.child_vb[p]})
            list(*v);
        for (const auto* v : {&w.back_task[p], &w.reach_task[p], &w.decision[p], &w.top_back[p], &w.top_reach[p]})
            list(*v);
        list(w.back_rec[p]);
        list(w.top_back_rec[p]);
        list(w.reach_rec[p]);
        list(w.top_reach_rec[p]);
        list(w.acc_rec[p]);
        list(w.leaf_rec[p]);
        list(w.pool_grp[p]);
        list(w.tower_blk[p]);
        list(w.tower_unit[p]);
        word(w.top_dec0[p]);
    }
    for (uint64_t x : {(uint64_t)w.jobs.size(), (uint64_t)w.reach_len, (uint64_t)w.vals_len, (uint64_t)w.ncells,
                       (uint64_t)w.root_values_len, (uint64_t)w.snapshot_configs, (uint64_t)w.nsub,
                       (uint64_t)w.lvl_len, (uint64_t)w.top_levels, (uint64_t)w.max_levels, (uint64_t)w.nroots_max,
                       (uint64_t)w.carry_slots, (uint64_t)w.max_vwin, (uint64_t)w.max_rwin, w.tower_len})
        word(x);
    return h;
}

// Every index a kernel dereferences, checked against the buffer it indexes.
// The device code relies on these bounds and performs no checks of its own.
bool pack_wave(std::vector<Job>&& jobs, WaveHost* out, std::string* err, uint32_t unit_slots, bool validated,
               bool fuse_top) {
    std::vector<std::shared_ptr<const Job>> shared(jobs.size());
    for (size_t k = 0; k < jobs.size(); k++) shared[k] = std::make_shared<const Job>(std::move(jobs[k]));
    jobs.clear();
    return pack_wave(std::move(shared), out, err, unit_slots, validated, fuse_top);
}

bool validate_shape(const WaveHost& w, std::string* err) {
    auto fail = [&](const char* m) {
        *err = std::string("wave bounds: ") + m;
        return false;
    };
    const uint64_t N = w.nodes();
    if (w.node_nc.size() != 2 * N || w.child_start.size() != N + 1 || w.legal_row_of.size() != N ||
        w.draw_off.size() != N || w.draw_row_off.size() != N || w.reach_base.size() != 2 * N ||
        w.vals_base.size() != 2 * N || w.parent.size() != N || w.rev_row_of.size() != N || w.rvd_row_of.size() != N)
        return fail("node arrays disagree");
    if (w.legal_value.size() != w.ncells || w.legal_off.empty() || w.legal_off.back() != w.ncells)
        return fail("cell arrays disagree");
    const uint64_t rows = w.rows();
    // An offset list starts at 0 and ends at its list's length; with every
    // difference equal to its count (checked per entry), no offset wraps.
    if (w.row_cfg_off.size() != 2 * rows + 1 || w.row_cfg_off[0] != 0 || w.row_cfg_off.back() != w.row_cfg.size())
        return fail("row_cfg_off");
    const uint64_t ncfg = w.cfg_key.size();
    if (w.cfg_emb.size() != (w.net.kind == MODEL_V5 ? 0 : ncfg * w.net.pool) ||
        w.pub_raw.size() != rows * w.net.row_bytes)
        return fail("row payload");
    if (w.net.kind == MODEL_MLP)
        for (uint32_t k : w.cfg_key)
            if (k >= w.net.heads) return fail("cfg_key");
    if (w.cfg_priv.size() != (w.net.kind == MODEL_TWO_TOWER ? ncfg * w.net.priv_in
                              : w.net.kind == MODEL_V5      ? ncfg * w.net.cfeat
                                                            : 0))
        return fail("cfg_priv");
    if (w.net.kind == MODEL_V5) {  // the v5 build's per-config and per-row job indices
        const uint64_t njobs = w.trees.size();
        if (w.cfg_job.size() != ncfg || w.cfg_owner.size() != ncfg || w.row_job.size() != rows ||
            w.card_feat.size() != njobs * w.net.card_feat || w.pub_raw.size() != uint64_t(rows) * w.net.row_bytes)
            return fail("v5 tables");
        for (uint64_t c = 0; c < ncfg; c++)
            if (w.cfg_job[c] >= njobs || w.cfg_owner[c] > 1) return fail("v5 config owner");
        for (uint32_t r : w.row_job)
            if (r >= njobs) return fail("v5 row job");
    }
    for (uint32_t t : w.term_node)
        if (t >= N || (w.node_meta[t] & 3u) != 2) return fail("term_node");
    const uint64_t nexit = w.exit_node.size();
    if (w.exit_coff.size() != 2 * nexit + 1 || w.exit_coff[0] != 0 || w.exit_coff.back() != w.snapshot_configs)
        return fail("exit_coff");
    if (w.exit_reach.size() != 2 * nexit) return fail("exit_reach");
    for (uint64_t e = 0; e < nexit; e++)
        for (int p = 0; p < 2; p++)
            if (w.exit_node[e] >= N || w.exit_coff[2 * e + p + 1] - w.exit_coff[2 * e + p] != w.nc(w.exit_node[e], p) ||
                w.exit_reach[2 * e + p] != w.reach_base[2 * size_t(w.exit_node[e]) + p])
                return fail("exit configs");
    for (int p = 0; p < 2; p++) {
        if (w.back_lvl[p].size() != w.lvl_len || w.reach_lvl[p].size() != w.lvl_len) return fail("level arrays");
        if (w.back_rec[p].size() != w.back_task[p].size() || w.top_back_rec[p].size() != w.top_back[p].size() ||
            w.reach_rec[p].size() != w.reach_task[p].size() || w.top_reach_rec[p].size() != w.top_reach[p].size() ||
            w.acc_rec[p].size() != w.decision[p].size())
            return fail("record counts");
    }
    if (w.unit_row.size() != rows || w.unit_term.size() != w.term_node.size()) return fail("unit leaf lists");
    for (uint32_t r : w.unit_row)
        if (r >= rows) return fail("unit_row");
    for (uint32_t te : w.unit_term)
        if ((te & TERM_INDEX) >= w.term_node.size()) return fail("unit_term");
    if (w.nsub > w.units.size()) return fail("unit counts");
    for (const UnitDev& u : w.units) {
        if (uint64_t(u.lvl0) + u.nlevels + 1 > w.lvl_len || u.tree >= w.trees.size()) return fail("unit range");
        for (int p = 0; p < 2; p++) {
            const auto& bl = w.back_lvl[p];
            const auto& rl = w.reach_lvl[p];
            for (uint32_t l = 0; l < u.nlevels; l++) {
                if (bl[u.lvl0 + l + 1] < bl[u.lvl0 + l] || bl[u.lvl0 + l + 1] > w.back_task[p].size())
                    return fail("back levels");
                if (rl[u.lvl0 + l + 1] < rl[u.lvl0 + l] || rl[u.lvl0 + l + 1] > w.reach_task[p].size())
                    return fail("reach levels");
            }
            if (u.dec0[p] > u.dec1[p] || u.dec1[p] > w.decision[p].size()) return fail("decision range");
            if (u.leaf0[p] > u.leaf1[p] || u.leaf1[p] > w.leaf_rec[p].size()) return fail("unit leaf range");
            // The kernels size each unit's LDS windows by the wave's widest.
            if (u.vwin_n[p] > w.max_vwin || u.rwin_n[p] > w.max_rwin || uint64_t(u.vwin[p]) + u.vwin_n[p] > w.vals_len)
                return fail("unit window size");
        }
        if (u.row0 > u.row1 || u.row1 > w.unit_row.size() || u.term0 > u.term1 || u.term1 > w.unit_term.size())
            return fail("unit leaf range");
    }
    for (int p = 0; p < 2; p++) {
        if (w.top_back_lvl[p].size() != w.top_levels + 1 || w.top_reach_lvl[p].size() != w.top_levels + 1)
            return fail("top levels");
        for (uint32_t l = 0; l < w.top_levels; l++)
            if (w.top_back_lvl[p][l + 1] < w.top_back_lvl[p][l] || w.top_reach_lvl[p][l + 1] < w.top_reach_lvl[p][l])
                return fail("top level order");
        if (w.top_back_lvl[p][w.top_levels] != w.top_back[p].size() ||
            w.top_reach_lvl[p][w.top_levels] != w.top_reach[p].size())
            return fail("top level bounds");
        // The value launches: every non-empty depth once, deepest first; a
        // fused pair's chunk bounds run through each depth's rows in order.
        const std::vector<uint32_t>& run = w.top_back_run[p];
        const std::vector<uint32_t>& off = w.top_back_chunk[p];
        if (run.size() % TOP_RUN) return fail("top back runs");
        uint32_t next = w.top_levels;  // depths below this one are still to come
        auto take = [&](uint32_t d) {
            if (d >= next) return false;
            for (uint32_t l = d + 1; l < next; l++)
                if (w.top_back_lvl[p][l + 1] > w.top_back_lvl[p][l]) return false;  // a depth left out
            next = d;
            return w.top_back_lvl[p][d + 1] > w.top_back_lvl[p][d];
        };
        for (size_t i = 0; i < run.size(); i += TOP_RUN) {
            const uint32_t a = run[i], b = run[i + 1], at = run[i + 2], nch = run[i + 3];
            if (!take(a)) return fail("top back runs");
            if (b == NONE) continue;
            if (!take(b) || nch == 0 || uint64_t(at) + 2 * (uint64_t(nch) + 1) > off.size())
                return fail("top back runs");
            for (int side = 0; side < 2; side++) {
                const uint32_t d = side ? b : a;
                const uint32_t* o = off.data() + at + side * (nch + 1);
                if (o[0] != w.top_back_lvl[p][d] || o[nch] != w.top_back_lvl[p][d + 1]) return fail("top back chunks");
                for (uint32_t k = 0; k < nch; k++)
                    if (o[k + 1] < o[k]) return fail("top back chunks");
            }
        }
        for (uint32_t l = 0; l < next; l++)
            if (w.top_back_lvl[p][l + 1] > w.top_back_lvl[p][l]) return fail("top back runs");
        // The reach launches: every non-empty depth once, top-down; a fused
        // pair's deeper bounds run through its rows, its parent lists through
        // top_reach_par, each entry a row of the shallower depth.
        const std::vector<uint32_t>& rrun = w.top_reach_run[p];
        const std::vector<uint32_t>& roff = w.top_reach_chunk[p];
        const std::vector<uint32_t>& rpar = w.top_reach_par[p];
        const std::vector<uint32_t>& rl = w.top_reach_lvl[p];
        if (rrun.size() % TOP_RUN) return fail("top reach runs");
        uint32_t from = 0;  // depths from this one on are still to come
        auto reach_take = [&](uint32_t d) {
            if (d < from || d >= w.top_levels) return false;
            for (uint32_t l = from; l < d; l++)
                if (rl[l + 1] > rl[l]) return false;  // a depth left out
            from = d + 1;
            return rl[d + 1] > rl[d];
        };
        for (size_t i = 0; i < rrun.size(); i += TOP_RUN) {
            const uint32_t d = rrun[i], e = rrun[i + 1], at = rrun[i + 2], nch = rrun[i + 3];
            if (!reach_take(d)) return fail("top reach runs");
            if (e == NONE) continue;
            if (!reach_take(e) || nch == 0 || uint64_t(at) + 2 * (uint64_t(nch) + 1) > roff.size())
                return fail("top reach runs");
            const uint32_t* o = roff.data() + at;
            if (o[0] != rl[e] || o[nch] != rl[e + 1]) return fail("top reach chunks");
            for (uint32_t k = 0; k < nch; k++)
                if (o[k + 1] < o[k]) return fail("top reach chunks");
            const uint32_t* q = o + nch + 1;
            if (q[nch] > rpar.size()) return fail("top reach chunks");
            for (uint32_t k = 0; k < nch; k++)
                if (q[k + 1] < q[k]) return fail("top reach chunks");
            for (uint32_t x = q[0]; x < q[nch]; x++)
                if (rpar[x] < rl[d] || rpar[x] >= rl[d + 1]) return fail("top reach parents");
        }
        for (uint32_t l = from; l < w.top_levels; l++)
            if (rl[l + 1] > rl[l]) return fail("top reach runs");
        if (w.top_dec0[p] > w.decision[p].size()) return fail("top decision rows");
        for (const UnitDev& u : w.units)
            if (u.dec1[p] > w.top_dec0[p]) return fail("unit decision rows overlap the top rows");
    }
    if (readout_net(w.net.kind))
        for (int p = 0; p < 2; p++) {
            for (const TowerBlock& b : w.tower_blk[p])
                if (b.r0 >= b.r1 || b.r1 > rows || b.clo >= b.chi || b.chi > ncfg ||
                    uint64_t(b.dbase) + uint64_t(b.r1 - b.r0) * (b.chi - b.clo) > w.tower_len)
                    return fail("tower block");
            for (const TowerUnit& u : w.tower_unit[p]) {
                if (u.block >= w.tower_blk[p].size()) return fail("tower unit");
                const TowerBlock& b = w.tower_blk[p][u.block];
                if (u.row % 16 || u.row + 16 <= b.r0 || u.row >= b.r1 || u.cfg < b.clo || u.cfg >= b.chi)
                    return fail("tower unit");
            }
        }
    for (const TreeDev& t : w.trees) {
        if (t.nodes == 0 || uint64_t(t.node0) + t.nodes > N) return fail("tree range");
        if (uint64_t(t.reach0) + t.reach_len > w.reach_len) return fail("reach range");
        if (t.n0 != w.nc(t.node0, 0) || t.n1 != w.nc(t.node0, 1)) return fail("root support");
        const uint64_t nr = uint64_t(t.n0) + t.n1;
        if (t.root0 + nr > w.roots.size() || t.carried0 + t.nroots * nr > w.carried.size() ||
            t.root_value0 + t.nroots * nr > w.root_values_len)
            return fail("root ranges");
        if (uint64_t(t.exit0) + t.nexit > nexit) return fail("exit range");
    }
    return true;
}

namespace {

// validate_deep's checks of the element tables, on host threads: the node
// lists (including the host-only lists the row records were built from), the
// tasks, the records and every element they name, the pool groups, the tower
// blocks' rows and the units' windows. They assume validate_shape passed.
bool validate_elements(const WaveHost& w, std::string* err) {
    auto fail = [&](const char* m) {
        *err = std::string("wave bounds: ") + m;
        return false;
    };
    // The first failure of check(i) over [0, n) in index order (nullptr: none),
    // checked in chunks on several host threads (small chunks for short lists
    // of heavy items such as units).
    auto first_fail = [&](uint64_t n, auto check) -> const char* {
        const uint64_t chunk = n < 65536 ? 16 : 4096, nch = (n + chunk - 1) / chunk;
        std::vector<const char*> e(nch, nullptr);
        parallel_for(nch, [&](size_t c) {
            for (uint64_t i = c * chunk; i < std::min<uint64_t>(n, (c + 1) * chunk); i++)
                if (const char* m = check(i)) {
                    e[c] = m;
                    return;
                }
        });
        for (const char* m : e)
            if (m) return m;
        return nullptr;
    };
    const uint64_t N = w.nodes(), rows = w.rows(), ncfg = w.cfg_key.size();
    auto node_check = [&](uint64_t i) -> const char* {
        uint32_t kind = w.node_meta[i] & 3u, actor = w.node_meta[i] >> 2;
        if (kind > 2 || actor > 1) return "node_meta";
        for (int p = 0; p < 2; p++) {
            uint64_t n = w.nc((uint32_t)i, p);
            if (uint64_t(w.reach_base[2 * i + p]) + n > w.reach_len) return "reach slot";
            if (uint64_t(w.vals_base[2 * i + p]) + n > w.vals_len) return "value slot";
        }
        if (w.child_start[i + 1] < w.child_start[i] || w.child_start[i + 1] > w.child.size()) return "child CSR";
        for (uint32_t x = w.child_start[i]; x < w.child_start[i + 1]; x++)
            if (w.child[x] >= N || w.parent[w.child[x]] != i) return "child index";
        if (kind == 0) {
            uint64_t r0 = w.legal_row_of[i], nc = w.nc((uint32_t)i, actor);
            if (r0 == NONE || r0 + nc + 1 > w.legal_off.size()) return "legal rows";
            for (uint64_t r = r0; r < r0 + nc; r++)
                if (w.legal_off[r + 1] < w.legal_off[r] || w.legal_off[r + 1] > w.ncells) return "legal_off";
            if (w.child_start[i + 1] == w.child_start[i]) return "decision node without children";
        } else if (kind == 1) {
            if (w.child_start[i + 1] != w.child_start[i] + 1) return "chance child";
            uint32_t ch = w.child[w.child_start[i]];
            uint64_t rb = w.draw_row_off[i], nc = w.nc((uint32_t)i, actor);
            if (rb + nc + 1 > w.draw_row_start.size()) return "draw rows";
            for (uint64_t c = 0; c < nc; c++) {
                uint64_t lo = w.draw_row_start[rb + c], hi = w.draw_row_start[rb + c + 1];
                if (hi < lo || uint64_t(w.draw_off[i]) + hi > w.draw_to.size()) return "draw entries";
                for (uint64_t x = lo; x < hi; x++)
                    if (w.draw_to[w.draw_off[i] + x] >= w.nc(ch, actor)) return "draw_to";
            }
        }
        uint32_t par = w.parent[i];
        if (par != NONE) {
            if (par >= N) return "parent";
            if ((w.node_meta[par] & 3u) > 2 || (w.node_meta[par] >> 2) > 1) return "node_meta";  // read before its own check
            int p = (int)(w.node_meta[par] >> 2);
            uint64_t nc = w.nc((uint32_t)i, p);
            if (w.rev_row_of[i] != NONE) {
                uint64_t r0 = w.rev_row_of[i];
                if (r0 + nc + 1 > w.rev_start.size()) return "rev rows";
                for (uint64_t c = 0; c < nc; c++)
                    for (uint64_t x = w.rev_start[r0 + c]; x < w.rev_start[r0 + c + 1]; x++)
                        if (x >= w.rev_src.size() || w.rev_src[x] >= w.nc(par, p) || w.rev_cell[x] >= w.ncells)
                            return "rev entry";
            } else if (w.rvd_row_of[i] != NONE) {
                uint64_t r0 = w.rvd_row_of[i];
                if (r0 + nc + 1 > w.rvd_start.size()) return "rvd rows";
                for (uint64_t c = 0; c < nc; c++)
                    for (uint64_t x = w.rvd_start[r0 + c]; x < w.rvd_start[r0 + c + 1]; x++)
                        if (x >= w.rvd_src.size() || w.rvd_src[x] >= w.nc(par, p)) return "rvd entry";
            } else {
                return "node without gather rows";
            }
        }
            return nullptr;
    };
    if (const char* m = first_fail(N, node_check)) return fail(m);
    if (first_fail(w.legal_value.size(), [&](uint64_t k) -> const char* {
            const uint32_t v = w.legal_value[k];
            return v != NONE && v >= w.vals_len ? "legal_value" : nullptr;
        }))
        return fail("legal_value");
    if (const char* m = first_fail(rows, [&](uint64_t r) -> const char* {
            const uint32_t node = w.row_node[r];
            if (node >= N || (w.node_meta[node] & 3u) != 2) return "row_node";
            for (int p = 0; p < 2; p++)
                if (w.row_cfg_off[2 * r + p + 1] - w.row_cfg_off[2 * r + p] != w.nc(node, p)) return "row configs";
            return nullptr;
        }))
        return fail(m);
    if (first_fail(w.row_cfg.size(), [&](uint64_t k) { return w.row_cfg[k] >= ncfg ? "row_cfg" : nullptr; }))
        return fail("row_cfg");
    {  // every row in exactly one group, with the group's list (the two players at once)
        const char* gm[2] = {nullptr, nullptr};
        parallel_for(2, [&](size_t p) {
            std::vector<uint8_t> seen(rows, 0);
            for (const PoolGroup& g : w.pool_grp[p]) {
                if (g.nrows == 0 || g.nrows > POOL_GROUP || (uint64_t)g.cfg + g.n > w.row_cfg.size()) {
                    gm[p] = "pool group";
                    return;
                }
                for (uint32_t i = 0; i < POOL_GROUP; i++) {
                    const uint32_t r = g.row[i < g.nrows ? i : 0];
                    if (r >= rows || g.rbase[i] != w.reach_base[2 * w.row_node[r] + p]) {
                        gm[p] = "pool group reach";
                        return;
                    }
                }
                for (uint32_t i = 0; i < g.nrows; i++) {
                    const uint32_t r = g.row[i];
                    if (r >= rows || seen[r]) {
                        gm[p] = "pool group row";
                        return;
                    }
                    seen[r] = 1;
                    const uint32_t a = w.row_cfg_off[2 * r + p];
                    if (w.row_cfg_off[2 * r + p + 1] - a != g.n ||
                        !std::equal(w.row_cfg.begin() + a, w.row_cfg.begin() + a + g.n, w.row_cfg.begin() + g.cfg)) {
                        gm[p] = "pool group list";
                        return;
                    }
                }
            }
            for (uint8_t v : seen)
                if (!v) {
                    gm[p] = "pool group cover";
                    return;
                }
        });
        for (const char* m : gm)
            if (m) return fail(m);
    }
    for (int p = 0; p < 2; p++) {
        if (first_fail(w.back_task[p].size(), [&](uint64_t k) {
                const Task& q = w.back_task[p][k];
                return q.node >= N || q.config >= w.nc(q.node, p) ? "x" : nullptr;
            }))
            return fail("back task");
        if (first_fail(w.reach_task[p].size(), [&](uint64_t k) {
                const Task& q = w.reach_task[p][k];
                return q.node >= N || q.config >= w.nc(q.node, p) || w.parent[q.node] == NONE ? "x" : nullptr;
            }))
            return fail("reach task");
        if (first_fail(w.decision[p].size(), [&](uint64_t k) {
                const Task& q = w.decision[p][k];
                return q.node >= N || q.config >= w.nc(q.node, p) || (w.node_meta[q.node] & 3u) != 0 ? "x" : nullptr;
            }))
            return fail("decision task");
    }
    for (int p = 0; p < 2; p++) {
        for (const Task& q : w.top_back[p])
            if (q.node >= N || q.config >= w.nc(q.node, p)) return fail("top back task");
        for (const Task& q : w.top_reach[p])
            if (q.node >= N || q.config >= w.nc(q.node, p) || w.parent[q.node] == NONE) return fail("top reach task");
    }
    // Row records: every slot and element they name.
    for (int p = 0; p < 2; p++) {
        auto back_ok = [&](const BackRec& r) {
            const uint64_t n = r.kn & REC_N, kind = r.kn >> 30;
            if (r.out >= w.vals_len) return false;
            if (kind == BACK_OWN) {
                if (uint64_t(r.start) + n > w.ncells) return false;
                for (uint64_t g = r.start; g < r.start + n; g++)
                    if (w.legal_value[g] != NONE && w.legal_value[g] >= w.vals_len) return false;
            } else if (kind == BACK_DRAW) {
                if (uint64_t(r.start) + n > w.draw_to.size()) return false;
                for (uint64_t x = r.start; x < r.start + n; x++)
                    if (uint64_t(r.arg) + w.draw_to[x] >= w.vals_len) return false;
            } else if (kind == BACK_OPP) {
                if (uint64_t(r.start) + n > w.child_vb[p].size()) return false;
                for (uint64_t x = r.start; x < r.start + n; x++)
                    if (uint64_t(w.child_vb[p][x]) + r.arg >= w.vals_len) return false;
            } else {
                return false;
            }
            return true;
        };
        auto reach_ok = [&](const ReachRec& r) {
            const uint64_t n = r.kn & REC_N;
            if (r.out >= w.reach_len) return false;
            if ((r.kn >> 31) == REACH_REV) {
                if (uint64_t(r.start) + n > w.rev_src.size()) return false;
                for (uint64_t x = r.start; x < r.start + n; x++)
                    if (uint64_t(r.pbase) + w.rev_src[x] >= w.reach_len || w.rev_cell[x] >= w.ncells) return false;
            } else {
                if (uint64_t(r.start) + n > w.rvd_src.size()) return false;
                for (uint64_t x = r.start; x < r.start + n; x++)
                    if (uint64_t(r.pbase) + w.rvd_src[x] >= w.reach_len) return false;
            }
            return true;
        };
        if (first_fail(w.back_rec[p].size(), [&](uint64_t k) { return back_ok(w.back_rec[p][k]) ? nullptr : "x"; }))
            return fail("back record");
        if (first_fail(w.top_back_rec[p].size(), [&](uint64_t k) { return back_ok(w.top_back_rec[p][k]) ? nullptr : "x"; }))
            return fail("top back record");
        if (first_fail(w.reach_rec[p].size(), [&](uint64_t k) { return reach_ok(w.reach_rec[p][k]) ? nullptr : "x"; }))
            return fail("reach record");
        if (first_fail(w.top_reach_rec[p].size(),
                       [&](uint64_t k) { return reach_ok(w.top_reach_rec[p][k]) ? nullptr : "x"; }))
            return fail("top reach record");
        if (first_fail(w.acc_rec[p].size(), [&](uint64_t k) {
                const AccRec& r = w.acc_rec[p][k];
                return r.ridx >= w.reach_len || uint64_t(r.lo) + r.n > w.ncells ? "x" : nullptr;
            }))
            return fail("accumulation record");
    }
    const uint64_t heads_end = readout_net(w.net.kind) ? w.tower_len : uint64_t(rows) * w.net.heads;
    for (int p = 0; p < 2; p++)
        if (first_fail(w.leaf_rec[p].size(), [&](uint64_t k) {
                const LeafRec& r = w.leaf_rec[p][k];
                return r.out >= w.vals_len || uint64_t(r.head) >= heads_end || r.mass >= 2 * rows ? "x" : nullptr;
            }))
            return fail("leaf record");
    if (readout_net(w.net.kind))
        for (int p = 0; p < 2; p++)
            for (const TowerBlock& b : w.tower_blk[p])
                for (uint32_t r = b.r0; r < b.r1; r++)
                    for (uint32_t x = w.row_cfg_off[2 * r + p]; x < w.row_cfg_off[2 * r + p + 1]; x++)
                        if (w.row_cfg[x] < b.clo || w.row_cfg[x] >= b.chi) return fail("tower block configs");
    // The subtree sweep keeps each unit's values in LDS: every slot a unit
    // writes (its leaves, its rows) and reads (its rows' children) must lie
    // inside the unit's window.
    auto unit_check = [&](uint64_t ui) -> const char* {
        const UnitDev& u = w.units[ui];
        for (int p = 0; p < 2; p++) {
            // The reach window: the unit's rows write inside it, and a row reads
            // a slot inside it only once a shallower level has written it.
            const uint64_t rlo = u.rwin[p], rn = u.rwin_n[p];
            if (rlo + rn > w.reach_len) return "unit reach window";
            std::vector<uint8_t> written(rn, 0);
            for (uint32_t l = 0; l < u.nlevels; l++) {
                const uint32_t b = w.reach_lvl[p][u.lvl0 + l], e = w.reach_lvl[p][u.lvl0 + l + 1];
                for (uint32_t x = b; x < e; x++) {
                    const ReachRec& r = w.reach_rec[p][x];
                    const uint32_t n = r.kn & REC_N;
                    for (uint32_t k = 0; k < n; k++) {
                        const uint64_t i = uint64_t(r.pbase) +
                                           ((r.kn >> 31) == REACH_REV ? w.rev_src[r.start + k] : w.rvd_src[r.start + k]);
                        if (i - rlo < rn && !written[i - rlo]) return "unit reach row reads an unwritten window slot";
                    }
                }
                for (uint32_t x = b; x < e; x++) {
                    const uint64_t o = w.reach_rec[p][x].out;
                    if (o - rlo >= rn) return "unit reach row writes outside its reach window";
                    written[o - rlo] = 1;
                }
            }
            const uint64_t lo = u.vwin[p], hi = lo + u.vwin_n[p];
            auto in = [&](uint64_t i) { return i >= lo && i < hi; };
            for (uint32_t k = u.leaf0[p]; k < u.leaf1[p]; k++)
                if (!in(w.leaf_rec[p][k].out)) return "unit leaf outside its value window";
            for (uint32_t k = u.term0; k < u.term1; k++) {
                uint32_t node = w.term_node[w.unit_term[k] & TERM_INDEX];
                if (w.nc(node, p) && (!in(w.vals_base[2 * node + p]) || !in(w.vals_base[2 * node + p] + w.nc(node, p) - 1)))
                    return "unit terminal outside its value window";
            }
            for (uint32_t x = w.back_lvl[p][u.lvl0]; x < w.back_lvl[p][u.lvl0 + u.nlevels]; x++) {
                const BackRec& r = w.back_rec[p][x];
                const uint32_t n = r.kn & REC_N, kind = r.kn >> 30;
                if (!in(r.out)) return "unit row outside its value window";
                for (uint32_t k = 0; k < n; k++) {
                    uint64_t i;
                    if (kind == BACK_OWN) {
                        if (w.legal_value[r.start + k] == NONE) continue;
                        i = w.legal_value[r.start + k];
                    } else if (kind == BACK_DRAW) {
                        i = uint64_t(r.arg) + w.draw_to[r.start + k];
                    } else {
                        i = uint64_t(w.child_vb[p][r.start + k]) + r.arg;
                    }
                    if (!in(i)) return "unit row reads outside its value window";
                }
            }
        }
        return nullptr;
    };
    if (const char* m = first_fail(w.units.size(), unit_check)) return fail(m);
    return true;
}

}  // namespace

bool validate_deep(const WaveHost& w, std::string* err) { return validate_shape(w, err) && validate_elements(w, err); }

bool check_chain_plan(const std::vector<ChainPass>& plan, const uint32_t* cols, uint32_t nrb, uint32_t heads,
                      std::string* err) {
    auto fail = [&](const char* m) {
        *err = m;
        return false;
    };
    std::vector<uint8_t> seen(nrb, 0);
    for (const ChainPass& ps : plan) {
        if (ps.n < 1 || ps.n > CHAIN_PASS_BLOCKS) return fail("value net plan: pass size");
        for (uint32_t j = 0; j < ps.n; j++) {
            const uint32_t rb = ps.rb[j];
            if (rb >= nrb || seen[rb]) return fail("value net plan: row block repeated or out of range");
            seen[rb] = 1;
            if (ps.cols < (cols ? cols[rb] : heads)) return fail("value net plan: head columns");
        }
    }
    for (uint32_t rb = 0; rb < nrb; rb++)
        if (!seen[rb]) return fail("value net plan: row block missing");
    return true;
}

std::vector<ChainPass> plan_chain(const uint32_t* cols, uint32_t nrb, uint32_t heads, uint32_t cus) {
    std::vector<ChainPass> out;
    if (!nrb) return out;
    cus = std::max(cus, 1u);
    auto width = [&](uint32_t rb) { return cols ? cols[rb] : heads; };
    std::vector<uint32_t> order(nrb);
    for (uint32_t i = 0; i < nrb; i++) order[i] = i;
    std::stable_sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) { return width(a) > width(b); });
    // Cost in units of one 16-row block's trunk: a pass costs about three of
    // them on top of its blocks (measured on the 512 -> 3 x 384 net). Each 16
    // head columns of a block are weighted 0.07, about three times their
    // measured share of a pass (0.024): the extra weight keeps the passes of
    // wide-head blocks, which finish last otherwise, short. Value net time per
    // wave of 256 subgames with 567 heads, by weight: 0.016 5.44 ms, 0.024
    // 5.20 ms, 0.07 4.90 ms, 0.15 5.25 ms.
    const double pass_cost = 3.0, col_cost = 0.07;
    std::vector<double> c(nrb);
    double total = 0.0, cmax = 0.0;
    for (uint32_t i = 0; i < nrb; i++) {
        c[i] = 1.0 + col_cost * ((width(order[i]) + 15) / 16);
        total += c[i];
        cmax = std::max(cmax, c[i]);
    }
    // A pass also closes before its cost would exceed that of a full pass of
    // narrow (64-column) blocks, so passes of wide-head blocks hold fewer rows
    // and the longest passes, which start first, stay short.
    const double cap = (pass_cost + CHAIN_PASS_BLOCKS * (1.0 + col_cost * 4)) * (1.0 + 1e-9);
    auto closes = [&](uint32_t pn, double pc, uint32_t i) {
        return pn == CHAIN_PASS_BLOCKS || (pn > 0 && pass_cost + pc + c[i] > cap);
    };
    // Shares of consecutive blocks under a cost bound t; returns their ends.
    auto deal = [&](double t, std::vector<uint32_t>* ends) {
        uint32_t shares = 0, i = 0;
        while (i < nrb) {
            double sum = 0.0, pc = 0.0;
            uint32_t n = 0, pn = 0;
            while (i < nrb) {
                const bool fresh = pn == 0 || closes(pn, pc, i);
                const double with = sum + (fresh ? pass_cost : 0.0) + c[i];
                if (n > 0 && with > t) break;
                if (fresh) pn = 0, pc = 0.0;
                sum = with;
                pc += c[i];
                pn++;
                n++;
                i++;
            }
            shares++;
            if (ends) ends->push_back(i);
        }
        return shares;
    };
    double lo = pass_cost + cmax, hi = pass_cost * nrb + total;
    for (int it = 0; it < 48 && hi - lo > 1e-6 * hi; it++) {  // the least bound that fits the CUs
        const double mid = 0.5 * (lo + hi);
        if (deal(mid, nullptr) <= cus)
            hi = mid;
        else
            lo = mid;
    }
    std::vector<uint32_t> ends;
    deal(hi, &ends);
    for (size_t k = 0; k < ends.size(); k++) {  // each share cut into passes by the same rule
        ChainPass ps{};
        double pc = 0.0;
        for (uint32_t i = k ? ends[k - 1] : 0; i < ends[k]; i++) {
            if (closes(ps.n, pc, i)) {
                out.push_back(ps);
                ps = ChainPass{};
                pc = 0.0;
            }
            ps.rb[ps.n++] = order[i];
            ps.cols = std::max(ps.cols, width(order[i]));
            pc += c[i];
        }
        if (ps.n) out.push_back(ps);
    }
    // Longest first: CUs that take the next pass as they free up then end
    // close together (the shares set the pass sizes).
    auto cost = [&](const ChainPass& ps) { return pass_cost + ps.n * (1.0 + col_cost * ((ps.cols + 15) / 16)); };
    std::stable_sort(out.begin(), out.end(),
                     [&](const ChainPass& a, const ChainPass& b) { return cost(a) > cost(b); });
    return out;
}

// Algorithmic HBM bytes of one CFR iteration (readout, backprop with the
// regret/DCFR update, reach gather, average accumulation) for traverser p:
//   44 C_p  legal cells of p: successor index 4, child value 4, cur read 4 +
//           write 4, regret read+write 8, sum read+write 8 (value sweep: 32);
//           accumulate: cur 4 + sum read+write 8 (accumulation: 12)
//   16 G_p  gather entries into p's reach: source 4, cell or probability 4,
//           parent reach 4, strategy 4
//    4 S_p  p's reach slots written
//   12 R_p  p's decision rows: row offsets 8 (value sweep), reach read by the
//           accumulation 4 (accumulation)
//    4 O_p  child-value reads at opponent decision nodes
//   12 H_p  draw entries at p's chance nodes: successor 4, probability 4, value 4
//    8 L_p  leaf value slots of p: net output read 4, value write 4
//    4 L_o  opponent reach read for the leaf reach mass
// A node's value-sweep bytes go to the kernel that sweeps its unit's values
// (subtree sweep or top sweep), its reach bytes to the kernel that gathers its
// reach (subtree reach or top sweep), its accumulation bytes to the leaf-input
// launch that runs every accumulation.
CfrBytes cfr_bytes_per_iter(const WaveHost& w, int p) {
    CfrBytes out;
    const uint32_t N = w.nodes();
    for (uint32_t i = 0; i < N; i++) {
        uint32_t kind = w.node_meta[i] & 3u, actor = w.node_meta[i] >> 2;
        uint32_t ncp = w.nc(i, p);
        const bool top = !w.node_top.empty() && w.node_top[i];
        uint64_t& back = out.part[top ? 1 : 0];
        uint64_t& reach = out.part[top ? 1 : 2];
        if (kind == 0 && actor == (uint32_t)p) {
            uint32_t r0 = w.legal_row_of[i];
            uint64_t C = w.legal_off[r0 + ncp] - w.legal_off[r0];
            back += 32 * C + 8 * uint64_t(ncp);
            out.part[3] += 12 * C + 4 * uint64_t(ncp);  // every accumulation runs in the leaf-input launch
        } else if (kind == 0) {
            back += 4 * uint64_t(ncp) * (w.child_start[i + 1] - w.child_start[i]);
        } else if (kind == 1 && actor == (uint32_t)p) {
            uint32_t rb = w.draw_row_off[i];
            back += 12 * uint64_t(w.draw_row_start[rb + ncp] - w.draw_row_start[rb]);
        } else if (kind == 2) {
            back += 8 * uint64_t(ncp) + 4 * uint64_t(w.nc(i, 1 - p));
        }
        uint32_t par = w.parent[i];
        if (par != NONE && (w.node_meta[par] >> 2) == (uint32_t)p) {
            uint64_t G;
            if (w.rev_row_of[i] != NONE) {
                uint32_t r0 = w.rev_row_of[i];
                G = w.rev_start[r0 + ncp] - w.rev_start[r0];
            } else {
                uint32_t r0 = w.rvd_row_of[i];
                G = w.rvd_start[r0 + ncp] - w.rvd_start[r0];
            }
            reach += 4 * uint64_t(ncp) + 16 * G;
        }
    }
    return out;
}

uint64_t leaf_input_bytes(const WaveHost& w, int p, uint32_t elem) {
    // Per network row: its reach over player p's configs (4 each) and its
    // outputs (the pooled block into both query inputs, and the mass); per
    // distinct config list, its config indices once (4 each); per distinct
    // config, its embedding once.
    const uint32_t pool = w.net.pool;
    uint64_t bytes = 0;
    std::vector<uint8_t> seen(w.cfg_key.size(), 0);
    for (uint32_t r = 0; r < w.rows(); r++) {
        const uint32_t lo = w.row_cfg_off[2 * r + p], hi = w.row_cfg_off[2 * r + p + 1];
        bytes += 4 * uint64_t(hi - lo) + 2 * uint64_t(pool) * elem + 4;
        for (uint32_t k = lo; k < hi; k++)
            if (w.row_cfg[k] < seen.size() && !seen[w.row_cfg[k]]) {
                seen[w.row_cfg[k]] = 1;
                bytes += 4 * uint64_t(pool);
            }
    }
    for (const PoolGroup& g : w.pool_grp[p]) bytes += 4 * uint64_t(g.n);
    return bytes;
}

}  // namespace wc
