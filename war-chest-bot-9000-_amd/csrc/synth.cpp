// Seeded synthetic subgames. The tables are packed the way
// `PackedTables::from_solver` packs a real solver (engine/src/serialize.rs:689-956):
// nodes in depth-first build order (engine/src/search.rs:942-1253 builds
// recursively, so a parent always precedes its children), config-major legal
// cells with ascending actions, observation groups numbered by first
// appearance, reverse gathers in the CPU accumulation order, BFS levels.
#include "synth.h"

#include "v5.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <deque>
#include <exception>
#include <map>
#include <mutex>
#include <stdexcept>
#include <thread>

namespace wc {

double Rng::normal() {
    double u1 = 1.0 - unit();  // (0, 1]
    double u2 = unit();
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

namespace {

enum : uint8_t { DEC = 0, CHANCE = 1, LEAF = 2 };

struct GNode {
    uint8_t kind = DEC;
    uint8_t player = 0;
    uint32_t parent = NONE;
    std::vector<uint32_t> child;
    uint32_t na = 0;
    std::vector<uint32_t> obs_child;  // action -> public-child position
};

// U[0,1) features with 30% of the dims (in expectation) replaced by one-hot blocks of 8.
void feature_floats(Rng& r, float* out, uint32_t width) {
    uint32_t full = width / 8 * 8;
    for (uint32_t b = 0; b < full; b += 8) {
        if (r.unit() < 0.3) {
            uint32_t hot = r.below(8);
            for (uint32_t k = 0; k < 8; k++) out[b + k] = k == hot ? 1.0f : 0.0f;
        } else {
            for (uint32_t k = 0; k < 8; k++) out[b + k] = (float)r.unit();
        }
    }
    for (uint32_t k = full; k < width; k++) out[k] = (float)r.unit();
}

// The same recipe quantised to bytes (value = byte / 255).
void feature_bytes(Rng& r, uint8_t* out, uint32_t width) {
    auto q = [](double u) { return (uint8_t)std::min(255.0, std::floor(u * 256.0)); };
    uint32_t full = width / 8 * 8;
    for (uint32_t b = 0; b < full; b += 8) {
        if (r.unit() < 0.3) {
            uint32_t hot = r.below(8);
            for (uint32_t k = 0; k < 8; k++) out[b + k] = k == hot ? 255 : 0;
        } else {
            for (uint32_t k = 0; k < 8; k++) out[b + k] = q(r.unit());
        }
    }
    for (uint32_t k = full; k < width; k++) out[k] = q(r.unit());
}

// One synthetic public row of the v5 contract (rebel.rs:966-986): hex
// occupants, stack heights and location markers, pile counts, the players'
// marker, hand, face-down and bag sizes, initiative, the player to act and
// the plies remaining.
void v5_public_row(Rng& r, uint8_t* raw) {
    for (uint32_t h = 0; h < 37; h++) {
        const double u = r.unit();
        const uint8_t owner = u < 0.2 ? 0 : u < 0.4 ? 1 : 255;
        raw[h] = owner;
        raw[37 + h] = owner == 255 ? 255 : (uint8_t)r.below(5);
        raw[74 + h] = owner == 255 ? 0 : (uint8_t)(1 + r.below(5));
        const double m = r.unit();
        raw[111 + h] = m < 0.15 ? 0 : m < 0.3 ? 1 : 255;
    }
    for (uint32_t k = 0; k < 40; k++) raw[148 + k] = (uint8_t)r.below(6);
    for (uint32_t p = 0; p < 2; p++) {
        raw[188 + p] = (uint8_t)r.below(7);
        raw[190 + p] = (uint8_t)r.below(4);
        raw[192 + p] = (uint8_t)r.below(15);
        raw[194 + p] = (uint8_t)r.below(19);
    }
    raw[196] = (uint8_t)r.below(2);
    raw[197] = (uint8_t)r.below(2);
    raw[198] = (uint8_t)r.below(2);
    const uint32_t plies = r.below(257);
    raw[199] = (uint8_t)(plies & 0xff);
    raw[200] = (uint8_t)(plies >> 8);
}

uint32_t lognormal_count(Rng& r, float median, float p99, uint32_t cap) {
    double sigma = std::log((double)p99 / (double)median) / 2.3263478740408408;
    double x = std::exp(std::log((double)median) + sigma * r.normal());
    long n = std::lround(x);
    if (n < 1) n = 1;
    if ((uint32_t)n > cap) n = cap;
    return (uint32_t)n;
}

// Number the observation groups of an action list by first appearance in action order.
void renumber_groups(std::vector<uint32_t>& g) {
    std::map<uint32_t, uint32_t> id;
    for (auto& x : g) {
        auto it = id.find(x);
        if (it == id.end()) it = id.emplace(x, (uint32_t)id.size()).first;
        x = it->second;
    }
}

std::vector<GNode> grow(Rng& r, const SynthSpec& s, uint32_t budget) {
    std::vector<GNode> g(1);
    g[0].kind = DEC;
    g[0].player = 0;
    std::deque<uint32_t> q{0};
    uint32_t count = 1, expanded = 0;
    std::vector<uint32_t> seq;
    if (s.exact_decisions > 0) {
        uint32_t slots = s.exact_decisions + s.exact_leaves - 1;
        if (slots < s.exact_decisions || slots > s.exact_decisions * std::max(s.act_hi, 1u))
            throw std::runtime_error("exact tree shape is not realisable");
        seq.assign(s.exact_decisions, 1);
        uint32_t left = slots - s.exact_decisions;
        while (left > 0) {
            uint32_t k = r.below(s.exact_decisions);
            if (seq[k] < s.act_hi) {
                seq[k]++;
                left--;
            }
        }
        budget = s.exact_decisions + s.exact_leaves;
    }
    while (!q.empty()) {
        uint32_t i = q.front();
        q.pop_front();
        if (g[i].kind == DEC) {
            uint32_t na, nch;
            std::vector<uint32_t> grp;
            if (s.exact_decisions > 0) {
                if (expanded >= s.exact_decisions) {
                    g[i].kind = LEAF;
                    continue;
                }
                nch = seq[expanded];
                na = r.range(std::max(s.act_lo, nch), std::max(s.act_hi, nch));
                std::vector<uint32_t> perm(na);
                for (uint32_t a = 0; a < na; a++) perm[a] = a;
                for (uint32_t a = na; a > 1; a--) std::swap(perm[a - 1], perm[r.below(a)]);
                grp.assign(na, 0);
                for (uint32_t a = 0; a < na; a++) grp[perm[a]] = a < nch ? a : r.below(nch);
                renumber_groups(grp);
            } else {
                na = r.range(s.act_lo, s.act_hi);
                grp.assign(na, 0);
                nch = 1;
                for (uint32_t a = 1; a < na; a++) grp[a] = r.unit() < s.collapse ? r.below(nch) : nch++;
            }
            // With chance interleaving every public child is a draw by the player
            // who just acted, followed by the other player's node; the pair is
            // created together so the frontier only ever holds decision nodes.
            const uint32_t cost = s.chance ? 2 * nch : nch;
            if (count + cost > budget) {
                g[i].kind = LEAF;
                continue;
            }
            expanded++;
            g[i].na = na;
            g[i].obs_child = grp;
            for (uint32_t c = 0; c < nch; c++) {
                uint32_t parent = i;
                if (s.chance) {
                    GNode draw;
                    draw.kind = CHANCE;
                    draw.player = g[i].player;
                    draw.parent = i;
                    parent = (uint32_t)g.size();
                    g.push_back(draw);
                    g[i].child.push_back(parent);
                    count++;
                }
                GNode ch;
                ch.kind = DEC;
                ch.player = 1 - g[i].player;
                ch.parent = parent;
                uint32_t id = (uint32_t)g.size();
                g.push_back(ch);
                g[parent].child.push_back(id);
                q.push_back(id);
                count++;
            }
        }
    }
    // Depth-first preorder numbering, children in public-child order.
    std::vector<uint32_t> order;
    order.reserve(g.size());
    std::vector<uint32_t> stack{0};
    while (!stack.empty()) {
        uint32_t i = stack.back();
        stack.pop_back();
        order.push_back(i);
        for (size_t k = g[i].child.size(); k > 0; k--) stack.push_back(g[i].child[k - 1]);
    }
    std::vector<uint32_t> id(g.size());
    for (uint32_t k = 0; k < order.size(); k++) id[order[k]] = k;
    std::vector<GNode> out(g.size());
    for (uint32_t k = 0; k < order.size(); k++) {
        out[k] = g[order[k]];
        out[k].parent = out[k].parent == NONE ? NONE : id[out[k].parent];
        for (auto& c : out[k].child) c = id[c];
    }
    return out;
}

struct Built {
    std::vector<uint32_t> S[2];
};

Job build_job(Rng& r, const SynthSpec& s, const NetShape& ns, bool whale) {
    uint32_t budget = whale ? s.whale_nodes : r.range(s.nodes_lo, s.nodes_hi);
    uint32_t nroot[2];
    for (int p = 0; p < 2; p++) {
        if (whale)
            nroot[p] = s.whale_info;
        else if (s.info_fixed > 0)
            nroot[p] = s.info_fixed;
        else
            nroot[p] = lognormal_count(r, s.info_median, s.info_p99, s.info_cap);
    }
    std::vector<GNode> g = grow(r, s, budget);
    const uint32_t N = (uint32_t)g.size();

    // Supports, legal cells, transitions and draw rows, top-down.
    std::vector<Built> sup(N);
    for (int p = 0; p < 2; p++)
        for (uint32_t k = 0; k < nroot[p]; k++) sup[0].S[p].push_back(k);

    struct Cell {
        uint32_t row, action, child_pos, trans;
    };
    std::vector<std::vector<Cell>> cells(N);
    struct DrawRow {
        std::vector<uint32_t> to;
        std::vector<float> p;
    };
    std::vector<std::vector<DrawRow>> draws(N);
    std::vector<float> util(N, 0.0f);
    std::vector<uint8_t> terminal(N, 0);

    for (uint32_t i = 0; i < N; i++) {
        GNode& n = g[i];
        const int me = n.player;
        const std::vector<uint32_t>& mine = sup[i].S[me];
        const uint32_t nc = (uint32_t)mine.size();
        if (n.kind == DEC) {
            const uint32_t na = n.na, nch = (uint32_t)n.child.size();
            std::vector<uint8_t> legal(size_t(nc) * na, 0);
            for (uint32_t c = 0; c < nc; c++) {
                bool any = false;
                for (uint32_t a = 0; a < na; a++)
                    if (r.unit() < s.legal_p) legal[c * na + a] = 1, any = true;
                if (!any) legal[c * na + r.below(na)] = 1;
            }
            if (nc > 0)
                for (uint32_t a = 0; a < na; a++) {
                    bool any = false;
                    for (uint32_t c = 0; c < nc && !any; c++) any = legal[c * na + a];
                    if (!any) legal[r.below(nc) * na + a] = 1;
                }
            std::vector<uint32_t> key;
            for (uint32_t c = 0; c < nc; c++)
                for (uint32_t a = 0; a < na; a++) {
                    if (!legal[c * na + a]) continue;
                    uint32_t k = NONE;
                    if (r.unit() >= s.notrans_p) {
                        k = mine[c];
                        if (r.unit() < s.shift_p) k = (k + 1) % nroot[me];
                    }
                    cells[i].push_back({c, a, n.obs_child[a], NONE});
                    key.push_back(k);
                }
            // Each public child's support is the sorted set of successor keys that
            // reach it; the idle player's support passes through unchanged.
            for (uint32_t ch = 0; ch < nch; ch++) {
                std::vector<uint32_t> ks;
                for (size_t x = 0; x < cells[i].size(); x++)
                    if (cells[i][x].child_pos == ch && key[x] != NONE) ks.push_back(key[x]);
                std::sort(ks.begin(), ks.end());
                ks.erase(std::unique(ks.begin(), ks.end()), ks.end());
                for (size_t x = 0; x < cells[i].size(); x++)
                    if (cells[i][x].child_pos == ch && key[x] != NONE)
                        cells[i][x].trans =
                            (uint32_t)(std::lower_bound(ks.begin(), ks.end(), key[x]) - ks.begin());
                uint32_t c = n.child[ch];
                sup[c].S[me] = ks;
                sup[c].S[1 - me] = sup[i].S[1 - me];
            }
        } else if (n.kind == CHANCE) {
            uint32_t c = n.child[0];
            uint32_t reach_keys = std::min(nroot[me], 2 * s.draw_hi + 1);
            std::vector<std::vector<uint32_t>> outs(nc);
            std::vector<uint32_t> all;
            for (uint32_t ci = 0; ci < nc; ci++) {
                uint32_t k = mine[ci];
                uint32_t nout = std::min(r.range(s.draw_lo, s.draw_hi), reach_keys);
                std::vector<uint32_t> o{k};
                while (o.size() < nout) {
                    uint32_t x = (k + r.range(1, 2 * s.draw_hi)) % nroot[me];
                    if (std::find(o.begin(), o.end(), x) == o.end()) o.push_back(x);
                }
                outs[ci] = o;
                all.insert(all.end(), o.begin(), o.end());
            }
            std::sort(all.begin(), all.end());
            all.erase(std::unique(all.begin(), all.end()), all.end());
            draws[i].resize(nc);
            for (uint32_t ci = 0; ci < nc; ci++) {
                std::vector<uint32_t> to;
                for (uint32_t x : outs[ci])
                    to.push_back((uint32_t)(std::lower_bound(all.begin(), all.end(), x) - all.begin()));
                std::sort(to.begin(), to.end());
                float pr = 1.0f / (float)to.size();
                draws[i][ci].to = to;
                draws[i][ci].p.assign(to.size(), pr);
            }
            sup[c].S[me] = all;
            sup[c].S[1 - me] = sup[i].S[1 - me];
        } else {
            if (s.terminal_p > 0.0f && r.unit() < s.terminal_p) {
                terminal[i] = 1;
                util[i] = (float)(2.0 * r.unit() - 1.0);
            }
        }
    }

    // Per-tree infostate features: the pooled-belief embedding (and, for the
    // two-tower net, the private-tower input) of every config key.
    std::vector<float> emb[2], priv[2];
    const bool v5 = ns.kind == MODEL_V5;
    for (int p = 0; p < 2 && v5; p++) {
        // v5: a config's hand, face-down and bag counts per coin slot, over the
        // count normaliser (search.rs:1433-1458, CNORM = 5)
        emb[p].resize(size_t(nroot[p]) * V5_CFEAT);
        for (uint32_t k = 0; k < nroot[p]; k++) {
            float* c = &emb[p][size_t(k) * V5_CFEAT];
            uint32_t hand = r.below(4), fd = r.below(5);
            for (uint32_t q = 0; q < V5_CFEAT; q++) c[q] = 0.0f;
            for (uint32_t x = 0; x < hand; x++) c[r.below(5)] += 1.0f;
            for (uint32_t x = 0; x < fd; x++) c[5 + r.below(5)] += 1.0f;
            for (uint32_t q = 0; q < 5; q++) c[10 + q] = (float)r.below(4);
            for (uint32_t q = 0; q < V5_CFEAT; q++) c[q] /= 5.0f;
        }
    }
    for (int p = 0; p < 2 && !v5; p++) {
        emb[p].resize(size_t(nroot[p]) * ns.pool);
        for (uint32_t k = 0; k < nroot[p]; k++) feature_floats(r, &emb[p][size_t(k) * ns.pool], ns.pool);
        if (ns.priv_in) {
            priv[p].resize(size_t(nroot[p]) * ns.priv_in);
            for (uint32_t k = 0; k < nroot[p]; k++)
                feature_floats(r, &priv[p][size_t(k) * ns.priv_in], ns.priv_in);
        }
    }

    Job job;
    Meta& m = job.meta;
    m.depth = s.depth;
    m.iters = s.iters;
    m.snapshots = s.snapshots != 0;
    m.cfr = s.cfr;
    m.snap_iters = snapshot_iters(s.iters);
    m.net_dims = s.net_dims;

    Tables& t = job.t;
    t.nodes = N;
    t.cfg_off.push_back(0);
    for (uint32_t i = 0; i < N; i++) {
        t.cfg_off.push_back(t.cfg_off.back() + (uint32_t)sup[i].S[0].size());
        t.cfg_off.push_back(t.cfg_off.back() + (uint32_t)sup[i].S[1].size());
    }
    t.node_parent.assign(N, NONE);
    t.rev_row_of.assign(N, NONE);
    t.rvd_row_of.assign(N, NONE);
    t.legal_row_of.assign(N, NONE);
    t.legal_off.push_back(0);
    t.rev_start.push_back(0);
    t.rvd_start.push_back(0);
    uint32_t reach_at = 0, cell_at = 0;
    for (uint32_t i = 0; i < N; i++) {
        const GNode& n = g[i];
        const int me = n.player;
        t.node_child_start.push_back((uint32_t)t.node_child.size());
        for (uint32_t c : n.child) {
            t.node_child.push_back(c);
            t.node_parent[c] = i;
        }
        t.node_kind.push_back(n.kind);
        t.node_player.push_back(n.player);
        t.obs_off.push_back((uint32_t)t.obs_start.size());
        t.draw_off.push_back((uint32_t)t.draw_to.size());
        t.draw_row_off.push_back((uint32_t)t.draw_row_start.size());
        t.reach_off.push_back(reach_at);
        reach_at += t.nc(i, 0) + t.nc(i, 1);
        t.soff.push_back(cell_at);
        if (n.kind == DEC) {
            const uint32_t na = n.na, nch = (uint32_t)n.child.size();
            // Observation CSR: actions of each public child in ascending order.
            std::vector<uint32_t> ostart(nch + 1, 0), oact(na);
            for (uint32_t a = 0; a < na; a++) ostart[n.obs_child[a] + 1]++;
            for (uint32_t c = 0; c < nch; c++) ostart[c + 1] += ostart[c];
            std::vector<uint32_t> fill(ostart.begin(), ostart.end() - 1);
            for (uint32_t a = 0; a < na; a++) oact[fill[n.obs_child[a]]++] = a;
            t.obs_start.insert(t.obs_start.end(), ostart.begin(), ostart.end());
            t.obs_act.insert(t.obs_act.end(), oact.begin(), oact.end());
            t.obs_child.insert(t.obs_child.end(), n.obs_child.begin(), n.obs_child.end());
            // Config-major legal rows.
            const uint32_t nc = t.nc(i, me);
            t.legal_row_of[i] = (uint32_t)t.legal_off.size() - 1;
            const std::vector<Cell>& cs = cells[i];
            size_t x = 0;
            for (uint32_t c = 0; c < nc; c++) {
                while (x < cs.size() && cs[x].row == c) {
                    t.legal_action.push_back(cs[x].action);
                    t.legal_child.push_back(n.child[cs[x].child_pos]);
                    t.legal_trans.push_back(cs[x].trans);
                    t.cell_row.push_back(c);
                    x++;
                }
                t.legal_off.push_back(cell_at + (uint32_t)x);
            }
            // Reverse gathers per public child, in the CPU's accumulation order:
            // actions in observation order, then legal cells of that action in
            // ascending cell (= config) order (serialize.rs:805-836).
            std::vector<std::vector<uint32_t>> action_cells(na);
            for (uint32_t k = 0; k < cs.size(); k++) action_cells[cs[k].action].push_back(k);
            for (uint32_t ch = 0; ch < nch; ch++) {
                uint32_t child = n.child[ch];
                uint32_t m_ch = t.nc(child, me);
                std::vector<std::vector<std::pair<uint32_t, uint32_t>>> gather(m_ch);
                for (uint32_t k = ostart[ch]; k < ostart[ch + 1]; k++) {
                    uint32_t a = oact[k];
                    for (uint32_t cell : action_cells[a]) {
                        if (cs[cell].trans == NONE) continue;
                        gather[cs[cell].trans].push_back({cs[cell].row, cell_at + cell});
                    }
                }
                t.rev_row_of[child] = (uint32_t)t.rev_start.size() - 1;
                for (auto& v : gather) {
                    for (auto& e : v) {
                        t.rev_src.push_back(e.first);
                        t.rev_cell.push_back(e.second);
                    }
                    t.rev_start.push_back((uint32_t)t.rev_src.size());
                }
            }
            cell_at += (uint32_t)cs.size();
        } else if (n.kind == CHANCE) {
            const uint32_t nc = t.nc(i, me);
            uint32_t local = 0;
            for (uint32_t c = 0; c < nc; c++) {
                t.draw_row_start.push_back(local);
                for (size_t k = 0; k < draws[i][c].to.size(); k++) {
                    t.draw_to.push_back(draws[i][c].to[k]);
                    t.draw_p.push_back(draws[i][c].p[k]);
                }
                local += (uint32_t)draws[i][c].to.size();
            }
            t.draw_row_start.push_back(local);
            uint32_t child = n.child[0];
            uint32_t m_ch = t.nc(child, me);
            std::vector<std::vector<std::pair<uint32_t, float>>> gather(m_ch);
            for (uint32_t c = 0; c < nc; c++)
                for (size_t k = 0; k < draws[i][c].to.size(); k++)
                    gather[draws[i][c].to[k]].push_back({c, draws[i][c].p[k]});
            t.rvd_row_of[child] = (uint32_t)t.rvd_start.size() - 1;
            for (auto& v : gather) {
                for (auto& e : v) {
                    t.rvd_src.push_back(e.first);
                    t.rvd_p.push_back(e.second);
                }
                t.rvd_start.push_back((uint32_t)t.rvd_src.size());
            }
        }
    }
    t.node_child_start.push_back((uint32_t)t.node_child.size());
    t.obs_off.push_back((uint32_t)t.obs_start.size());
    t.draw_off.push_back((uint32_t)t.draw_to.size());
    t.draw_row_off.push_back((uint32_t)t.draw_row_start.size());
    t.reach_off.push_back(reach_at);
    t.soff.push_back(cell_at);
    t.ncells = cell_at;

    // Leaves: network rows first in node order, then terminals in node order.
    std::map<uint64_t, uint32_t> intern;
    for (uint32_t i = 0; i < N; i++) {
        if (g[i].kind != LEAF) continue;
        if (terminal[i]) {
            t.term_leaves.push_back(i);
            t.terminal_utility.push_back(util[i]);
            continue;
        }
        t.leaf_rows.push_back(i);
        for (int p = 0; p < 2; p++) {
            t.leaf_coff.push_back((uint32_t)t.leaf_cidx.size());
            for (uint32_t key : sup[i].S[p]) {
                uint64_t k = (uint64_t(p) << 32) | key;
                auto it = intern.find(k);
                if (it == intern.end()) {
                    uint32_t idx = (uint32_t)t.cplayer.size();
                    it = intern.emplace(k, idx).first;
                    t.cplayer.push_back((uint8_t)p);
                    if (v5) {
                        const float* e = &emb[p][size_t(key) * V5_CFEAT];
                        t.cphi.insert(t.cphi.end(), e, e + V5_CFEAT);
                    } else {
                        t.cphi.push_back((float)key);
                        const float* e = &emb[p][size_t(key) * ns.pool];
                        t.cphi.insert(t.cphi.end(), e, e + ns.pool);
                        if (ns.priv_in) {
                            const float* q = &priv[p][size_t(key) * ns.priv_in];
                            t.cphi.insert(t.cphi.end(), q, q + ns.priv_in);
                        }
                    }
                }
                t.leaf_cidx.push_back(it->second);
            }
        }
    }
    t.leaf_coff.push_back((uint32_t)t.leaf_cidx.size());
    t.rows = (uint32_t)t.leaf_rows.size();
    t.ncfg = (uint32_t)t.cplayer.size();
    t.leaf_raw.resize(size_t(t.rows) * ns.row_bytes);
    for (uint32_t row = 0; row < t.rows; row++) {
        uint8_t* raw = &t.leaf_raw[size_t(row) * ns.row_bytes];
        if (v5)
            v5_public_row(r, raw);
        else
            feature_bytes(r, raw, ns.row_bytes);
    }
    if (v5) {  // the printed facts of the ten coin types in play (units.rs:71-110 widths)
        t.card_feat.resize(V5_CARD_FEAT);
        for (uint32_t ty = 0; ty < 10; ty++) {
            float* f = &t.card_feat[size_t(ty) * 25];
            for (uint32_t q = 0; q < 10; q++) f[q] = r.unit() < 0.3 ? 1.0f : 0.0f;
            for (uint32_t q = 10; q < 22; q++) f[q] = (float)r.below(6) / 5.0f;
            for (uint32_t q = 22; q < 24; q++) f[q] = r.unit() < 0.5 ? 1.0f : 0.0f;
            f[24] = (float)r.unit();
        }
    }
    uint32_t snap_at = 0;
    auto exits = t.leaf_rows;
    exits.insert(exits.end(), t.term_leaves.begin(), t.term_leaves.end());
    for (uint32_t i : exits)
        for (int p = 0; p < 2; p++) {
            t.snap_coff.push_back(snap_at);
            snap_at += t.nc(i, p);
        }
    t.snap_coff.push_back(snap_at);

    // BFS levels (serialize.rs:898-917).
    t.level_start.push_back(0);
    std::vector<uint32_t> frontier{0};
    while (!frontier.empty()) {
        std::vector<uint32_t> next;
        for (uint32_t i : frontier) {
            t.bfs_order.push_back(i);
            for (uint32_t c : g[i].child) next.push_back(c);
        }
        frontier.swap(next);
        t.level_start.push_back((uint32_t)t.bfs_order.size());
    }

    // Root beliefs and carried roots.
    for (int p = 0; p < 2; p++) {
        uint32_t n = nroot[p];
        std::vector<float> b(n);
        if (s.dirichlet) {
            std::vector<double> x(n);
            double sum = 0.0;
            for (uint32_t k = 0; k < n; k++) {
                x[k] = -std::log(1.0 - r.unit());
                sum += x[k];
            }
            for (uint32_t k = 0; k < n; k++) b[k] = (float)(x[k] / sum);
        } else {
            for (uint32_t k = 0; k < n; k++) b[k] = 1.0f / (float)n;
        }
        job.root[p] = b;
    }
    for (uint32_t k = 0; k < std::max(s.nroots, 1u); k++)
        for (int p = 0; p < 2; p++) {
            if (k == 0) {
                job.carried[p].push_back(job.root[p]);
                continue;
            }
            // A skewed copy of the root belief (the pattern of engine/src/gpu/tests.rs:56-70).
            std::vector<float> x(job.root[p]);
            float sum = 0.0f;
            for (size_t c = 0; c < x.size(); c++) {
                if (c % (k + 1) == 0) x[c] += 0.5f;
                sum += x[c];
            }
            for (auto& v : x) v /= sum;
            job.carried[p].push_back(x);
        }
    return job;
}

}  // namespace

std::vector<Job> synth_jobs(const SynthSpec& spec) {
    NetShape ns;
    std::string err;
    if (!ns.parse(spec.net_dims, &err)) throw std::runtime_error(err);
    // Tree k's stream is the k-th draw of the master stream, so the trees are
    // independent and built on several host threads.
    Rng master(spec.seed);
    std::vector<uint64_t> seeds(spec.trees);
    for (uint32_t k = 0; k < spec.trees; k++) seeds[k] = master.next();
    std::vector<Job> jobs(spec.trees);
    std::atomic<uint32_t> next{0};
    std::exception_ptr failure;
    std::mutex failure_mu;
    auto work = [&]() {
        for (uint32_t k; (k = next.fetch_add(1)) < spec.trees;) {
            try {
                Rng r(seeds[k]);
                bool whale = spec.whale_frac > 0.0f && r.unit() < spec.whale_frac;
                jobs[k] = build_job(r, spec, ns, whale);
            } catch (...) {
                std::lock_guard<std::mutex> g(failure_mu);
                if (!failure) failure = std::current_exception();
            }
        }
    };
    const uint32_t threads = std::max(1u, std::min({std::thread::hardware_concurrency(), 16u, spec.trees}));
    std::vector<std::thread> pool;
    for (uint32_t t = 1; t < threads; t++) pool.emplace_back(work);
    work();
    for (auto& t : pool) t.join();
    if (failure) std::rethrow_exception(failure);
    return jobs;
}

void synth_weights(const std::vector<uint32_t>& dims, uint64_t seed, std::vector<float>* w,
                   std::vector<float>* b) {
    NetShape ns;
    std::string err;
    if (!ns.parse(dims, &err)) throw std::runtime_error(err);
    Rng r(seed);
    w->clear();
    b->clear();
    auto mat = [&](uint32_t rows, uint32_t cols, uint32_t fan_in) {
        double sd = std::sqrt(2.0 / (double)fan_in);
        for (size_t k = 0; k < size_t(rows) * cols; k++) w->push_back((float)(sd * r.normal()));
    };
    auto bias = [&](uint32_t n) {
        for (uint32_t k = 0; k < n; k++) b->push_back((float)(0.2 * r.unit() - 0.1));
    };
    if (ns.kind == MODEL_MLP) {
        mat(ns.in, ns.hidden, ns.in);
        for (uint32_t l = 1; l < ns.layers; l++) mat(ns.hidden, ns.hidden, ns.hidden);
        mat(ns.heads, ns.hidden, ns.hidden);
        for (uint32_t l = 0; l < ns.layers; l++) bias(ns.hidden);
        bias(ns.heads);
    } else if (ns.kind == MODEL_TWO_TOWER) {
        mat(ns.in, ns.hidden, ns.in);
        for (uint32_t l = 1; l < ns.layers; l++) mat(ns.hidden, ns.hidden, ns.hidden);
        mat(ns.priv_in, ns.hidden, ns.priv_in);
        for (uint32_t l = 1; l < ns.priv_layers; l++) mat(ns.hidden, ns.hidden, ns.hidden);
        mat(1, ns.hidden, ns.hidden);
        for (uint32_t l = 0; l < ns.layers; l++) bias(ns.hidden);
        for (uint32_t l = 0; l < ns.priv_layers; l++) bias(ns.hidden);
        bias(1);
    } else {
        // v5 (net.rs:272-316): every matrix Kaiming-normal over its fan-in,
        // the seat and position embeddings N(0, 0.25), biases U[-0.1, 0.1].
        const v5::Layout L = v5::layout();
        w->assign(L.w_len, 0.0f);
        b->assign(L.b_len, 0.0f);
        auto fill = [&](const v5::Span& sp) {
            const double sd = std::sqrt(2.0 / (double)sp.i);
            for (size_t k = 0; k < size_t(sp.i) * sp.o; k++) (*w)[sp.w + k] = (float)(sd * r.normal());
            if (sp.bias)
                for (uint32_t k = 0; k < sp.o; k++) (*b)[sp.b + k] = (float)(0.2 * r.unit() - 0.1);
        };
        auto embed = [&](uint32_t at, uint32_t n) {
            for (uint32_t k = 0; k < n; k++) (*w)[at + k] = (float)(0.5 * r.normal());
        };
        fill(L.card[0]);
        fill(L.card[1]);
        fill(L.pile);
        embed(L.seat, 2 * v5::TYPE);
        fill(L.hex_stem);
        fill(L.tok_stem);
        embed(L.pos, v5::HEXES * v5::C);
        fill(L.glob_stem);
        for (uint32_t i = 0; i < v5::BLOCKS; i++) {
            fill(L.mix[i]);
            fill(L.pool[i]);
            fill(L.out[i]);
        }
        for (const v5::Span* sp : {&L.board_out, &L.cfg1, &L.cfg_f, &L.cfg_g, &L.cfg_m, &L.join_p, &L.join_b})
            fill(*sp);
        for (uint32_t i = 0; i < v5::JBLOCKS; i++) fill(L.join_w[i]);
        fill(L.join_out);
        (*b)[L.value_bias] = (float)(0.2 * r.unit() - 0.1);
    }
}

void synth_norms(const std::vector<uint32_t>& dims, uint64_t seed, std::vector<float>* ln) {
    NetShape ns;
    std::string err;
    if (!ns.parse(dims, &err)) throw std::runtime_error(err);
    ln->clear();
    if (ns.kind != MODEL_V5) return;
    const v5::Layout L = v5::layout();
    Rng r(seed ^ 0x4c4e4c4e4c4e4c4eull);
    ln->assign(L.ln_len, 0.0f);
    for (uint32_t i = 0; i < v5::NORMS; i++)
        for (uint32_t k = 0; k < L.norm_width[i]; k++) {
            (*ln)[L.norm_g[i] + k] = (float)(1.0 + 0.1 * r.normal());
            (*ln)[L.norm_b[i] + k] = (float)(0.1 * r.normal());
        }
}

void synth_features(uint32_t rows, uint32_t width, uint64_t seed, std::vector<float>* x) {
    Rng r(seed);
    x->assign(size_t(rows) * width, 0.0f);
    for (uint32_t i = 0; i < rows; i++) feature_floats(r, &(*x)[size_t(i) * width], width);
}

}  // namespace wc
