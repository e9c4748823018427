// WCJ8 codec and structural validation for the job contract.
// Byte order: engine/src/serialize.rs:1052-1129 (writer), 1131-1261 (reader).
#include "job.h"

#include <cstring>

namespace wc {

bool NetShape::parse(const std::vector<uint32_t>& dims, std::string* err) {
    *this = NetShape{};
    if (dims.empty()) {
        if (err) *err = "net_dims is empty";
        return false;
    }
    kind = dims[0];
    if (kind == MODEL_V5) {
        // engine/src/net.rs:41 MODEL_TAG = [5]; v5 payload widths.
        if (dims.size() != 1) {
            if (err) *err = "v5 net_dims must be exactly [5]";
            return false;
        }
        // The join reads both pooled beliefs and the seat; the trunk reads the
        // row's public bytes (rebel.rs:966-986); the readout is 256 wide.
        in = 2 * 64 + 1;
        hidden = 256;
        pool = 64;
        row_bytes = V5_ROW_BYTES;
        cfeat = V5_CFEAT;
        card_feat = V5_CARD_FEAT;
        return true;
    }
    if (kind == MODEL_MLP) {
        if (dims.size() != 6) {
            if (err) *err = "MLP net_dims must be [101, in, hidden, layers, heads, pool]";
            return false;
        }
        in = dims[1];
        hidden = dims[2];
        layers = dims[3];
        heads = dims[4];
        pool = dims[5];
        if (in < 2 * pool + 1 || hidden == 0 || layers == 0 || heads == 0 || pool == 0) {
            if (err) *err = "MLP net_dims out of range";
            return false;
        }
        row_bytes = in - 2 * pool - 1;
        cfeat = 1 + pool;
        card_feat = 0;
        return true;
    }
    if (kind == MODEL_TWO_TOWER) {
        if (dims.size() != 7) {
            if (err) *err = "two-tower net_dims must be [102, in, width, pub_layers, priv_in, priv_layers, pool]";
            return false;
        }
        in = dims[1];
        hidden = dims[2];
        layers = dims[3];
        priv_in = dims[4];
        priv_layers = dims[5];
        pool = dims[6];
        if (in < 2 * pool + 1 || hidden == 0 || layers == 0 || priv_in == 0 || priv_layers == 0) {
            if (err) *err = "two-tower net_dims out of range";
            return false;
        }
        row_bytes = in - 2 * pool - 1;
        cfeat = 1 + pool + priv_in;
        card_feat = 0;
        return true;
    }
    if (err) *err = "unknown network tag " + std::to_string(kind);
    return false;
}

std::vector<uint32_t> snapshot_iters(uint32_t iters) {
    std::vector<uint32_t> out;
    for (uint32_t t = 0; t <= iters; t++)
        if (t == 0 || (t & (t - 1)) == 0 || t == iters) out.push_back(t);
    return out;
}

namespace {

struct W {
    std::vector<uint8_t> b;
    void u32(uint32_t v) {
        uint8_t x[4] = {uint8_t(v), uint8_t(v >> 8), uint8_t(v >> 16), uint8_t(v >> 24)};
        b.insert(b.end(), x, x + 4);
    }
    void f32(float v) {
        uint32_t u;
        std::memcpy(&u, &v, 4);
        u32(u);
    }
    void u8s(const std::vector<uint8_t>& v) {
        u32((uint32_t)v.size());
        b.insert(b.end(), v.begin(), v.end());
    }
    // Arrays of 32-bit words, little-endian: one block copy on a little-endian
    // host, word by word elsewhere.
    template <class T>
    void words(const std::vector<T>& v) {
        static_assert(sizeof(T) == 4, "32-bit words");
        u32((uint32_t)v.size());
#if defined(__BYTE_ORDER__) && __BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__
        const uint8_t* p = (const uint8_t*)v.data();
        b.insert(b.end(), p, p + v.size() * 4);
#else
        for (const T& x : v) {
            uint32_t u;
            std::memcpy(&u, &x, 4);
            u32(u);
        }
#endif
    }
    void u32s(const std::vector<uint32_t>& v) { words(v); }
    void f32s(const std::vector<float>& v) { words(v); }
};

struct R {
    const uint8_t* b;
    size_t n, at = 0;
    std::string* err;
    bool ok = true;
    bool take(size_t k, const char* what) {
        if (!ok) return false;
        if (k > n - at) {
            if (err) *err = std::string("job truncated reading ") + what;
            ok = false;
            return false;
        }
        return true;
    }
    uint32_t u32(const char* what) {
        if (!take(4, what)) return 0;
        uint32_t v = uint32_t(b[at]) | uint32_t(b[at + 1]) << 8 | uint32_t(b[at + 2]) << 16 |
                     uint32_t(b[at + 3]) << 24;
        at += 4;
        return v;
    }
    float f32(const char* what) {
        uint32_t u = u32(what);
        float f;
        std::memcpy(&f, &u, 4);
        return f;
    }
    uint8_t u8(const char* what) {
        if (!take(1, what)) return 0;
        return b[at++];
    }
    void u8s(std::vector<uint8_t>& v, const char* what) {
        uint32_t k = u32(what);
        if (!take(k, what)) return;
        v.assign(b + at, b + at + k);
        at += k;
    }
    // Arrays of little-endian 32-bit words: one block copy on a little-endian
    // host, word by word elsewhere.
    template <class T>
    void words(std::vector<T>& v, const char* what) {
        static_assert(sizeof(T) == 4, "32-bit words");
        uint32_t k = u32(what);
        if (!take(size_t(k) * 4, what)) return;
        v.resize(k);
#if defined(__BYTE_ORDER__) && __BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__
        if (k) std::memcpy(v.data(), b + at, size_t(k) * 4);
        at += size_t(k) * 4;
#else
        for (uint32_t i = 0; i < k; i++) {
            uint32_t u = u32(what);
            std::memcpy(&v[i], &u, 4);
        }
#endif
    }
    void u32s(std::vector<uint32_t>& v, const char* what) { words(v, what); }
    void f32s(std::vector<float>& v, const char* what) { words(v, what); }
};

bool check(size_t got, size_t want, const char* what, std::string* err) {
    if (got != want) {
        if (err)
            *err = std::string("job ") + what + ": count " + std::to_string(got) + " != expected " +
                   std::to_string(want);
        return false;
    }
    return true;
}

}  // namespace

std::vector<uint8_t> to_bytes(const Job& job) {
    W w;
    w.u32(JOB_MAGIC);
    w.u32(JOB_VERSION);
    const Meta& m = job.meta;
    w.u32(m.depth);
    w.u32(m.iters);
    w.b.push_back(m.snapshots ? 1 : 0);
    w.f32(m.cfr.alpha);
    w.f32(m.cfr.beta);
    w.f32(m.cfr.gamma);
    w.f32(m.cfr.predict);
    w.u32s(m.snap_iters);
    w.u32s(m.net_dims);
    const Tables& t = job.t;
    w.u32(t.nodes);
    w.u32(t.ncfg);
    w.u32(t.rows);
    w.u32(t.ncells);
    w.u8s(t.node_kind);
    w.u8s(t.node_player);
    w.u32s(t.node_child_start);
    w.u32s(t.node_child);
    w.u32s(t.obs_off);
    w.u32s(t.obs_start);
    w.u32s(t.obs_act);
    w.u32s(t.obs_child);
    w.u32s(t.legal_row_of);
    w.u32s(t.legal_off);
    w.u32s(t.legal_action);
    w.u32s(t.legal_child);
    w.u32s(t.legal_trans);
    w.u32s(t.cell_row);
    w.u32s(t.draw_off);
    w.u32s(t.draw_to);
    w.f32s(t.draw_p);
    w.u32s(t.draw_row_off);
    w.u32s(t.draw_row_start);
    w.u32s(t.cfg_off);
    w.u32s(t.reach_off);
    w.u32s(t.soff);
    w.u32s(t.node_parent);
    w.u32s(t.rev_row_of);
    w.u32s(t.rev_start);
    w.u32s(t.rev_src);
    w.u32s(t.rev_cell);
    w.u32s(t.rvd_row_of);
    w.u32s(t.rvd_start);
    w.u32s(t.rvd_src);
    w.f32s(t.rvd_p);
    w.u32s(t.leaf_rows);
    w.u32s(t.term_leaves);
    w.f32s(t.terminal_utility);
    w.u32s(t.leaf_coff);
    w.u32s(t.leaf_cidx);
    w.u32s(t.snap_coff);
    w.u8s(t.leaf_raw);
    w.f32s(t.card_feat);
    w.f32s(t.cphi);
    w.u8s(t.cplayer);
    w.u32s(t.bfs_order);
    w.u32s(t.level_start);
    w.f32s(job.root[0]);
    w.f32s(job.root[1]);
    w.u32(job.nroots());
    for (uint32_t r = 0; r < job.nroots(); r++) {
        w.f32s(job.carried[0][r]);
        w.f32s(job.carried[1][r]);
    }
    return w.b;
}

bool from_bytes(const uint8_t* b, size_t n, Job* out, std::string* err) {
    R r{b, n, 0, err};
    Job job;
    if (r.u32("magic") != JOB_MAGIC) {
        if (r.ok && err) *err = "job: bad magic";
        return false;
    }
    if (r.u32("version") != JOB_VERSION) {
        if (r.ok && err) *err = "job: unsupported version";
        return false;
    }
    Meta& m = job.meta;
    m.depth = r.u32("depth");
    m.iters = r.u32("iters");
    m.snapshots = r.u8("snapshots") != 0;
    m.cfr.alpha = r.f32("alpha");
    m.cfr.beta = r.f32("beta");
    m.cfr.gamma = r.f32("gamma");
    m.cfr.predict = r.f32("predict");
    r.u32s(m.snap_iters, "snap_iters");
    r.u32s(m.net_dims, "net_dims");
    Tables& t = job.t;
    t.nodes = r.u32("nodes");
    t.ncfg = r.u32("ncfg");
    t.rows = r.u32("rows");
    t.ncells = r.u32("ncells");
    r.u8s(t.node_kind, "node_kind");
    r.u8s(t.node_player, "node_player");
    r.u32s(t.node_child_start, "node_child_start");
    r.u32s(t.node_child, "node_child");
    r.u32s(t.obs_off, "obs_off");
    r.u32s(t.obs_start, "obs_start");
    r.u32s(t.obs_act, "obs_act");
    r.u32s(t.obs_child, "obs_child");
    r.u32s(t.legal_row_of, "legal_row_of");
    r.u32s(t.legal_off, "legal_off");
    r.u32s(t.legal_action, "legal_action");
    r.u32s(t.legal_child, "legal_child");
    r.u32s(t.legal_trans, "legal_trans");
    r.u32s(t.cell_row, "cell_row");
    r.u32s(t.draw_off, "draw_off");
    r.u32s(t.draw_to, "draw_to");
    r.f32s(t.draw_p, "draw_p");
    r.u32s(t.draw_row_off, "draw_row_off");
    r.u32s(t.draw_row_start, "draw_row_start");
    r.u32s(t.cfg_off, "cfg_off");
    r.u32s(t.reach_off, "reach_off");
    r.u32s(t.soff, "soff");
    r.u32s(t.node_parent, "node_parent");
    r.u32s(t.rev_row_of, "rev_row_of");
    r.u32s(t.rev_start, "rev_start");
    r.u32s(t.rev_src, "rev_src");
    r.u32s(t.rev_cell, "rev_cell");
    r.u32s(t.rvd_row_of, "rvd_row_of");
    r.u32s(t.rvd_start, "rvd_start");
    r.u32s(t.rvd_src, "rvd_src");
    r.f32s(t.rvd_p, "rvd_p");
    r.u32s(t.leaf_rows, "leaf_rows");
    r.u32s(t.term_leaves, "term_leaves");
    r.f32s(t.terminal_utility, "terminal_utility");
    r.u32s(t.leaf_coff, "leaf_coff");
    r.u32s(t.leaf_cidx, "leaf_cidx");
    r.u32s(t.snap_coff, "snap_coff");
    r.u8s(t.leaf_raw, "leaf_raw");
    r.f32s(t.card_feat, "card_feat");
    r.f32s(t.cphi, "cphi");
    r.u8s(t.cplayer, "cplayer");
    r.u32s(t.bfs_order, "bfs_order");
    r.u32s(t.level_start, "level_start");
    if (!r.ok) return false;

    NetShape ns;
    if (!ns.parse(m.net_dims, err)) return false;
    const size_t nodes = t.nodes;
    if (!check(t.node_kind.size(), nodes, "node_kind", err) ||
        !check(t.node_player.size(), nodes, "node_player", err) ||
        !check(t.legal_row_of.size(), nodes, "legal_row_of", err) ||
        !check(t.node_child_start.size(), nodes + 1, "node_child_start", err) ||
        !check(t.obs_off.size(), nodes + 1, "obs_off", err) ||
        !check(t.draw_off.size(), nodes + 1, "draw_off", err) ||
        !check(t.draw_row_off.size(), nodes + 1, "draw_row_off", err) ||
        !check(t.reach_off.size(), nodes + 1, "reach_off", err) ||
        !check(t.soff.size(), nodes + 1, "soff", err) ||
        !check(t.cfg_off.size(), 2 * nodes + 1, "cfg_off", err) ||
        !check(t.cphi.size(), size_t(t.ncfg) * ns.cfeat, "cphi", err) ||
        !check(t.cplayer.size(), t.ncfg, "cplayer", err) ||
        !check(t.leaf_raw.size(), size_t(t.rows) * ns.row_bytes, "leaf_raw", err) ||
        !check(t.card_feat.size(), ns.card_feat, "card_feat", err) ||
        !check(t.leaf_coff.size(), 2 * size_t(t.rows) + 1, "leaf_coff", err) ||
        !check(t.node_parent.size(), nodes, "node_parent", err) ||
        !check(t.rev_row_of.size(), nodes, "rev_row_of", err) ||
        !check(t.rvd_row_of.size(), nodes, "rvd_row_of", err) ||
        !check(t.rev_src.size(), t.rev_cell.size(), "rev_cell", err) ||
        !check(t.rvd_src.size(), t.rvd_p.size(), "rvd_p", err) ||
        !check(t.legal_action.size(), t.ncells, "legal_action", err) ||
        !check(t.legal_child.size(), t.ncells, "legal_child", err) ||
        !check(t.legal_trans.size(), t.ncells, "legal_trans", err) ||
        !check(t.cell_row.size(), t.ncells, "cell_row", err) ||
        !check(t.legal_off.empty() ? 0 : t.legal_off.back(), t.ncells, "legal_off", err) ||
        !check(t.snap_coff.size(), 2 * (t.leaf_rows.size() + t.term_leaves.size()) + 1, "snap_coff", err) ||
        !check(t.rows, t.leaf_rows.size(), "rows", err) ||
        !check(t.terminal_utility.size(), t.term_leaves.size(), "terminal_utility", err) ||
        !check(t.level_start.empty() ? 1 : 0, 0, "level_start", err))
        return false;
    r.f32s(job.root[0], "root0");
    r.f32s(job.root[1], "root1");
    uint32_t nroots = r.u32("nroots");
    if (!r.ok) return false;
    for (uint32_t k = 0; k < nroots; k++) {
        std::vector<float> a, c;
        r.f32s(a, "carried0");
        r.f32s(c, "carried1");
        if (!r.ok) return false;
        job.carried[0].push_back(std::move(a));
        job.carried[1].push_back(std::move(c));
    }
    if (r.at != n) {
        if (err) *err = "job: trailing bytes";
        return false;
    }
    *out = std::move(job);
    return true;
}

bool validate(const Job& job, std::string* err) {
    const Tables& t = job.t;
    auto fail = [&](const std::string& m) {
        if (err) *err = "invalid job: " + m;
        return false;
    };
    const uint32_t N = t.nodes;
    if (N == 0) return fail("no nodes");
    for (uint32_t x : job.meta.snap_iters)
        if (x > job.meta.iters) return fail("snap_iters beyond iters");
    NetShape ns;
    std::string nerr;
    if (!ns.parse(job.meta.net_dims, &nerr)) return fail(nerr);
    if (ns.kind != MODEL_V5)
        for (uint32_t c = 0; c < t.ncfg; c++) {
            uint32_t row;
            if (!head_row(t.cphi[size_t(c) * ns.cfeat], ns.heads, &row)) return fail("config head index out of range");
        }
    if (t.cfg_off[0] != 0) return fail("cfg_off[0] != 0");
    for (size_t i = 0; i + 1 < t.cfg_off.size(); i++)
        if (t.cfg_off[i + 1] < t.cfg_off[i]) return fail("cfg_off not monotone");
    if (t.node_child_start[0] != 0 || t.node_child_start[N] != t.node_child.size())
        return fail("node_child_start bounds");
    if (t.soff[0] != 0 || t.soff[N] != t.ncells) return fail("soff bounds");
    if (t.draw_off[0] != 0 || t.draw_off[N] != t.draw_to.size() || t.draw_p.size() != t.draw_to.size())
        return fail("draw_off bounds");
    if (t.reach_off[0] != 0) return fail("reach_off[0] != 0");
    if (t.node_parent[0] != NONE) return fail("root has a parent");
    if (job.root[0].size() != t.nc(0, 0) || job.root[1].size() != t.nc(0, 1))
        return fail("root belief length != root support");
    for (uint32_t r = 0; r < job.nroots(); r++)
        if (job.carried[0][r].size() != t.nc(0, 0) || job.carried[1][r].size() != t.nc(0, 1))
            return fail("carried root length != root support");
    // Every node but the root is exactly one node's child.
    if (t.node_child.size() != size_t(N) - 1) return fail("child lists do not name every node once");
    {
        std::vector<uint8_t> seen(N, 0);
        for (uint32_t ch : t.node_child)
            if (ch == 0 || ch >= N || seen[ch]++) return fail("child lists do not name every node once");
    }
    // The per-node offset lists, whole, before the loop below reads through
    // them: with both ends bounded and every step non-negative, every entry
    // lies inside its list.
    for (uint32_t i = 0; i < N; i++) {
        if (t.node_child_start[i + 1] < t.node_child_start[i]) return fail("child CSR");
        if (t.soff[i + 1] < t.soff[i]) return fail("soff not monotone");
        if (t.draw_off[i + 1] < t.draw_off[i]) return fail("draw_off not monotone");
    }
    for (uint32_t i = 0; i < N; i++) {
        if (t.node_kind[i] > 2) return fail("node_kind");
        if (t.node_player[i] > 1) return fail("node_player");
        if (t.reach_off[i + 1] - t.reach_off[i] != t.nc(i, 0) + t.nc(i, 1)) return fail("reach_off");
        const uint32_t c0 = t.node_child_start[i], c1 = t.node_child_start[i + 1];
        for (uint32_t k = c0; k < c1; k++) {
            uint32_t ch = t.node_child[k];
            if (ch >= N || ch <= i) return fail("child index (children must follow parents)");
            if (t.node_parent[ch] != i) return fail("node_parent disagrees with children");
        }
        const int me = t.node_player[i];
        if (t.node_kind[i] == 2) {
            if (c1 != c0) return fail("leaf with children");
            if (t.soff[i + 1] != t.soff[i]) return fail("leaf owns strategy cells");
        } else if (t.node_kind[i] == 1) {
            if (c1 != c0 + 1) return fail("chance node needs exactly one child");
            if (t.soff[i + 1] != t.soff[i]) return fail("chance node owns strategy cells");
            uint32_t ch = t.node_child[c0];
            uint32_t rb = t.draw_row_off[i];
            if (size_t(rb) + t.nc(i, me) + 1 > t.draw_row_start.size())
                return fail("draw rows out of range");
            uint32_t d0 = t.draw_off[i], d1 = t.draw_off[i + 1];
            for (uint32_t c = 0; c < t.nc(i, me); c++) {
                uint32_t lo = t.draw_row_start[rb + c], hi = t.draw_row_start[rb + c + 1];
                if (hi < lo || uint64_t(d0) + hi > d1) return fail("draw row bounds");
                for (uint32_t x = lo; x < hi; x++)
                    if (t.draw_to[d0 + x] >= t.nc(ch, me)) return fail("draw_to out of child support");
            }
            if (t.nc(ch, 1 - me) != t.nc(i, 1 - me)) return fail("chance changed the idle support");
            if (t.rvd_row_of[ch] == NONE) return fail("chance child without rvd rows");
        } else {
            if (c1 == c0) return fail("decision node without children");
            uint32_t row0 = t.legal_row_of[i];
            if (row0 == NONE) return fail("decision node without legal rows");
            if (size_t(row0) + t.nc(i, me) >= t.legal_off.size()) return fail("legal rows out of range");
            if (t.legal_off[row0] != t.soff[i] || t.legal_off[row0 + t.nc(i, me)] != t.soff[i + 1])
                return fail("legal rows disagree with soff");
            for (uint32_t c = 0; c < t.nc(i, me); c++) {
                uint32_t lo = t.legal_off[row0 + c], hi = t.legal_off[row0 + c + 1];
                if (hi < lo || hi > t.soff[i + 1]) return fail("legal_off not monotone");
                for (uint32_t x = lo; x < hi; x++) {
                    if (t.cell_row[x] != c) return fail("cell_row disagrees with legal_off");
                    uint32_t ch = t.legal_child[x];
                    if (ch >= N || t.node_parent[ch] != i) return fail("legal_child is not a child");
                    if (t.legal_trans[x] != NONE && t.legal_trans[x] >= t.nc(ch, me))
                        return fail("legal_trans out of child support");
                }
            }
            for (uint32_t k = c0; k < c1; k++) {
                uint32_t ch = t.node_child[k];
                if (t.nc(ch, 1 - me) != t.nc(i, 1 - me)) return fail("decision changed the idle support");
                if (t.rev_row_of[ch] == NONE) return fail("decision child without rev rows");
            }
        }
    }
    for (size_t k = 0; k < t.rev_src.size(); k++)
        if (t.rev_cell[k] >= t.ncells) return fail("rev_cell out of range");
    for (uint32_t i = 1; i < N; i++) {
        uint32_t par = t.node_parent[i];
        if (par >= i) return fail("parent after child");
        int me = t.node_player[par];
        if (t.rev_row_of[i] != NONE) {
            uint32_t row0 = t.rev_row_of[i];
            if (size_t(row0) + t.nc(i, me) >= t.rev_start.size()) return fail("rev rows out of range");
            for (uint32_t c = 0; c < t.nc(i, me); c++) {
                const uint32_t lo = t.rev_start[row0 + c], hi = t.rev_start[row0 + c + 1];
                if (hi < lo || hi > t.rev_src.size()) return fail("rev_start");  // the packer takes hi - lo
                for (uint32_t x = lo; x < hi; x++)
                    if (t.rev_src[x] >= t.nc(par, me)) return fail("rev_src");
            }
        } else if (t.rvd_row_of[i] != NONE) {
            uint32_t row0 = t.rvd_row_of[i];
            if (size_t(row0) + t.nc(i, me) >= t.rvd_start.size()) return fail("rvd rows out of range");
            for (uint32_t c = 0; c < t.nc(i, me); c++) {
                const uint32_t lo = t.rvd_start[row0 + c], hi = t.rvd_start[row0 + c + 1];
                if (hi < lo || hi > t.rvd_src.size()) return fail("rvd_start");
                for (uint32_t x = lo; x < hi; x++)
                    if (t.rvd_src[x] >= t.nc(par, me)) return fail("rvd_src");
            }
        } else {
            return fail("non-root node without gather rows");
        }
    }
    for (uint32_t r = 0; r < t.rows; r++)
        if (t.leaf_rows[r] >= N || t.node_kind[t.leaf_rows[r]] != 2) return fail("leaf_rows");
    for (size_t r = 0; r < t.term_leaves.size(); r++)
        if (t.term_leaves[r] >= N || t.node_kind[t.term_leaves[r]] != 2) return fail("term_leaves");
    {  // every leaf is valued once: a network row or a terminal, not both, not twice
        std::vector<uint8_t> seen(N, 0);
        for (uint32_t x : t.leaf_rows)
            if (seen[x]++) return fail("leaf listed twice");
        for (uint32_t x : t.term_leaves)
            if (seen[x]++) return fail("leaf listed twice");
        for (uint32_t i = 0; i < N; i++)
            if (t.node_kind[i] == 2 && !seen[i]) return fail("leaf neither a network row nor a terminal");
    }
    // The carry store's layout: the exits (network leaves, then terminal
    // leaves), each one's configs of player 0 then player 1.
    if (t.snap_coff[0] != 0) return fail("snap_coff[0] != 0");
    for (size_t e = 0; e < t.leaf_rows.size() + t.term_leaves.size(); e++) {
        const uint32_t node = e < t.leaf_rows.size() ? t.leaf_rows[e] : t.term_leaves[e - t.leaf_rows.size()];
        for (int p = 0; p < 2; p++)
            if (t.snap_coff[2 * e + p + 1] - t.snap_coff[2 * e + p] != t.nc(node, p))
                return fail("snap_coff span != support");
    }
    for (uint32_t r = 0; r < t.rows; r++)
        for (int p = 0; p < 2; p++) {
            uint32_t lo = t.leaf_coff[2 * r + p], hi = t.leaf_coff[2 * r + p + 1];
            if (hi < lo || hi > t.leaf_cidx.size()) return fail("leaf_coff");
            if (hi - lo != t.nc(t.leaf_rows[r], p)) return fail("leaf_coff span != support");
            for (uint32_t x = lo; x < hi; x++)
                if (t.leaf_cidx[x] >= t.ncfg || t.cplayer[t.leaf_cidx[x]] != p) return fail("leaf_cidx");
        }
    // BFS levels cover every node exactly once.
    if (t.bfs_order.size() != N || t.level_start.back() != N) return fail("bfs_order size");
    std::vector<uint8_t> seen(N, 0);
    for (uint32_t x : t.bfs_order) {
        if (x >= N || seen[x]) return fail("bfs_order not a permutation");
        seen[x] = 1;
    }
    // Levels are depths: the root alone at level 0, every child one level below its parent.
    if (t.level_start.size() < 2 || t.level_start[0] != 0 || t.level_start[1] != 1 || t.bfs_order[0] != 0)
        return fail("level 0 must hold the root alone");
    std::vector<uint32_t> level(N, 0);
    for (size_t l = 0; l + 1 < t.level_start.size(); l++) {
        if (t.level_start[l + 1] < t.level_start[l] || t.level_start[l + 1] > N) return fail("level_start not monotone");
        for (uint32_t k = t.level_start[l]; k < t.level_start[l + 1]; k++) level[t.bfs_order[k]] = (uint32_t)l;
    }
    for (uint32_t i = 1; i < N; i++)
        if (level[i] != level[t.node_parent[i]] + 1) return fail("levels disagree with parents");
    return true;
}

}  // namespace wc
