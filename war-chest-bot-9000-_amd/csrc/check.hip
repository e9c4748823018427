// Element checks of an uploaded wave, written for gfx950: one pass over each
// element table with every index compared against the size of the table it
// indexes (the same conditions as validate_deep's host scans, in wave-global
// terms). A check reads an entry only after comparing the index that leads
// to it with that table's size, so the checks themselves stay in bounds on any
// table contents. Failures raise a flag word (an atomic max of CHECK_BASE -
// code: the lowest code wins); nothing else is written but the pool-group
// row counters.
#include "check.h"

namespace wc {

namespace {

constexpr int CBLOCK = 256;
constexpr unsigned CGRID_MAX = 8192;

unsigned cgrid(uint64_t n) {
    const uint64_t g = (n + CBLOCK - 1) / CBLOCK;
    return (unsigned)(g < 1 ? 1 : g > CGRID_MAX ? CGRID_MAX : g);
}

__device__ __forceinline__ void raise_flag(const CheckArgs& a, uint32_t code) { atomicMax(a.flag, CHECK_BASE - code); }

// Grid-stride loop over [0, n).
#define FOR_EACH(i, n) \
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (n); i += (uint64_t)gridDim.x * blockDim.x)

__global__ __launch_bounds__(CBLOCK) void k_check_nodes(CheckArgs a) {
    FOR_EACH(i, a.nodes) {
        const uint32_t meta = a.w.node_meta[i];
        if ((meta & 3u) > 2 || (meta >> 2) > 1) raise_flag(a, CK_NODE_META);
        for (int p = 0; p < 2; p++) {
            const uint64_t n = a.w.nc[2 * i + p];
            if (a.w.reach_base[2 * i + p] + n > a.reach_len) raise_flag(a, CK_REACH_SLOT);
            if (a.w.vals_base[2 * i + p] + n > a.vals_len) raise_flag(a, CK_VALUE_SLOT);
        }
    }
}

__global__ __launch_bounds__(CBLOCK) void k_check_cells(CheckArgs a) {
    FOR_EACH(k, a.ncells) {
        const uint32_t v = a.w.legal_value[k];
        if (v != NONE && v >= a.vals_len) raise_flag(a, CK_LEGAL_VALUE);
    }
}

// Each network row names a leaf node, and lists exactly that node's configs
// of each player.
__global__ __launch_bounds__(CBLOCK) void k_check_rows(CheckArgs a) {
    FOR_EACH(r, a.rows) {
        const uint32_t node = a.w.row_node[r];
        if (node >= a.nodes || (a.w.node_meta[node] & 3u) != 2) {
            raise_flag(a, CK_ROW_NODE);
            continue;
        }
        for (int p = 0; p < 2; p++)
            if (a.w.row_cfg_off[2 * r + p + 1] - a.w.row_cfg_off[2 * r + p] != a.w.nc[2 * (uint64_t)node + p])
                raise_flag(a, CK_ROW_CONFIGS);
    }
}

__global__ __launch_bounds__(CBLOCK) void k_check_row_cfg(CheckArgs a) {
    FOR_EACH(k, a.row_cfg_n) {
        if (a.w.row_cfg[k] >= a.ncfg) raise_flag(a, CK_ROW_CFG);
    }
}

// One pool group per wavefront: its list inside the config lists, each row's
// reach base (lane i < 15 takes entry i; the padding entries repeat row 0's),
// each row's own list equal to the group's (lanes across the list), and every
// row counted for the cover check.
__global__ __launch_bounds__(CBLOCK) void k_check_groups(CheckArgs a) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t n0 = a.w.npool[0], ng = n0 + a.w.npool[1];
    const uint64_t waves = (uint64_t)gridDim.x * (CBLOCK / 64);
    for (uint64_t k = (uint64_t)blockIdx.x * (CBLOCK / 64) + threadIdx.x / 64; k < ng; k += waves) {
        const int p = k < n0 ? 0 : 1;
        const PoolGroup& g = a.w.pool_grp[p][p ? k - n0 : k];
        const uint32_t nrows = g.nrows, cfg = g.cfg, n = g.n;
        if (nrows == 0 || nrows > POOL_GROUP || (uint64_t)cfg + n > a.row_cfg_n) {
            if (lane == 0) raise_flag(a, CK_POOL_GROUP);
            continue;
        }
        bool bad = false;
        if (lane < POOL_GROUP) {
            const uint32_t r = g.row[lane < nrows ? lane : 0];
            if (r >= a.rows) {
                raise_flag(a, CK_POOL_REACH);
                bad = true;
            } else {
                const uint32_t node = a.w.row_node[r];
                if (node >= a.nodes)  // the row check reports it
                    bad = true;
                else if (g.rbase[lane] != a.w.reach_base[2 * (uint64_t)node + p]) {
                    raise_flag(a, CK_POOL_REACH);
                    bad = true;
                }
            }
        }
        if (__any(bad)) continue;  // (wave-uniform)
        if (lane < nrows) atomicAdd(a.cover + (uint64_t)p * a.rows + g.row[lane], 1u);
        for (uint32_t i = 0; i < nrows; i++) {
            const uint32_t r = g.row[i];
            const uint32_t lo = a.w.row_cfg_off[2 * (uint64_t)r + p], hi = a.w.row_cfg_off[2 * (uint64_t)r + p + 1];
            if (hi - lo != n || (uint64_t)lo + n > a.row_cfg_n) {
                if (lane == 0) raise_flag(a, CK_POOL_LIST);
                continue;
            }
            bool diff = false;
            for (uint32_t j = lane; j < n; j += 64) diff = diff || a.w.row_cfg[lo + j] != a.w.row_cfg[cfg + j];
            if (diff) raise_flag(a, CK_POOL_LIST);
        }
    }
}

// Every (player, row) pooled by exactly one group.
__global__ __launch_bounds__(CBLOCK) void k_check_cover(CheckArgs a) {
    FOR_EACH(k, 2 * a.rows) {
        const uint32_t c = a.cover[k];
        if (c == 0)
            raise_flag(a, CK_POOL_COVER);
        else if (c > 1)
            raise_flag(a, CK_POOL_ROW);
    }
}

// A value row's output slot, element range and every value slot it reads.
__device__ bool back_ok(const CheckArgs& a, const BackRec& r, int p) {
    const uint64_t n = r.kn & REC_N, kind = r.kn >> 30, start = r.start;
    if (r.out >= a.vals_len) return false;
    if (kind == BACK_OWN) {
        if (start + n > a.ncells) return false;
        for (uint64_t g = start; g < start + n; g++) {
            const uint32_t v = a.w.legal_value[g];
            if (v != NONE && v >= a.vals_len) return false;
        }
    } else if (kind == BACK_DRAW) {
        if (start + n > a.draw_to_n) return false;
        for (uint64_t x = start; x < start + n; x++)
            if ((uint64_t)r.arg + a.w.draw_to[x] >= a.vals_len) return false;
    } else if (kind == BACK_OPP) {
        if (start + n > a.child_vb_n[p]) return false;
        for (uint64_t x = start; x < start + n; x++)
            if ((uint64_t)a.w.child_vb[p][x] + r.arg >= a.vals_len) return false;
    } else {
        return false;
    }
    return true;
}

// A reach row's output slot, gather range and every reach slot and cell it reads.
__device__ bool reach_ok(const CheckArgs& a, const ReachRec& r) {
    const uint64_t n = r.kn & REC_N, start = r.start;
    if (r.out >= a.reach_len) return false;
    if ((r.kn >> 31) == REACH_REV) {
        if (start + n > a.rev_n) return false;
        for (uint64_t x = start; x < start + n; x++)
            if ((uint64_t)r.pbase + a.w.rev_src[x] >= a.reach_len || a.w.rev_cell[x] >= a.ncells) return false;
    } else {
        if (start + n > a.rvd_n) return false;
        for (uint64_t x = start; x < start + n; x++)
            if ((uint64_t)r.pbase + a.w.rvd_src[x] >= a.reach_len) return false;
    }
    return true;
}

__global__ __launch_bounds__(CBLOCK) void k_check_back(CheckArgs a, const BackRec* rec, uint64_t n, int p,
                                                      uint32_t code) {
    FOR_EACH(k, n) {
        if (!back_ok(a, rec[k], p)) raise_flag(a, code);
    }
}

__global__ __launch_bounds__(CBLOCK) void k_check_reach(CheckArgs a, const ReachRec* rec, uint64_t n, uint32_t code) {
    FOR_EACH(k, n) {
        if (!reach_ok(a, rec[k])) raise_flag(a, code);
    }
}

__global__ __launch_bounds__(CBLOCK) void k_check_acc_leaf(CheckArgs a, int p) {
    const uint64_t nacc = a.nacc[p];
    FOR_EACH(k, nacc + a.w.nleaf[p]) {
        if (k < nacc) {
            const AccRec r = a.w.acc_rec[p][k];
            if (r.ridx >= a.reach_len || (uint64_t)r.lo + r.n > a.ncells) raise_flag(a, CK_ACC_REC);
        } else {
            const LeafRec r = a.w.leaf_rec[p][k - nacc];
            if (r.out >= a.vals_len || r.head >= a.heads_end || r.mass >= 2 * a.rows) raise_flag(a, CK_LEAF_REC);
        }
    }
}

// One workgroup per readout block of player p: each of its rows names only
// configs of the block (the block's own ranges are checked on the host).
__global__ __launch_bounds__(CBLOCK) void k_check_tower(CheckArgs a, int p) {
    const TowerBlock b = a.w.tower_blk[p][blockIdx.x];
    for (uint32_t r = b.r0 + threadIdx.x; r < b.r1; r += blockDim.x) {
        const uint32_t lo = a.w.row_cfg_off[2 * (uint64_t)r + p], hi = a.w.row_cfg_off[2 * (uint64_t)r + p + 1];
        if (hi < lo || hi > a.row_cfg_n) continue;  // the row checks report it
        for (uint32_t x = lo; x < hi; x++) {
            const uint32_t c = a.w.row_cfg[x];
            if (c < b.clo || c >= b.chi) {
                raise_flag(a, CK_TOWER_CONFIGS);
                break;
            }
        }
    }
}

// One workgroup per subtree unit. The kernels keep a unit's windows in LDS:
// each of its reach rows, level by level, may read a window slot only after
// a shallower level wrote it (a bitmap of the window's slots in LDS, a
// barrier between the reads and the writes of a level) and writes inside the
// window; its leaves, terminals and value rows write and read inside its
// value window. The unit's own level and leaf ranges were checked on the host.
__global__ __launch_bounds__(CBLOCK) void k_check_units(CheckArgs a) {
    extern __shared__ uint32_t written[];  // one bit per reach window slot
    const UnitDev u = a.w.units[blockIdx.x];
    const uint32_t t = threadIdx.x, nt = blockDim.x;
    for (int p = 0; p < 2; p++) {
        const uint64_t rlo = p ? u.rwin[1] : u.rwin[0], rn = p ? u.rwin_n[1] : u.rwin_n[0];
        const uint32_t* lvl = a.w.reach_lvl[p] + u.lvl0;
        const ReachRec* rec = a.w.reach_rec[p];
        if (rlo + rn > a.reach_len || rn > a.max_rwin) {  // (the bitmap is sized for max_rwin)
            if (t == 0) raise_flag(a, CK_UNIT_RWIN);
        } else {
            for (uint64_t k = t; k < (rn + 31) / 32; k += nt) written[k] = 0;
            __syncthreads();
            for (uint32_t l = 0; l < u.nlevels; l++) {
                const uint32_t b = lvl[l], e = lvl[l + 1];
                for (uint32_t x = b + t; x < e; x += nt) {
                    const ReachRec r = rec[x];
                    const uint64_t n = r.kn & REC_N;
                    const bool rev = (r.kn >> 31) == REACH_REV;
                    if (r.start + n > (rev ? a.rev_n : a.rvd_n)) continue;  // the record check reports it
                    for (uint64_t k = 0; k < n; k++) {
                        const uint64_t i = (uint64_t)r.pbase + (rev ? a.w.rev_src[r.start + k] : a.w.rvd_src[r.start + k]);
                        const uint64_t s = i - rlo;
                        if (s < rn && !((written[s >> 5] >> (s & 31)) & 1u)) {
                            raise_flag(a, CK_UNIT_UNWRITTEN);
                            break;
                        }
                    }
                }
                __syncthreads();
                for (uint32_t x = b + t; x < e; x += nt) {
                    const uint64_t s = (uint64_t)rec[x].out - rlo;
                    if (s >= rn)
                        raise_flag(a, CK_UNIT_WRITES_OUT);
                    else
                        atomicOr(&written[s >> 5], 1u << (s & 31));
                }
                __syncthreads();
            }
        }
        const uint64_t lo = p ? u.vwin[1] : u.vwin[0], hi = lo + (p ? u.vwin_n[1] : u.vwin_n[0]);
        auto in = [&](uint64_t i) { return i >= lo && i < hi; };
        const uint32_t leaf0 = p ? u.leaf0[1] : u.leaf0[0], leaf1 = p ? u.leaf1[1] : u.leaf1[0];
        for (uint32_t k = leaf0 + t; k < leaf1; k += nt)
            if (!in(a.w.leaf_rec[p][k].out)) raise_flag(a, CK_UNIT_LEAF_OUT);
        for (uint32_t k = u.term0 + t; k < u.term1; k += nt) {
            const uint32_t node = a.w.term_node[a.w.unit_term[k] & TERM_INDEX];
            const uint64_t n = a.w.nc[2 * (uint64_t)node + p], vb = a.w.vals_base[2 * (uint64_t)node + p];
            if (n && (!in(vb) || !in(vb + n - 1))) raise_flag(a, CK_UNIT_TERM_OUT);
        }
        const uint32_t* bl = a.w.back_lvl[p] + u.lvl0;
        for (uint32_t x = bl[0] + t; x < bl[u.nlevels]; x += nt) {
            const BackRec r = a.w.back_rec[p][x];
            const uint64_t n = r.kn & REC_N, kind = r.kn >> 30, start = r.start;
            if (!in(r.out)) raise_flag(a, CK_UNIT_ROW_OUT);
            if (start + n > (kind == BACK_OWN ? a.ncells : kind == BACK_DRAW ? a.draw_to_n
                                                       : kind == BACK_OPP    ? a.child_vb_n[p]
                                                                             : 0))
                continue;  // the record check reports it
            for (uint64_t k = 0; k < n; k++) {
                uint64_t i;
                if (kind == BACK_OWN) {
                    const uint32_t v = a.w.legal_value[start + k];
                    if (v == NONE) continue;
                    i = v;
                } else if (kind == BACK_DRAW) {
                    i = (uint64_t)r.arg + a.w.draw_to[start + k];
                } else {
                    i = (uint64_t)a.w.child_vb[p][start + k] + r.arg;
                }
                if (!in(i)) {
                    raise_flag(a, CK_UNIT_ROW_READS_OUT);
                    break;
                }
            }
        }
        __syncthreads();  // the bitmap is cleared again for the next player
    }
}

}  // namespace

const char* check_message(uint32_t code) {
    static const char* const msg[CK_COUNT] = {
        "none",
        "node_meta",
        "reach slot",
        "value slot",
        "legal_value",
        "row_node",
        "row configs",
        "row_cfg",
        "pool group",
        "pool group reach",
        "pool group row",
        "pool group list",
        "pool group cover",
        "back record",
        "top back record",
        "reach record",
        "top reach record",
        "accumulation record",
        "leaf record",
        "tower block configs",
        "unit reach window",
        "unit reach row reads an unwritten window slot",
        "unit reach row writes outside its reach window",
        "unit leaf outside its value window",
        "unit terminal outside its value window",
        "unit row outside its value window",
        "unit row reads outside its value window",
    };
    return code < CK_COUNT ? msg[code] : nullptr;
}

CheckArgs check_args(const WaveHost& h, const WaveDev& w, const BackRec* const top_back[2],
                     const ReachRec* const top_reach[2], uint32_t* flag, uint32_t* cover) {
    CheckArgs a{};
    a.w = w;
    a.flag = flag;
    a.cover = cover;
    a.nodes = h.nodes();
    a.ncells = h.ncells;
    a.reach_len = h.reach_len;
    a.vals_len = h.vals_len;
    a.rows = h.rows();
    a.ncfg = h.cfg_key.size();
    a.row_cfg_n = h.row_cfg.size();
    a.draw_to_n = h.draw_to.size();
    a.rev_n = h.rev_src.size();
    a.rvd_n = h.rvd_src.size();
    a.heads_end = readout_net(h.net.kind) ? h.tower_len : uint64_t(h.rows()) * h.net.heads;
    a.term_n = h.term_node.size();
    for (int p = 0; p < 2; p++) {
        a.top_back[p] = top_back[p];
        a.top_reach[p] = top_reach[p];
        a.child_vb_n[p] = h.child_vb[p].size();
        a.nback[p] = h.back_rec[p].size();
        a.ntop_back[p] = h.top_back_rec[p].size();
        a.nreach[p] = h.reach_rec[p].size();
        a.ntop_reach[p] = h.top_reach_rec[p].size();
        a.nacc[p] = h.acc_rec[p].size();
    }
    a.max_rwin = h.max_rwin;
    a.tower = readout_net(h.net.kind) ? 1u : 0u;
    return a;
}

void launch_check(const CheckArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_check_nodes, dim3(cgrid(a.nodes)), dim3(CBLOCK), 0, s, a);
    hipLaunchKernelGGL(k_check_cells, dim3(cgrid(a.ncells)), dim3(CBLOCK), 0, s, a);
    hipLaunchKernelGGL(k_check_rows, dim3(cgrid(a.rows)), dim3(CBLOCK), 0, s, a);
    hipLaunchKernelGGL(k_check_row_cfg, dim3(cgrid(a.row_cfg_n)), dim3(CBLOCK), 0, s, a);
    hipLaunchKernelGGL(k_check_groups, dim3(cgrid(64 * ((uint64_t)a.w.npool[0] + a.w.npool[1]))), dim3(CBLOCK), 0, s,
                       a);
    hipLaunchKernelGGL(k_check_cover, dim3(cgrid(2 * a.rows)), dim3(CBLOCK), 0, s, a);
    for (int p = 0; p < 2; p++) {
        hipLaunchKernelGGL(k_check_back, dim3(cgrid(a.nback[p])), dim3(CBLOCK), 0, s, a, a.w.back_rec[p], a.nback[p],
                           p, (uint32_t)CK_BACK_REC);
        hipLaunchKernelGGL(k_check_back, dim3(cgrid(a.ntop_back[p])), dim3(CBLOCK), 0, s, a, a.top_back[p],
                           a.ntop_back[p], p, (uint32_t)CK_TOP_BACK_REC);
        hipLaunchKernelGGL(k_check_reach, dim3(cgrid(a.nreach[p])), dim3(CBLOCK), 0, s, a, a.w.reach_rec[p],
                           a.nreach[p], (uint32_t)CK_REACH_REC);
        hipLaunchKernelGGL(k_check_reach, dim3(cgrid(a.ntop_reach[p])), dim3(CBLOCK), 0, s, a, a.top_reach[p],
                           a.ntop_reach[p], (uint32_t)CK_TOP_REACH_REC);
        hipLaunchKernelGGL(k_check_acc_leaf, dim3(cgrid(a.nacc[p] + a.w.nleaf[p])), dim3(CBLOCK), 0, s, a, p);
        if (a.tower && a.w.ntower_blk[p])
            hipLaunchKernelGGL(k_check_tower, dim3(a.w.ntower_blk[p]), dim3(CBLOCK), 0, s, a, p);
    }
    if (a.w.nunits) {
        const size_t lds = ((size_t)a.max_rwin + 31) / 32 * 4;
        hipLaunchKernelGGL(k_check_units, dim3(a.w.nunits), dim3(CBLOCK), lds ? lds : 4, s, a);
    }
}

}  // namespace wc
