// HIP kernels of the wave executor, written for gfx950 (wave64).
//
// Every reduction whose result the CPU solver also forms is taken by one lane
// in the solver's order, with no contraction into FMA (the library is built
// with -ffp-contract=off): per-row regret updates in ascending action order,
// reverse gathers in their stored order, child sums in child order, leaf masses
// and belief normalisations in config order. That makes the CFR state
// bit-identical to the CPU restatement whenever the leaf values are.
#include "kernels.h"

#include <hip/hip_fp16.h>

#include <algorithm>

#include "../../include/wc_wave.h"

namespace wc {

// MFMA operand and accumulator vectors.
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

#define EPSF 1e-6f       // regret-matching floor (engine/src/search.rs:1658)
#define SMOOTHF 1e-30f   // belief normalisation floor (engine/src/rebel.rs:359)

constexpr int BLOCK = 256;
// The subtree sweep stages a unit's values in LDS when the widest window fits this.
constexpr size_t SWEEP_LDS_MAX = 64 * 1024;
constexpr size_t REACH_LDS_MAX = 32 * 1024;  // the reach pass keeps a unit's reach window in LDS up to this

static inline unsigned grid_for(size_t n, int block = BLOCK) { return (unsigned)((n + block - 1) / block); }

// ------------------------------------------------------------------ helpers

__global__ void k_zero(float* p, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = 0.0f;
}

void launch_zero(float* p, size_t n, hipStream_t s) {
    if (n == 0) return;
    unsigned g = grid_for(n);
    if (g > 4096) g = 4096;
    hipLaunchKernelGGL(k_zero, dim3(g), dim3(BLOCK), 0, s, p, n);
}

__device__ __forceinline__ const AccRec& decision_row(const WaveDev& w, uint32_t i, int* p) {
    if (i < w.ndec[0]) {
        *p = 0;
        return w.acc_rec[0][i];
    }
    *p = 1;
    return w.acc_rec[1][i - w.ndec[0]];
}

// ------------------------------------------------------------- CFR state

// cur = 1/len over each acting row (engine/src/search.rs:826-836).
__global__ void k_init_strategy(WaveDev w) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= w.ndec[0] + w.ndec[1]) return;
    int p;
    AccRec q = decision_row(w, i, &p);
    float u = 1.0f / (float)q.n;
    for (uint32_t g = q.lo; g < q.lo + q.n; g++) w.cur[g] = u;
}

void launch_init_strategy(const WaveDev& w, hipStream_t s) {
    uint32_t n = w.ndec[0] + w.ndec[1];
    if (n) hipLaunchKernelGGL(k_init_strategy, dim3(grid_for(n)), dim3(BLOCK), 0, s, w);
}

// Zero one tree's reach span and write its root (or carried root k) beliefs.
// Root beliefs into the zeroed reach (launch_seed_reach clears it first).
__global__ void k_seed_reach(WaveDev w, float* reach, int root_index) {
    const TreeDev t = w.trees[blockIdx.x];
    if (root_index >= (int)t.nroots) return;
    const float* src = root_index < 0 ? w.roots + t.root0 : w.carried + t.carried0 + (size_t)root_index * (t.n0 + t.n1);
    for (uint32_t i = threadIdx.x; i < t.n0 + t.n1; i += blockDim.x) {
        int p = i >= t.n0;
        uint32_t c = p ? i - t.n0 : i;
        reach[w.reach_base[2 * t.node0 + p] + c] = src[i];
    }
}

void launch_seed_reach(const WaveDev& w, float* reach, size_t reach_len, int root_index, hipStream_t s) {
    launch_zero(reach, reach_len, s);  // every tree's reach span: the trees tile [0, reach_len)
    hipLaunchKernelGGL(k_seed_reach, dim3(w.ntrees), dim3(BLOCK), 0, s, w, reach, root_index);
}

// Row elements are handled ROW_BATCH at a time: a batch's loads are issued
// together (indices, then the values they name) and its part of the reduction
// is taken after, in element order, so every sum keeps the CPU's order.
constexpr uint32_t ROW_BATCH = 12;   // value rows: decision rows up to 12 actions in one pass
constexpr uint32_t REACH_BATCH = 8;  // reach gathers and average accumulation
// Network-leaf slots in flight per thread in the sweep's leaf phase.
constexpr uint32_t LEAF_BATCH = 4;

// One child config's reach: the reverse gather in stored order (the CPU's
// scatter order, engine/src/serialize.rs:714-723). With LDSR the unit's reach
// window [rw, rw + rn) is also kept in LDS at lr: parent reach inside it is
// read from there, and the row's result goes to both.
template <bool LDSR = false>
__device__ __forceinline__ void reach_row(const WaveDev& w, float* reach, const float* strat, ReachRec q,
                                          float* lr = nullptr, uint32_t rw = 0, uint32_t rn = 0) {
    const uint32_t lo = q.start, n = q.kn & REC_N, base = q.pbase;
    auto parent = [&](uint32_t i) { return LDSR && i - rw < rn ? lr[i - rw] : reach[i]; };
    float v = 0.0f;
    if ((q.kn >> 31) == REACH_REV) {
        for (uint32_t c0 = 0; c0 < n; c0 += REACH_BATCH) {
            const uint32_t m = n - c0 < REACH_BATCH ? n - c0 : REACH_BATCH;
            uint32_t src[REACH_BATCH], cell[REACH_BATCH];
            float a[REACH_BATCH], b[REACH_BATCH];
#pragma unroll
            for (uint32_t k = 0; k < REACH_BATCH; k++)
                if (k < m) {
                    src[k] = w.rev_src[lo + c0 + k];
                    cell[k] = w.rev_cell[lo + c0 + k];
                }
#pragma unroll
            for (uint32_t k = 0; k < REACH_BATCH; k++)
                if (k < m) {
                    a[k] = parent(base + src[k]);
                    b[k] = strat[cell[k]];
                }
#pragma unroll
            for (uint32_t k = 0; k < REACH_BATCH; k++)
                if (k < m) v += a[k] * b[k];
        }
    } else {
        for (uint32_t c0 = 0; c0 < n; c0 += REACH_BATCH) {
            const uint32_t m = n - c0 < REACH_BATCH ? n - c0 : REACH_BATCH;
            uint32_t src[REACH_BATCH];
            float a[REACH_BATCH], pr[REACH_BATCH];
#pragma unroll
            for (uint32_t k = 0; k < REACH_BATCH; k++)
                if (k < m) {
                    src[k] = w.rvd_src[lo + c0 + k];
                    pr[k] = w.rvd_p[lo + c0 + k];
                }
#pragma unroll
            for (uint32_t k = 0; k < REACH_BATCH; k++)
                if (k < m) a[k] = parent(base + src[k]);
#pragma unroll
            for (uint32_t k = 0; k < REACH_BATCH; k++)
                if (k < m) v += a[k] * pr[k];
        }
    }
    reach[q.out] = v;
    if (LDSR) lr[q.out - rw] = v;
}

// sum = sum * ds + reach * cur over one decision row: the DCFR discount of the
// traverser's average-strategy sum (search.rs:1770-1779, applied at the
// backprop) and this iteration's accumulation (engine/src/search.rs:1818-1835),
// the same two rounded steps in the same order, taken in one pass.
__device__ __forceinline__ void accumulate_row(const WaveDev& w, AccRec q, float ds) {
    const float r = w.reach[q.ridx];
    const uint32_t lo = q.lo, n = q.n;
    for (uint32_t c0 = 0; c0 < n; c0 += REACH_BATCH) {
        const uint32_t m = n - c0 < REACH_BATCH ? n - c0 : REACH_BATCH;
        float cu[REACH_BATCH], sm[REACH_BATCH];
#pragma unroll
        for (uint32_t j = 0; j < REACH_BATCH; j++)
            if (j < m) {
                cu[j] = w.cur[lo + c0 + j];
                sm[j] = w.sum[lo + c0 + j];
            }
#pragma unroll
        for (uint32_t j = 0; j < REACH_BATCH; j++)
            if (j < m) w.sum[lo + c0 + j] = sm[j] * ds + r * cu[j];
    }
}

// Both players' top-down reach of one unit, level by level under block
// barriers (their rows of a level are independent), parents read from L2:
// both players' reach windows in LDS (32 KB at the default unit budget) would
// leave room for five workgroups per CU instead of eight (88.6 against 76.4 µs
// per launch).
__device__ __forceinline__ void reach_unit_both(const WaveDev& w, const UnitDev& u, float* reach, const float* strat) {
    for (uint32_t l = 0; l < u.nlevels; l++) {
        uint32_t b0 = w.reach_lvl[0][u.lvl0 + l], e0 = w.reach_lvl[0][u.lvl0 + l + 1];
        uint32_t b1 = w.reach_lvl[1][u.lvl0 + l], e1 = w.reach_lvl[1][u.lvl0 + l + 1];
        uint32_t n0 = e0 - b0, n = n0 + (e1 - b1);
        for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
            if (k < n0)
                reach_row(w, reach, strat, w.reach_rec[0][b0 + k]);
            else
                reach_row(w, reach, strat, w.reach_rec[1][b1 + k - n0]);
        }
        __syncthreads();
    }
}

// One player's top-down reach of one unit, the next level's bounds and each
// thread's first record of it fetched while the current level runs; with
// LDSR the unit's reach window lives in LDS as well (every slot of it is
// written by a level above the rows that read it).
template <bool LDSR>
__device__ __forceinline__ void reach_unit_one(const WaveDev& w, const UnitDev& u, float* reach, const float* strat,
                                               int p, float* lr) {
    // The player's fields by select: indexing them with the run-time p would
    // place the record in scratch memory.
    const uint32_t rw = p ? u.rwin[1] : u.rwin[0], rn = p ? u.rwin_n[1] : u.rwin_n[0];
    const ReachRec* rec = w.reach_rec[p];
    const uint32_t* lvl = w.reach_lvl[p] + u.lvl0;
    const uint32_t L = u.nlevels, t = threadIdx.x;
    uint32_t b = L ? lvl[0] : 0, e = L ? lvl[1] : 0;
    ReachRec q{};
    if (L && b + t < e) q = rec[b + t];
    for (uint32_t l = 0; l < L; l++) {
        const uint32_t lb = b, le = e;
        const bool more = l + 1 < L;
        if (more) {
            b = le;
            e = lvl[l + 2];
        }
        // Each thread's rows form one stream across the levels: the record of
        // its next row (in this level, else its first in the next level) is
        // fetched while the current row runs.
        if (lb + t >= le && more && b + t < e) q = rec[b + t];
        for (uint32_t k = lb + t; k < le;) {
            const uint32_t kn = k + blockDim.x;
            ReachRec qn{};
            if (kn < le)
                qn = rec[kn];
            else if (more && b + t < e)
                qn = rec[b + t];
            reach_row<LDSR>(w, reach, strat, q, lr, rw, rn);
            q = qn;
            k = kn;
        }
        __syncthreads();
    }
}

// Subtree units' reach: one player's, one unit per workgroup with its reach
// window in LDS when LDSR; both players' (player < 0) either as one
// workgroup per (unit, player), windows in LDS, or one per unit from L2. With
// reach2 (player >= 0), workgroup 3 u + k takes unit u's rows of player
// `player` under strat into reach (k = 0) or of player k - 1 under strat2
// into reach2: independent computations, one launch.
template <bool LDSR>
__global__ __launch_bounds__(BLOCK) void k_reach(WaveDev w, uint32_t unit0, float* reach, const float* strat,
                                               int player, float* reach2, const float* strat2) {
    extern __shared__ float lds_reach[];  // the unit's reach window of the player (when LDSR)
    if (player >= 0 && reach2) {
        const uint32_t k = blockIdx.x % 3;
        const UnitDev u = w.units[unit0 + blockIdx.x / 3];
        if (k == 0)
            reach_unit_one<LDSR>(w, u, reach, strat, player, lds_reach);
        else
            reach_unit_one<LDSR>(w, u, reach2, strat2, (int)k - 1, lds_reach);
        return;
    }
    if (LDSR && player < 0) {  // the players' rows are independent: workgroup 2 u + p
        const UnitDev u = w.units[unit0 + blockIdx.x / 2];
        reach_unit_one<true>(w, u, reach, strat, (int)(blockIdx.x & 1), lds_reach);
        return;
    }
    const UnitDev u = w.units[unit0 + blockIdx.x];
    if (player < 0)
        reach_unit_both(w, u, reach, strat);
    else
        reach_unit_one<LDSR>(w, u, reach, strat, player, lds_reach);
}

void launch_reach(const WaveDev& w, uint32_t unit0, uint32_t n, float* reach, const float* strat, int player,
                  hipStream_t s, float* reach2, const float* strat2) {
    if (!n) return;
    if (player < 0) reach2 = nullptr;  // both players already
    const size_t lds = (size_t)w.max_rwin * sizeof(float);
    const bool in_lds = w.unit_lds && lds <= REACH_LDS_MAX;
    const uint32_t grid = reach2 ? 3 * n : player < 0 && in_lds ? 2 * n : n;
    if (in_lds)
        hipLaunchKernelGGL(k_reach<true>, dim3(grid), dim3(BLOCK), lds, s, w, unit0, reach, strat, player, reach2,
                           strat2);
    else
        hipLaunchKernelGGL(k_reach<false>, dim3(grid), dim3(BLOCK), 0, s, w, unit0, reach, strat, player, reach2,
                           strat2);
}

// The average-strategy accumulation of player `acc` over all its decision rows
// (units' and top regions'), one row per thread, in workgroups of a leaf-input
// launch (both only read the final reach). The launch's pool_blocks pooling
// workgroups come longest config lists first; the accumulation's workgroups
// are dealt after the first quarter of them, so the streaming accumulation
// runs beside the long lists rather than trailing the launch (3.94 -> 3.78 ms
// per 256-subgame wave; right after the first eighth or half: 3.86 / 3.89).
// Returns true for an accumulation workgroup, else sets *pool_block to the
// workgroup's index among the pooling ones.
__device__ __forceinline__ bool accumulate_blocks(const WaveDev& w, int acc, float ds, uint32_t pool_blocks,
                                                  uint32_t* pool_block) {
    const uint32_t nacc = acc >= 0 ? gridDim.x - pool_blocks : 0, q1 = pool_blocks / 4;
    if (blockIdx.x >= q1 && blockIdx.x < q1 + nacc) {
        const uint32_t k = (blockIdx.x - q1) * blockDim.x + threadIdx.x;
        if (k < w.ndec[acc]) accumulate_row(w, w.acc_rec[acc][k], ds);
        return true;
    }
    *pool_block = blockIdx.x < q1 ? blockIdx.x : blockIdx.x - nacc;
    return false;
}

// Top-region reach at one depth, all trees together: one row per thread, the
// rows of up to three independent sets (players, reach computations).
__global__ __launch_bounds__(BLOCK) void k_reach_rows(WaveDev w, ReachSet a, ReachSet b, ReachSet c) {
    uint32_t k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k < a.n) {
        reach_row(w, a.reach, a.strat, a.rows[k]);
        return;
    }
    k -= a.n;
    if (k < b.n) {
        reach_row(w, b.reach, b.strat, b.rows[k]);
        return;
    }
    k -= b.n;
    if (k < c.n) reach_row(w, c.reach, c.strat, c.rows[k]);
}

// A top depth holds 10k-50k rows, one per thread: one-wavefront workgroups
// spread them over four times as many CUs as 256-thread ones, so each CU's
// memory pipeline serves fewer of the rows' dependent loads (0.33 ms per wave
// of 256 subgames over 1,120 launches).
constexpr int TOP_BLOCK = 64;

void launch_reach_rows(const WaveDev& w, const ReachSet& a, const ReachSet& b, const ReachSet& c, hipStream_t s) {
    const size_t n = (size_t)a.n + b.n + c.n;
    if (n) hipLaunchKernelGGL(k_reach_rows, dim3(grid_for(n, TOP_BLOCK)), dim3(TOP_BLOCK), 0, s, w, a, b, c);
}

// Top-region reach at two depths in one launch, up to three independent sets
// (players, reach computations) one after another in the grid. A shallower
// row named by two chunks is computed by both: reach rows keep no state, and
// both write the same value, so each chunk reads its own result or the
// other's equal one after its barrier. A chunk names up to about 85
// shallower rows for its 64 deeper ones, so its workgroup has two wavefronts:
// one shallower row per thread (20.34 ms per 256-subgame wave, against 20.65
// with one wavefront, two rows on some threads, and 20.45 without the fused
// reach launches).
__global__ __launch_bounds__(BLOCK) void k_reach_pair(WaveDev w, ReachPair a, ReachPair b, ReachPair c) {
    uint32_t k = blockIdx.x;
    ReachPair s = a;
    if (k >= a.chunks) {
        k -= a.chunks;
        s = b;
        if (k >= b.chunks) {
            k -= b.chunks;
            s = c;
        }
    }
    const uint32_t* q = s.off + s.chunks + 1;
    for (uint32_t i = q[k] + threadIdx.x; i < q[k + 1]; i += blockDim.x)
        reach_row(w, s.reach, s.strat, s.rows[s.par[i]]);
    __syncthreads();
    for (uint32_t i = s.off[k] + threadIdx.x; i < s.off[k + 1]; i += blockDim.x)
        reach_row(w, s.reach, s.strat, s.rows[i]);
}

void launch_reach_pair(const WaveDev& w, const ReachPair& a, const ReachPair& b, const ReachPair& c, hipStream_t s) {
    const uint32_t n = a.chunks + b.chunks + c.chunks;
    if (n) hipLaunchKernelGGL(k_reach_pair, dim3(n), dim3(2 * TOP_BLOCK), 0, s, w, a, b, c);
}

// sum = reach * cur: one reach-weighted uniform strategy (engine/src/search.rs:854-870).
__global__ void k_seed_sum(WaveDev w) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= w.ndec[0] + w.ndec[1]) return;
    int p;
    AccRec q = decision_row(w, i, &p);
    float r = w.reach[q.ridx];
    for (uint32_t g = q.lo; g < q.lo + q.n; g++) w.sum[g] = r * w.cur[g];
}

void launch_seed_sum(const WaveDev& w, hipStream_t s) {
    uint32_t n = w.ndec[0] + w.ndec[1];
    if (n) hipLaunchKernelGGL(k_seed_sum, dim3(grid_for(n)), dim3(BLOCK), 0, s, w);
}

// --------------------------------------------------------------- leaf input

__device__ __forceinline__ uint16_t f32_to_bf16_rn(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u | 0x00400000u) >> 16);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_rn(float x) {
    _Float16 h = (_Float16)x;
    return __builtin_bit_cast(uint16_t, h);
}

// One query-input element. Compensated f16 keeps two planes `plane` elements
// apart: hi = f16(v) and lo = f16(v - hi).
template <int PREC>
__device__ __forceinline__ void store_operand(void* base, size_t i, float v, size_t plane) {
    if (PREC == WC_PRECISE) {
        ((float*)base)[i] = v;
    } else if (PREC == WC_F16) {
        ((uint16_t*)base)[i] = f32_to_f16_rn(v);
    } else if (PREC == WC_BF16) {
        ((uint16_t*)base)[i] = f32_to_bf16_rn(v);
    } else {
        const uint16_t hi = f32_to_f16_rn(v);
        ((uint16_t*)base)[i] = hi;
        ((uint16_t*)base)[i + plane] = f32_to_f16_rn(v - (float)__builtin_bit_cast(_Float16, hi));
    }
}

// Query inputs are row-major float32 for the exact net, fragment-major 16-bit for MFMA.
template <int PREC>
__device__ __forceinline__ size_t operand_at(uint32_t row, uint32_t k, uint32_t K) {
    return PREC == WC_PRECISE ? (size_t)row * K + k : frag_off(row, k, K);
}

__device__ __forceinline__ float lane_value(float v, uint32_t j) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)j));
}
__device__ __forceinline__ uint32_t lane_value(uint32_t v, uint32_t j) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)j);
}

// tot + v's lanes 0 .. m - 1 (m <= 64), added one at a time in lane order.
// Eight lanes are read per step (independent reads ahead of the dependent
// adds); the caller sets lanes m .. 63 to +0.0, and adding +0.0 leaves a sum
// that started at +0.0 unchanged (such a sum is never -0.0), so the result is
// the plain sequential sum.
__device__ __forceinline__ float lane_sum_in_order(float tot, float v, uint32_t m) {
    for (uint32_t k0 = 0; k0 < m; k0 += 8) {
        float y[8];
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) y[i] = lane_value(v, k0 + i);
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) tot += y[i];
    }
    return tot;
}

// Float32 net: one wavefront per (network row, player). The leaf's reach
// mass, and the pooled belief sum_c beta(c) e(c) with beta the normalised
// reach (normalize_weights, engine/src/rebel.rs:1054-1068; accumulate,
// net.rs:161-170). Lanes load 64 configs at a time; both reductions then run
// in config order with every lane holding the running value, so the result is
// the CPU's sequential sum. The pooled block goes straight into the two query
// inputs that carry it: [pooled_q | pooled_{1-q} | seat | public] for
// traverser q.
__global__ __launch_bounds__(BLOCK) void k_pool_exact(WaveDev w, int player, float* x0, float* x1, int acc,
                                                    float ds, uint32_t pool_blocks) {
    uint32_t pbk;
    if (accumulate_blocks(w, acc, ds, pool_blocks, &pbk)) return;
    const uint32_t task = __builtin_amdgcn_readfirstlane((pbk * blockDim.x + threadIdx.x) >> 6);
    const uint32_t lane = threadIdx.x & 63;
    uint32_t row, p;
    if (player < 0) {
        row = task >> 1;
        p = task & 1;
    } else {
        row = task;
        p = (uint32_t)player;
    }
    if (row >= w.rows) return;  // wave-uniform
    const uint32_t node = w.row_node[row];
    const uint32_t n = w.nc[2 * node + p];
    const float* r = w.reach + w.reach_base[2 * node + p];
    const uint32_t* cfgs = w.row_cfg + w.row_cfg_off[2 * row + p];
    float tot = 0.0f;
    for (uint32_t c0 = 0; c0 < n; c0 += 64) {
        float v = c0 + lane < n ? r[c0 + lane] : 0.0f;
        tot = lane_sum_in_order(tot, v, n - c0 < 64 ? n - c0 : 64);
    }
    float scale, flat;
    if (tot > SMOOTHF) {
        scale = 1.0f / tot;
        flat = 0.0f;
    } else {
        scale = 0.0f;
        flat = 1.0f / (float)(n > 0 ? n : 1);
    }
    if (lane == 0) w.mass[2 * row + p] = tot;
    const uint32_t pool = w.pool, in = w.in;
    float* own = p ? x1 : x0;    // pooled_p is the first block of traverser p's query
    float* other = p ? x0 : x1;  // and the second block of the other traverser's
    for (uint32_t k0 = 0; k0 < pool; k0 += 64) {
        const uint32_t k = k0 + lane;
        const bool live = k < pool;
        float acc = 0.0f;
        for (uint32_t c0 = 0; c0 < n; c0 += 64) {
            uint32_t cf = c0 + lane < n ? cfgs[c0 + lane] : 0u;
            float beta = c0 + lane < n ? r[c0 + lane] * scale + flat : 0.0f;
            uint32_t m = n - c0 < 64 ? n - c0 : 64;
            uint32_t j = 0;
            for (; j + 8 <= m; j += 8) {
                float e[8], b[8];
#pragma unroll
                for (uint32_t t = 0; t < 8; t++) {
                    uint32_t cj = lane_value(cf, j + t);
                    b[t] = lane_value(beta, j + t);
                    e[t] = live ? w.cfg_emb[(size_t)cj * pool + k] : 0.0f;
                }
#pragma unroll
                for (uint32_t t = 0; t < 8; t++) acc += b[t] * e[t];
            }
            for (; j < m; j++) {
                uint32_t cj = lane_value(cf, j);
                float e = live ? w.cfg_emb[(size_t)cj * pool + k] : 0.0f;
                acc += lane_value(beta, j) * e;
            }
        }
        if (live) {
            own[(size_t)row * in + k] = acc;
            other[(size_t)row * in + pool + k] = acc;
        }
    }
}

// 16-bit nets: one wavefront per pool group (up to POOL_GROUP rows of one
// player whose configs are the same list), on the f32 MFMA. With A the
// group's reach rows (row 15: ones) and B the configs' embeddings, four
// 16x16x4 products per 4 configs accumulate U[r][k] = sum_c reach_r(c) e_c(k)
// and, in row 15, S[k] = sum_c e_c(k); each row's mass is summed on the VALU
// from the same reach values. Then pooled = U / mass, or S / n where
// the mass is below the smoothing floor (the uniform weights of
// normalize_weights). Each config's embedding is read once for the group.
// Products are exact f32; only the summation order differs from the CPU's,
// far below the 16-bit rounding of the stored query input.
template <int PREC>
__global__ __launch_bounds__(BLOCK) void k_pool_mfma(WaveDev w, int player, uint16_t* x0, uint16_t* x1, int acc,
                                                   float ds, uint32_t pool_blocks) {
    uint32_t pbk;
    if (accumulate_blocks(w, acc, ds, pool_blocks, &pbk)) return;
    uint32_t g = __builtin_amdgcn_readfirstlane((pbk * blockDim.x + threadIdx.x) >> 6);
    const uint32_t lane = threadIdx.x & 63;
    uint32_t p = player < 0 ? 0u : (uint32_t)player;
    if (player < 0 && g >= w.npool[0]) {
        g -= w.npool[0];
        p = 1;
    }
    if (g >= w.npool[p]) return;  // wave-uniform
    const PoolGroup* grp = w.pool_grp[p] + g;
    const uint32_t n = grp->n, G = grp->nrows;
    const uint32_t i = lane & 15, q = lane >> 4;  // A row / B column, and config within a 4-step
    const float* ra = w.reach + grp->rbase[i < POOL_GROUP ? i : 0];  // lane row 15 reads no reach
    const float aconst = i == 15 ? 1.0f : 0.0f;  // rows G..14 are zero, row 15 sums the embeddings
    const uint32_t* cfgs = w.row_cfg + grp->cfg;
    const uint32_t pool = w.pool, in = w.in;
    uint16_t* own = p ? x1 : x0;
    uint16_t* other = p ? x0 : x1;
    float tot[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // mass of rows 4q .. 4q + 3
    for (uint32_t k0 = 0; k0 < pool; k0 += 64) {
        float4v acc[4];
#pragma unroll
        for (int t = 0; t < 4; t++) acc[t] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
        bool kl[4];
#pragma unroll
        for (int t = 0; t < 4; t++) kl[t] = k0 + 16 * t + i < pool;
        float tpart = 0.0f;  // this lane's share of row i's mass: configs 4 s + q
        // 64 configs per chunk: one coalesced load of their indices, the reach
        // gathers of all 16 steps in flight together, each step's index handed
        // to its lanes by a shuffle, then 8 steps' embeddings at a time. Steps
        // past the end of the list are skipped.
        for (uint32_t c0 = 0; c0 < n; c0 += 64) {
            const uint32_t cfl = c0 + lane < n ? cfgs[c0 + lane] : 0xffffffffu;
            float a[16];
#pragma unroll
            for (int s = 0; s < 16; s++) {
                const uint32_t c = c0 + 4 * s + q;
                a[s] = c < n ? (i < G ? ra[c] : aconst) : 0.0f;
            }
#pragma unroll
            for (int s = 0; s < 16; s++) tpart += a[s];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                if (c0 + 32 * h >= n) break;  // wave-uniform
                uint32_t cf[8];
                float b[8][4];
#pragma unroll
                for (int s = 0; s < 8; s++) cf[s] = (uint32_t)__shfl((int)cfl, 4 * (8 * h + s) + (int)q, 64);
#pragma unroll
                for (int s = 0; s < 8; s++) {
                    const bool live = cf[s] != 0xffffffffu;
                    const float* e = w.cfg_emb + (size_t)(live ? cf[s] : 0u) * pool + k0 + i;
#pragma unroll
                    for (int t = 0; t < 4; t++) b[s][t] = live && kl[t] ? e[16 * t] : 0.0f;
                }
#pragma unroll
                for (int s = 0; s < 8; s++) {
                    if (c0 + 4 * (8 * h + s) >= n) break;  // wave-uniform
#pragma unroll
                    for (int t = 0; t < 4; t++)
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[8 * h + s], b[s][t], acc[t], 0, 0, 0);
                }
            }
        }
        if (k0 == 0) {
            // Row i's mass: lanes i, i + 16, i + 32, i + 48 hold its partial sums.
            float ti = tpart + __shfl_xor(tpart, 16, 64);
            ti += __shfl_xor(ti, 32, 64);
#pragma unroll
            for (int v = 0; v < 4; v++) tot[v] = __shfl(ti, (int)(4 * q + v), 64);
            if (q == 0 && i < G) w.mass[2 * grp->row[i] + p] = ti;
        }
        const float inv_n = 1.0f / (float)(n > 0 ? n : 1);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float S = __shfl(acc[t][3], (int)(48 + i), 64);  // row 15 of this column
            const uint32_t k = k0 + 16 * t + i;
            if (!kl[t]) continue;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const uint32_t rr = 4 * q + v;
                if (rr >= G) continue;
                const float y = tot[v] > SMOOTHF ? acc[t][v] * (1.0f / tot[v]) : S * inv_n;
                const uint32_t row = grp->row[rr];
                store_operand<PREC>(own, frag_off(row, k, in), y, w.xplane);
                store_operand<PREC>(other, frag_off(row, pool + k, in), y, w.xplane);
            }
        }
    }
}

void launch_pool(const WaveDev& w, int player, int precision, void* x0, void* x1, hipStream_t s, int acc,
                 float ds) {
    const uint32_t accb = acc >= 0 ? grid_for(w.ndec[acc]) : 0;
    if (precision == WC_PRECISE) {
        size_t waves = (size_t)w.rows * (player < 0 ? 2 : 1);
        const uint32_t pb = grid_for(waves * 64);
        if (pb + accb)
            hipLaunchKernelGGL(k_pool_exact, dim3(pb + accb), dim3(BLOCK), 0, s, w, player, (float*)x0, (float*)x1,
                               acc, ds, pb);
        return;
    }
    size_t waves = player < 0 ? (size_t)w.npool[0] + w.npool[1] : w.npool[player];
    const uint32_t pb = grid_for(waves * 64);
    if (!(pb + accb)) return;
    dim3 g(pb + accb);
    if (precision == WC_F16)
        hipLaunchKernelGGL(k_pool_mfma<WC_F16>, g, dim3(BLOCK), 0, s, w, player, (uint16_t*)x0, (uint16_t*)x1, acc,
                           ds, pb);
    else if (precision == WC_BF16)
        hipLaunchKernelGGL(k_pool_mfma<WC_BF16>, g, dim3(BLOCK), 0, s, w, player, (uint16_t*)x0, (uint16_t*)x1, acc,
                           ds, pb);
    else
        hipLaunchKernelGGL(k_pool_mfma<WC_F16X>, g, dim3(BLOCK), 0, s, w, player, (uint16_t*)x0, (uint16_t*)x1, acc,
                           ds, pb);
}

// The fixed part of both traversers' query inputs: the seat (-1 for player 0,
// +1 for player 1) and the row's public features / 255.
template <int PREC>
__global__ void k_query_static(WaveDev w, void* x0, void* x1) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t width = w.in - 2 * w.pool;
    if (i >= (size_t)w.rows * width) return;
    uint32_t row = (uint32_t)(i / width), k = (uint32_t)(i % width);
    size_t at = operand_at<PREC>(row, 2 * w.pool + k, w.in);
    if (k == 0) {
        store_operand<PREC>(x0, at, -1.0f, w.xplane);
        store_operand<PREC>(x1, at, 1.0f, w.xplane);
    } else {
        // public features; columns past them (a 16-bit operand's k padding) are zero
        const float v = k - 1 < w.row_bytes ? (float)w.pub_raw[(size_t)row * w.row_bytes + (k - 1)] / 255.0f : 0.0f;
        store_operand<PREC>(x0, at, v, w.xplane);
        store_operand<PREC>(x1, at, v, w.xplane);
    }
}

void launch_query_static(const WaveDev& w, int precision, void* x0, void* x1, hipStream_t s) {
    size_t n = (size_t)w.rows * (w.in - 2 * w.pool);
    if (!n) return;
    if (precision == WC_PRECISE)
        hipLaunchKernelGGL(k_query_static<WC_PRECISE>, dim3(grid_for(n)), dim3(BLOCK), 0, s, w, x0, x1);
    else if (precision == WC_F16)
        hipLaunchKernelGGL(k_query_static<WC_F16>, dim3(grid_for(n)), dim3(BLOCK), 0, s, w, x0, x1);
    else if (precision == WC_BF16)
        hipLaunchKernelGGL(k_query_static<WC_BF16>, dim3(grid_for(n)), dim3(BLOCK), 0, s, w, x0, x1);
    else
        hipLaunchKernelGGL(k_query_static<WC_F16X>, dim3(grid_for(n)), dim3(BLOCK), 0, s, w, x0, x1);
}

// ------------------------------------------------------------- the sweep

// One value row of traverser p (engine/src/search.rs:1672-1803).
// Values come from the unit's LDS window when LDSV (slot i at lv[i - vw]),
// else from HBM; results go to both.
template <int MODE, bool LDSV>
__device__ __forceinline__ void backprop_row(const WaveDev& w, int p, BackRec q, float da, float db, float predict,
                                             const float* strat, float* lv, uint32_t vw) {
    float* vals = w.vals;
    // A staged unit keeps its values in LDS; only values read outside the
    // unit (REC_EXPORT) also go to HBM.
    const bool to_hbm = !LDSV || (q.kn & REC_EXPORT);
    auto get = [&](uint32_t i) { return LDSV ? lv[i - vw] : vals[i]; };
    auto put = [&](uint32_t i, float v) {
        if (to_hbm) vals[i] = v;
        if (LDSV) lv[i - vw] = v;
    };
    const uint32_t kind = q.kn >> 30, n = q.kn & REC_N, lo = q.start;
    if (kind == BACK_DRAW) {  // the traverser draws: push values through the outcome row
        const uint32_t cb = q.arg;
        float v = 0.0f;
        for (uint32_t c0 = 0; c0 < n; c0 += ROW_BATCH) {
            const uint32_t m = n - c0 < ROW_BATCH ? n - c0 : ROW_BATCH;
            uint32_t to[ROW_BATCH];
            float pr[ROW_BATCH], cv[ROW_BATCH];
#pragma unroll
            for (uint32_t k = 0; k < ROW_BATCH; k++)
                if (k < m) {
                    to[k] = w.draw_to[lo + c0 + k];
                    pr[k] = w.draw_p[lo + c0 + k];
                }
#pragma unroll
            for (uint32_t k = 0; k < ROW_BATCH; k++)
                if (k < m) cv[k] = get(cb + to[k]);
#pragma unroll
            for (uint32_t k = 0; k < ROW_BATCH; k++)
                if (k < m) v += pr[k] * cv[k];
        }
        put(q.out, v);
        return;
    }
    if (kind == BACK_OPP) {  // opponent decision: sum the children in child order
        const uint32_t c = q.arg;
        const uint32_t* cvb = w.child_vb[p] + lo;
        float v = 0.0f;
        for (uint32_t c0 = 0; c0 < n; c0 += ROW_BATCH) {
            const uint32_t m = n - c0 < ROW_BATCH ? n - c0 : ROW_BATCH;
            uint32_t cb[ROW_BATCH];
            float cv[ROW_BATCH];
#pragma unroll
            for (uint32_t k = 0; k < ROW_BATCH; k++)
                if (k < m) cb[k] = cvb[c0 + k];
#pragma unroll
            for (uint32_t k = 0; k < ROW_BATCH; k++)
                if (k < m) cv[k] = get(cb[k] + c);
#pragma unroll
            for (uint32_t k = 0; k < ROW_BATCH; k++)
                if (k < m) v += cv[k];
        }
        put(q.out, v);
        return;
    }
    // The traverser's own row: base = sum of child value x strategy in action
    // order, then the fused regret matching with DCFR discounting
    // (search.rs:1742-1779): r = old (old > 0 ? da : db) + delta, cur = max(r +
    // predict delta, EPS), normalised by a reciprocal multiply. The sum's
    // discount (sum *= ds) is taken with the accumulation in the reach sweep.
    const float* st = MODE == MODE_VALUE ? strat : w.cur;
    if (n <= ROW_BATCH) {  // one batch: everything stays in registers
        uint32_t lvi[ROW_BATCH];
        float sv[ROW_BATCH], qv[ROW_BATCH], old[ROW_BATCH];
#pragma unroll
        for (uint32_t k = 0; k < ROW_BATCH; k++)
            if (k < n) {
                lvi[k] = w.legal_value[lo + k];
                sv[k] = st[lo + k];
                if (MODE == MODE_REGRET) old[k] = w.regret[lo + k];
            }
#pragma unroll
        for (uint32_t k = 0; k < ROW_BATCH; k++)
            if (k < n) qv[k] = lvi[k] != 0xffffffffu ? get(lvi[k]) : 0.0f;
        float base = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < ROW_BATCH; k++)
            if (k < n && lvi[k] != 0xffffffffu) base += qv[k] * sv[k];
        put(q.out, base);
        if (MODE == MODE_VALUE) return;
        float total = 0.0f, v[ROW_BATCH];
#pragma unroll
        for (uint32_t k = 0; k < ROW_BATCH; k++)
            if (k < n) {
                float delta = 0.0f;
                if (lvi[k] != 0xffffffffu) delta += qv[k];
                delta -= base;
                float r = old[k] * (old[k] > 0.0f ? da : db) + delta;
                w.regret[lo + k] = r;
                v[k] = fmaxf(r + predict * delta, EPSF);
                total += v[k];
            }
        float inv = total > 0.0f ? 1.0f / total : 1.0f;
#pragma unroll
        for (uint32_t k = 0; k < ROW_BATCH; k++)
            if (k < n) w.cur[lo + k] = total > 0.0f ? v[k] * inv : v[k];
        return;
    }
    // Longer rows: the same arithmetic in three batched passes (base; update,
    // with cur holding the unnormalised value; normalisation).
    float base = 0.0f;
    for (uint32_t c0 = 0; c0 < n; c0 += ROW_BATCH) {
        const uint32_t m = n - c0 < ROW_BATCH ? n - c0 : ROW_BATCH;
        uint32_t lvi[ROW_BATCH];
        float sv[ROW_BATCH], qv[ROW_BATCH];
#pragma unroll
        for (uint32_t k = 0; k < ROW_BATCH; k++)
            if (k < m) {
                lvi[k] = w.legal_value[lo + c0 + k];
                sv[k] = st[lo + c0 + k];
            }
#pragma unroll
        for (uint32_t k = 0; k < ROW_BATCH; k++)
            if (k < m) qv[k] = lvi[k] != 0xffffffffu ? get(lvi[k]) : 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < ROW_BATCH; k++)
            if (k < m && lvi[k] != 0xffffffffu) base += qv[k] * sv[k];
    }
    put(q.out, base);
    if (MODE == MODE_VALUE) return;
    float total = 0.0f;
    for (uint32_t c0 = 0; c0 < n; c0 += ROW_BATCH) {
        const uint32_t m = n - c0 < ROW_BATCH ? n - c0 : ROW_BATCH;
        uint32_t lvi[ROW_BATCH];
        float qv[ROW_BATCH], old[ROW_BATCH];
#pragma unroll
        for (uint32_t k = 0; k < ROW_BATCH; k++)
            if (k < m) {
                lvi[k] = w.legal_value[lo + c0 + k];
                old[k] = w.regret[lo + c0 + k];
            }
#pragma unroll
        for (uint32_t k = 0; k < ROW_BATCH; k++)
            if (k < m) qv[k] = lvi[k] != 0xffffffffu ? get(lvi[k]) : 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < ROW_BATCH; k++)
            if (k < m) {
                float delta = 0.0f;
                if (lvi[k] != 0xffffffffu) delta += qv[k];
                delta -= base;
                float r = old[k] * (old[k] > 0.0f ? da : db) + delta;
                w.regret[lo + c0 + k] = r;
                float v = fmaxf(r + predict * delta, EPSF);
                w.cur[lo + c0 + k] = v;
                total += v;
            }
    }
    if (total > 0.0f) {
        const float inv = 1.0f / total;
        for (uint32_t c0 = 0; c0 < n; c0 += ROW_BATCH) {
            const uint32_t m = n - c0 < ROW_BATCH ? n - c0 : ROW_BATCH;
            float cu[ROW_BATCH];
#pragma unroll
            for (uint32_t k = 0; k < ROW_BATCH; k++)
                if (k < m) cu[k] = w.cur[lo + c0 + k];
#pragma unroll
            for (uint32_t k = 0; k < ROW_BATCH; k++)
                if (k < m) w.cur[lo + c0 + k] = cu[k] * inv;
        }
    }
}

// Leaf values and the bottom-up value sweep of one subtree unit for traverser
// p, one workgroup per unit: leaf values first (net value x opponent reach
// mass, engine/src/search.rs:1587-1636), then levels from the deepest up, with
// the fused regret/DCFR update at the traverser's rows.
template <int MODE, bool LDSV>
__global__ __launch_bounds__(BLOCK) void k_sweep(WaveDev w, uint32_t unit0, const float* head_out, uint32_t heads,
                                               int p, float da, float db, float predict) {
    extern __shared__ float lds_vals[];  // the unit's value window of player p (when LDSV)
    const UnitDev u = w.units[unit0 + blockIdx.x];
    const int opp = 1 - p;
    // The player's fields by select, not by index: indexing the record's
    // arrays with the run-time p would place the record in scratch memory.
    const uint32_t vw = p ? u.vwin[1] : u.vwin[0];
    const uint32_t leaf0 = p ? u.leaf0[1] : u.leaf0[0], leaf1 = p ? u.leaf1[1] : u.leaf1[0];
    // The deepest level's bounds and each thread's first record of it are
    // fetched before the leaf phase: they do not depend on its values.
    const BackRec* back = w.back_rec[p];
    const uint32_t* blvl = w.back_lvl[p] + u.lvl0;
    const uint32_t t = threadIdx.x;
    uint32_t l = u.nlevels;
    uint32_t e = l ? blvl[l] : 0, b = l ? blvl[l - 1] : 0;
    BackRec q{};
    if (l && b + t < e) q = back[b + t];
    // Network leaves: one value slot per thread, LEAF_BATCH slots per thread
    // in flight (their records, then the values they name).
    for (uint32_t k0 = leaf0; k0 < leaf1; k0 += LEAF_BATCH * BLOCK) {
        LeafRec lr[LEAF_BATCH];
        float h[LEAF_BATCH], m[LEAF_BATCH];
#pragma unroll
        for (uint32_t j = 0; j < LEAF_BATCH; j++) {
            const uint32_t k = k0 + j * BLOCK + threadIdx.x;
            if (k < leaf1) lr[j] = w.leaf_rec[p][k];
        }
#pragma unroll
        for (uint32_t j = 0; j < LEAF_BATCH; j++)
            if (k0 + j * BLOCK + threadIdx.x < leaf1) {
                h[j] = head_out[lr[j].head];
                m[j] = w.mass[lr[j].mass];
            }
#pragma unroll
        for (uint32_t j = 0; j < LEAF_BATCH; j++)
            if (k0 + j * BLOCK + threadIdx.x < leaf1) {
                const float v = h[j] * m[j];
                if (!LDSV || lr[j].exported) w.vals[lr[j].out] = v;
                if (LDSV) lds_vals[lr[j].out - vw] = v;
            }
    }
    for (uint32_t x = u.term0 + threadIdx.x; x < u.term1; x += blockDim.x) {
        const uint32_t te = w.unit_term[x], k = te & TERM_INDEX;
        const bool to_hbm = !LDSV || (te & term_export(p));
        uint32_t node = w.term_node[k];
        const float* ro = w.reach + w.reach_base[2 * node + opp];
        float m = 0.0f;
        for (uint32_t c = 0; c < w.nc[2 * node + opp]; c++) m += ro[c];
        float uu = (w.node_meta[node] >> 2) == (uint32_t)p ? w.term_util[k] : -w.term_util[k];
        const uint32_t ob = w.vals_base[2 * node + p];
        for (uint32_t c = 0; c < w.nc[2 * node + p]; c++) {
            if (to_hbm) w.vals[ob + c] = uu * m;
            if (LDSV) lds_vals[ob + c - vw] = uu * m;
        }
    }
    __syncthreads();
    // Levels from the deepest up. Each thread's rows form one stream across
    // the levels: the record of its next row (in this level, else its first
    // in the next level up) is fetched while the current row runs.
    while (l-- > 0) {
        const uint32_t lb = b, le = e;
        if (l) {
            e = lb;
            b = blvl[l - 1];
        }
        if (lb + t >= le && l && b + t < e) q = back[b + t];
        for (uint32_t k = lb + t; k < le;) {
            const uint32_t kn = k + blockDim.x;
            BackRec qn{};
            if (kn < le)
                qn = back[kn];
            else if (l && b + t < e)
                qn = back[b + t];
            backprop_row<MODE, LDSV>(w, p, q, da, db, predict, w.snap, lds_vals, vw);
            q = qn;
            k = kn;
        }
        __syncthreads();
    }
}

void launch_sweep(const WaveDev& w, uint32_t unit0, uint32_t n, const float* head_out, uint32_t heads, int traverser,
                  int mode, float da, float db, float predict, hipStream_t s) {
    if (!n) return;
    const size_t lds = (size_t)w.max_vwin * sizeof(float);
    const bool staged = w.unit_lds && lds <= SWEEP_LDS_MAX;
#define WC_SWEEP(M, L)                                                                                          \
    hipLaunchKernelGGL((k_sweep<M, L>), dim3(n), dim3(BLOCK), L ? lds : 0, s, w, unit0, head_out, heads, traverser, \
                       da, db, predict)
    if (mode == MODE_VALUE) {
        if (staged)
            WC_SWEEP(MODE_VALUE, true);
        else
            WC_SWEEP(MODE_VALUE, false);
    } else {
        if (staged)
            WC_SWEEP(MODE_REGRET, true);
        else
            WC_SWEEP(MODE_REGRET, false);
    }
#undef WC_SWEEP
}

// Top-region values at one depth, all trees together: one row per thread.
template <int MODE>
__global__ __launch_bounds__(BLOCK) void k_back_rows(WaveDev w, const BackRec* rows, uint32_t n, int p, float da,
                                                   float db, float predict) {
    uint32_t k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k < n) backprop_row<MODE, false>(w, p, rows[k], da, db, predict, w.snap, nullptr, 0);
}

void launch_back_rows(const WaveDev& w, const BackRec* rows, uint32_t n, int traverser, int mode, float da,
                      float db, float predict, hipStream_t s) {
    if (!n) return;
    if (mode == MODE_VALUE)
        hipLaunchKernelGGL(k_back_rows<MODE_VALUE>, dim3(grid_for(n, TOP_BLOCK)), dim3(TOP_BLOCK), 0, s, w, rows, n,
                           traverser, da, db, predict);
    else
        hipLaunchKernelGGL(k_back_rows<MODE_REGRET>, dim3(grid_for(n, TOP_BLOCK)), dim3(TOP_BLOCK), 0, s, w, rows, n,
                           traverser, da, db, predict);
}

// Two top depths in one launch: each workgroup takes one chunk's rows of the
// deeper depth, then (after a block barrier: the values it wrote are read by
// the same workgroup) that chunk's rows of the shallower depth. Sparing the
// launch boundary saves its fixed cost, about as long as a depth's own rows
// take.
template <int MODE>
__global__ __launch_bounds__(BLOCK) void k_back_pair(WaveDev w, const BackRec* rows, const uint32_t* off,
                                                   uint32_t chunks, int p, float da, float db, float predict) {
    const uint32_t k = blockIdx.x;
    for (uint32_t i = off[k] + threadIdx.x; i < off[k + 1]; i += blockDim.x)
        backprop_row<MODE, false>(w, p, rows[i], da, db, predict, w.snap, nullptr, 0);
    __syncthreads();
    const uint32_t* o = off + chunks + 1;
    for (uint32_t i = o[k] + threadIdx.x; i < o[k + 1]; i += blockDim.x)
        backprop_row<MODE, false>(w, p, rows[i], da, db, predict, w.snap, nullptr, 0);
}

void launch_back_pair(const WaveDev& w, const BackRec* rows, const uint32_t* off, uint32_t chunks, int traverser,
                      int mode, float da, float db, float predict, hipStream_t s) {
    if (!chunks) return;
    if (mode == MODE_VALUE)
        hipLaunchKernelGGL(k_back_pair<MODE_VALUE>, dim3(chunks), dim3(TOP_BLOCK), 0, s, w, rows, off, chunks,
                           traverser, da, db, predict);
    else
        hipLaunchKernelGGL(k_back_pair<MODE_REGRET>, dim3(chunks), dim3(TOP_BLOCK), 0, s, w, rows, off, chunks,
                           traverser, da, db, predict);
}

// Average strategy: sum / row sum, uniform when the sum is not positive, the
// literal current strategy for a player whose sum was never updated
// (engine/src/search.rs:899-938).
__global__ void k_normalize(WaveDev w, int touched0, int touched1) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= w.ndec[0] + w.ndec[1]) return;
    int p;
    AccRec q = decision_row(w, i, &p);
    uint32_t lo = q.lo, hi = q.lo + q.n;
    const bool touched = p ? touched1 : touched0;
    if (q.n <= ROW_BATCH) {  // the row's loads issued together, then the same sum and quotients
        const float* src = touched ? w.sum : w.cur;
        float x[ROW_BATCH];
#pragma unroll
        for (uint32_t k = 0; k < ROW_BATCH; k++)
            if (k < q.n) x[k] = src[lo + k];
        if (!touched) {
#pragma unroll
            for (uint32_t k = 0; k < ROW_BATCH; k++)
                if (k < q.n) w.snap[lo + k] = x[k];
            return;
        }
        float s = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < ROW_BATCH; k++)
            if (k < q.n) s += x[k];
        const float u = 1.0f / (float)(q.n ? q.n : 1);
#pragma unroll
        for (uint32_t k = 0; k < ROW_BATCH; k++)
            if (k < q.n) w.snap[lo + k] = s > 0.0f ? x[k] / s : u;
        return;
    }
    if (!touched) {
        for (uint32_t g = lo; g < hi; g++) w.snap[g] = w.cur[g];
        return;
    }
    float s = 0.0f;
    for (uint32_t g = lo; g < hi; g++) s += w.sum[g];
    float k = (float)(hi > lo ? hi - lo : 1);
    for (uint32_t g = lo; g < hi; g++) w.snap[g] = s > 0.0f ? w.sum[g] / s : 1.0f / k;
}

void launch_normalize(const WaveDev& w, int touched0, int touched1, hipStream_t s) {
    uint32_t n = w.ndec[0] + w.ndec[1];
    if (n) hipLaunchKernelGGL(k_normalize, dim3(grid_for(n)), dim3(BLOCK), 0, s, w, touched0, touched1);
}

// Normalised beliefs at every exit, f16 (the carry store, engine/src/gpu/client.rs:20-111).
// One wavefront per (exit, player), task 2 e + p: its reach slot and carry
// offsets (scalar loads), then 64 configs at a time; the mass is summed in
// config order from the lanes' values.
__global__ __launch_bounds__(64) void k_gather_carry(WaveDev w, const float* reach, int slot) {
    const uint32_t lane = threadIdx.x, t = blockIdx.x;
    if (t >= 2 * w.nexit) return;  // wave-uniform
    const float* r = reach + w.exit_reach[t];
    const uint32_t cb = w.exit_coff[t], n = w.exit_coff[t + 1] - cb;
    const float v0 = lane < n ? r[lane] : 0.0f;
    float tot = 0.0f;
    for (uint32_t c0 = 0; c0 < n; c0 += 64) {
        const float x = c0 ? (c0 + lane < n ? r[c0 + lane] : 0.0f) : v0;
        tot = lane_sum_in_order(tot, x, n - c0 < 64 ? n - c0 : 64);
    }
    float scale, flat;
    if (tot > SMOOTHF) {
        scale = 1.0f / tot;
        flat = 0.0f;
    } else {
        scale = 0.0f;
        flat = 1.0f / (float)(n > 0 ? n : 1);
    }
    uint16_t* dst = w.carry + (size_t)slot * w.snapshot_configs + cb;
    for (uint32_t c = lane; c < n; c += 64) dst[c] = f32_to_f16_rn((c < 64 ? v0 : r[c]) * scale + flat);
}

void launch_gather_carry(const WaveDev& w, const float* reach, int slot, hipStream_t s) {
    const size_t tasks = (size_t)w.nexit * 2;
    // one wavefront per task, one per workgroup: a wavefront that finishes
    // frees its slot at once
    if (tasks) hipLaunchKernelGGL(k_gather_carry, dim3((uint32_t)tasks), dim3(64), 0, s, w, reach, slot);
}

__global__ void k_collect_root(WaveDev w, int root, int p) {
    const TreeDev t = w.trees[blockIdx.x];
    if (root >= (int)t.nroots) return;
    uint32_t n = p ? t.n1 : t.n0;
    float* dst = w.root_values + t.root_value0 + (size_t)root * (t.n0 + t.n1) + (p ? t.n0 : 0);
    const float* src = w.vals + w.vals_base[2 * t.node0 + p];
    for (uint32_t c = threadIdx.x; c < n; c += blockDim.x) dst[c] = src[c];
}

void launch_collect_root(const WaveDev& w, int root, int player, hipStream_t s) {
    hipLaunchKernelGGL(k_collect_root, dim3(w.ntrees), dim3(BLOCK), 0, s, w, root, player);
}

// ------------------------------------------------------- leaf MLP (exact)

// y[r, j] = relu(sum_p x[r, p] W[p, j] + b[j]): per output, from zero over
// ascending inputs, zero inputs skipped (engine/src/net.rs:102-122).
__global__ void k_dense_exact(const float* X, uint32_t K, const float* W, const float* b, uint32_t N, float* Y,
                              uint32_t rows) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows * N) return;
    uint32_t r = (uint32_t)(i / N), j = (uint32_t)(i % N);
    const float* x = X + (size_t)r * K;
    float acc = 0.0f;
    for (uint32_t p = 0; p < K; p++) {
        float a = x[p];
        if (a == 0.0f) continue;
        acc += a * W[(size_t)p * N + j];
    }
    float v = acc + b[j];
    Y[i] = v > 0.0f ? v : 0.0f;
}

void launch_dense_exact(const float* X, uint32_t K, const float* W, const float* b, uint32_t N, float* Y,
                        uint32_t rows, hipStream_t s) {
    size_t n = (size_t)rows * N;
    if (n) hipLaunchKernelGGL(k_dense_exact, dim3(grid_for(n)), dim3(BLOCK), 0, s, X, K, W, b, N, Y, rows);
}

// out[r, k] = b[k] + sum_j Wh[k, j] H[r, j] (Net::values, engine/src/net.rs:844-853).
__global__ void k_head_exact(const float* H, uint32_t hidden, const float* Wh, const float* bh, uint32_t heads,
                             float* out, uint32_t rows) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows * heads) return;
    uint32_t r = (uint32_t)(i / heads), k = (uint32_t)(i % heads);
    const float* h = H + (size_t)r * hidden;
    const float* wr = Wh + (size_t)k * hidden;
    float v = bh[k];
    for (uint32_t j = 0; j < hidden; j++) v += wr[j] * h[j];
    out[i] = v;
}

void launch_head_exact(const float* H, uint32_t hidden, const float* Wh, const float* bh, uint32_t heads,
                       float* out, uint32_t rows, hipStream_t s) {
    size_t n = (size_t)rows * heads;
    if (n) hipLaunchKernelGGL(k_head_exact, dim3(grid_for(n)), dim3(BLOCK), 0, s, H, hidden, Wh, bh, heads, out, rows);
}

// ------------------------------------------------------- leaf MLP (MFMA)


template <int PREC>
__global__ void k_to16(const float* src, uint16_t* dst, uint32_t rows, uint32_t K, int transposed, size_t plane) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows * K) return;
    uint32_t r = (uint32_t)(i / K), k = (uint32_t)(i % K);
    float v = transposed ? src[(size_t)k * rows + r] : src[i];
    store_operand<PREC>(dst, frag_off(r, k, K), v, plane);
}

void launch_to16(int precision, const float* src, void* dst, uint32_t rows, uint32_t K, bool transposed,
                 hipStream_t s) {
    size_t n = (size_t)rows * K;
    if (!n) return;
    const size_t plane = (size_t)gemm_rows(rows) * K;  // compensated f16: the lo plane follows the hi plane
#define WC_TO16(P)                                                                                              \
    hipLaunchKernelGGL(k_to16<P>, dim3(grid_for(n)), dim3(BLOCK), 0, s, src, (uint16_t*)dst, rows, K, (int)transposed, \
                       plane)
    if (precision == WC_F16)
        WC_TO16(WC_F16);
    else if (precision == WC_BF16)
        WC_TO16(WC_BF16);
    else
        WC_TO16(WC_F16X);
#undef WC_TO16
}

// 16x16x32 MFMA step over a 64 x 64 wave tile: acc[a][b] += A(a) B(b)^T.
template <int PREC>
__device__ __forceinline__ void mfma_step(float4v (&acc)[4][4], const uint4 (&af)[4], const uint4 (&bf)[4]) {
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            if (PREC == WC_F16)
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, af[a]),
                                                                   __builtin_bit_cast(half8, bf[b]), acc[a][b], 0, 0,
                                                                   0);
            else
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[a]),
                                                                    __builtin_bit_cast(bf16x8, bf[b]), acc[a][b], 0,
                                                                    0, 0);
        }
}

// One 16x16x32 MFMA: acc += A(a) B(b)^T.
template <int PREC>
__device__ __forceinline__ float4v mfma_step16(const uint4& a, const uint4& b, const float4v& acc) {
    if (PREC == WC_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), acc,
                                                      0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       acc, 0, 0, 0);
}

// Fragment-major MFMA GEMM. A 128 x 128 output tile per workgroup, 64 x 64 per
// wavefront (4 x 4 16x16x32 tiles). Both operands are fragment-major, so each
// of a step's 8 fragment loads is one contiguous 1 KB read. Two fragment sets
// ping-pong: while one step's 16 MFMAs run, the next step's loads are in
// flight (the loop is unrolled by two so the compiler waits only for the set
// it is about to use). The epilogue adds the bias, applies ReLU and stores
// either the next layer's 16-bit fragment-major operand or row-major f32.
template <int PREC, bool RELU, bool OUT16>
__global__ __launch_bounds__(256) void k_gemm(const uint16_t* __restrict__ X, uint32_t K,
                                              const uint16_t* __restrict__ Wt, const float* __restrict__ bias,
                                              uint32_t N, void* __restrict__ Y, uint32_t M,
                                              const uint32_t* __restrict__ tile_n) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (tile_n && blockIdx.y * GEMM_ROWS >= tile_n[blockIdx.x]) return;  // block-uniform
    const uint32_t m0 = blockIdx.x * GEMM_ROWS + (wave & 1) * 64;
    const uint32_t n0 = blockIdx.y * GEMM_ROWS + (wave >> 1) * 64;
    const uint32_t ks = K >> 5;  // 32-wide k steps
    float4v acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    // Fragment (block, step) lives at ((block * ks + step) * 64 + lane) * 8.
    const uint16_t* ap = X + ((size_t)(m0 >> 4) * ks * 64 + lane) * 8;
    const uint16_t* bp = Wt + ((size_t)(n0 >> 4) * ks * 64 + lane) * 8;
    const size_t blk = (size_t)ks * 64 * 8;  // halves between consecutive 16-row blocks
    uint4 af[4], bf[4], an[4], bn[4];
    auto load = [&](uint4 (&fa)[4], uint4 (&fb)[4], uint32_t step) {
#pragma unroll
        for (int a = 0; a < 4; a++) fa[a] = *(const uint4*)(ap + a * blk + (size_t)step * 512);
#pragma unroll
        for (int b = 0; b < 4; b++) fb[b] = *(const uint4*)(bp + b * blk + (size_t)step * 512);
    };
    load(af, bf, 0);
    uint32_t st = 0;
    for (; st + 2 <= ks; st += 2) {
        load(an, bn, st + 1);
        __builtin_amdgcn_sched_barrier(0);
        mfma_step<PREC>(acc, af, bf);
        __builtin_amdgcn_sched_barrier(0);
        load(af, bf, st + 2 < ks ? st + 2 : st + 1);  // past the end: re-read a valid step, unused
        __builtin_amdgcn_sched_barrier(0);
        mfma_step<PREC>(acc, an, bn);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (st < ks) mfma_step<PREC>(acc, af, bf);  // odd step count: af holds the last step
    const uint32_t li = lane & 15, kb = lane >> 4;
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            uint32_t col = n0 + b * 16 + li;
            if (col >= N) continue;
            float bv = bias[col];
#pragma unroll
            for (int v = 0; v < 4; v++) {
                uint32_t row = m0 + a * 16 + kb * 4 + v;
                if (row >= M) continue;
                float y = acc[a][b][v] + bv;
                if (RELU) y = y > 0.0f ? y : 0.0f;
                if (OUT16)
                    ((uint16_t*)Y)[frag_off(row, col, N)] = PREC == WC_F16 ? f32_to_f16_rn(y) : f32_to_bf16_rn(y);
                else
                    ((float*)Y)[(size_t)row * N + col] = y;
            }
        }
}

// Compensated f16 GEMM: each operand is an f16 pair hi + lo in two planes
// (xplane / wplane elements apart), each product is taken as lo hi + hi lo +
// hi hi (f32 accumulation), the output likewise split when 16-bit. Tiles as
// k_gemm, without its load pipelining: this is the accuracy mode.
template <bool RELU, bool OUT16>
__global__ __launch_bounds__(256) void k_gemm_x(const uint16_t* __restrict__ X, uint32_t K,
                                                const uint16_t* __restrict__ Wt, const float* __restrict__ bias,
                                                uint32_t N, void* __restrict__ Y, uint32_t M,
                                                const uint32_t* __restrict__ tile_n, size_t xplane, size_t wplane,
                                                size_t yplane) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (tile_n && blockIdx.y * GEMM_ROWS >= tile_n[blockIdx.x]) return;  // block-uniform
    const uint32_t m0 = blockIdx.x * GEMM_ROWS + (wave & 1) * 64;
    const uint32_t n0 = blockIdx.y * GEMM_ROWS + (wave >> 1) * 64;
    const uint32_t ks = K >> 5;
    float4v acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    const uint16_t* ap = X + ((size_t)(m0 >> 4) * ks * 64 + lane) * 8;
    const uint16_t* bp = Wt + ((size_t)(n0 >> 4) * ks * 64 + lane) * 8;
    const size_t blk = (size_t)ks * 64 * 8;
    for (uint32_t st = 0; st < ks; st++) {
        uint4 ah[4], al[4], bh[4], bl[4];
#pragma unroll
        for (int a = 0; a < 4; a++) {
            ah[a] = *(const uint4*)(ap + a * blk + (size_t)st * 512);
            al[a] = *(const uint4*)(ap + xplane + a * blk + (size_t)st * 512);
        }
#pragma unroll
        for (int b = 0; b < 4; b++) {
            bh[b] = *(const uint4*)(bp + b * blk + (size_t)st * 512);
            bl[b] = *(const uint4*)(bp + wplane + b * blk + (size_t)st * 512);
        }
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                acc[a][b] = mfma_step16<WC_F16>(al[a], bh[b], acc[a][b]);
                acc[a][b] = mfma_step16<WC_F16>(ah[a], bl[b], acc[a][b]);
                acc[a][b] = mfma_step16<WC_F16>(ah[a], bh[b], acc[a][b]);
            }
    }
    const uint32_t li = lane & 15, kb = lane >> 4;
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            uint32_t col = n0 + b * 16 + li;
            if (col >= N) continue;
            float bv = bias[col];
#pragma unroll
            for (int v = 0; v < 4; v++) {
                uint32_t row = m0 + a * 16 + kb * 4 + v;
                if (row >= M) continue;
                float y = acc[a][b][v] + bv;
                if (RELU) y = y > 0.0f ? y : 0.0f;
                if (OUT16)
                    store_operand<WC_F16X>(Y, frag_off(row, col, N), y, yplane);
                else
                    ((float*)Y)[(size_t)row * N + col] = y;
            }
        }
}

void launch_gemm16(int precision, const void* X, uint32_t K, const void* Wt, const float* b, uint32_t N, void* Y,
                   uint32_t M, bool relu, bool out16, hipStream_t s, const uint32_t* tile_n) {
    if (M == 0 || N == 0) return;
    dim3 grid(gemm_rows(M) / GEMM_ROWS, gemm_rows(N) / GEMM_ROWS);
    if (precision == WC_F16X) {
        const size_t xp = (size_t)gemm_rows(M) * K, wp = (size_t)gemm_rows(N) * K, yp = (size_t)gemm_rows(M) * N;
        const uint16_t* x = (const uint16_t*)X;
        const uint16_t* wt = (const uint16_t*)Wt;
#define WC_GEMMX(R, O) \
    hipLaunchKernelGGL((k_gemm_x<R, O>), grid, dim3(256), 0, s, x, K, wt, b, N, Y, M, tile_n, xp, wp, yp)
        if (relu && out16)
            WC_GEMMX(true, true);
        else if (relu)
            WC_GEMMX(true, false);
        else if (out16)
            WC_GEMMX(false, true);
        else
            WC_GEMMX(false, false);
#undef WC_GEMMX
        return;
    }
    const uint16_t* x = (const uint16_t*)X;
    const uint16_t* wt = (const uint16_t*)Wt;
#define WC_GEMM(P, R, O) hipLaunchKernelGGL((k_gemm<P, R, O>), grid, dim3(256), 0, s, x, K, wt, b, N, Y, M, tile_n)
    if (precision == WC_F16) {
        if (relu && out16)
            WC_GEMM(WC_F16, true, true);
        else if (relu)
            WC_GEMM(WC_F16, true, false);
        else if (out16)
            WC_GEMM(WC_F16, false, true);
        else
            WC_GEMM(WC_F16, false, false);
    } else {
        if (relu && out16)
            WC_GEMM(WC_BF16, true, true);
        else if (relu)
            WC_GEMM(WC_BF16, true, false);
        else if (out16)
            WC_GEMM(WC_BF16, false, true);
        else
            WC_GEMM(WC_BF16, false, false);
    }
#undef WC_GEMM
}


// ------------------------------------------------------------ two-tower net
//
// The two-tower leaf value of row r and infostate c is <f(c), h(r)> + b_read
// with h the public tower's output for the row's query and f(c) the private
// tower's output for the infostate's features times the readout weight
// (elementwise). f is formed once per wave and weight bank.

// F[c][k] = Hp[c][k] * wread[k]; the 16-bit nets round the product to the
// operand type (Hp fragment-major with K = width, F row-major), float32 keeps it.
template <int PREC>
__global__ void k_tower_f(const void* __restrict__ Hp, uint32_t width, uint32_t ncfg, const float* __restrict__ wread,
                          void* __restrict__ F) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)ncfg * width) return;
    const uint32_t c = (uint32_t)(i / width), k = (uint32_t)(i % width);
    if (PREC == WC_PRECISE) {
        ((float*)F)[i] = ((const float*)Hp)[i] * wread[k];
        return;
    }
    const uint16_t hv = ((const uint16_t*)Hp)[frag_off(c, k, width)];
    float h;
    if (PREC == WC_F16)
        h = (float)__builtin_bit_cast(_Float16, hv);
    else
        h = __uint_as_float((uint32_t)hv << 16);
    const float f = h * wread[k];
    ((uint16_t*)F)[i] = PREC == WC_F16 ? f32_to_f16_rn(f) : f32_to_bf16_rn(f);
}

void launch_tower_f(int precision, const void* Hp, uint32_t width, uint32_t ncfg, const float* wread, void* F,
                    hipStream_t s) {
    const size_t n = (size_t)ncfg * width;
    if (!n) return;
    if (precision == WC_PRECISE)
        hipLaunchKernelGGL(k_tower_f<WC_PRECISE>, dim3(grid_for(n)), dim3(BLOCK), 0, s, Hp, width, ncfg, wread, F);
    else if (precision == WC_F16)
        hipLaunchKernelGGL(k_tower_f<WC_F16>, dim3(grid_for(n)), dim3(BLOCK), 0, s, Hp, width, ncfg, wread, F);
    else
        hipLaunchKernelGGL(k_tower_f<WC_BF16>, dim3(grid_for(n)), dim3(BLOCK), 0, s, Hp, width, ncfg, wread, F);
}

// Float32 readout: one workgroup per readout block of player p, one thread
// per (row, config) entry, the sum from b_read in k order as the CPU net forms
// it (engine/src/net.rs:844-853 pattern: bias, then += f[k] h[k]).
__global__ __launch_bounds__(BLOCK) void k_tower_dense_exact(WaveDev w, int p, const float* __restrict__ H,
                                                           uint32_t width, const float* __restrict__ F, float bread,
                                                           float* __restrict__ tv) {
    const TowerBlock b = w.tower_blk[p][blockIdx.x];
    const uint32_t nc = b.chi - b.clo, n = (b.r1 - b.r0) * nc;
    for (uint32_t x = threadIdx.x; x < n; x += blockDim.x) {
        const uint32_t r = b.r0 + x / nc, c = b.clo + x % nc;
        const float* h = H + (size_t)r * width;
        const float* f = F + (size_t)c * width;
        float acc = bread;
        for (uint32_t j = 0; j < width; j++) acc += f[j] * h[j];
        tv[b.dbase + x] = acc;
    }
}

// 16-bit readout on MFMA: one wavefront per 64 x 64 tile of a readout block,
// 4 x 4 16x16x32 tiles over the width. A = 16-row blocks of the public-tower
// output H (whole fragments: tile rows are 16-aligned; blocks past the tree's
// last row re-read its last block), B = 16 configs' F rows per tile (configs
// past the block re-read its last config). Entries outside the block are not
// stored.
template <int PREC>
__global__ __launch_bounds__(BLOCK) void k_tower_dense(WaveDev w, int p, const uint16_t* __restrict__ H,
                                                     uint32_t width, const uint16_t* __restrict__ F, float bread,
                                                     float* __restrict__ tv) {
    const uint32_t k = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    if (k >= w.ntower_unit[p]) return;  // wave-uniform
    const uint32_t lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    const TowerUnit u = w.tower_unit[p][k];
    const TowerBlock b = w.tower_blk[p][u.block];
    const uint32_t ks = width >> 5, last_blk = (b.r1 - 1) & ~15u;
    const uint16_t* ap[4];
    const uint16_t* bp[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t rb = min(u.row + 16 * t, last_blk);
        ap[t] = H + ((size_t)(rb >> 4) * ks * 64 + lane) * 8;  // fragment (block, step) at + step * 512
        const uint32_t c = min(u.cfg + 16 * t + i, b.chi - 1);
        bp[t] = F + (size_t)c * width + 8 * q;  // this lane's 8 columns of step s at + 32 s
    }
    float4v acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[a][c] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    uint4 fa[4], fb[4], na[4], nb[4];
    auto load = [&](uint4 (&xa)[4], uint4 (&xb)[4], uint32_t s) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            xa[t] = *(const uint4*)(ap[t] + (size_t)s * 512);
            xb[t] = *(const uint4*)(bp[t] + 32 * s);
        }
    };
    auto step = [&](const uint4 (&xa)[4], const uint4 (&xb)[4]) {
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int c = 0; c < 4; c++) acc[a][c] = mfma_step16<PREC>(xa[a], xb[c], acc[a][c]);
    };
    load(fa, fb, 0);
    uint32_t s = 0;
    for (; s + 2 <= ks; s += 2) {
        load(na, nb, s + 1);
        __builtin_amdgcn_sched_barrier(0);
        step(fa, fb);
        __builtin_amdgcn_sched_barrier(0);
        load(fa, fb, s + 2 < ks ? s + 2 : s + 1);  // past the end: re-read a valid step, unused
        __builtin_amdgcn_sched_barrier(0);
        step(na, nb);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (s < ks) step(fa, fb);
    const uint32_t nc = b.chi - b.clo;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t cfg = u.cfg + 16 * c + i;
        if (cfg >= b.chi) continue;
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const uint32_t r = u.row + 16 * a + 4 * q + v;
                if (r >= b.r0 && r < b.r1) tv[b.dbase + (r - b.r0) * nc + (cfg - b.clo)] = acc[a][c][v] + bread;
            }
    }
}

void launch_tower_head(const WaveDev& w, int player, int precision, const void* H, uint32_t width, const void* F,
                       float bread, float* tv, hipStream_t s) {
    if (precision == WC_PRECISE) {
        if (w.ntower_blk[player])
            hipLaunchKernelGGL(k_tower_dense_exact, dim3(w.ntower_blk[player]), dim3(BLOCK), 0, s, w, player,
                               (const float*)H, width, (const float*)F, bread, tv);
        return;
    }
    if (!w.ntower_unit[player]) return;
    dim3 g(grid_for((size_t)w.ntower_unit[player] * 64));
    if (precision == WC_F16)
        hipLaunchKernelGGL(k_tower_dense<WC_F16>, g, dim3(BLOCK), 0, s, w, player, (const uint16_t*)H, width,
                           (const uint16_t*)F, bread, tv);
    else
        hipLaunchKernelGGL(k_tower_dense<WC_BF16>, g, dim3(BLOCK), 0, s, w, player, (const uint16_t*)H, width,
                           (const uint16_t*)F, bread, tv);
}

// ------------------------------------------------------- fused leaf network
//
// One launch runs the whole MLP, one pass of up to eight 16-row blocks per
// workgroup (the passes come from plan_chain): the pass's input operand is
// staged into LDS once, every trunk layer reads its input from LDS and writes
// its bias + ReLU output back over it (fragment-major, 16-bit: the next
// layer's operand), and the head writes row-major f32. Only the pass's input,
// the weights (shared by every pass, L2-resident) and the head outputs touch
// HBM.
//
// Products are computed transposed, D = W X^T: the weight fragment is the
// MFMA's A operand and the activation fragment its B operand, so lane l holds
// four consecutive output features 4 (l / 16) .. + 3 of one row l % 16 --
// one 8-byte LDS store per 16x16 tile in the next layer's fragment layout.
// Every output is the same f32 sum over the same 32-wide k steps, in the same
// order, as the layer-by-layer k_gemm, except in the partial-start mode, whose
// first layer adds the pooled columns' steps to the precomputed sum over the
// fixed columns (the same products, summed in another order).

constexpr uint32_t CHAIN_LDS_HALVES = GEMM_ROWS * CHAIN_MAX_WIDTH;

bool chain_fits(uint32_t in, uint32_t hidden, uint32_t layers) {
    return in % 32 == 0 && in <= CHAIN_MAX_WIDTH && hidden % 32 == 0 &&
           hidden <= CHAIN_WAVES * CHAIN_NB * 16 && layers >= 1 && layers <= CHAIN_MAX_LAYERS;
}

template <int PREC>
__device__ __forceinline__ float4v mfma16(const uint4& a, const uint4& b, const float4v& c) {
    if (PREC == WC_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c,
                                                      0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
}

// acc[a][b] (a < RB, b < NB) = sum over ks steps of W(block b) X(rows 16a..)^T.
// xs: the LDS operand at this lane's fragment slot (fragment (a, s) at xs + (a
// ks + s) 512); wp: the wavefront's first weight block at this lane's slot
// (block b at wp + b wstride). Weight fragments (from L2) are fetched two
// steps ahead through a ring of four sets, activation fragments (from LDS) one
// step ahead through two; the loop is unrolled by four so every set keeps a
// fixed role. Loads past the last step re-read the last step (in bounds,
// unused).
template <int PREC, int NB, int RB, bool ZERO = true>
__device__ __forceinline__ void chain_kloop(float4v (&acc)[8][CHAIN_NB], const uint16_t* xs, uint32_t ks,
                                            const uint16_t* __restrict__ wp, size_t wstride) {
    if (ZERO) {  // else acc arrives holding the product's starting value
#pragma unroll
        for (int a = 0; a < RB; a++)
#pragma unroll
            for (int b = 0; b < NB; b++) acc[a][b] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    }
    uint4 xa[RB], xb[RB], w0[NB], w1[NB], w2[NB], w3[NB];
    auto ldw = [&](uint4 (&fw)[NB], uint32_t s) {
        s = s < ks ? s : ks - 1;
#pragma unroll
        for (int b = 0; b < NB; b++) fw[b] = *(const uint4*)(wp + b * wstride + (size_t)s * 512);
    };
    auto ldx = [&](uint4 (&fx)[RB], uint32_t s) {
        s = s < ks ? s : ks - 1;
#pragma unroll
        for (int a = 0; a < RB; a++) fx[a] = *(const uint4*)(xs + ((size_t)a * ks + s) * 512);
    };
    auto step = [&](const uint4 (&fx)[RB], const uint4 (&fw)[NB]) {
#pragma unroll
        for (int a = 0; a < RB; a++)
#pragma unroll
            for (int b = 0; b < NB; b++) acc[a][b] = mfma16<PREC>(fw[b], fx[a], acc[a][b]);
    };
    ldw(w0, 0);
    ldw(w1, 1);
    ldx(xa, 0);
    uint32_t s = 0;
    for (; s + 4 <= ks; s += 4) {
        ldw(w2, s + 2);
        ldx(xb, s + 1);
        __builtin_amdgcn_sched_barrier(0);
        step(xa, w0);
        __builtin_amdgcn_sched_barrier(0);
        ldw(w3, s + 3);
        ldx(xa, s + 2);
        __builtin_amdgcn_sched_barrier(0);
        step(xb, w1);
        __builtin_amdgcn_sched_barrier(0);
        ldw(w0, s + 4);
        ldx(xb, s + 3);
        __builtin_amdgcn_sched_barrier(0);
        step(xa, w2);
        __builtin_amdgcn_sched_barrier(0);
        ldw(w1, s + 5);
        ldx(xa, s + 4);
        __builtin_amdgcn_sched_barrier(0);
        step(xb, w3);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (; s < ks; s++) {  // K not a multiple of 128: the last steps one at a time
        ldw(w0, s);
        ldx(xa, s);
        step(xa, w0);
    }
}

// The wavefront's share of one layer: 16-feature blocks blk0, blk0 + bstep,
// ... (nb of them, 0..CHAIN_NB) of RB row blocks from the LDS operand at lds,
// which holds ks k steps per row block: weight steps w0 .. w0 + ks of
// matrices with kw steps (all of them when ks == kw).
template <int PREC, int RB, bool ZERO = true>
__device__ __forceinline__ void chain_blocks(float4v (&acc)[8][CHAIN_NB], uint32_t nb, const uint16_t* lds,
                                             uint32_t ks, const uint16_t* __restrict__ W, uint32_t blk0,
                                             uint32_t bstep, uint32_t lane, uint32_t kw = 0, uint32_t w0 = 0) {
    if (!kw) kw = ks;
    const uint16_t* xs = lds + lane * 8;
    const uint16_t* wp = W + ((size_t)blk0 * kw * 64 + lane) * 8 + (size_t)w0 * 512;
    const size_t wstride = (size_t)bstep * kw * 512;
    static_assert(CHAIN_NB == 3, "dispatch below covers 1..3 blocks");
    if (nb == 1)
        chain_kloop<PREC, 1, RB, ZERO>(acc, xs, ks, wp, wstride);
    else if (nb == 2)
        chain_kloop<PREC, 2, RB, ZERO>(acc, xs, ks, wp, wstride);
    else if (nb == 3)
        chain_kloop<PREC, 3, RB, ZERO>(acc, xs, ks, wp, wstride);
}

// One (row block, feature block) tile of a first-layer partial product: the
// lane's four accumulator values.
__device__ __forceinline__ size_t part_tile(uint32_t rb, uint32_t fb, uint32_t hblk, uint32_t lane) {
    return ((size_t)rb * hblk + fb) * 256 + lane * 4;
}

__device__ __forceinline__ uint32_t pack16(uint16_t lo, uint16_t hi) { return (uint32_t)lo | ((uint32_t)hi << 16); }

// The head over the pass's RB row blocks (LDS operand, K = hidden): rg row
// groups of RBW blocks each (RBW = ceil(RB / rg); a group's blocks past RB are
// computed from in-bounds LDS and not stored) by 8 / rg column groups; the
// wavefront's column blocks are c, c + 8 / rg, ... in steps of CHAIN_NB of
// them. Row-major f32 out.
template <int PREC, int RB, int RBW>
__device__ __forceinline__ void chain_head(const ChainNet& net, uint32_t rows, float* __restrict__ out,
                                           const ChainPass* __restrict__ ps, uint32_t nt, uint32_t rg,
                                           const uint16_t* lds, uint32_t lane, uint32_t wave) {
    const uint32_t q = lane >> 4, r = lane & 15, ksn = net.hidden >> 5;
    const uint32_t cg = CHAIN_WAVES / rg, g = wave / cg, c = wave % cg, a0 = g * RBW;
    const uint16_t* wh = net.w[net.layers];
    const float* bh = net.b[net.layers];
    const uint16_t* xs = lds + (size_t)a0 * ksn * 512;
    float4v acc[8][CHAIN_NB];
    for (uint32_t c0 = 0; c0 < nt; c0 += cg * CHAIN_NB) {
        const uint32_t end = min(nt, c0 + cg * CHAIN_NB);
        const uint32_t hb = end > c0 + c ? (end - c0 - c + cg - 1) / cg : 0;
        chain_blocks<PREC, RBW>(acc, hb, xs, ksn, wh, c0 + c, cg, lane);
#pragma unroll
        for (int b = 0; b < CHAIN_NB; b++) {
            if ((uint32_t)b >= hb) break;
            const uint32_t n = (c0 + c + cg * b) * 16 + 4 * q;
            float bv[4];
#pragma unroll
            for (int v = 0; v < 4; v++) bv[v] = n + v < net.heads ? bh[n + v] : 0.0f;
            // The row indices are recomputed per column step from an opaque
            // copy of the lane's row: kept live across the loop, they spill.
            uint32_t rr = r;
            asm volatile("" : "+v"(rr));
#pragma unroll
            for (int a = 0; a < RBW; a++) {
                if (a0 + a >= RB) break;
                const uint32_t m = ps->rb[a0 + a] * 16 + rr;
                if (m >= rows) continue;
                float* o = out + (size_t)m * net.heads + n;
#pragma unroll
                for (int v = 0; v < 4; v++)
                    if (n + v < net.heads) o[v] = acc[a][b][v] + bv[v];
            }
        }
    }
}

// One pass of the whole network over the pass's RB 16-row blocks (RB <= 8):
// stage their input operand in LDS, run the trunk layers in place, write the
// head.
// Modes: the whole net; the whole net with the first layer started from a
// precomputed partial product; the partial product alone.
constexpr int CHAIN_FULL = 0, CHAIN_PART = 1, CHAIN_STATIC = 2;
template <int PREC, int RB, int MODE>
__device__ __forceinline__ void chain_pass(const ChainNet& net, const uint16_t* __restrict__ X, uint32_t rows,
                                           float* __restrict__ out, const ChainPass* __restrict__ ps,
                                           uint16_t* lds, uint32_t lane, uint32_t wave) {
    const uint32_t q = lane >> 4, r = lane & 15;
    const uint32_t hblk = net.hidden >> 4, ksn = net.hidden >> 5;
    const uint32_t nb = hblk > wave ? (hblk - wave + CHAIN_WAVES - 1) / CHAIN_WAVES : 0;
    const uint32_t nt = (min(ps->cols, net.heads) + 15) >> 4;  // head column blocks the pass needs
    // The first layer's k steps [s0, s0 + sn) of each row block (a contiguous
    // run of 1 KB steps in X), packed in LDS in pass order: all of them, the
    // first dsteps (partial start) or the rest (the static product).
    const uint32_t ks0 = net.in >> 5;
    constexpr bool part = MODE == CHAIN_PART;
    const uint32_t s0 = MODE == CHAIN_STATIC ? net.dsteps : 0;
    const uint32_t sn = MODE == CHAIN_STATIC ? ks0 - net.dsteps : part ? net.dsteps : ks0;
    const uint32_t per = sn * 64;  // uint4 per row block
#pragma unroll
    for (int a = 0; a < RB; a++) {
        const uint4* src = (const uint4*)(X + ((size_t)ps->rb[a] * ks0 + s0) * 512);
        uint4* dst = (uint4*)lds + a * per;
        for (uint32_t i = threadIdx.x; i < per; i += CHAIN_WAVES * 64) dst[i] = src[i];
    }
    float4v acc[8][CHAIN_NB];
    if constexpr (part) {  // the first layer starts from the precomputed product of its other columns
#pragma unroll
        for (int a = 0; a < RB; a++)
#pragma unroll
            for (int b = 0; b < CHAIN_NB; b++)
                if ((uint32_t)b < nb)
                    acc[a][b] = *(const float4v*)(net.part + part_tile(ps->rb[a], wave + CHAIN_WAVES * b, hblk, lane));
    }
    __syncthreads();
    if constexpr (MODE == CHAIN_STATIC) {
        chain_blocks<PREC, RB>(acc, nb, lds, sn, net.w[0], wave, CHAIN_WAVES, lane, ks0, s0);
#pragma unroll
        for (int a = 0; a < RB; a++)
#pragma unroll
            for (int b = 0; b < CHAIN_NB; b++)
                if ((uint32_t)b < nb)
                    *(float4v*)(out + part_tile(ps->rb[a], wave + CHAIN_WAVES * b, hblk, lane)) = acc[a][b];
        return;
    }
    uint32_t K = net.in;
    for (uint32_t l = 0; l < net.layers; l++) {
        if constexpr (part) {  // the later layers start from zero
            if (l > 0)
#pragma unroll
                for (int a = 0; a < RB; a++)
#pragma unroll
                    for (int b = 0; b < CHAIN_NB; b++) acc[a][b] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
        }
        // (sn = ks0 without the partial start: the same call for every layer)
        chain_blocks<PREC, RB, !part>(acc, nb, lds, l ? K >> 5 : sn, net.w[l], wave, CHAIN_WAVES, lane,
                                      l ? 0 : ks0, 0);
        __syncthreads();  // the layer input is dead from here on
        // bias + ReLU, stored over the input as the next operand (K = hidden)
        const float* bias = net.b[l];
#pragma unroll
        for (int b = 0; b < CHAIN_NB; b++) {
            if ((uint32_t)b >= nb) break;
            const uint32_t n = (wave + CHAIN_WAVES * b) * 16 + 4 * q;
            const float b0 = bias[n], b1 = bias[n + 1], b2 = bias[n + 2], b3 = bias[n + 3];
            const size_t col = (size_t)(n >> 5) * 64 + r + ((n & 31) >> 3) * 16;
#pragma unroll
            for (int a = 0; a < RB; a++) {
                float y0 = acc[a][b][0] + b0, y1 = acc[a][b][1] + b1, y2 = acc[a][b][2] + b2,
                      y3 = acc[a][b][3] + b3;
                y0 = y0 > 0.0f ? y0 : 0.0f;
                y1 = y1 > 0.0f ? y1 : 0.0f;
                y2 = y2 > 0.0f ? y2 : 0.0f;
                y3 = y3 > 0.0f ? y3 : 0.0f;
                uint2 v;
                if (PREC == WC_F16) {
                    v.x = pack16(f32_to_f16_rn(y0), f32_to_f16_rn(y1));
                    v.y = pack16(f32_to_f16_rn(y2), f32_to_f16_rn(y3));
                } else {
                    v.x = pack16(f32_to_bf16_rn(y0), f32_to_bf16_rn(y1));
                    v.y = pack16(f32_to_bf16_rn(y2), f32_to_bf16_rn(y3));
                }
                *(uint2*)(lds + (((size_t)a * ksn * 64 + col) * 8 + (n & 7))) = v;
            }
        }
        __syncthreads();
        K = net.hidden;
    }
    // Head: the columns the pass's rows need, nt 16-column blocks. Few blocks go to groups of wavefronts that split the rows (rg
    // row groups of RB / rg blocks, 8 / rg blocks per column step), so that
    // every wavefront has work and reads fewer operand fragments per product.
    if (nt <= 6 && RB >= 4)
        chain_head<PREC, RB, (RB + 3) / 4>(net, rows, out, ps, nt, 4, lds, lane, wave);
    else if (nt <= 12 && RB >= 2)
        chain_head<PREC, RB, (RB + 1) / 2>(net, rows, out, ps, nt, 2, lds, lane, wave);
    else
        chain_head<PREC, RB, RB>(net, rows, out, ps, nt, 1, lds, lane, wave);
}

// One workgroup per pass of the plan (plan_chain orders the passes so that
// the costly ones start first).
template <int PREC, int MODE>
__global__ __launch_bounds__(CHAIN_WAVES * 64) __attribute__((amdgpu_waves_per_eu(CHAIN_WAVES / 4, CHAIN_WAVES / 4))) void k_chain(
    ChainNet net, const uint16_t* __restrict__ X, uint32_t rows, float* __restrict__ out,
    const ChainPass* __restrict__ plan) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[CHAIN_LDS_HALVES];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const ChainPass* ps = plan + blockIdx.x;
    switch (min(CHAIN_PASS_BLOCKS, ps->n)) {
        case 8: chain_pass<PREC, 8, MODE>(net, X, rows, out, ps, lds, lane, wave); break;
        case 7: chain_pass<PREC, 7, MODE>(net, X, rows, out, ps, lds, lane, wave); break;
        case 6: chain_pass<PREC, 6, MODE>(net, X, rows, out, ps, lds, lane, wave); break;
        case 5: chain_pass<PREC, 5, MODE>(net, X, rows, out, ps, lds, lane, wave); break;
        case 4: chain_pass<PREC, 4, MODE>(net, X, rows, out, ps, lds, lane, wave); break;
        case 3: chain_pass<PREC, 3, MODE>(net, X, rows, out, ps, lds, lane, wave); break;
        case 2: chain_pass<PREC, 2, MODE>(net, X, rows, out, ps, lds, lane, wave); break;
        case 1: chain_pass<PREC, 1, MODE>(net, X, rows, out, ps, lds, lane, wave); break;
        default: break;
    }
}

void launch_chain(int precision, const ChainNet& net, const void* X, uint32_t rows, float* out,
                  const ChainPass* plan, uint32_t npass, hipStream_t s) {
    if (rows == 0 || npass == 0) return;
    dim3 grid(npass), block(CHAIN_WAVES * 64);
    const uint16_t* x = (const uint16_t*)X;
    if (precision == WC_F16) {
        if (net.part)
            hipLaunchKernelGGL((k_chain<WC_F16, CHAIN_PART>), grid, block, 0, s, net, x, rows, out, plan);
        else
            hipLaunchKernelGGL((k_chain<WC_F16, CHAIN_FULL>), grid, block, 0, s, net, x, rows, out, plan);
    } else {
        if (net.part)
            hipLaunchKernelGGL((k_chain<WC_BF16, CHAIN_PART>), grid, block, 0, s, net, x, rows, out, plan);
        else
            hipLaunchKernelGGL((k_chain<WC_BF16, CHAIN_FULL>), grid, block, 0, s, net, x, rows, out, plan);
    }
}

void launch_chain_static(int precision, const ChainNet& net, const void* X, float* part, const ChainPass* plan,
                         uint32_t npass, hipStream_t s) {
    if (npass == 0) return;
    dim3 grid(npass), block(CHAIN_WAVES * 64);
    if (precision == WC_F16)
        hipLaunchKernelGGL((k_chain<WC_F16, CHAIN_STATIC>), grid, block, 0, s, net, (const uint16_t*)X, 0u, part,
                           plan);
    else
        hipLaunchKernelGGL((k_chain<WC_BF16, CHAIN_STATIC>), grid, block, 0, s, net, (const uint16_t*)X, 0u, part,
                           plan);
}

}  // namespace wc
