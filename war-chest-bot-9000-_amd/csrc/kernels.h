// Device-side view of a packed wave: table and arena pointers passed to every
// kernel by value.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "wave.h"

namespace wc {

enum : int { MODE_REGRET = 0, MODE_VALUE = 1 };

// Fragment-major layout of a 16-bit GEMM operand with K columns: every
// (16-row block, 32-column step) is one contiguous 1 KB block holding the 64
// lanes' 16-byte MFMA fragments in lane order (lane l: row l % 16, columns
// 8 (l / 16) .. + 7 of the step), so one fragment load is one coalesced read.
// Rows are padded to a multiple of GEMM_ROWS; K must be a multiple of 32.
constexpr uint32_t GEMM_ROWS = 128;
__host__ __device__ inline size_t frag_off(uint32_t row, uint32_t k, uint32_t K) {
    return ((size_t)((row >> 4) * (K >> 5) + (k >> 5)) * 64 + (row & 15) + ((k & 31) >> 3) * 16) * 8 + (k & 7);
}
inline uint32_t gemm_rows(uint32_t rows) { return (rows + GEMM_ROWS - 1) / GEMM_ROWS * GEMM_ROWS; }

struct WaveDev {
    // immutable tables (the ones the kernels read; row records carry the
    // offsets into the element arrays)
    const uint32_t *node_meta, *nc, *legal_value, *draw_to;
    const float* draw_p;
    const uint32_t *reach_base, *vals_base;
    const uint32_t *rev_src, *rev_cell, *rvd_src;
    const float* rvd_p;
    const uint32_t *row_node, *row_cfg_off, *row_cfg;
    const float* cfg_emb;
    const uint8_t* pub_raw;
    const uint32_t* term_node;
    const float* term_util;
    const float *roots, *carried;
    const uint32_t *exit_node, *exit_coff, *exit_reach;
    const TreeDev* trees;
    const UnitDev* units;
    const BackRec* back_rec[2];
    const ReachRec* reach_rec[2];
    const AccRec* acc_rec[2];  // every decision row; the top regions' rows close each list
    const LeafRec* leaf_rec[2];
    const PoolGroup* pool_grp[2];
    const uint32_t* child_vb[2];
    const uint32_t *back_lvl[2], *reach_lvl[2];
    const uint32_t* unit_term;
    // mutable arena
    float *regret, *cur, *sum, *snap;
    float *reach, *snap_reach, *vals;
    float *mass, *root_values;
    uint16_t* carry;
    // sizes
    uint32_t ntrees, nunits, nsub, rows, pool, in, row_bytes, snapshot_configs, nexit, ncells;
    uint32_t max_vwin;  // widest unit value window (floats)
    uint32_t max_rwin;  // widest unit reach window (floats)
    uint32_t unit_lds;  // 1: the sweep and reach passes keep unit windows in LDS when they fit
    uint32_t ndec[2];
    uint32_t npool[2];  // pool groups of each player
    uint32_t nleaf[2];  // network-leaf slots of each player (leaf_rec entries)
    const TowerBlock* tower_blk[2];  // two-tower readout blocks and tiles of each player
    const TowerUnit* tower_unit[2];
    uint32_t ntower_blk[2], ntower_unit[2];
    uint64_t xplane;  // compensated f16: elements between a query input's hi and lo planes
};

// Launchers (kernels.hip). All take the executor's stream.
void launch_zero(float* p, size_t n, hipStream_t s);
void launch_init_strategy(const WaveDev& w, hipStream_t s);
// Zero `reach` (reach_len floats), then write every tree's root beliefs
// (root_index < 0) or its carried root `root_index`.
void launch_seed_reach(const WaveDev& w, float* reach, size_t reach_len, int root_index, hipStream_t s);
// Top-down reach of subtree units [unit0, unit0 + n) under `strat`, for one
// player or both (player < 0). With reach2 (player >= 0), the same launch also
// computes both players' reach under strat2 into reach2: a second, independent
// reach computation over the same units (a snapshot's, under the average
// strategy).
void launch_reach(const WaveDev& w, uint32_t unit0, uint32_t n, float* reach, const float* strat, int player,
                  hipStream_t s, float* reach2 = nullptr, const float* strat2 = nullptr);
// One set of top-region reach rows of one depth: their records, the reach they
// write and the strategy they read.
struct ReachSet {
    const ReachRec* rows = nullptr;
    uint32_t n = 0;
    float* reach = nullptr;
    const float* strat = nullptr;
};
// Top-region reach at one depth: up to three independent row sets in one launch.
void launch_reach_rows(const WaveDev& w, const ReachSet& a, const ReachSet& b, const ReachSet& c, hipStream_t s);
// One reach computation's rows of two top depths, chunk by chunk
// (WaveHost::top_reach_run): workgroup k of the set computes the shallower
// rows rows[par[off[chunks + 1 + k] .. off[chunks + 2 + k])], then the deeper
// rows rows[off[k] .. off[k + 1]), which read no shallower row of another
// chunk.
struct ReachPair {
    const ReachRec* rows;
    const uint32_t* off;
    const uint32_t* par;
    uint32_t chunks;
    float* reach;
    const float* strat;
};
void launch_reach_pair(const WaveDev& w, const ReachPair& a, const ReachPair& b, const ReachPair& c, hipStream_t s);
void launch_seed_sum(const WaveDev& w, hipStream_t s);
// Leaf reach masses and pooled beliefs of one player (-1 = both), written into
// the query inputs x0 (traverser 0) and x1 (traverser 1) in the operand precision.
// With acc >= 0, the same launch also takes player acc's average-strategy
// accumulation, sum = sum * ds + reach * cur over all its decision rows (the
// discount and this iteration's addition, search.rs:1770-1779,1818-1835), in
// workgroups of their own: it reads only the final reach and cur, as the
// leaf input does.
void launch_pool(const WaveDev& w, int player, int precision, void* x0, void* x1, hipStream_t s, int acc = -1,
                 float ds = 1.0f);
// Seat and public features of both query inputs (once per upload).
void launch_query_static(const WaveDev& w, int precision, void* x0, void* x1, hipStream_t s);
// Leaf values and the bottom-up sweep of subtree units [unit0, unit0 + n) for the traverser.
void launch_sweep(const WaveDev& w, uint32_t unit0, uint32_t n, const float* head_out, uint32_t heads, int traverser,
                  int mode, float da, float db, float predict, hipStream_t s);
// Top-region values at one depth for the traverser.
void launch_back_rows(const WaveDev& w, const BackRec* rows, uint32_t n, int traverser, int mode, float da,
                      float db, float predict, hipStream_t s);
// Top-region values at two depths in one launch of `chunks` workgroups:
// workgroup k runs rows[off[k] .. off[k + 1]) of the deeper depth, then
// rows[off[chunks + 1 + k] .. off[chunks + 2 + k]) of the shallower one,
// which read no deeper row of another chunk (WaveHost::top_back_run).
void launch_back_pair(const WaveDev& w, const BackRec* rows, const uint32_t* off, uint32_t chunks, int traverser,
                      int mode, float da, float db, float predict, hipStream_t s);
void launch_normalize(const WaveDev& w, int touched0, int touched1, hipStream_t s);
void launch_gather_carry(const WaveDev& w, const float* reach, int slot, hipStream_t s);
void launch_collect_root(const WaveDev& w, int root, int player, hipStream_t s);

// Leaf MLP.
// Exact float32 dense ReLU layer in the CPU loop order: Y = relu(X W + b), W [K x N] row-major.
void launch_dense_exact(const float* X, uint32_t K, const float* W, const float* b, uint32_t N, float* Y,
                        uint32_t rows, hipStream_t s);
// Exact float32 head: out[r, k] = b[k] + sum_j Wh[k, j] H[r, j], Wh [heads x hidden].
void launch_head_exact(const float* H, uint32_t hidden, const float* Wh, const float* bh, uint32_t heads,
                       float* out, uint32_t rows, hipStream_t s);
// MFMA GEMM: Y[M, N] = act(X[M, K] Wt[N, K]^T + b); 16-bit fragment-major
// operands (X with gemm_rows(M) rows, Wt with gemm_rows(N) rows), f32
// accumulate. precision WC_F16 / WC_BF16; relu selects the activation; out16
// selects a 16-bit fragment-major output with K = N (the next layer's operand,
// N % 32 == 0) or a row-major f32 output. tile_n (optional, one entry per
// 128-row tile) bounds the columns each row tile needs; the rest are not computed.
void launch_gemm16(int precision, const void* X, uint32_t K, const void* Wt, const float* b, uint32_t N,
                   void* Y, uint32_t M, bool relu, bool out16, hipStream_t s, const uint32_t* tile_n = nullptr);
// Whole-network MLP in one launch (16-bit operands, f32 accumulate): one
// workgroup per pass of a plan (plan_chain), each running its up to 128 rows
// through every layer with the activations resident in LDS; writes out[r, k]
// (row-major f32, `heads` columns) for r < rows and the columns k < the pass's
// cols. X is the fragment-major input with gemm_rows(rows) rows; w/b hold the
// trunk layers and then the head, as launch_gemm16 takes them. Applies when
// chain_fits(in, hidden, layers).
constexpr uint32_t CHAIN_MAX_LAYERS = 8, CHAIN_MAX_WIDTH = 512;
// Eight wavefronts per tile, each owning up to CHAIN_NB 16-feature blocks of a layer.
constexpr uint32_t CHAIN_WAVES = 8, CHAIN_NB = 3;
struct ChainNet {
    const uint16_t* w[CHAIN_MAX_LAYERS + 1];
    const float* b[CHAIN_MAX_LAYERS + 1];
    uint32_t in, hidden, layers, heads;
    // With part set, the first layer takes only its first dsteps 32-column
    // k steps from X and starts from part, the product of the remaining
    // columns computed beforehand by launch_chain_static (f32, one 16 x 16
    // tile of 1 KB per (row block, feature block), in the MFMA accumulator's
    // lane order).
    const float* part = nullptr;
    uint32_t dsteps = 0;
};
bool chain_fits(uint32_t in, uint32_t hidden, uint32_t layers);
void launch_chain(int precision, const ChainNet& net, const void* X, uint32_t rows, float* out,
                  const ChainPass* plan, uint32_t npass, hipStream_t s);
// The first layer's product over X's columns from k step net.dsteps on (the
// columns that stay fixed while a wave is solved: seat and public features),
// without bias, into part (the layout ChainNet::part describes), for every
// row block of the plan.
void launch_chain_static(int precision, const ChainNet& net, const void* X, float* part, const ChainPass* plan,
                         uint32_t npass, hipStream_t s);
// Two-tower net: F = private-tower output (ncfg rows, fragment-major 16-bit or
// row-major f32) times the readout weight, row-major; then player p's readout
// blocks, tv[entry (row, config)] = <F[config], H[row]> + bread, from the
// public-tower output H (fragment-major 16-bit or row-major f32).
void launch_tower_f(int precision, const void* Hp, uint32_t width, uint32_t ncfg, const float* wread, void* F,
                    hipStream_t s);
void launch_tower_head(const WaveDev& w, int player, int precision, const void* H, uint32_t width, const void* F,
                       float bread, float* tv, hipStream_t s);
// Convert f32 -> a 16-bit fragment-major operand of `rows` rows and K columns;
// element (r, k) is src[k * rows + r] when `transposed`, else src[r * K + k].
void launch_to16(int precision, const float* src, void* dst, uint32_t rows, uint32_t K, bool transposed,
                 hipStream_t s);

}  // namespace wc
