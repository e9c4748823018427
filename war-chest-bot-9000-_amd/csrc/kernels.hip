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

#include "../../include/wc_wave.h"

namespace wc {

#define EPSF 1e-6f       // regret-matching floor (engine/src/search.rs:1658)
#define SMOOTHF 1e-30f   // belief normalisation floor (engine/src/rebel.rs:359)

constexpr int BLOCK = 256;

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

__device__ __forceinline__ const Task& decision_task(const WaveDev& w, uint32_t i, int* p) {
    if (i < w.ndec0) {
        *p = 0;
        return w.decision0[i];
    }
    *p = 1;
    return w.decision1[i - w.ndec0];
}

// ------------------------------------------------------------- CFR state

// cur = 1/len over each acting row (engine/src/search.rs:826-836).
__global__ void k_init_strategy(WaveDev w) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= w.ndec0 + w.ndec1) return;
    int p;
    Task q = decision_task(w, i, &p);
    uint32_t row = w.legal_row_of[q.node] + q.config;
    uint32_t lo = w.legal_off[row], hi = w.legal_off[row + 1];
    float u = 1.0f / (float)(hi - lo);
    for (uint32_t g = lo; g < hi; g++) w.cur[g] = u;
}

void launch_init_strategy(const WaveDev& w, hipStream_t s) {
    uint32_t n = w.ndec0 + w.ndec1;
    if (n) hipLaunchKernelGGL(k_init_strategy, dim3(grid_for(n)), dim3(BLOCK), 0, s, w);
}

// Zero one tree's reach span and write its root (or carried root k) beliefs.
__global__ void k_seed_reach(WaveDev w, float* reach, int root_index) {
    const TreeDev t = w.trees[blockIdx.x];
    for (uint32_t i = threadIdx.x; i < t.reach_len; i += blockDim.x) reach[t.reach0 + i] = 0.0f;
    __syncthreads();
    if (root_index >= (int)t.nroots) return;
    const float* src = root_index < 0 ? w.roots + t.root0 : w.carried + t.carried0 + (size_t)root_index * (t.n0 + t.n1);
    for (uint32_t i = threadIdx.x; i < t.n0 + t.n1; i += blockDim.x) {
        int p = i >= t.n0;
        uint32_t c = p ? i - t.n0 : i;
        reach[w.reach_base[2 * t.node0 + p] + c] = src[i];
    }
}

void launch_seed_reach(const WaveDev& w, float* reach, int root_index, hipStream_t s) {
    hipLaunchKernelGGL(k_seed_reach, dim3(w.ntrees), dim3(BLOCK), 0, s, w, reach, root_index);
}

// One child config's reach: the reverse gather in stored order (the CPU's
// scatter order, engine/src/serialize.rs:714-723).
__device__ __forceinline__ void reach_task(const WaveDev& w, float* reach, const float* strat, int p, Task q) {
    uint32_t node = q.node, c = q.config;
    uint32_t base = w.reach_base[2 * w.parent[node] + p];
    float v = 0.0f;
    uint32_t rr = w.rev_row_of[node];
    if (rr != 0xffffffffu) {
        uint32_t row = rr + c;
        for (uint32_t x = w.rev_start[row]; x < w.rev_start[row + 1]; x++)
            v += reach[base + w.rev_src[x]] * strat[w.rev_cell[x]];
    } else {
        uint32_t row = w.rvd_row_of[node] + c;
        for (uint32_t x = w.rvd_start[row]; x < w.rvd_start[row + 1]; x++)
            v += reach[base + w.rvd_src[x]] * w.rvd_p[x];
    }
    reach[w.reach_base[2 * node + p] + c] = v;
}

// Both players' reach under one fixed strategy, one workgroup per tree, top-down
// levels separated by block barriers.
__global__ __launch_bounds__(BLOCK) void k_reach_both(WaveDev w, float* reach, const float* strat) {
    const TreeDev t = w.trees[blockIdx.x];
    for (uint32_t l = 1; l < t.nlevels; l++) {
        uint32_t b0 = w.reach_lvl0[t.lvl0 + l], e0 = w.reach_lvl0[t.lvl0 + l + 1];
        uint32_t b1 = w.reach_lvl1[t.lvl0 + l], e1 = w.reach_lvl1[t.lvl0 + l + 1];
        uint32_t n0 = e0 - b0, n = n0 + (e1 - b1);
        for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
            if (k < n0)
                reach_task(w, reach, strat, 0, w.reach_task0[b0 + k]);
            else
                reach_task(w, reach, strat, 1, w.reach_task1[b1 + k - n0]);
        }
        __syncthreads();
    }
}

void launch_reach_both(const WaveDev& w, float* reach, const float* strat, hipStream_t s) {
    hipLaunchKernelGGL(k_reach_both, dim3(w.ntrees), dim3(BLOCK), 0, s, w, reach, strat);
}

// sum = reach * cur: one reach-weighted uniform strategy (engine/src/search.rs:854-870).
__global__ void k_seed_sum(WaveDev w) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= w.ndec0 + w.ndec1) return;
    int p;
    Task q = decision_task(w, i, &p);
    uint32_t row = w.legal_row_of[q.node] + q.config;
    float r = w.reach[w.reach_base[2 * q.node + p] + q.config];
    for (uint32_t g = w.legal_off[row]; g < w.legal_off[row + 1]; g++) w.sum[g] = r * w.cur[g];
}

void launch_seed_sum(const WaveDev& w, hipStream_t s) {
    uint32_t n = w.ndec0 + w.ndec1;
    if (n) hipLaunchKernelGGL(k_seed_sum, dim3(grid_for(n)), dim3(BLOCK), 0, s, w);
}

// --------------------------------------------------------------- leaf input

// One wavefront per (network row, player): the leaf's reach mass, and the
// pooled belief sum_c beta(c) e(c) with beta the normalised reach
// (normalize_weights, engine/src/rebel.rs:1054-1068; accumulate, net.rs:161-170).
// Every lane forms the mass in config order; lane k owns pooled[k].
__global__ __launch_bounds__(BLOCK) void k_pool(WaveDev w, int player) {
    uint32_t task = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    uint32_t lane = threadIdx.x & 63;
    uint32_t row, p;
    if (player < 0) {
        row = task >> 1;
        p = task & 1;
    } else {
        row = task;
        p = (uint32_t)player;
    }
    if (row >= w.rows) return;
    uint32_t node = w.row_node[row];
    uint32_t n = w.nc[2 * node + p];
    const float* r = w.reach + w.reach_base[2 * node + p];
    float tot = 0.0f;
    for (uint32_t c = 0; c < n; c++) tot += r[c];
    float scale, flat;
    if (tot > SMOOTHF) {
        scale = 1.0f / tot;
        flat = 0.0f;
    } else {
        scale = 0.0f;
        flat = 1.0f / (float)(n > 0 ? n : 1);
    }
    uint32_t q = 2 * row + p;
    if (lane == 0) w.mass[q] = tot;
    const uint32_t* cfgs = w.row_cfg + w.row_cfg_off[q];
    for (uint32_t k = lane; k < w.pool; k += 64) {
        float acc = 0.0f;
        for (uint32_t c = 0; c < n; c++) {
            float wc = r[c] * scale + flat;
            acc += wc * w.cfg_emb[(size_t)cfgs[c] * w.pool + k];
        }
        w.pooled[(size_t)q * w.pool + k] = acc;
    }
}

void launch_pool(const WaveDev& w, int player, hipStream_t s) {
    size_t waves = (size_t)w.rows * (player < 0 ? 2 : 1);
    if (waves) hipLaunchKernelGGL(k_pool, dim3(grid_for(waves * 64)), dim3(BLOCK), 0, s, w, player);
}

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

// Query rows for traverser q: [pooled_q | pooled_{1-q} | seat | public / 255].
template <int PREC>
__global__ void k_build_x(WaveDev w, int q, void* xout) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t total = (size_t)w.rows * w.in;
    if (i >= total) return;
    uint32_t row = (uint32_t)(i / w.in), k = (uint32_t)(i % w.in);
    uint32_t pool = w.pool;
    float v;
    if (k < pool)
        v = w.pooled[(size_t)(2 * row + q) * pool + k];
    else if (k < 2 * pool)
        v = w.pooled[(size_t)(2 * row + 1 - q) * pool + (k - pool)];
    else if (k == 2 * pool)
        v = q ? 1.0f : -1.0f;
    else
        v = (float)w.pub_raw[(size_t)row * w.row_bytes + (k - 2 * pool - 1)] / 255.0f;
    if (PREC == WC_PRECISE)
        ((float*)xout)[i] = v;
    else if (PREC == WC_F16)
        ((uint16_t*)xout)[i] = f32_to_f16_rn(v);
    else
        ((uint16_t*)xout)[i] = f32_to_bf16_rn(v);
}

void launch_build_x(const WaveDev& w, int traverser, int precision, void* x, hipStream_t s) {
    size_t n = (size_t)w.rows * w.in;
    if (!n) return;
    if (precision == WC_PRECISE)
        hipLaunchKernelGGL(k_build_x<WC_PRECISE>, dim3(grid_for(n)), dim3(BLOCK), 0, s, w, traverser, x);
    else if (precision == WC_F16)
        hipLaunchKernelGGL(k_build_x<WC_F16>, dim3(grid_for(n)), dim3(BLOCK), 0, s, w, traverser, x);
    else
        hipLaunchKernelGGL(k_build_x<WC_BF16>, dim3(grid_for(n)), dim3(BLOCK), 0, s, w, traverser, x);
}

// ------------------------------------------------------------- the sweep

// One backprop task for traverser p (engine/src/search.rs:1672-1803).
__device__ __forceinline__ void backprop_task(const WaveDev& w, int p, Task q, int mode, float da, float db,
                                              float ds, float predict, const float* strat) {
    uint32_t node = q.node, c = q.config;
    uint32_t meta = w.node_meta[node];
    uint32_t kind = meta & 3u, actor = meta >> 2;
    float* vals = w.vals;
    uint32_t vb = w.vals_base[2 * node + p];
    if (kind == 1) {  // the traverser draws: push values through the outcome row
        uint32_t child = w.child[w.child_start[node]];
        uint32_t d0 = w.draw_off[node], rb = w.draw_row_off[node];
        uint32_t lo = w.draw_row_start[rb + c], hi = w.draw_row_start[rb + c + 1];
        uint32_t cb = w.vals_base[2 * child + p];
        float v = 0.0f;
        for (uint32_t x = lo; x < hi; x++) v += w.draw_p[d0 + x] * vals[cb + w.draw_to[d0 + x]];
        vals[vb + c] = v;
        return;
    }
    if (actor != (uint32_t)p) {  // opponent decision: sum the children in child order
        float v = 0.0f;
        for (uint32_t x = w.child_start[node]; x < w.child_start[node + 1]; x++)
            v += vals[w.vals_base[2 * w.child[x] + p] + c];
        vals[vb + c] = v;
        return;
    }
    uint32_t row = w.legal_row_of[node] + c;
    uint32_t lo = w.legal_off[row], hi = w.legal_off[row + 1];
    const float* st = mode == MODE_VALUE ? strat : w.cur;
    float base = 0.0f;
    for (uint32_t g = lo; g < hi; g++) {
        uint32_t lv = w.legal_value[g];
        if (lv != 0xffffffffu) base += vals[lv] * st[g];
    }
    vals[vb + c] = base;
    if (mode == MODE_VALUE) return;
    // Fused regret matching with DCFR discounting (search.rs:1742-1779).
    float total = 0.0f;
    for (uint32_t g = lo; g < hi; g++) {
        uint32_t lv = w.legal_value[g];
        float delta = 0.0f;
        if (lv != 0xffffffffu) delta += vals[lv];
        delta -= base;
        float old = w.regret[g];
        float r = old * (old > 0.0f ? da : db) + delta;
        w.regret[g] = r;
        float v = fmaxf(r + predict * delta, EPSF);
        w.cur[g] = v;
        total += v;
        w.sum[g] *= ds;
    }
    if (total > 0.0f) {
        float inv = 1.0f / total;
        for (uint32_t g = lo; g < hi; g++) w.cur[g] *= inv;
    }
}

// One CFR iteration (or one fixed-strategy value pass) for traverser p, one
// workgroup per tree: leaf values, bottom-up values with the regret update,
// top-down reach under the new strategy, average accumulation.
template <int MODE>
__global__ __launch_bounds__(BLOCK) void k_cfr(WaveDev w, const float* head_out, uint32_t heads, int p, float da,
                                             float db, float ds, float predict) {
    constexpr int mode = MODE;
    const TreeDev t = w.trees[blockIdx.x];
    const int opp = 1 - p;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    // Leaf values: net value x opponent reach mass (search.rs:1587-1636).
    for (uint32_t r = t.row0 + wave; r < t.row0 + t.rows; r += nwaves) {
        uint32_t node = w.row_node[r];
        uint32_t n = w.nc[2 * node + p];
        float m = w.mass[2 * r + opp];
        const uint32_t* cfgs = w.row_cfg + w.row_cfg_off[2 * r + p];
        float* out = w.vals + w.vals_base[2 * node + p];
        const float* h = head_out + (size_t)r * heads;
        for (uint32_t c = lane; c < n; c += 64) out[c] = h[w.cfg_key[cfgs[c]]] * m;
    }
    for (uint32_t k = t.term0 + threadIdx.x; k < t.term0 + t.nterm; k += blockDim.x) {
        uint32_t node = w.term_node[k];
        const float* ro = w.reach + w.reach_base[2 * node + opp];
        float m = 0.0f;
        for (uint32_t c = 0; c < w.nc[2 * node + opp]; c++) m += ro[c];
        float u = (w.node_meta[node] >> 2) == (uint32_t)p ? w.term_util[k] : -w.term_util[k];
        float* out = w.vals + w.vals_base[2 * node + p];
        for (uint32_t c = 0; c < w.nc[2 * node + p]; c++) out[c] = u * m;
    }
    __syncthreads();
    const Task* back = p ? w.back_task1 : w.back_task0;
    const uint32_t* blvl = p ? w.back_lvl1 : w.back_lvl0;
    for (uint32_t l = t.nlevels; l-- > 0;) {
        uint32_t b = blvl[t.lvl0 + l], e = blvl[t.lvl0 + l + 1];
        for (uint32_t k = b + threadIdx.x; k < e; k += blockDim.x)
            backprop_task(w, p, back[k], mode, da, db, ds, predict, w.snap);
        __syncthreads();
    }
    if (mode == MODE_VALUE) return;
    const Task* rt = p ? w.reach_task1 : w.reach_task0;
    const uint32_t* rlvl = p ? w.reach_lvl1 : w.reach_lvl0;
    for (uint32_t l = 1; l < t.nlevels; l++) {
        uint32_t b = rlvl[t.lvl0 + l], e = rlvl[t.lvl0 + l + 1];
        for (uint32_t k = b + threadIdx.x; k < e; k += blockDim.x) reach_task(w, w.reach, w.cur, p, rt[k]);
        __syncthreads();
    }
    // Average-strategy accumulation over p's decision rows (search.rs:1818-1835).
    const Task* dec = p ? w.decision1 : w.decision0;
    for (uint32_t k = t.dec0[p] + threadIdx.x; k < t.dec1[p]; k += blockDim.x) {
        Task q = dec[k];
        uint32_t row = w.legal_row_of[q.node] + q.config;
        float r = w.reach[w.reach_base[2 * q.node + p] + q.config];
        for (uint32_t g = w.legal_off[row]; g < w.legal_off[row + 1]; g++) w.sum[g] += r * w.cur[g];
    }
}

void launch_cfr(const WaveDev& w, const float* head_out, uint32_t heads, int traverser, int mode, float da,
                float db, float ds, float predict, hipStream_t s) {
    if (mode == MODE_VALUE)
        hipLaunchKernelGGL(k_cfr<MODE_VALUE>, dim3(w.ntrees), dim3(BLOCK), 0, s, w, head_out, heads, traverser, da,
                           db, ds, predict);
    else
        hipLaunchKernelGGL(k_cfr<MODE_REGRET>, dim3(w.ntrees), dim3(BLOCK), 0, s, w, head_out, heads, traverser, da,
                           db, ds, predict);
}

// Average strategy: sum / row sum, uniform when the sum is not positive, the
// literal current strategy for a player whose sum was never updated
// (engine/src/search.rs:899-938).
__global__ void k_normalize(WaveDev w, int touched0, int touched1) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= w.ndec0 + w.ndec1) return;
    int p;
    Task q = decision_task(w, i, &p);
    uint32_t row = w.legal_row_of[q.node] + q.config;
    uint32_t lo = w.legal_off[row], hi = w.legal_off[row + 1];
    if (!(p ? touched1 : touched0)) {
        for (uint32_t g = lo; g < hi; g++) w.snap[g] = w.cur[g];
        return;
    }
    float s = 0.0f;
    for (uint32_t g = lo; g < hi; g++) s += w.sum[g];
    float k = (float)(hi > lo ? hi - lo : 1);
    for (uint32_t g = lo; g < hi; g++) w.snap[g] = s > 0.0f ? w.sum[g] / s : 1.0f / k;
}

void launch_normalize(const WaveDev& w, int touched0, int touched1, hipStream_t s) {
    uint32_t n = w.ndec0 + w.ndec1;
    if (n) hipLaunchKernelGGL(k_normalize, dim3(grid_for(n)), dim3(BLOCK), 0, s, w, touched0, touched1);
}

// Normalised beliefs at every exit, f16 (the carry store, engine/src/gpu/client.rs:20-111).
__global__ __launch_bounds__(BLOCK) void k_gather_carry(WaveDev w, const float* reach, int slot) {
    uint32_t task = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    uint32_t lane = threadIdx.x & 63;
    uint32_t e = task >> 1, p = task & 1;
    if (e >= w.nexit) return;
    uint32_t node = w.exit_node[e];
    uint32_t n = w.nc[2 * node + p];
    const float* r = reach + w.reach_base[2 * node + p];
    float tot = 0.0f;
    for (uint32_t c = 0; c < n; c++) tot += r[c];
    float scale, flat;
    if (tot > SMOOTHF) {
        scale = 1.0f / tot;
        flat = 0.0f;
    } else {
        scale = 0.0f;
        flat = 1.0f / (float)(n > 0 ? n : 1);
    }
    uint16_t* dst = w.carry + (size_t)slot * w.snapshot_configs + w.exit_coff[2 * e + p];
    for (uint32_t c = lane; c < n; c += 64) dst[c] = f32_to_f16_rn(r[c] * scale + flat);
}

void launch_gather_carry(const WaveDev& w, const float* reach, int slot, hipStream_t s) {
    size_t waves = (size_t)w.nexit * 2;
    if (waves) hipLaunchKernelGGL(k_gather_carry, dim3(grid_for(waves * 64)), dim3(BLOCK), 0, s, w, reach, slot);
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

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

template <int PREC>
__global__ void k_to16(const float* src, uint16_t* dst, uint32_t rows, uint32_t cols, int transpose) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows * cols) return;
    uint32_t r = (uint32_t)(i / cols), c = (uint32_t)(i % cols);
    float v = src[i];
    uint16_t h = PREC == WC_F16 ? f32_to_f16_rn(v) : f32_to_bf16_rn(v);
    if (transpose)
        dst[(size_t)c * rows + r] = h;
    else
        dst[i] = h;
}

void launch_to16(int precision, const float* src, void* dst, uint32_t rows, uint32_t cols, bool transpose,
                 hipStream_t s) {
    size_t n = (size_t)rows * cols;
    if (!n) return;
    if (precision == WC_F16)
        hipLaunchKernelGGL(k_to16<WC_F16>, dim3(grid_for(n)), dim3(BLOCK), 0, s, src, (uint16_t*)dst, rows, cols,
                           (int)transpose);
    else
        hipLaunchKernelGGL(k_to16<WC_BF16>, dim3(grid_for(n)), dim3(BLOCK), 0, s, src, (uint16_t*)dst, rows, cols,
                           (int)transpose);
}

// 16x16x32 MFMA tile GEMM, 128 x 128 output per workgroup (4 wavefronts in a
// 2 x 2 grid, 64 x 64 each = 4 x 4 MFMA tiles). Both operands are K-contiguous
// (X row-major [M, K], Wt [N, K]), so each lane's 8-element fragment is one
// 16-byte load. Lane l holds A[l % 16][8 (l / 16) ..] and B[..][l % 16]; the
// 4 accumulators of lane l are D[4 (l / 16) + v][l % 16].
template <int PREC, bool RELU, bool OUT16>
__global__ __launch_bounds__(256) void k_gemm16(const uint16_t* __restrict__ X, uint32_t K,
                                                const uint16_t* __restrict__ Wt, const float* __restrict__ bias,
                                                uint32_t N, void* __restrict__ Y, uint32_t M) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t m0 = blockIdx.x * 128 + (wave & 1) * 64;
    const uint32_t n0 = blockIdx.y * 128 + (wave >> 1) * 64;
    const uint32_t li = lane & 15, kb = lane >> 4;
    float4v acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    const uint4 zero = make_uint4(0, 0, 0, 0);
    for (uint32_t k0 = 0; k0 < K; k0 += 32) {
        uint4 af[4], bfr[4];
#pragma unroll
        for (int a = 0; a < 4; a++) {
            uint32_t row = m0 + a * 16 + li;
            af[a] = row < M ? *(const uint4*)(X + (size_t)row * K + k0 + kb * 8) : zero;
        }
#pragma unroll
        for (int b = 0; b < 4; b++) {
            uint32_t col = n0 + b * 16 + li;
            bfr[b] = col < N ? *(const uint4*)(Wt + (size_t)col * K + k0 + kb * 8) : zero;
        }
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                if (PREC == WC_F16)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, af[a]),
                                                                       __builtin_bit_cast(half8, bfr[b]), acc[a][b],
                                                                       0, 0, 0);
                else
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[a]),
                                                                        __builtin_bit_cast(bf16x8, bfr[b]),
                                                                        acc[a][b], 0, 0, 0);
            }
    }
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
                    ((uint16_t*)Y)[(size_t)row * N + col] = PREC == WC_F16 ? f32_to_f16_rn(y) : f32_to_bf16_rn(y);
                else
                    ((float*)Y)[(size_t)row * N + col] = y;
            }
        }
}

void launch_gemm16(int precision, const void* X, uint32_t K, const void* Wt, const float* b, uint32_t N, void* Y,
                   uint32_t M, bool relu, bool out16, hipStream_t s) {
    if (M == 0 || N == 0) return;
    dim3 grid((M + 127) / 128, (N + 127) / 128);
    const uint16_t* x = (const uint16_t*)X;
    const uint16_t* wt = (const uint16_t*)Wt;
#define WC_GEMM(P, R, O) hipLaunchKernelGGL((k_gemm16<P, R, O>), grid, dim3(256), 0, s, x, K, wt, b, N, Y, M)
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

}  // namespace wc
