// The v5 leaf network on the device (engine/src/net.rs; the reference's
// device path: engine/src/gpu/device.rs:836-1106 per wave, 1218-1305 per
// iteration, wave_kernels.cu:301-579,778-830).
//
// Layout in HBM. Per wave: the card tokens of both seat views and their bag
// rows per job, the board vector P (D floats) and its join projection Jp (JW
// floats) per network row, f(c) (D) and g(c) (POOL) per interned config. The
// trunk's activations (37 hexes x 96 channels per row) never leave LDS: one
// workgroup carries a row from its raw bytes to P and Jp. Per iteration: the
// join's activations stay in LDS too, one workgroup per tile of rows, from the
// pooled query input to h.
//
// Arithmetic. WC_PRECISE follows the CPU net's loop order exactly (every
// product of a Lin summed from the start value over ascending inputs,
// skipping zero inputs, then the bias; LayerNorm and GELU in net.rs order;
// tanh by the restatement's own formula below), so float32 results are
// bit-identical to the CPU restatement. The 16-bit precisions round the
// operands of the GEMMs the reference's fast mode runs on tensor cores.
#include "v5.h"

#include <algorithm>
#include <cmath>
#include <type_traits>

#include "../../include/wc_wave.h"
#include "kernels.h"

namespace wc {
namespace v5 {

// ------------------------------------------------------------- host side

namespace {
struct Cursor {
    uint32_t w = 0, b = 0, ln = 0;
    Span lin(uint32_t i, uint32_t o, bool bias) {
        Span s;
        s.w = w;
        s.b = bias ? b : 0;
        s.i = i;
        s.o = o;
        s.bias = bias;
        w += i * o;
        if (bias) b += o;
        return s;
    }
    uint32_t embed(uint32_t n) {
        const uint32_t at = w;
        w += n;
        return at;
    }
};
}  // namespace

Layout layout() {
    Layout L;
    Cursor c;
    L.card[0] = c.lin(CARD_FEATS, TYPE, true);
    L.card[1] = c.lin(TYPE, TYPE, true);
    L.pile = c.lin(PILE_COUNTS, TYPE, false);
    L.seat = c.embed(2 * TYPE);
    L.hex_stem = c.lin(HEX_FACTS, C, true);
    L.tok_stem = c.lin(TYPE, C, false);
    L.pos = c.embed(HEXES * C);
    L.glob_stem = c.lin(LOOSE, C, false);
    for (uint32_t i = 0; i < BLOCKS; i++) {
        L.mix[i] = c.lin(2 * C, C, true);
        L.pool[i] = c.lin(2 * C, C, true);
        L.out[i] = c.lin(C, C, true);
    }
    L.board_out = c.lin(2 * C + LOOSE, D, true);
    L.cfg1 = c.lin(3 + TYPE, CFGH, true);
    L.cfg_f = c.lin(CFGH, D, true);
    L.cfg_g = c.lin(CFGH, POOL, true);
    L.cfg_m = c.lin(TYPE, 3 * POOL, false);
    L.join_p = c.lin(D, JW, false);
    L.join_b = c.lin(JOIN_IN, JW, true);
    for (uint32_t i = 0; i < JBLOCKS; i++) L.join_w[i] = c.lin(JW, JW, true);
    L.join_out = c.lin(JW, D, true);
    L.value_bias = c.b;
    c.b += 1;
    uint32_t k = 0;
    for (uint32_t i = 0; i < BLOCKS; i++) {
        L.norm_width[k++] = C;
        L.norm_width[k++] = C;
    }
    L.norm_width[k++] = C;     // trunk
    L.norm_width[k++] = CFGH;  // config encoder
    for (uint32_t i = 0; i < JBLOCKS; i++) L.norm_width[k++] = JW;
    L.norm_width[k++] = JW;  // join output
    L.norm_width[k++] = D;   // h
    for (uint32_t i = 0; i < NORMS; i++) {
        L.norm_g[i] = c.ln;
        L.norm_b[i] = c.ln + L.norm_width[i];
        c.ln += 2 * L.norm_width[i];
    }
    L.w_len = c.w;
    L.b_len = c.b;
    L.ln_len = c.ln;
    return L;
}

Board board() {
    // The radius-3 hexagon around (3, 3) in axial coordinates, hexes in
    // row-major (y, then x) order (board.rs:1-6); directions as board.rs:14.
    static const int dir[6][2] = {{1, 0}, {-1, 0}, {0, 1}, {0, -1}, {1, -1}, {-1, 1}};
    static const int locs[10][2] = {{4, 0}, {6, 1}, {0, 5}, {2, 6}, {2, 1}, {3, 2}, {5, 3}, {1, 3}, {3, 4}, {4, 5}};
    int hx[HEXES], hy[HEXES], n = 0;
    auto valid = [](int x, int y) { return std::abs(x - 3) <= 3 && std::abs(y - 3) <= 3 && std::abs(x + y - 6) <= 3; };
    for (int y = 0; y <= 6; y++)
        for (int x = 0; x <= 6; x++)
            if (valid(x, y)) {
                hx[n] = x;
                hy[n] = y;
                n++;
            }
    auto at = [&](int x, int y) -> int {
        for (int h = 0; h < (int)HEXES; h++)
            if (hx[h] == x && hy[h] == y) return h;
        return (int)HEXES;
    };
    Board b{};
    for (uint32_t h = 0; h < HEXES; h++)
        for (int d = 0; d < 6; d++) b.nb[h][d] = (uint8_t)at(hx[h] + dir[d][0], hy[h] + dir[d][1]);
    for (const auto& l : locs) b.loc[at(l[0], l[1])] = 1;
    return b;
}

Span mat_span(const Layout& L, uint32_t m) {
    if (m == M_CARD0) return L.card[0];
    if (m == M_CARD1) return L.card[1];
    if (m == M_CFG_M) return L.cfg_m;
    if (m >= M_MIX0 && m < M_MIX0 + BLOCKS) return L.mix[m - M_MIX0];
    if (m >= M_POOL0 && m < M_POOL0 + BLOCKS) return L.pool[m - M_POOL0];
    if (m >= M_OUT0 && m < M_OUT0 + BLOCKS) return L.out[m - M_OUT0];
    if (m == M_BOARD) return L.board_out;
    if (m == M_JOIN_P) return L.join_p;
    if (m == M_CFG1) return L.cfg1;
    if (m == M_CFG_F) return L.cfg_f;
    if (m == M_CFG_G) return L.cfg_g;
    if (m == M_JOIN_B) return L.join_b;
    if (m >= M_JOIN_W0 && m < M_JOIN_W0 + JBLOCKS) return L.join_w[m - M_JOIN_W0];
    return L.join_out;
}

// ----------------------------------------------------------- device side

namespace {

constexpr int NBLK = 192;  // trunk and config workgroups
__host__ __device__ constexpr uint32_t kpad_dev(uint32_t k) { return (k + 31) / 32 * 32; }
constexpr int JROWS = 8;   // rows per join workgroup (float32 path)

// The blob layout, computed at compile time for the kernels (the same
// cursor as layout(), which the host uses and a test compares).
struct DevLayout {
    Layout L;
    constexpr DevLayout() : L() {
        uint32_t w = 0, b = 0, ln = 0;
        auto lin = [&](Span& s, uint32_t i, uint32_t o, bool bias) {
            s.w = w;
            s.b = bias ? b : 0;
            s.i = i;
            s.o = o;
            s.bias = bias;
            w += i * o;
            if (bias) b += o;
        };
        lin(L.card[0], CARD_FEATS, TYPE, true);
        lin(L.card[1], TYPE, TYPE, true);
        lin(L.pile, PILE_COUNTS, TYPE, false);
        L.seat = w;
        w += 2 * TYPE;
        lin(L.hex_stem, HEX_FACTS, C, true);
        lin(L.tok_stem, TYPE, C, false);
        L.pos = w;
        w += HEXES * C;
        lin(L.glob_stem, LOOSE, C, false);
        for (uint32_t i = 0; i < BLOCKS; i++) {
            lin(L.mix[i], 2 * C, C, true);
            lin(L.pool[i], 2 * C, C, true);
            lin(L.out[i], C, C, true);
        }
        lin(L.board_out, 2 * C + LOOSE, D, true);
        lin(L.cfg1, 3 + TYPE, CFGH, true);
        lin(L.cfg_f, CFGH, D, true);
        lin(L.cfg_g, CFGH, POOL, true);
        lin(L.cfg_m, TYPE, 3 * POOL, false);
        lin(L.join_p, D, JW, false);
        lin(L.join_b, JOIN_IN, JW, true);
        for (uint32_t i = 0; i < JBLOCKS; i++) lin(L.join_w[i], JW, JW, true);
        lin(L.join_out, JW, D, true);
        L.value_bias = b;
        b += 1;
        uint32_t k = 0;
        for (uint32_t i = 0; i < BLOCKS; i++) {
            L.norm_width[k++] = C;
            L.norm_width[k++] = C;
        }
        L.norm_width[k++] = C;
        L.norm_width[k++] = CFGH;
        for (uint32_t i = 0; i < JBLOCKS; i++) L.norm_width[k++] = JW;
        L.norm_width[k++] = JW;
        L.norm_width[k++] = D;
        for (uint32_t i = 0; i < NORMS; i++) {
            L.norm_g[i] = ln;
            L.norm_b[i] = ln + L.norm_width[i];
            ln += 2 * L.norm_width[i];
        }
        L.w_len = w;
        L.b_len = b;
        L.ln_len = ln;
    }
};
constexpr DevLayout DL{};
#define LY (DL.L)

// tanh by the restatement's formula: e^x for x <= 0 by Cody-Waite reduction
// (ln2 = 0.693145751953125 + 1.428606765330187e-6) and the degree-7 Taylor
// polynomial on |r| <= ln2/2, then tanh|x| = (1 - e^{-2|x|}) / (1 + e^{-2|x|}).
__device__ __forceinline__ float exp_neg(float x) {
    const float n = rintf(x * 1.44269504f);
    const float r = (x - n * 0.693145751953125f) - n * 1.428606765330187e-6f;
    float p = 1.0f / 5040.0f;
    p = 1.0f / 720.0f + r * p;
    p = 1.0f / 120.0f + r * p;
    p = 1.0f / 24.0f + r * p;
    p = 1.0f / 6.0f + r * p;
    p = 0.5f + r * p;
    p = 1.0f + r * p;
    p = 1.0f + r * p;
    return ldexpf(p, (int)n);
}
__device__ __forceinline__ float tanh_r(float x) {
    const float a = fabsf(x);
    if (a > 20.0f) return x > 0.0f ? 1.0f : -1.0f;
    const float t = exp_neg(-2.0f * a);
    const float y = (1.0f - t) / (1.0f + t);
    return x < 0.0f ? -y : y;
}
// net.rs:125-128
__device__ __forceinline__ float gelu(float x) {
    const float inner = 0.79788456f * (x + 0.044715f * x * x * x);
    return 0.5f * x * (1.0f + tanh_r(inner));
}

__device__ __forceinline__ float bf16_round(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return __uint_as_float((u | 0x00400000u) & 0xffff0000u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return __uint_as_float(u & 0xffff0000u);
}
// An operand of a 16-bit GEMM, as the matrix cores see it.
template <int PREC>
__device__ __forceinline__ float qop(float x) {
    if (PREC == WC_F16) return (float)(_Float16)x;
    if (PREC == WC_BF16) return bf16_round(x);
    return x;
}
template <int PREC>
__device__ __forceinline__ uint16_t to16(float x) {
    if (PREC == WC_F16) return __builtin_bit_cast(uint16_t, (_Float16)x);
    return (uint16_t)(__float_as_uint(bf16_round(x)) >> 16);
}

// Output j of one Lin over an input vector x (LDS) of length k with matrix
// W [k x o] row-major: `gemm` then Lin::bias. FAST marks a product the 16-bit
// path runs with rounded operands (summed in float32 from zero, then the
// start value, then the bias); otherwise the float32 CPU order (from the start
// value, then the bias).
template <int PREC, bool FAST>
__device__ __forceinline__ float lin_out(const float* x, uint32_t k, const float* W, uint32_t o, uint32_t j,
                                         float start, const float* bias) {
    // Weight loads are unconditional (every index is in range) so that the
    // unrolled loop keeps several in flight; a zero input skips the addition.
    if (PREC == WC_PRECISE || !FAST) {
        float acc = start;
#pragma unroll 8
        for (uint32_t p = 0; p < k; p++) {
            const float a = x[p], w = W[(size_t)p * o + j];
            acc = a != 0.0f ? acc + a * w : acc;
        }
        if (bias) acc += bias[j];
        return acc;
    }
    float acc = 0.0f;
#pragma unroll 8
    for (uint32_t p = 0; p < k; p++) {
        const float a = qop<PREC>(x[p]), w = qop<PREC>(W[(size_t)p * o + j]);
        acc = a != 0.0f ? acc + a * w : acc;
    }
    float v = start + acc;
    if (bias) v += bias[j];
    return v;
}

// LayerNorm statistics of one row in the CPU order (net.rs:380-405): mean,
// then 1 / sqrt(var + 1e-5).
__device__ __forceinline__ void norm_stats(const float* x, uint32_t width, float* mean_out, float* inv_out) {
    float sum = 0.0f;
    for (uint32_t j = 0; j < width; j++) sum += x[j];
    const float mean = sum / (float)width;
    float sq = 0.0f;
    for (uint32_t j = 0; j < width; j++) sq += (x[j] - mean) * (x[j] - mean);
    const float var = sq / (float)width;
    *mean_out = mean;
    *inv_out = 1.0f / sqrtf(var + 1e-5f);
}
__device__ __forceinline__ float norm_apply(float x, float mean, float inv, const float* ln, uint32_t which, uint32_t j,
                                            bool act) {
    const float v = (x - mean) * inv * ln[LY.norm_g[which] + j] + ln[LY.norm_b[which] + j];
    return act ? gelu(v) : v;
}

__device__ __forceinline__ int physical_type(int view, int t) {
    return (view ? 1 - t / (int)NSLOT : t / (int)NSLOT) * (int)NSLOT + t % (int)NSLOT;
}

// --------------------------------------------------------------- cards

// Net::cards (net.rs:459-471) for one (job, view, token), and the token's
// count-weighted bag row cfg_m (net.rs:779-784). 192 threads.
template <int PREC>
__global__ __launch_bounds__(NBLK) void k_cards(Net net, WaveIn in, WaveOut out) {
    __shared__ float facts[CARD_FEATS], hid[TYPE], card[TYPE];
    const uint32_t id = blockIdx.x, t = id % NTYPE, view = (id / NTYPE) & 1, job = id / (2 * NTYPE);
    const uint32_t j = threadIdx.x;
    const float* cf = in.card_feat + (size_t)job * NTYPE * CARD_FEATS + (size_t)physical_type(view, t) * CARD_FEATS;
    if (j < CARD_FEATS) facts[j] = cf[j];
    __syncthreads();
    if (j < TYPE)
        hid[j] = gelu(lin_out<PREC, true>(facts, CARD_FEATS, net.w + LY.card[0].w, TYPE, j, 0.0f, net.b + LY.card[0].b));
    __syncthreads();
    if (j < TYPE) {
        card[j] = lin_out<PREC, true>(hid, TYPE, net.w + LY.card[1].w, TYPE, j, 0.0f, net.b + LY.card[1].b);
        out.cards[(size_t)id * TYPE + j] = card[j];
    }
    __syncthreads();
    for (uint32_t m = j; m < 3 * POOL; m += NBLK)
        out.bag[(size_t)id * 3 * POOL + m] = lin_out<PREC, true>(card, TYPE, net.w + LY.cfg_m.w, 3 * POOL, m, 0.0f, nullptr);
}

// -------------------------------------------------------------- configs

// Net::configs (net.rs:735-797) for one config. 192 threads.
template <int PREC>
__global__ __launch_bounds__(NBLK) void k_configs(Net net, WaveIn in, WaveOut out) {
    __shared__ float slot[NSLOT][3 + TYPE], hid[NSLOT][CFGH], u[CFGH], phi[CFEAT], stats[2];
    const uint32_t c = blockIdx.x, j = threadIdx.x;
    const uint32_t job = in.cfg_job[c], owner = in.cfg_owner[c];
    if (j < CFEAT) phi[j] = in.phi[(size_t)c * CFEAT + j];
    __syncthreads();
    const float* cards = out.cards + ((size_t)job * 2 + owner) * NTYPE * TYPE;  // the owner's view: its slot k is token k
    for (uint32_t x = j; x < NSLOT * (3 + TYPE); x += NBLK) {
        const uint32_t k = x / (3 + TYPE), q = x % (3 + TYPE);
        slot[k][q] = q < 3 ? phi[q * NSLOT + k] : cards[(size_t)k * TYPE + (q - 3)];
    }
    __syncthreads();
    if (j < CFGH)
        for (uint32_t k = 0; k < NSLOT; k++)
            hid[k][j] = gelu(lin_out<PREC, true>(slot[k], 3 + TYPE, net.w + LY.cfg1.w, CFGH, j, 0.0f, net.b + LY.cfg1.b));
    __syncthreads();
    if (j < CFGH) {
        float v = 0.0f;
        for (uint32_t k = 0; k < NSLOT; k++) v += hid[k][j];
        u[j] = v;
    }
    __syncthreads();
    if (j == 0) norm_stats(u, CFGH, &stats[0], &stats[1]);
    __syncthreads();
    if (j < CFGH) u[j] = norm_apply(u[j], stats[0], stats[1], net.ln, LN_CFG, j, true);
    __syncthreads();
    for (uint32_t x = j; x < D; x += NBLK) {
        const float f = lin_out<PREC, true>(u, CFGH, net.w + LY.cfg_f.w, D, x, 0.0f, net.b + LY.cfg_f.b);
        if (PREC == WC_PRECISE)
            ((float*)out.F)[(size_t)c * D + x] = f;
        else
            ((uint16_t*)out.F)[(size_t)c * D + x] = to16<PREC>(f);
    }
    if (j < POOL) {
        float g = lin_out<PREC, true>(u, CFGH, net.w + LY.cfg_g.w, POOL, j, 0.0f, net.b + LY.cfg_g.b);
        const float* bag = out.bag + ((size_t)job * 2 + owner) * NTYPE * 3 * POOL;
        for (uint32_t k = 0; k < NSLOT; k++)
            for (uint32_t zone = 0; zone < 3; zone++) {
                const float count = phi[zone * NSLOT + k];
                if (count == 0.0f) continue;
                g += count * bag[(size_t)k * 3 * POOL + zone * POOL + j];
            }
        out.G[(size_t)c * POOL + j] = g;
    }
}

// ---------------------------------------------------------------- trunk

// Net::board + join_cache (net.rs:474-730) for one network row, every
// activation in LDS. 192 threads: in the hex-wide products thread j % 96
// owns channel j of every other hex.
template <int PREC>
__global__ __launch_bounds__(NBLK) void k_trunk(Net net, WaveIn in, WaveOut out) {
    __shared__ float x[HEXES][C], a[HEXES][C], ns[HEXES][C], y[HEXES][C];
    __shared__ float tok[NTYPE][TYPE], proj[NTYPE][C], tp[C], glob[C], loose[LOOSE], facts[HEXES][HEX_FACTS];
    __shared__ float pooled[2 * C], gb[C], bin[2 * C + LOOSE], P[D], mean[HEXES], inv[HEXES];
    __shared__ int occ[HEXES];
    const uint32_t r = blockIdx.x, tid = threadIdx.x;
    const uint32_t job = in.row_job[r];
    const uint8_t* raw = in.raw + (size_t)r * ROW_BYTES;
    const float* cards = out.cards + (size_t)job * 2 * NTYPE * TYPE;  // view 0
    const float* W = net.w;
    // tokens (net.rs:474-495)
    for (uint32_t i = tid; i < NTYPE * TYPE; i += NBLK) {
        const uint32_t t = i / TYPE, j = i % TYPE;
        float piles[PILE_COUNTS];
        for (uint32_t f = 0; f < PILE_COUNTS; f++) piles[f] = (float)raw[GR_PILES + t * PILE_COUNTS + f] / 5.0f;
        const float v = lin_out<PREC, false>(piles, PILE_COUNTS, W + LY.pile.w, TYPE, j, 0.0f, nullptr);
        tok[t][j] = v + (cards[(size_t)t * TYPE + j] + W[LY.seat + (t / NSLOT) * TYPE + j]);
    }
    // hex facts and loose scalars (wave_kernels.cu:254-296; rebel.rs:1174-1231)
    if (tid < HEXES) {
        const uint32_t h = tid;
        const int owner = raw[GR_HEX_OWNER + h], marker = raw[GR_HEX_MARKER + h], sl = raw[GR_HEX_SLOT + h];
        facts[h][0] = owner == 0 ? 1.0f : 0.0f;
        facts[h][1] = owner == 1 ? 1.0f : 0.0f;
        facts[h][2] = (float)raw[GR_HEX_HEIGHT + h] / 5.0f;
        facts[h][3] = marker == 0 ? 1.0f : 0.0f;
        facts[h][4] = marker == 1 ? 1.0f : 0.0f;
        facts[h][5] = (float)net.loc[h];
        occ[h] = owner < 2 && sl < (int)NSLOT ? owner * (int)NSLOT + sl : -1;
    } else if (tid >= 64 && tid < 64 + LOOSE) {
        const uint32_t q = tid - 64;
        float v;
        if (q < 12) {
            const uint32_t p = q / 6, k = q % 6;
            const int markers = raw[GR_MARKERS + p];
            if (k == 0) v = (float)markers / 6.0f;
            else if (k == 1) v = (float)(6 - markers) / 6.0f;
            else if (k == 2) v = (float)raw[GR_HAND + p] / 3.0f;
            else if (k == 3) v = (float)raw[GR_FD + p] / 21.0f;
            else if (k == 4) v = (float)raw[GR_BAG + p] / 21.0f;
            else v = raw[GR_INITIATIVE] == p ? 1.0f : 0.0f;
        } else if (q == 12) {
            v = (float)((int)raw[GR_PLIES] | (int)raw[GR_PLIES + 1] << 8) / 256.0f;
        } else if (q == 13) {
            v = raw[GR_INIT_MOVED] ? 1.0f : 0.0f;
        } else {
            v = raw[GR_TO_ACT] == 0 ? 1.0f : 0.0f;
        }
        loose[q] = v;
    }
    __syncthreads();
    // stem (net.rs:499-543)
    for (uint32_t i = tid; i < NTYPE * C; i += NBLK) {
        const uint32_t t = i / C, j = i % C;
        proj[t][j] = lin_out<PREC, false>(tok[t], TYPE, W + LY.tok_stem.w, C, j, 0.0f, nullptr);
    }
    __syncthreads();
    if (tid < C) {
        float v = 0.0f;
        for (uint32_t t = 0; t < NTYPE; t++) v += gelu(proj[t][tid]) / (float)NTYPE;
        tp[tid] = v;
        glob[tid] = lin_out<PREC, false>(loose, LOOSE, W + LY.glob_stem.w, C, tid, 0.0f, nullptr);
    }
    __syncthreads();
    for (uint32_t i = tid; i < HEXES * C; i += NBLK) {
        const uint32_t h = i / C, j = i % C;
        const float v = lin_out<PREC, false>(facts[h], HEX_FACTS, W + LY.hex_stem.w, C, j, 0.0f, net.b + LY.hex_stem.b);
        const float o = occ[h] >= 0 ? proj[occ[h]][j] : 0.0f;
        x[h][j] = v + (((o + W[LY.pos + h * C + j]) + glob[j]) + tp[j]);
    }
    __syncthreads();
    const uint32_t j = tid % C, h0 = tid / C;  // hex-wide products: channel j of hexes h0, h0 + 2, ...
    auto norm_rows = [&](float (*src)[C], float (*dst)[C], uint32_t which, bool act) {
        if (tid < HEXES) norm_stats(src[tid], C, &mean[tid], &inv[tid]);
        __syncthreads();
        for (uint32_t i = tid; i < HEXES * C; i += NBLK) {
            const uint32_t h = i / C, q = i % C;
            dst[h][q] = norm_apply(src[h][q], mean[h], inv[h], net.ln, which, q, act);
        }
        __syncthreads();
    };
    for (uint32_t blk = 0; blk < BLOCKS; blk++) {
        norm_rows(x, a, 2 * blk, true);
        // neighbour sums (a zero start, directions in board order) and the
        // mean / max pool (net.rs:553-585)
        for (uint32_t i = tid; i < HEXES * C; i += NBLK) {
            const uint32_t h = i / C, q = i % C;
            float v = 0.0f;
            for (int d = 0; d < 6; d++) {
                const uint32_t n = net.nb[h * 6 + d];
                if (n < HEXES) v += a[n][q];
            }
            ns[h][q] = v;
        }
        if (tid < C) {
            float mn = 0.0f, top = -INFINITY;
            for (uint32_t h = 0; h < HEXES; h++) {
                mn += a[h][tid] / (float)HEXES;
                top = fmaxf(top, a[h][tid]);
            }
            pooled[tid] = mn;
            pooled[C + tid] = top;
        }
        __syncthreads();
        if (tid < C)
            gb[tid] = lin_out<PREC, true>(pooled, 2 * C, W + LY.pool[blk].w, C, tid, 0.0f, net.b + LY.pool[blk].b);
        // mix: [a, ns] (192 inputs) -> C, then the pool bias broadcast
        {
            const float* Wm = W + LY.mix[blk].w;
            float acc[(HEXES + 1) / 2];
#pragma unroll
            for (uint32_t m = 0; m < (HEXES + 1) / 2; m++) acc[m] = 0.0f;
            for (uint32_t p = 0; p < 2 * C; p++) {
                const float wv = PREC == WC_PRECISE ? Wm[(size_t)p * C + j] : qop<PREC>(Wm[(size_t)p * C + j]);
#pragma unroll
                for (uint32_t m = 0; m < (HEXES + 1) / 2; m++) {
                    const uint32_t h = h0 + 2 * m;
                    if (h < HEXES) {
                        const float av = qop<PREC>(p < C ? a[h][p] : ns[h][p - C]);
                        if (av != 0.0f) acc[m] += av * wv;
                    }
                }
            }
            __syncthreads();  // gb ready
#pragma unroll
            for (uint32_t m = 0; m < (HEXES + 1) / 2; m++) {
                const uint32_t h = h0 + 2 * m;
                if (h < HEXES) y[h][j] = (acc[m] + net.b[LY.mix[blk].b + j]) + gb[j];
            }
        }
        __syncthreads();
        norm_rows(y, y, 2 * blk + 1, true);
        // out: C -> C, the residual add
        {
            const float* Wo = W + LY.out[blk].w;
            float acc[(HEXES + 1) / 2];
#pragma unroll
            for (uint32_t m = 0; m < (HEXES + 1) / 2; m++) acc[m] = 0.0f;
            for (uint32_t p = 0; p < C; p++) {
                const float wv = PREC == WC_PRECISE ? Wo[(size_t)p * C + j] : qop<PREC>(Wo[(size_t)p * C + j]);
#pragma unroll
                for (uint32_t m = 0; m < (HEXES + 1) / 2; m++) {
                    const uint32_t h = h0 + 2 * m;
                    if (h < HEXES) {
                        const float av = qop<PREC>(y[h][p]);
                        if (av != 0.0f) acc[m] += av * wv;
                    }
                }
            }
#pragma unroll
            for (uint32_t m = 0; m < (HEXES + 1) / 2; m++) {
                const uint32_t h = h0 + 2 * m;
                if (h < HEXES) x[h][j] += acc[m] + net.b[LY.out[blk].b + j];
            }
        }
        __syncthreads();
    }
    norm_rows(x, a, LN_TRUNK, true);
    // the board vector (net.rs:704-722) and its join projection
    if (tid < C) {
        float mn = 0.0f, top = -INFINITY;
        for (uint32_t h = 0; h < HEXES; h++) {
            mn += a[h][tid] / (float)HEXES;
            top = fmaxf(top, a[h][tid]);
        }
        bin[tid] = mn;
        bin[C + tid] = top;
    } else if (tid < C + LOOSE) {
        bin[2 * C + (tid - C)] = loose[tid - C];
    }
    __syncthreads();
    for (uint32_t q = tid; q < D; q += NBLK) {
        P[q] = lin_out<PREC, true>(bin, 2 * C + LOOSE, W + LY.board_out.w, D, q, 0.0f, net.b + LY.board_out.b);
        out.P[(size_t)r * D + q] = P[q];
    }
    __syncthreads();
    if (tid < JW) out.Jp[(size_t)r * JW + tid] = lin_out<PREC, true>(P, D, W + LY.join_p.w, JW, tid, 0.0f, nullptr);
}

// ----------------------------------------------------------------- join

// Net::join (net.rs:801-841) for JROWS rows, float32 or rounded operands,
// every activation in LDS. 128 threads: thread j owns column j (and j + 128
// of the 256-wide output) of every row of the tile.
template <int PREC>
__global__ __launch_bounds__(JW) void k_join(Net net, uint32_t rows, const float* X, const float* P, const float* Jp,
                                             float* H) {
    __shared__ float xin[JROWS][JOIN_IN], z[JROWS][JW], t[JROWS][JW], h[JROWS][D], mean[JROWS], inv[JROWS];
    const uint32_t r0 = blockIdx.x * JROWS, j = threadIdx.x;
    const uint32_t nr = min((uint32_t)JROWS, rows - r0);
    for (uint32_t i = j; i < nr * JOIN_IN; i += JW) xin[i / JOIN_IN][i % JOIN_IN] = X[(size_t)r0 * JOIN_IN + i];
    __syncthreads();
    for (uint32_t r = 0; r < nr; r++)
        z[r][j] = lin_out<PREC, true>(xin[r], JOIN_IN, net.w + LY.join_b.w, JW, j, Jp[(size_t)(r0 + r) * JW + j],
                                      net.b + LY.join_b.b);
    __syncthreads();
    auto norm_tile = [&](float (*src)[JW], float (*dst)[JW], uint32_t which) {
        if (j < nr) norm_stats(src[j], JW, &mean[j], &inv[j]);
        __syncthreads();
        for (uint32_t r = 0; r < nr; r++) dst[r][j] = norm_apply(src[r][j], mean[r], inv[r], net.ln, which, j, true);
        __syncthreads();
    };
    for (uint32_t blk = 0; blk < JBLOCKS; blk++) {
        norm_tile(z, t, LN_JOIN + blk);
        for (uint32_t r = 0; r < nr; r++)
            z[r][j] += lin_out<PREC, true>(t[r], JW, net.w + LY.join_w[blk].w, JW, j, 0.0f, net.b + LY.join_w[blk].b);
        __syncthreads();
    }
    norm_tile(z, z, LN_JOUT);
    for (uint32_t r = 0; r < nr; r++)
        for (uint32_t q = j; q < D; q += JW)
            h[r][q] = lin_out<PREC, true>(z[r], JW, net.w + LY.join_out.w, D, q, P[(size_t)(r0 + r) * D + q],
                                          net.b + LY.join_out.b);
    __syncthreads();
    if (j < nr) norm_stats(h[j], D, &mean[j], &inv[j]);
    __syncthreads();
    for (uint32_t r = 0; r < nr; r++)
        for (uint32_t q = j; q < D; q += JW) {
            const float v = norm_apply(h[r][q], mean[r], inv[r], net.ln, LN_H, q, false);
            if (PREC == WC_PRECISE)
                H[(size_t)(r0 + r) * D + q] = v;
            else
                ((uint16_t*)H)[frag_off(r0 + r, q, D)] = to16<PREC>(v);
        }
}

// ------------------------------------------------------- join on MFMA

typedef _Float16 v5half8 __attribute__((ext_vector_type(8)));
typedef __bf16 v5bf8 __attribute__((ext_vector_type(8)));
typedef float v5f4 __attribute__((ext_vector_type(4)));

template <int PREC>
__device__ __forceinline__ v5f4 mma(const uint4& a, const uint4& b, const v5f4& c) {
    if (PREC == WC_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v5half8, a), __builtin_bit_cast(v5half8, b),
                                                      c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v5bf8, a), __builtin_bit_cast(v5bf8, b), c, 0,
                                                   0, 0);
}

// GELU of the 16-bit path (the operands it feeds are rounded to 16 bits
// anyway): 0.5 x (1 + tanh u) = x / (1 + e^(-2u)), through the hardware
// base-2 exponential and reciprocal (about one ulp each). Large |u| reach the
// limits: e^(-2u) = inf gives x * 0, e^(-2u) = 0 gives x.
__device__ __forceinline__ float gelu_fast(float x) {
    const float u = 0.79788456f * (x + 0.044715f * x * x * x);
    const float e = __builtin_amdgcn_exp2f(-2.88539008f * u);  // -2 log2(e) u
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// The sum of x over each 16-lane row of the wavefront, in every lane of the
// row: four DPP butterfly steps (lanes xor 1 and xor 2 by quad permutes, then
// the half-row and row mirrors), no LDS traffic.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_mov<0xB1>(x);   // quad_perm [1, 0, 3, 2]
    x += dpp_mov<0x4E>(x);   // quad_perm [2, 3, 0, 1]
    x += dpp_mov<0x141>(x);  // row_half_mirror: lane i <-> 7 - i within 8
    x += dpp_mov<0x140>(x);  // row_mirror: lane i <-> 15 - i
    return x;
}
// row16_sum of N independent values, step by step across them: a DPP step
// that reads the previous step's result needs two wait states, which the
// other values' steps fill instead of s_nop. The same sums, bit for bit.
template <int N>
__device__ __forceinline__ void row16_sum_n(float (&x)[N]) {
#pragma unroll
    for (int k = 0; k < N; k++) x[k] += dpp_mov<0xB1>(x[k]);
#pragma unroll
    for (int k = 0; k < N; k++) x[k] += dpp_mov<0x4E>(x[k]);
#pragma unroll
    for (int k = 0; k < N; k++) x[k] += dpp_mov<0x141>(x[k]);
#pragma unroll
    for (int k = 0; k < N; k++) x[k] += dpp_mov<0x140>(x[k]);
}

constexpr int JT_ROWS = 32;          // rows per join workgroup
constexpr int JT_WAVES = 8;          // wavefront w owns columns 16 w .. 16 w + 15 of the 128-wide stream
constexpr int JT_LD = JW + 8;        // LDS row stride of the 16-bit operand (halves)
constexpr int JT_RB = JT_ROWS / 16;  // row blocks per tile

// Net::join for a 64-row tile on the matrix cores (16x16x32, 16-bit operands,
// f32 accumulate). Eight wavefronts: wavefront w owns one 16-column block of
// the 128-wide residual stream z (in its accumulator registers) and two of
// the 256-wide output. LayerNorm statistics are summed per row across the
// wavefronts through LDS; each GELU output becomes the next product's A
// operand in LDS. Every product's B fragments (the wave's column block, all
// k steps) are loaded before the norm that precedes the product, so their L2
// latency overlaps it. In the accumulator layout lane l holds rows
// 4 (l / 16) + v, column l % 16 of each 16 x 16 tile; an A fragment is 8
// consecutive k of row l % 16.
template <int PREC>
__global__ __launch_bounds__(JT_WAVES * 64) void k_join_mfma(Net net, uint32_t rows, const uint16_t* __restrict__ X,
                                                            const float* __restrict__ P, const float* __restrict__ Jp,
                                                            uint16_t* __restrict__ H) {
    __shared__ __attribute__((aligned(16))) uint16_t tA[JT_ROWS * JT_LD];
    __shared__ float part[JT_WAVES][JT_ROWS], part2[JT_WAVES][JT_ROWS], mean[JT_ROWS], inv[JT_ROWS];
    const uint32_t wv = threadIdx.x >> 6, l = threadIdx.x & 63, q = l >> 4, i = l & 15;
    const uint32_t r0 = blockIdx.x * JT_ROWS;
    const uint32_t col = wv * 16 + i;  // this lane's column of the 128-wide stream
    // Per-row statistics of the wave's accumulators (NC column blocks each),
    // combined across the wavefronts: mean, then 1 / sqrt(var + 1e-5).
    // Each wavefront's sum and sum of squared deviations from its own mean
    // (over its NC x 16 columns), combined across the wavefronts by the
    // pairwise-variance formula (Chan, Golub and LeVeque) in one exchange.
    auto row_stats = [&](auto& z, auto ncb, float width) {
        constexpr uint32_t NC = decltype(ncb)::value;
        constexpr float NW = 16.0f * NC;  // columns per wavefront
        float sw[JT_RB * 4], dw[JT_RB * 4];  // the rows' sums, then squared deviations (rb, v)
#pragma unroll
        for (uint32_t rb = 0; rb < JT_RB; rb++)
#pragma unroll
            for (uint32_t v = 0; v < 4; v++) {
                float sacc = 0.0f;
#pragma unroll
                for (uint32_t cb = 0; cb < NC; cb++) sacc += z[rb][cb][v];
                sw[rb * 4 + v] = sacc;
            }
        row16_sum_n(sw);
#pragma unroll
        for (uint32_t rb = 0; rb < JT_RB; rb++)
#pragma unroll
            for (uint32_t v = 0; v < 4; v++) {
                const float mw = sw[rb * 4 + v] * (1.0f / NW);
                float dacc = 0.0f;
#pragma unroll
                for (uint32_t cb = 0; cb < NC; cb++) {
                    const float d = z[rb][cb][v] - mw;
                    dacc += d * d;
                }
                dw[rb * 4 + v] = dacc;
            }
        row16_sum_n(dw);
#pragma unroll
        for (uint32_t rb = 0; rb < JT_RB; rb++)
#pragma unroll
            for (uint32_t v = 0; v < 4; v++)
                if (i == 0) {
                    part[wv][rb * 16 + 4 * q + v] = sw[rb * 4 + v];
                    part2[wv][rb * 16 + 4 * q + v] = dw[rb * 4 + v];
                }
        __syncthreads();
        if (threadIdx.x < JT_ROWS) {
            float t = 0.0f;
#pragma unroll
            for (uint32_t w2 = 0; w2 < JT_WAVES; w2++) t += part[w2][threadIdx.x];
            const float m = t / width;
            float m2 = 0.0f;
#pragma unroll
            for (uint32_t w2 = 0; w2 < JT_WAVES; w2++) {
                const float dm = part[w2][threadIdx.x] * (1.0f / NW) - m;
                m2 += part2[w2][threadIdx.x] + NW * dm * dm;
            }
            mean[threadIdx.x] = m;
            inv[threadIdx.x] = 1.0f / sqrtf(m2 / width + 1e-5f);
        }
        __syncthreads();
    };
    // gelu(LN(z)) of the 128-wide stream into the A operand in LDS (16-bit).
    auto to_operand = [&](float (&z)[JT_RB][1][4], uint32_t which) {
        row_stats(z, std::integral_constant<uint32_t, 1>{}, (float)JW);
        const float g = net.ln[LY.norm_g[which] + col], bt = net.ln[LY.norm_b[which] + col];
#pragma unroll
        for (uint32_t rb = 0; rb < JT_RB; rb++)
#pragma unroll
            for (uint32_t v = 0; v < 4; v++) {
                const uint32_t r = rb * 16 + 4 * q + v;
                tA[r * JT_LD + col] = to16<PREC>(gelu_fast((z[rb][0][v] - mean[r]) * inv[r] * g + bt));
            }
        __syncthreads();
    };
    // B fragments of column blocks cb0 .. cb0 + NC - 1 over KS k steps.
    auto load_b = [&](auto& bf, const uint16_t* W, uint32_t cb0) {
        constexpr uint32_t KS = sizeof(bf) / sizeof(bf[0]);
        constexpr uint32_t NC = sizeof(bf[0]) / sizeof(uint4);
#pragma unroll
        for (uint32_t s = 0; s < KS; s++)
#pragma unroll
            for (uint32_t cb = 0; cb < NC; cb++)
                bf[s][cb] = *(const uint4*)(W + ((size_t)(cb0 + cb) * KS * 64 + (size_t)s * 64 + l) * 8);
    };
    // acc[rb][cb] = A B^T: A from the LDS operand (or the fragment-major X).
    auto gemm = [&](auto& acc, const auto& bf, bool from_x) {
        constexpr uint32_t KS = sizeof(bf) / sizeof(bf[0]);
        constexpr uint32_t NC = sizeof(bf[0]) / sizeof(uint4);
#pragma unroll
        for (uint32_t rb = 0; rb < JT_RB; rb++)
#pragma unroll
            for (uint32_t cb = 0; cb < NC; cb++) acc[rb][cb] = v5f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t s = 0; s < KS; s++) {
            uint4 af[JT_RB];
#pragma unroll
            for (uint32_t rb = 0; rb < JT_RB; rb++)
                af[rb] = from_x ? *(const uint4*)(X + ((size_t)((r0 >> 4) + rb) * KS * 64 + (size_t)s * 64 + l) * 8)
                                : *(const uint4*)(tA + (rb * 16 + i) * JT_LD + s * 32 + 8 * q);
#pragma unroll
            for (uint32_t rb = 0; rb < JT_RB; rb++)
#pragma unroll
                for (uint32_t cb = 0; cb < NC; cb++) acc[rb][cb] = mma<PREC>(af[rb], bf[s][cb], acc[rb][cb]);
        }
    };
    // z = Jp + X join_b + b
    float z[JT_RB][1][4];
    uint4 bw[JW / 32][1];
    {
        uint4 bb[JOIN_IN_PAD / 32][1];
        load_b(bb, net.m16[M_JOIN_B], wv);
        v5f4 acc[JT_RB][1];
        gemm(acc, bb, true);
        const float bias = net.b[LY.join_b.b + col];
#pragma unroll
        for (uint32_t rb = 0; rb < JT_RB; rb++)
#pragma unroll
            for (uint32_t v = 0; v < 4; v++) {
                const uint32_t row = r0 + rb * 16 + 4 * q + v;
                const float jp = row < rows ? Jp[(size_t)row * JW + col] : 0.0f;
                z[rb][0][v] = (jp + acc[rb][0][v]) + bias;
            }
    }
    for (uint32_t blk = 0; blk < JBLOCKS; blk++) {
        load_b(bw, net.m16[M_JOIN_W0 + blk], wv);
        to_operand(z, LN_JOIN + blk);
        v5f4 acc[JT_RB][1];
        gemm(acc, bw, false);
        __syncthreads();  // every wave has read the operand before the next one is written
        const float bias = net.b[LY.join_w[blk].b + col];
#pragma unroll
        for (uint32_t rb = 0; rb < JT_RB; rb++)
#pragma unroll
            for (uint32_t v = 0; v < 4; v++) z[rb][0][v] += acc[rb][0][v] + bias;
    }
    // h = LN_H(P + z join_out + b), 256 wide: column blocks 2 w and 2 w + 1
    uint4 bo[JW / 32][2];
    load_b(bo, net.m16[M_JOIN_OUT], 2 * wv);
    to_operand(z, LN_JOUT);
    v5f4 acc[JT_RB][2];
    gemm(acc, bo, false);
    float h[JT_RB][2][4];
#pragma unroll
    for (uint32_t rb = 0; rb < JT_RB; rb++)
#pragma unroll
        for (uint32_t cb = 0; cb < 2; cb++) {
            const uint32_t c2 = (2 * wv + cb) * 16 + i;
            const float bias = net.b[LY.join_out.b + c2];
#pragma unroll
            for (uint32_t v = 0; v < 4; v++) {
                const uint32_t row = r0 + rb * 16 + 4 * q + v;
                const float pv = row < rows ? P[(size_t)row * D + c2] : 0.0f;
                h[rb][cb][v] = (pv + acc[rb][cb][v]) + bias;
            }
        }
    row_stats(h, std::integral_constant<uint32_t, 2>{}, (float)D);
#pragma unroll
    for (uint32_t cb = 0; cb < 2; cb++) {
        const uint32_t c2 = (2 * wv + cb) * 16 + i;
        const float g = net.ln[LY.norm_g[LN_H] + c2], bt = net.ln[LY.norm_b[LN_H] + c2];
#pragma unroll
        for (uint32_t rb = 0; rb < JT_RB; rb++)
#pragma unroll
            for (uint32_t v = 0; v < 4; v++) {
                const uint32_t r = rb * 16 + 4 * q + v, row = r0 + r;
                if (row < rows) H[frag_off(row, c2, D)] = to16<PREC>((h[rb][cb][v] - mean[r]) * inv[r] * g + bt);
            }
    }
}

// ------------------------------------------------------ trunk on MFMA

constexpr int TT_ROWS = 2;                        // network rows per group of wavefronts
constexpr int TT_GROUPS = 2;                      // groups per workgroup
constexpr int TT_CELLS = TT_ROWS * HEXES;         // 74 hex cells
constexpr int TT_RB = (TT_CELLS + 15) / 16;       // 5 row blocks of 16 cells
constexpr int TT_WAVES = C / 16;                  // one 16-channel column block per wavefront
constexpr int TT_LD = 2 * C + 8;                  // LDS row stride of the 16-bit operand (halves)
constexpr int TT_BIN = 2 * C + LOOSE;             // board input width
constexpr int TT_SLD = D + 8;                     // LDS row stride of the per-row operand (halves)

// Net::board + join_cache (net.rs:474-730) for two network rows on the
// matrix cores: the mix (192 -> 96) and out (96 -> 96) products of every
// residual block run as 16x16x32 MFMA over the 74 hex cells (five 16-cell
// blocks), wavefront w owning channels 16 w .. 16 w + 15 with the residual
// stream x in its accumulator registers. The post-norm activations a stay in
// LDS in float32 (the neighbour sums and the mean / max pool read them); the
// GEMM A operand ([a, neighbours], then the mid-block activations) in LDS in
// 16 bits. The stem, the pool bias, the board vector and the join cache are
// one or two rows each and stay scalar, with rounded operands where the
// reference's fast mode runs them on tensor cores.
template <int PREC>
__global__ __launch_bounds__(TT_GROUPS * TT_WAVES * 64) __attribute__((amdgpu_waves_per_eu(3, 3))) void k_trunk_mfma(
    Net net, WaveIn in, WaveOut out) {  // twelve waves: three per SIMD, one workgroup per CU
    // Two groups of six wavefronts, each with its own pair of rows and its own
    // LDS below; they share only the barriers and the neighbour table.
    __shared__ __attribute__((aligned(16))) float aF_g[TT_GROUPS][TT_RB * 16][C];
    __shared__ __attribute__((aligned(16))) uint16_t A16_g[TT_GROUPS][TT_RB * 16 * TT_LD];
    __shared__ float part_g[TT_GROUPS][TT_WAVES][TT_RB * 16], part2_g[TT_GROUPS][TT_WAVES][TT_RB * 16];
    __shared__ __attribute__((aligned(16))) float mean_g[TT_GROUPS][TT_RB * 16], inv_g[TT_GROUPS][TT_RB * 16];
    __shared__ float gb_g[TT_GROUPS][TT_ROWS][C];
    __shared__ float loose_g[TT_GROUPS][TT_ROWS][LOOSE], tp_g[TT_GROUPS][TT_ROWS][C], glob_g[TT_GROUPS][TT_ROWS][C];
    // The A operand of the per-row products (pool bias, board vector, join
    // cache): one 16-row block whose rows past TT_ROWS stay zero.
    __shared__ __attribute__((aligned(16))) uint16_t S16_g[TT_GROUPS][16 * TT_SLD];
    __shared__ int occ_g[TT_GROUPS][TT_CELLS];
    __shared__ uint8_t nbc[TT_RB * 16][6];  // each cell's neighbour cells (the zero padding cell when off board)
    const uint32_t grp = threadIdx.x / (TT_WAVES * 64);
    float(&aF)[TT_RB * 16][C] = aF_g[grp];
    uint16_t* A16 = A16_g[grp];
    float(&part)[TT_WAVES][TT_RB * 16] = part_g[grp];
    float(&part2)[TT_WAVES][TT_RB * 16] = part2_g[grp];
    float* mean = mean_g[grp];
    float* inv = inv_g[grp];
    float(&gb)[TT_ROWS][C] = gb_g[grp];
    float(&loose)[TT_ROWS][LOOSE] = loose_g[grp];
    float(&tp)[TT_ROWS][C] = tp_g[grp];
    float(&glob)[TT_ROWS][C] = glob_g[grp];
    uint16_t* S16 = S16_g[grp];
    int* occ = occ_g[grp];
    // stem scratch in the operand's space: tokens, projected tokens, hex facts
    float* tok = (float*)A16;                           // [TT_ROWS][NTYPE][TYPE]
    float* proj = tok + TT_ROWS * NTYPE * TYPE;         // [TT_ROWS][NTYPE][C]
    float* facts = proj + TT_ROWS * NTYPE * C;          // [TT_CELLS][HEX_FACTS]
    static_assert(sizeof(float) * (TT_ROWS * NTYPE * (TYPE + C) + TT_CELLS * HEX_FACTS) <= sizeof(A16_g[0]),
                  "stem scratch");
    const uint32_t tid = threadIdx.x % (TT_WAVES * 64), wv = tid >> 6, l = tid & 63, q = l >> 4, i = l & 15;
    const uint32_t row0 = (blockIdx.x * TT_GROUPS + grp) * TT_ROWS;
    const uint32_t nrow = row0 < in.rows ? min((uint32_t)TT_ROWS, in.rows - row0) : 0;  // 0: an empty group
    const float* W = net.w;
    for (uint32_t x2 = tid; x2 < 16 * TT_SLD; x2 += TT_WAVES * 64) S16[x2] = 0;
    static_assert(TT_RB * 16 > TT_CELLS, "a zero padding cell stands for a missing neighbour");
    for (uint32_t x2 = threadIdx.x; x2 < TT_RB * 16 * 6; x2 += TT_GROUPS * TT_WAVES * 64) {
        const uint32_t cell = x2 / 6, d = x2 % 6;
        uint32_t n = TT_RB * 16 - 1;
        if (cell < TT_CELLS) {
            const uint32_t h = cell % HEXES, nh = net.nb[h * 6 + d];
            if (nh < HEXES) n = cell - h + nh;
        }
        nbc[cell][d] = (uint8_t)n;
    }
    // out[r][n] (r < TT_ROWS) of the per-row operand S16 (K columns) times Wt
    // (N outputs): this wave's 16-column blocks, one 16x16x32 MFMA per k step;
    // emit(r, n, acc) receives each valid entry.
    auto row_gemm = [&](const uint16_t* Wt, uint32_t K, uint32_t N, auto emit) {
        const uint32_t ks = K / 32;
        for (uint32_t cb = wv; cb < N / 16; cb += TT_WAVES) {
            v5f4 c = v5f4{0.0f, 0.0f, 0.0f, 0.0f};
            for (uint32_t st = 0; st < ks; st++) {
                const uint4 af = *(const uint4*)(S16 + i * TT_SLD + st * 32 + 8 * q);
                const uint4 bf = *(const uint4*)(Wt + ((size_t)cb * ks * 64 + (size_t)st * 64 + l) * 8);
                c = mma<PREC>(af, bf, c);
            }
            if (q == 0)
#pragma unroll
                for (uint32_t v = 0; v < TT_ROWS; v++) emit(v, cb * 16 + i, c[v]);
        }
    };
    // ---- stem (net.rs:474-543), float32 loops
    for (uint32_t x = tid; x < TT_ROWS * NTYPE * TYPE; x += TT_WAVES * 64) {
        const uint32_t rr = x / (NTYPE * TYPE), t = (x / TYPE) % NTYPE, j = x % TYPE;
        if (rr >= nrow) {  // the last workgroup's missing row: zeros
            tok[x] = 0.0f;
            continue;
        }
        const uint8_t* raw = in.raw + (size_t)(row0 + rr) * ROW_BYTES;
        const float* cards = out.cards + (size_t)in.row_job[row0 + rr] * 2 * NTYPE * TYPE;  // view 0
        float piles[PILE_COUNTS];
        for (uint32_t f = 0; f < PILE_COUNTS; f++) piles[f] = (float)raw[GR_PILES + t * PILE_COUNTS + f] / 5.0f;
        const float v = lin_out<PREC, false>(piles, PILE_COUNTS, W + LY.pile.w, TYPE, j, 0.0f, nullptr);
        tok[x] = v + (cards[(size_t)t * TYPE + j] + W[LY.seat + (t / NSLOT) * TYPE + j]);
    }
    for (uint32_t x = tid; x < TT_CELLS; x += TT_WAVES * 64) {
        const uint32_t rr = x / HEXES, h = x % HEXES;
        if (rr >= nrow) {
            occ[x] = -1;
            for (uint32_t f = 0; f < HEX_FACTS; f++) facts[x * HEX_FACTS + f] = 0.0f;
            continue;
        }
        const uint8_t* raw = in.raw + (size_t)(row0 + rr) * ROW_BYTES;
        const int owner = raw[GR_HEX_OWNER + h], marker = raw[GR_HEX_MARKER + h], sl = raw[GR_HEX_SLOT + h];
        float* fx = facts + x * HEX_FACTS;
        fx[0] = owner == 0 ? 1.0f : 0.0f;
        fx[1] = owner == 1 ? 1.0f : 0.0f;
        fx[2] = (float)raw[GR_HEX_HEIGHT + h] / 5.0f;
        fx[3] = marker == 0 ? 1.0f : 0.0f;
        fx[4] = marker == 1 ? 1.0f : 0.0f;
        fx[5] = (float)net.loc[h];
        occ[x] = owner < 2 && sl < (int)NSLOT ? owner * (int)NSLOT + sl : -1;
    }
    if (tid < TT_ROWS * LOOSE) {
        const uint32_t rr = tid / LOOSE, qq = tid % LOOSE;
        float v = 0.0f;
        if (rr < nrow) {
            const uint8_t* raw = in.raw + (size_t)(row0 + rr) * ROW_BYTES;
            if (qq < 12) {
                const uint32_t p = qq / 6, k = qq % 6;
                const int markers = raw[GR_MARKERS + p];
                if (k == 0) v = (float)markers / 6.0f;
                else if (k == 1) v = (float)(6 - markers) / 6.0f;
                else if (k == 2) v = (float)raw[GR_HAND + p] / 3.0f;
                else if (k == 3) v = (float)raw[GR_FD + p] / 21.0f;
                else if (k == 4) v = (float)raw[GR_BAG + p] / 21.0f;
                else v = raw[GR_INITIATIVE] == p ? 1.0f : 0.0f;
            } else if (qq == 12) {
                v = (float)((int)raw[GR_PLIES] | (int)raw[GR_PLIES + 1] << 8) / 256.0f;
            } else if (qq == 13) {
                v = raw[GR_INIT_MOVED] ? 1.0f : 0.0f;
            } else {
                v = raw[GR_TO_ACT] == 0 ? 1.0f : 0.0f;
            }
        }
        loose[rr][qq] = v;
    }
    // tok_stem's matrix (64 x 96 float32) staged in the activations' space,
    // which the stem does not use: one round of independent loads
    float* wtok = &aF[0][0];
    static_assert(TYPE * C <= sizeof(aF) / sizeof(float) && (TYPE * C) % (TT_WAVES * 64) == 0, "tok_stem staging");
#pragma unroll
    for (uint32_t k = 0; k < TYPE * C / (TT_WAVES * 64); k++)
        wtok[tid + k * TT_WAVES * 64] = W[LY.tok_stem.w + tid + k * TT_WAVES * 64];
    __syncthreads();
    {
        // tok_stem (float32, no bias): a thread's outputs tid + k * 384 share
        // the channel, so each weight is read once for all of them
        constexpr uint32_t NT = TT_WAVES * 64, NOUT = TT_ROWS * NTYPE * C / NT;
        static_assert(TT_ROWS * NTYPE * C % NT == 0 && NT % C == 0, "projection mapping");
        const uint32_t j = tid % C;
        float acc[NOUT];
#pragma unroll
        for (uint32_t k = 0; k < NOUT; k++) acc[k] = 0.0f;
#pragma unroll 8
        for (uint32_t p = 0; p < TYPE; p++) {
            const float wv2 = wtok[p * C + j];
#pragma unroll
            for (uint32_t k = 0; k < NOUT; k++) {
                const float a = tok[((tid + k * NT) / C) * TYPE + p];
                acc[k] = a != 0.0f ? acc[k] + a * wv2 : acc[k];
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < NOUT; k++) proj[tid + k * NT] = acc[k];
    }
    __syncthreads();
    for (uint32_t x = tid; x < TT_ROWS * C; x += TT_WAVES * 64) {
        const uint32_t rr = x / C, j = x % C;
        float v = 0.0f;
        for (uint32_t t = 0; t < NTYPE; t++) v += gelu_fast(proj[(rr * NTYPE + t) * C + j]) * (1.0f / (float)NTYPE);
        tp[rr][j] = v;
        glob[rr][j] = lin_out<PREC, false>(loose[rr], LOOSE, W + LY.glob_stem.w, C, j, 0.0f, nullptr);
    }
    __syncthreads();
    const uint32_t col = wv * 16 + i;
    float x[TT_RB][4];
    float whex[HEX_FACTS];
#pragma unroll
    for (uint32_t f = 0; f < HEX_FACTS; f++) whex[f] = W[LY.hex_stem.w + f * C + col];
    const float bhex = net.b[LY.hex_stem.b + col];
#pragma unroll
    for (uint32_t rb = 0; rb < TT_RB; rb++)
#pragma unroll
        for (uint32_t v = 0; v < 4; v++) {
            const uint32_t cell = rb * 16 + 4 * q + v;
            float val = 0.0f;
            if (cell < TT_CELLS) {
                const uint32_t rr = cell / HEXES, h = cell % HEXES;
                float st = 0.0f;  // hex_stem: the float32 loop, then the bias
#pragma unroll
                for (uint32_t f = 0; f < HEX_FACTS; f++) {
                    const float a = facts[cell * HEX_FACTS + f];
                    st = a != 0.0f ? st + a * whex[f] : st;
                }
                st += bhex;
                const float o = occ[cell] >= 0 ? proj[(rr * NTYPE + occ[cell]) * C + col] : 0.0f;
                val = st + (((o + W[LY.pos + h * C + col]) + glob[rr][col]) + tp[rr][col]);
            }
            x[rb][v] = val;
        }
    __syncthreads();  // the stem scratch is free: the operand space is reused below
    // Per-cell LayerNorm statistics of a 96-wide stream held as [rb][v] per lane
    // (channel `col`): each wavefront's sum and sum of squared deviations from
    // its own 16-channel mean, combined over the six wavefronts by the
    // pairwise-variance formula (Chan, Golub and LeVeque): one exchange
    // through LDS instead of one per pass.
    auto cell_stats = [&](float (&z)[TT_RB][4]) {
#pragma unroll
        for (uint32_t rb = 0; rb < TT_RB; rb++)
#pragma unroll
            for (uint32_t v = 0; v < 4; v++) {
                const uint32_t cell = rb * 16 + 4 * q + v;
                const float sw = row16_sum(z[rb][v]);
                const float d = z[rb][v] - sw * (1.0f / 16.0f);
                const float m2 = row16_sum(d * d);
                if (i == 0) {
                    part[wv][cell] = sw;
                    part2[wv][cell] = m2;
                }
            }
        __syncthreads();
        if (tid < TT_RB * 16) {
            float t = 0.0f;
            for (uint32_t w2 = 0; w2 < TT_WAVES; w2++) t += part[w2][tid];
            const float m = t * (1.0f / (float)C);
            float m2 = 0.0f;
            for (uint32_t w2 = 0; w2 < TT_WAVES; w2++) {
                const float dm = part[w2][tid] * (1.0f / 16.0f) - m;
                m2 += part2[w2][tid] + 16.0f * dm * dm;
            }
            mean[tid] = m;
            inv[tid] = 1.0f / sqrtf(m2 * (1.0f / (float)C) + 1e-5f);
        }
        __syncthreads();
    };
    // gelu(LayerNorm(z)) of this lane's four cells 4 q .. 4 q + 3 of row block rb (their mean and
    // 1 / std read as one 16-byte LDS load each), gain g and bias bt of channel `col`
    auto norm4 = [&](const float (&z)[4], uint32_t rb, float g, float bt, float (&out)[4]) {
        const float4 m4 = *(const float4*)&mean[rb * 16 + 4 * q], i4 = *(const float4*)&inv[rb * 16 + 4 * q];
        const float m[4] = {m4.x, m4.y, m4.z, m4.w}, iv[4] = {i4.x, i4.y, i4.z, i4.w};
#pragma unroll
        for (uint32_t v = 0; v < 4; v++) out[v] = gelu_fast((z[v] - m[v]) * iv[v] * g + bt);
    };
    // This wave's B fragments (its 16-column block) of a K-column matrix,
    // loaded ahead of the product that uses them.
    auto load_b = [&](uint4* bf, const uint16_t* Wt, auto kk) {
        constexpr uint32_t ks = decltype(kk)::value / 32;
#pragma unroll
        for (uint32_t st = 0; st < ks; st++) bf[st] = *(const uint4*)(Wt + ((size_t)wv * ks * 64 + (size_t)st * 64 + l) * 8);
    };
    // acc[rb] = A16 (K columns) B^T for this wave's column block.
    auto gemm = [&](float (&acc)[TT_RB][4], const uint4* bf, auto kk) {
        constexpr uint32_t ks = decltype(kk)::value / 32;
        v5f4 c[TT_RB];
#pragma unroll
        for (uint32_t rb = 0; rb < TT_RB; rb++) c[rb] = v5f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t st = 0; st < ks; st++)
#pragma unroll
            for (uint32_t rb = 0; rb < TT_RB; rb++) {
                const uint4 af = *(const uint4*)(A16 + (rb * 16 + i) * TT_LD + st * 32 + 8 * q);
                c[rb] = mma<PREC>(af, bf[st], c[rb]);
            }
#pragma unroll
        for (uint32_t rb = 0; rb < TT_RB; rb++)
#pragma unroll
            for (uint32_t v = 0; v < 4; v++) acc[rb][v] = c[rb][v];
    };
    using K96 = std::integral_constant<uint32_t, C>;
    using K192 = std::integral_constant<uint32_t, 2 * C>;
    for (uint32_t blk = 0; blk < BLOCKS; blk++) {
        uint4 bmix[2 * C / 32], bpool[2 * C / 32];
        cell_stats(x);
        {
            const float g = net.ln[LY.norm_g[2 * blk] + col], bt = net.ln[LY.norm_b[2 * blk] + col];
#pragma unroll
            for (uint32_t rb = 0; rb < TT_RB; rb++) {
                float a4[4];
                norm4(x[rb], rb, g, bt, a4);
#pragma unroll
                for (uint32_t v = 0; v < 4; v++) {
                    const uint32_t cell = rb * 16 + 4 * q + v;
                    const float a = cell < TT_CELLS ? a4[v] : 0.0f;
                    aF[cell][col] = a;
                    A16[cell * TT_LD + col] = to16<PREC>(a);
                }
            }
        }
        __syncthreads();
        load_b(bpool, net.m16[M_POOL0 + blk], K192{});
        load_b(bmix, net.m16[M_MIX0 + blk], K192{});
        // neighbour sums (zero start, directions in board order) into the
        // operand's upper half, and the mean / max pool of each row
        {
            // a thread per (cell, quarter of the channels): 24 channels as six
            // float4 reads per neighbour, summed per channel from zero in
            // board direction order (off board reads the zero cell)
            constexpr uint32_t QW = C / 4;
            static_assert(TT_RB * 16 * 4 <= TT_WAVES * 64 && QW % 8 == 0, "neighbour mapping");
            if (tid < TT_RB * 16 * 4) {
                const uint32_t cell = tid >> 2;
                uint32_t nb[6];
#pragma unroll
                for (int d = 0; d < 6; d++) nb[d] = nbc[cell][d];
                // 8 channels at a time: two float4 per neighbour, one 16-byte store
#pragma unroll 1
                for (uint32_t c0 = (tid & 3) * QW; c0 < (tid & 3) * QW + QW; c0 += 8) {
                    float4 lo = make_float4(0.0f, 0.0f, 0.0f, 0.0f), hi = lo;
#pragma unroll
                    for (int d = 0; d < 6; d++) {
                        const float4 a0 = *(const float4*)&aF[nb[d]][c0], a1 = *(const float4*)&aF[nb[d]][c0 + 4];
                        lo.x += a0.x;
                        lo.y += a0.y;
                        lo.z += a0.z;
                        lo.w += a0.w;
                        hi.x += a1.x;
                        hi.y += a1.y;
                        hi.z += a1.z;
                        hi.w += a1.w;
                    }
                    uint4 w4;
                    w4.x = (uint32_t)to16<PREC>(lo.x) | (uint32_t)to16<PREC>(lo.y) << 16;
                    w4.y = (uint32_t)to16<PREC>(lo.z) | (uint32_t)to16<PREC>(lo.w) << 16;
                    w4.z = (uint32_t)to16<PREC>(hi.x) | (uint32_t)to16<PREC>(hi.y) << 16;
                    w4.w = (uint32_t)to16<PREC>(hi.z) | (uint32_t)to16<PREC>(hi.w) << 16;
                    *(uint4*)(A16 + cell * TT_LD + C + c0) = w4;
                }
            }
        }
        for (uint32_t x2 = tid; x2 < TT_ROWS * C; x2 += TT_WAVES * 64) {
            const uint32_t rr = x2 / C, j = x2 % C;
            float mn = 0.0f, top = -INFINITY;
            for (uint32_t h = 0; h < HEXES; h++) {
                const float v = aF[rr * HEXES + h][j];
                mn += v * (1.0f / (float)HEXES);
                top = fmaxf(top, v);
            }
            S16[rr * TT_SLD + j] = to16<PREC>(mn);
            S16[rr * TT_SLD + C + j] = to16<PREC>(top);
        }
        __syncthreads();
        {  // the pool bias: one 16-column block per wave (C / 16 = TT_WAVES)
            v5f4 c = v5f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t st = 0; st < 2 * C / 32; st++)
                c = mma<PREC>(*(const uint4*)(S16 + i * TT_SLD + st * 32 + 8 * q), bpool[st], c);
            if (q == 0)
#pragma unroll
                for (uint32_t v = 0; v < TT_ROWS; v++) gb[v][col] = c[v] + net.b[LY.pool[blk].b + col];
        }
        float y[TT_RB][4];
        gemm(y, bmix, K192{});
        uint4 bout[C / 32];
        load_b(bout, net.m16[M_OUT0 + blk], K96{});
        __syncthreads();  // gb written; every wave has read the operand
        {
            const float bm = net.b[LY.mix[blk].b + col];
#pragma unroll
            for (uint32_t rb = 0; rb < TT_RB; rb++)
#pragma unroll
                for (uint32_t v = 0; v < 4; v++) {
                    const uint32_t cell = rb * 16 + 4 * q + v;
                    y[rb][v] = (y[rb][v] + bm) + (cell < TT_CELLS ? gb[cell / HEXES][col] : 0.0f);
                }
        }
        cell_stats(y);
        {
            const float g = net.ln[LY.norm_g[2 * blk + 1] + col], bt = net.ln[LY.norm_b[2 * blk + 1] + col];
#pragma unroll
            for (uint32_t rb = 0; rb < TT_RB; rb++) {
                float a4[4];
                norm4(y[rb], rb, g, bt, a4);
#pragma unroll
                for (uint32_t v = 0; v < 4; v++) {
                    const uint32_t cell = rb * 16 + 4 * q + v;
                    A16[cell * TT_LD + col] = to16<PREC>(cell < TT_CELLS ? a4[v] : 0.0f);
                }
            }
        }
        __syncthreads();
        float z[TT_RB][4];
        gemm(z, bout, K96{});
        __syncthreads();  // every wave has read the operand before the next block writes it
        const float bo = net.b[LY.out[blk].b + col];
#pragma unroll
        for (uint32_t rb = 0; rb < TT_RB; rb++)
#pragma unroll
            for (uint32_t v = 0; v < 4; v++) x[rb][v] += z[rb][v] + bo;
    }
    cell_stats(x);
    {
        const float g = net.ln[LY.norm_g[LN_TRUNK] + col], bt = net.ln[LY.norm_b[LN_TRUNK] + col];
#pragma unroll
        for (uint32_t rb = 0; rb < TT_RB; rb++) {
            float a4[4];
            norm4(x[rb], rb, g, bt, a4);
#pragma unroll
            for (uint32_t v = 0; v < 4; v++) {
                const uint32_t cell = rb * 16 + 4 * q + v;
                aF[cell][col] = cell < TT_CELLS ? a4[v] : 0.0f;
            }
        }
    }
    __syncthreads();
    // the board vector (net.rs:704-722) and its join projection, per row:
    // [mean, max, loose] (zero-padded to whole k steps) as the operand
    for (uint32_t x2 = tid; x2 < TT_ROWS * C; x2 += TT_WAVES * 64) {
        const uint32_t rr = x2 / C, j = x2 % C;
        float mn = 0.0f, top = -INFINITY;
        for (uint32_t h = 0; h < HEXES; h++) {
            const float v = aF[rr * HEXES + h][j];
            mn += v * (1.0f / (float)HEXES);
            top = fmaxf(top, v);
        }
        S16[rr * TT_SLD + j] = to16<PREC>(mn);
        S16[rr * TT_SLD + C + j] = to16<PREC>(top);
    }
    for (uint32_t x2 = tid; x2 < TT_ROWS * (kpad_dev(TT_BIN) - 2 * C); x2 += TT_WAVES * 64) {
        const uint32_t rr = x2 / (kpad_dev(TT_BIN) - 2 * C), qq = x2 % (kpad_dev(TT_BIN) - 2 * C);
        S16[rr * TT_SLD + 2 * C + qq] = to16<PREC>(qq < LOOSE ? loose[rr][qq] : 0.0f);
    }
    __syncthreads();
    float* Pf = aF[0];  // the two rows' board vectors, float32, in the activations' space
    row_gemm(net.m16[M_BOARD], kpad_dev(TT_BIN), D, [&](uint32_t r, uint32_t n, float acc) {
        const float v = acc + net.b[LY.board_out.b + n];
        Pf[r * D + n] = v;
        if (r < nrow) out.P[(size_t)(row0 + r) * D + n] = v;
    });
    __syncthreads();
    for (uint32_t x2 = tid; x2 < TT_ROWS * D; x2 += TT_WAVES * 64) S16[(x2 / D) * TT_SLD + x2 % D] = to16<PREC>(Pf[x2]);
    __syncthreads();
    row_gemm(net.m16[M_JOIN_P], D, JW, [&](uint32_t r, uint32_t n, float acc) {
        if (r < nrow) out.Jp[(size_t)(row0 + r) * JW + n] = acc;
    });
}

// The 16-bit query input (fragment-major, K = JOIN_IN_PAD) back to float32
// rows of JOIN_IN for the rounded-operand join.
template <int PREC>
__global__ void k_unpack_x(const uint16_t* X, uint32_t rows, float* out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows * JOIN_IN) return;
    const uint32_t r = (uint32_t)(i / JOIN_IN), k = (uint32_t)(i % JOIN_IN);
    const uint16_t v = X[frag_off(r, k, JOIN_IN_PAD)];
    out[i] = PREC == WC_F16 ? (float)__builtin_bit_cast(_Float16, v) : __uint_as_float((uint32_t)v << 16);
}

}  // namespace

static_assert(sizeof(Net) < 1024, "kernel argument");

void launch_build(int precision, const Net& net, const WaveIn& in, const WaveOut& out, hipStream_t s) {
    const uint32_t tokens = in.jobs * 2 * NTYPE;
#define V5_BUILD(P)                                                                                          \
    do {                                                                                                     \
        if (tokens) hipLaunchKernelGGL(k_cards<P>, dim3(tokens), dim3(NBLK), 0, s, net, in, out);            \
        if (in.ncfg) hipLaunchKernelGGL(k_configs<P>, dim3(in.ncfg), dim3(NBLK), 0, s, net, in, out);        \
        if (in.rows && P != WC_PRECISE && net.m16[M_MIX0])                                                   \
            hipLaunchKernelGGL(k_trunk_mfma<P>, dim3((in.rows + TT_GROUPS * TT_ROWS - 1) / (TT_GROUPS * TT_ROWS)), \
                               dim3(TT_GROUPS * TT_WAVES * 64), 0, s, net, in, out);                         \
        else if (in.rows)                                                                                    \
            hipLaunchKernelGGL(k_trunk<P>, dim3(in.rows), dim3(NBLK), 0, s, net, in, out);                   \
    } while (0)
    if (precision == WC_PRECISE)
        V5_BUILD(WC_PRECISE);
    else if (precision == WC_F16)
        V5_BUILD(WC_F16);
    else
        V5_BUILD(WC_BF16);
#undef V5_BUILD
}

void launch_join(int precision, const Net& net, uint32_t rows, const void* X, const float* P, const float* Jp,
                 void* H, float* xf, hipStream_t s) {
    if (!rows) return;
    const dim3 g((rows + JROWS - 1) / JROWS);
    if (precision == WC_PRECISE) {
        hipLaunchKernelGGL(k_join<WC_PRECISE>, g, dim3(JW), 0, s, net, rows, (const float*)X, P, Jp, (float*)H);
        return;
    }
    if (net.m16[M_JOIN_B]) {  // the matrix-core join
        const dim3 gt((rows + JT_ROWS - 1) / JT_ROWS);
        if (precision == WC_F16)
            hipLaunchKernelGGL(k_join_mfma<WC_F16>, gt, dim3(JT_WAVES * 64), 0, s, net, rows, (const uint16_t*)X, P,
                               Jp, (uint16_t*)H);
        else
            hipLaunchKernelGGL(k_join_mfma<WC_BF16>, gt, dim3(JT_WAVES * 64), 0, s, net, rows, (const uint16_t*)X, P,
                               Jp, (uint16_t*)H);
        return;
    }
    const size_t n = (size_t)rows * JOIN_IN;
    const dim3 gx((unsigned)((n + 255) / 256));
    if (precision == WC_F16) {
        hipLaunchKernelGGL(k_unpack_x<WC_F16>, gx, dim3(256), 0, s, (const uint16_t*)X, rows, xf);
        hipLaunchKernelGGL(k_join<WC_F16>, g, dim3(JW), 0, s, net, rows, xf, P, Jp, (float*)H);
    } else {
        hipLaunchKernelGGL(k_unpack_x<WC_BF16>, gx, dim3(256), 0, s, (const uint16_t*)X, rows, xf);
        hipLaunchKernelGGL(k_join<WC_BF16>, g, dim3(JW), 0, s, net, rows, xf, P, Jp, (float*)H);
    }
}

}  // namespace v5
}  // namespace wc
