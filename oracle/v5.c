/*
 * ORACLE — test infrastructure only (see oracle.c's header).
 *
 * The v5 leaf network (engine/src/net.rs) in the CPU loop order of net.rs:
 *   - every Lin is the row-major `gemm` of net.rs:102-122 (per output, start
 *     from zero or from the existing value, add a*w over ascending inputs,
 *     skipping zero inputs) followed by Lin::bias (net.rs:339-348);
 *   - LayerNorm in net.rs:380-405 order: mean = sum / width, var = sum of
 *     squared deviations / width, inv = 1 / sqrt(var + 1e-5),
 *     y = (x - mean) * inv * g + b, then GELU where `apply` asks for it;
 *   - GELU in net.rs:125-128 order: 0.5 x (1 + tanh(0.79788456 (x + 0.044715 x x x))).
 *
 * The public inputs are expanded from the GPU row bytes exactly as the
 * reference's device expansion defines them (engine/src/gpu/wave_kernels.cu
 * hex_facts / loose_feature, 254-296; the same values write_public_features_raw
 * produces, rebel.rs:1144-1233).
 *
 * tanh. The reference's CPU net calls the C library's tanhf through Rust's
 * f32::tanh. This restatement evaluates tanh by its own formula,
 * tanh|x| = (1 - t) / (1 + t) with t = exp(-2|x|), and exp by Cody-Waite range
 * reduction (x = n ln2 + r, ln2 split into a 15-bit head and a tail) and the
 * degree-7 Taylor polynomial of e^r on |r| <= ln2/2 scaled by 2^n: only
 * additions, multiplications, one division, rint and ldexp, so the GPU
 * executor evaluates it to the same bits. The absolute error of this tanh is
 * a few units in the last place of 1, which is what GELU's (1 + tanh) needs.
 * With libm_tanh set, GELU calls tanhf instead (the reference's own
 * arithmetic): tests/test_v5_pins.py measures how far that moves a solve.
 *
 * Arithmetic models (NET_*): F32 is the CPU loop bit for bit. In the reduced
 * models the GEMMs the reference runs on tensor cores in its fast mode
 * (device.rs gemm(): cards, configs, trunk blocks, board, join) take operands
 * rounded to the 16-bit type and a wide (double) or, for F16A and BF16A
 * (bfloat16 operands), an ascending float32 sum, then the existing value (for
 * an accumulating GEMM) and the bias; the small stem products (pile, hex, token, global) stay float32 loops
 * in every model, as the device computes them.
 */
#include "v5.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum { NET_EMPTY = 0, NET_F32 = 1, NET_F16 = 2, NET_BF16 = 3, NET_F16A = 4, NET_F16X = 5, NET_F32W = 6, NET_BF16A = 7 };

float oracle_round_f16(float x);
float oracle_round_bf16(float x);

/* ----------------------------------------------------------------- board */

/* engine/src/board.rs:1-6,14-28: the radius-3 hexagon around (3,3), hexes in
 * row-major (y, then x) order of their axial coordinates. */
static const int NB_OFF[6][2] = {{1, 0}, {-1, 0}, {0, 1}, {0, -1}, {1, -1}, {-1, 1}};
static const int LOC[10][2] = {{4, 0}, {6, 1}, {0, 5}, {2, 6}, {2, 1}, {3, 2}, {5, 3}, {1, 3}, {3, 4}, {4, 5}};

static int g_board_ready;
static int g_hx[V5_HEXES], g_hy[V5_HEXES];
static int g_nb[V5_HEXES][6]; /* neighbour hex or -1 */
static float g_loc[V5_HEXES];

static int valid_coord(int x, int y) { return abs(x - 3) <= 3 && abs(y - 3) <= 3 && abs(x + y - 6) <= 3; }
static int hex_at(int x, int y) {
    for (int h = 0; h < V5_HEXES; h++)
        if (g_hx[h] == x && g_hy[h] == y) return h;
    return -1;
}
static void board_init(void) {
    if (g_board_ready) return;
    int n = 0;
    for (int y = 0; y <= 6; y++)
        for (int x = 0; x <= 6; x++)
            if (valid_coord(x, y)) {
                g_hx[n] = x;
                g_hy[n] = y;
                n++;
            }
    for (int h = 0; h < V5_HEXES; h++) {
        for (int d = 0; d < 6; d++) g_nb[h][d] = hex_at(g_hx[h] + NB_OFF[d][0], g_hy[h] + NB_OFF[d][1]);
        g_loc[h] = 0.0f;
    }
    for (int l = 0; l < 10; l++) g_loc[hex_at(LOC[l][0], LOC[l][1])] = 1.0f;
    g_board_ready = 1;
}

/* The board as the pins see it: neighbours (-1 = off board) and locations. */
void oracle_v5_board_geometry(int32_t* nb, float* loc) {
    board_init();
    for (int h = 0; h < V5_HEXES; h++) {
        for (int d = 0; d < 6; d++) nb[6 * h + d] = g_nb[h][d];
        loc[h] = g_loc[h];
    }
}

/* ---------------------------------------------------------------- layout */

typedef struct {
    size_t w, b;
    uint32_t i, o;
    int bias;
} Span;

typedef struct {
    size_t w, b, ln;
} Cursor;

static Span lin(Cursor* c, uint32_t i, uint32_t o, int bias) {
    Span s = {c->w, bias ? c->b : 0, i, o, bias};
    c->w += (size_t)i * o;
    if (bias) c->b += o;
    return s;
}
static size_t embed(Cursor* c, size_t n) {
    size_t at = c->w;
    c->w += n;
    return at;
}

typedef struct {
    Span card[2], pile;
    size_t seat;
    Span hex_stem, tok_stem;
    size_t pos;
    Span glob_stem;
    Span mix[V5_BLOCKS], poolm[V5_BLOCKS], out[V5_BLOCKS];
    Span board_out, cfg1, cfg_f, cfg_g, cfg_m, join_p, join_b, join_w[V5_JBLOCKS], join_out;
    size_t value_bias;
    size_t ng[V5_NORMS], nbeta[V5_NORMS];
    uint32_t nwidth[V5_NORMS];
    size_t w_len, b_len, ln_len;
} Layout;

/* NetLayout::new (net.rs:272-316), in blob order. */
static void layout(Layout* L) {
    Cursor c = {0, 0, 0};
    L->card[0] = lin(&c, V5_CARD_FEATS, V5_TYPE, 1);
    L->card[1] = lin(&c, V5_TYPE, V5_TYPE, 1);
    L->pile = lin(&c, V5_PILE_COUNTS, V5_TYPE, 0);
    L->seat = embed(&c, 2 * V5_TYPE);
    L->hex_stem = lin(&c, V5_HEX_FACTS, V5_C, 1);
    L->tok_stem = lin(&c, V5_TYPE, V5_C, 0);
    L->pos = embed(&c, (size_t)V5_HEXES * V5_C);
    L->glob_stem = lin(&c, V5_LOOSE, V5_C, 0);
    for (int i = 0; i < V5_BLOCKS; i++) {
        L->mix[i] = lin(&c, 2 * V5_C, V5_C, 1);
        L->poolm[i] = lin(&c, 2 * V5_C, V5_C, 1);
        L->out[i] = lin(&c, V5_C, V5_C, 1);
    }
    L->board_out = lin(&c, 2 * V5_C + V5_LOOSE, V5_D, 1);
    L->cfg1 = lin(&c, 3 + V5_TYPE, V5_CFGH, 1);
    L->cfg_f = lin(&c, V5_CFGH, V5_D, 1);
    L->cfg_g = lin(&c, V5_CFGH, V5_POOL, 1);
    L->cfg_m = lin(&c, V5_TYPE, 3 * V5_POOL, 0);
    L->join_p = lin(&c, V5_D, V5_JW, 0);
    L->join_b = lin(&c, V5_JOIN_IN, V5_JW, 1);
    for (int i = 0; i < V5_JBLOCKS; i++) L->join_w[i] = lin(&c, V5_JW, V5_JW, 1);
    L->join_out = lin(&c, V5_JW, V5_D, 1);
    L->value_bias = c.b;
    c.b += 1;
    /* norm_widths (net.rs:233-242) */
    int k = 0;
    for (int i = 0; i < V5_BLOCKS; i++) {
        L->nwidth[k++] = V5_C;
        L->nwidth[k++] = V5_C;
    }
    L->nwidth[k++] = V5_C;    /* trunk */
    L->nwidth[k++] = V5_CFGH; /* config */
    for (int i = 0; i < V5_JBLOCKS; i++) L->nwidth[k++] = V5_JW;
    L->nwidth[k++] = V5_JW; /* join output */
    L->nwidth[k++] = V5_D;  /* h */
    for (int i = 0; i < V5_NORMS; i++) {
        L->ng[i] = c.ln;
        L->nbeta[i] = c.ln + L->nwidth[i];
        c.ln += 2 * (size_t)L->nwidth[i];
    }
    L->w_len = c.w;
    L->b_len = c.b;
    L->ln_len = c.ln;
}

void v5_sizes(size_t* nw, size_t* nb, size_t* nln) {
    Layout L;
    layout(&L);
    *nw = L.w_len;
    *nb = L.b_len;
    *nln = L.ln_len;
}

/* Norm indices (net.rs:214-219). */
static int ln_block(int i, int half) { return 2 * i + half; }
enum { LN_TRUNK = 2 * V5_BLOCKS, LN_CFG = LN_TRUNK + 1, LN_JOIN = LN_CFG + 1, LN_JOUT = LN_JOIN + V5_JBLOCKS,
       LN_H = LN_JOUT + 1 };

struct V5 {
    int mode, libm_tanh;
    Layout L;
    const float *w, *b, *ln;
    float* wq; /* the 16-bit models' rounded matrix copy */
};

static int reduced(const V5* n) { return n->mode != NET_F32; }
static int rounded_ops(const V5* n) {
    return n->mode == NET_F16 || n->mode == NET_BF16 || n->mode == NET_F16A || n->mode == NET_BF16A;
}
/* The models that sum in float32 in ascending order (the others in double). */
static int ascending(const V5* n) { return n->mode == NET_F16A || n->mode == NET_BF16A; }
static float qv(const V5* n, float x) {
    if (n->mode == NET_F16 || n->mode == NET_F16A) return oracle_round_f16(x);
    if (n->mode == NET_BF16 || n->mode == NET_BF16A) return oracle_round_bf16(x);
    return x;
}

V5* v5_new(int mode, const float* w, size_t nw, const float* b, size_t nb, const float* ln, size_t nln,
           int libm_tanh, char* err, size_t errlen) {
    board_init();
    if (mode != NET_F32 && mode != NET_F16 && mode != NET_BF16 && mode != NET_F16A && mode != NET_F32W &&
        mode != NET_BF16A) {
        snprintf(err, errlen, "the v5 restatement models F32, F16, BF16, F16A, BF16A and F32W");
        return NULL;
    }
    V5* n = (V5*)calloc(1, sizeof *n);
    layout(&n->L);
    if (nw != n->L.w_len || nb != n->L.b_len || nln != n->L.ln_len) {
        snprintf(err, errlen, "v5 weights: got %zu/%zu/%zu floats, want %zu/%zu/%zu", nw, nb, nln, n->L.w_len,
                 n->L.b_len, n->L.ln_len);
        free(n);
        return NULL;
    }
    n->mode = mode;
    n->libm_tanh = libm_tanh;
    n->w = w;
    n->b = b;
    n->ln = ln;
    if (rounded_ops(n)) {
        n->wq = (float*)malloc(nw * sizeof(float));
        for (size_t k = 0; k < nw; k++) n->wq[k] = qv(n, w[k]);
    }
    return n;
}

void v5_free(V5* n) {
    if (!n) return;
    free(n->wq);
    free(n);
}

/* ------------------------------------------------------------ arithmetic */

/* e^x for x <= 0 (Cody-Waite reduction, degree-7 Taylor polynomial). */
static float exp_neg(float x) {
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

static float own_tanh(float x) {
    const float a = fabsf(x);
    if (a > 20.0f) return x > 0.0f ? 1.0f : -1.0f;
    const float t = exp_neg(-2.0f * a);
    const float y = (1.0f - t) / (1.0f + t);
    return x < 0.0f ? -y : y;
}

float v5_gelu(const V5* n, float x) {
    const float inner = 0.79788456f * (x + 0.044715f * x * x * x);
    return 0.5f * x * (1.0f + (n->libm_tanh ? tanhf(inner) : own_tanh(inner)));
}

/* y = init (or 0) + x W (row-major [i x o]), then + bias: `gemm` then
 * Lin::bias. `fast` marks a product the reference's fast mode runs on tensor
 * cores (the reduced models round its operands). */
static void apply_lin(const V5* n, Span s, int fast, const float* x, const float* init, float* y) {
    const float* bias = s.bias ? n->b + s.b : NULL;
    if (!fast || !reduced(n)) {
        const float* W = n->w + s.w;
        for (uint32_t j = 0; j < s.o; j++) y[j] = init ? init[j] : 0.0f;
        for (uint32_t p = 0; p < s.i; p++) {
            const float a = x[p];
            if (a == 0.0f) continue;
            const float* row = W + (size_t)p * s.o;
            for (uint32_t j = 0; j < s.o; j++) y[j] += a * row[j];
        }
        if (bias)
            for (uint32_t j = 0; j < s.o; j++) y[j] += bias[j];
        return;
    }
    const float* W = (n->wq ? n->wq : n->w) + s.w;
    if (ascending(n)) {
        float* acc = (float*)calloc(s.o, sizeof(float));
        for (uint32_t p = 0; p < s.i; p++) {
            const float a = qv(n, x[p]);
            if (a == 0.0f) continue;
            const float* row = W + (size_t)p * s.o;
            for (uint32_t j = 0; j < s.o; j++) acc[j] += a * row[j];
        }
        for (uint32_t j = 0; j < s.o; j++) {
            float v = acc[j];
            if (init) v = init[j] + v;
            if (bias) v += bias[j];
            y[j] = v;
        }
        free(acc);
        return;
    }
    double* acc = (double*)calloc(s.o, sizeof(double));
    for (uint32_t p = 0; p < s.i; p++) {
        const double a = (double)qv(n, x[p]);
        if (a == 0.0) continue;
        const float* row = W + (size_t)p * s.o;
        for (uint32_t j = 0; j < s.o; j++) acc[j] += a * (double)row[j];
    }
    for (uint32_t j = 0; j < s.o; j++) {
        float v = (float)acc[j];
        if (init) v = init[j] + v;
        if (bias) v += bias[j];
        y[j] = v;
    }
    free(acc);
}

/* Norm::apply (act) or Norm::plain over one row (net.rs:380-405). */
static void norm(const V5* n, int which, float* x, int act) {
    const uint32_t width = n->L.nwidth[which];
    const float* g = n->ln + n->L.ng[which];
    const float* bt = n->ln + n->L.nbeta[which];
    float sum = 0.0f;
    for (uint32_t j = 0; j < width; j++) sum += x[j];
    const float mean = sum / (float)width;
    float sq = 0.0f;
    for (uint32_t j = 0; j < width; j++) sq += (x[j] - mean) * (x[j] - mean);
    const float var = sq / (float)width;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
    for (uint32_t j = 0; j < width; j++) {
        const float v = (x[j] - mean) * inv * g[j] + bt[j];
        x[j] = act ? v5_gelu(n, v) : v;
    }
}

/* --------------------------------------------------------- public inputs */

enum { GR_HEX_OWNER = 0, GR_HEX_SLOT = 37, GR_HEX_HEIGHT = 74, GR_HEX_MARKER = 111, GR_PILES = 148,
       GR_MARKERS = 188, GR_HAND = 190, GR_FD = 192, GR_BAG = 194, GR_INITIATIVE = 196, GR_INIT_MOVED = 197,
       GR_TO_ACT = 198, GR_PLIES = 199 };
#define CNORM 5.0f       /* rebel.rs:74 */
#define MAX_COINS 21.0f  /* rebel.rs:883 */
#define MAX_PLIES 256.0f /* state.rs:13, MAX_MAIN_PLAYS */

/* Seat-zero view of hex h: six facts and the occupant's coin type (-1: none)
 * (wave_kernels.cu hex_facts; rebel.rs:1174-1192). */
static void hex_facts(const uint8_t* src, int h, float* out, int* occupant) {
    const int owner = src[GR_HEX_OWNER + h], marker = src[GR_HEX_MARKER + h], slot = src[GR_HEX_SLOT + h];
    out[0] = owner == 0 ? 1.0f : 0.0f;
    out[1] = owner == 1 ? 1.0f : 0.0f;
    out[2] = (float)src[GR_HEX_HEIGHT + h] / CNORM;
    out[3] = marker == 0 ? 1.0f : 0.0f;
    out[4] = marker == 1 ? 1.0f : 0.0f;
    out[5] = g_loc[h];
    *occupant = owner < 2 && slot < V5_NSLOT ? owner * V5_NSLOT + slot : -1;
}

/* Seat-zero loose scalars (wave_kernels.cu loose_feature; rebel.rs:1211-1231). */
static void loose_features(const uint8_t* src, float* out) {
    for (int j = 0; j < 12; j++) {
        const int p = j / 6, k = j % 6;
        const int markers = src[GR_MARKERS + p];
        float v;
        if (k == 0) v = (float)markers / 6.0f;
        else if (k == 1) v = (float)(6 - markers) / 6.0f;
        else if (k == 2) v = (float)src[GR_HAND + p] / 3.0f;
        else if (k == 3) v = (float)src[GR_FD + p] / MAX_COINS;
        else if (k == 4) v = (float)src[GR_BAG + p] / MAX_COINS;
        else v = src[GR_INITIATIVE] == p ? 1.0f : 0.0f;
        out[j] = v;
    }
    const int plies = src[GR_PLIES] | (int)src[GR_PLIES + 1] << 8;
    out[12] = (float)plies / MAX_PLIES;
    out[13] = src[GR_INIT_MOVED] ? 1.0f : 0.0f;
    out[14] = src[GR_TO_ACT] == 0 ? 1.0f : 0.0f;
}

/* View v's token t is physical coin type (wave_kernels.cu physical_type). */
static int physical_type(int v, int t) {
    return (v ? 1 - t / V5_NSLOT : t / V5_NSLOT) * V5_NSLOT + t % V5_NSLOT;
}

/* ----------------------------------------------------------------- pieces */

void v5_cards(const V5* n, const float* card_feat, float* cards) {
    float hid[V5_TYPE];
    for (int v = 0; v < 2; v++)
        for (int t = 0; t < V5_NTYPE; t++) {
            const float* facts = card_feat + (size_t)physical_type(v, t) * V5_CARD_FEATS;
            apply_lin(n, n->L.card[0], 1, facts, NULL, hid);
            for (int j = 0; j < V5_TYPE; j++) hid[j] = v5_gelu(n, hid[j]);
            apply_lin(n, n->L.card[1], 1, hid, NULL, cards + ((size_t)v * V5_NTYPE + t) * V5_TYPE);
        }
}

/* Residual block i over one row's hexes, in place on x [HEXES][C]; a and y
 * are [HEXES][C] scratch, z [C] (net.rs:548-595). */
static void trunk_block(const V5* n, int i, float* x, float* a, float* y, float* z) {
    const Layout* L = &n->L;
    enum { H = V5_HEXES, C = V5_C };
    float mixed[2 * V5_C], pooled[2 * V5_C], gb[V5_C];
    memcpy(a, x, sizeof(float) * H * C);
    for (int h = 0; h < H; h++) norm(n, ln_block(i, 0), a + (size_t)h * C, 1);
    for (int j = 0; j < C; j++) {
        float mean = 0.0f, top = -INFINITY;
        for (int h = 0; h < H; h++) {
            const float v = a[(size_t)h * C + j];
            mean += v / (float)H;
            top = fmaxf(top, v);
        }
        pooled[j] = mean;
        pooled[C + j] = top;
    }
    apply_lin(n, L->poolm[i], 1, pooled, NULL, gb);
    for (int h = 0; h < H; h++) {
        memcpy(mixed, a + (size_t)h * C, sizeof(float) * C);
        for (int j = 0; j < C; j++) mixed[C + j] = 0.0f;
        for (int d = 0; d < 6; d++) {
            const int nh = g_nb[h][d];
            if (nh < 0) continue;
            for (int j = 0; j < C; j++) mixed[C + j] += a[(size_t)nh * C + j];
        }
        float* yh = y + (size_t)h * C;
        apply_lin(n, L->mix[i], 1, mixed, NULL, yh);
        for (int j = 0; j < C; j++) yh[j] += gb[j];
        norm(n, ln_block(i, 1), yh, 1);
        apply_lin(n, L->out[i], 1, yh, NULL, z);
        for (int j = 0; j < C; j++) x[(size_t)h * C + j] += z[j];
    }
}

void v5_board(const V5* n, const uint8_t* raw, const float* cards, float* P, float* Jp) {
    const Layout* L = &n->L;
    enum { H = V5_HEXES, C = V5_C };
    float* tok = (float*)malloc(sizeof(float) * V5_NTYPE * V5_TYPE);
    float* proj = (float*)malloc(sizeof(float) * V5_NTYPE * C);
    float* x = (float*)malloc(sizeof(float) * H * C);
    float* a = (float*)malloc(sizeof(float) * H * C);
    float* y = (float*)malloc(sizeof(float) * H * C);
    float* z = (float*)malloc(sizeof(float) * C);
    float tp[V5_C], glob[V5_C], loose[V5_LOOSE], piles[V5_PILE_COUNTS];
    float facts[V5_HEX_FACTS];
    int occ[V5_HEXES];
    /* tokens (net.rs:474-495): pile counts through `pile`, then card + seat */
    for (int t = 0; t < V5_NTYPE; t++) {
        float* dst = tok + (size_t)t * V5_TYPE;
        for (int f = 0; f < V5_PILE_COUNTS; f++) piles[f] = (float)raw[GR_PILES + t * V5_PILE_COUNTS + f] / CNORM;
        float zero[V5_TYPE];
        memset(zero, 0, sizeof zero);
        apply_lin(n, L->pile, 0, piles, zero, dst);
        const float* card = cards + (size_t)t * V5_TYPE; /* seat-zero view */
        const float* seat = n->w + L->seat + (size_t)(t / V5_NSLOT) * V5_TYPE;
        for (int j = 0; j < V5_TYPE; j++) dst[j] += card[j] + seat[j];
    }
    /* stem (net.rs:499-543) */
    for (int t = 0; t < V5_NTYPE; t++) apply_lin(n, L->tok_stem, 0, tok + (size_t)t * V5_TYPE, NULL, proj + (size_t)t * C);
    for (int j = 0; j < C; j++) tp[j] = 0.0f;
    for (int t = 0; t < V5_NTYPE; t++)
        for (int j = 0; j < C; j++) tp[j] += v5_gelu(n, proj[(size_t)t * C + j]) / (float)V5_NTYPE;
    loose_features(raw, loose);
    for (int h = 0; h < H; h++) {
        hex_facts(raw, h, facts, &occ[h]);
        apply_lin(n, L->hex_stem, 0, facts, NULL, x + (size_t)h * C);
    }
    apply_lin(n, L->glob_stem, 0, loose, NULL, glob);
    const float* pos = n->w + L->pos;
    for (int h = 0; h < H; h++)
        for (int j = 0; j < C; j++) {
            const float o = occ[h] >= 0 ? proj[(size_t)occ[h] * C + j] : 0.0f;
            x[(size_t)h * C + j] += o + pos[(size_t)h * C + j] + glob[j] + tp[j];
        }
    for (int i = 0; i < V5_BLOCKS; i++) trunk_block(n, i, x, a, y, z);
    for (int h = 0; h < H; h++) norm(n, LN_TRUNK, x + (size_t)h * C, 1);
    /* board vector (net.rs:700-723) and the join cache (net.rs:728-730) */
    float input[2 * V5_C + V5_LOOSE];
    for (int j = 0; j < C; j++) {
        input[j] = 0.0f;
        input[C + j] = -INFINITY;
    }
    for (int h = 0; h < H; h++)
        for (int j = 0; j < C; j++) {
            const float v = x[(size_t)h * C + j];
            input[j] += v / (float)H;
            input[C + j] = fmaxf(input[C + j], v);
        }
    memcpy(input + 2 * C, loose, sizeof loose);
    apply_lin(n, L->board_out, 1, input, NULL, P);
    apply_lin(n, L->join_p, 1, P, NULL, Jp);
    free(tok);
    free(proj);
    free(x);
    free(a);
    free(y);
    free(z);
}

void v5_config(const V5* n, const float* phi, int owner, const float* cards, float* f, float* g) {
    const Layout* L = &n->L;
    float slot[3 + V5_TYPE], hid[V5_NSLOT][V5_CFGH], u[V5_CFGH], bag[3 * V5_POOL];
    for (int k = 0; k < V5_NSLOT; k++) {
        slot[0] = phi[k];
        slot[1] = phi[V5_NSLOT + k];
        slot[2] = phi[2 * V5_NSLOT + k];
        memcpy(slot + 3, cards + ((size_t)owner * V5_NTYPE + k) * V5_TYPE, sizeof(float) * V5_TYPE);
        apply_lin(n, L->cfg1, 1, slot, NULL, hid[k]);
        for (int j = 0; j < V5_CFGH; j++) hid[k][j] = v5_gelu(n, hid[k][j]);
    }
    for (int j = 0; j < V5_CFGH; j++) u[j] = 0.0f;
    for (int k = 0; k < V5_NSLOT; k++)
        for (int j = 0; j < V5_CFGH; j++) u[j] += hid[k][j];
    norm(n, LN_CFG, u, 1);
    apply_lin(n, L->cfg_f, 1, u, NULL, f);
    apply_lin(n, L->cfg_g, 1, u, NULL, g);
    /* the count-weighted card half of g (net.rs:779-796) */
    for (int k = 0; k < V5_NSLOT; k++) {
        apply_lin(n, L->cfg_m, 1, cards + ((size_t)owner * V5_NTYPE + k) * V5_TYPE, NULL, bag);
        for (int zone = 0; zone < 3; zone++) {
            const float count = phi[zone * V5_NSLOT + k];
            if (count == 0.0f) continue;
            for (int j = 0; j < V5_POOL; j++) g[j] += count * bag[zone * V5_POOL + j];
        }
    }
}

void v5_join(const V5* n, const float* P, const float* Jp, const float* pooled_me, const float* pooled_opp,
             int player, float* h) {
    const Layout* L = &n->L;
    float in[V5_JOIN_IN], z[V5_JW], t[V5_JW], d[V5_JW];
    memcpy(in, pooled_me, sizeof(float) * V5_POOL);
    memcpy(in + V5_POOL, pooled_opp, sizeof(float) * V5_POOL);
    in[2 * V5_POOL] = player == 0 ? -1.0f : 1.0f;
    apply_lin(n, L->join_b, 1, in, Jp, z);
    for (int i = 0; i < V5_JBLOCKS; i++) {
        memcpy(t, z, sizeof z);
        norm(n, LN_JOIN + i, t, 1);
        apply_lin(n, L->join_w[i], 1, t, NULL, d);
        for (int j = 0; j < V5_JW; j++) z[j] += d[j];
    }
    norm(n, LN_JOUT, z, 1);
    apply_lin(n, L->join_out, 1, z, P, h);
    norm(n, LN_H, h, 0);
}

float v5_value(const V5* n, const float* f, const float* h) {
    const float bias = n->b[n->L.value_bias];
    if (n->mode == NET_F32) {
        float v = bias;
        for (int j = 0; j < V5_D; j++) v += f[j] * h[j];
        return v;
    }
    if (ascending(n)) {
        float v = 0.0f;
        for (int j = 0; j < V5_D; j++) v += qv(n, f[j]) * qv(n, h[j]);
        return v + bias;
    }
    double v = 0.0;
    for (int j = 0; j < V5_D; j++) v += (double)qv(n, f[j]) * (double)qv(n, h[j]);
    return (float)v + bias;
}

/* ------------------------------------------------- pieces for the pins */

const char* oracle_last_error(void);

static V5* piece_net(int mode, const float* w, size_t nw, const float* b, size_t nb, const float* ln, size_t nln,
                     int libm) {
    static __thread char err[256];
    V5* n = v5_new(mode, w, nw, b, nb, ln, nln, libm, err, sizeof err);
    if (!n) fprintf(stderr, "v5 oracle: %s\n", err);
    return n;
}

int oracle_v5_sizes(size_t* nw, size_t* nb, size_t* nln) {
    v5_sizes(nw, nb, nln);
    return 0;
}

/* cards: [2][NTYPE][TYPE] from card_feat [NTYPE][CARD_FEATS]. */
int oracle_v5_cards(int mode, const float* w, size_t nw, const float* b, size_t nb, const float* ln, size_t nln,
                    int libm, const float* card_feat, float* cards) {
    V5* n = piece_net(mode, w, nw, b, nb, ln, nln, libm);
    if (!n) return -1;
    v5_cards(n, card_feat, cards);
    v5_free(n);
    return 0;
}

/* Per row r < rows: P [rows][D], Jp [rows][JW] from raw [rows][ROW_BYTES]. */
int oracle_v5_board(int mode, const float* w, size_t nw, const float* b, size_t nb, const float* ln, size_t nln,
                    int libm, const uint8_t* raw, uint32_t rows, const float* cards, float* P, float* Jp) {
    V5* n = piece_net(mode, w, nw, b, nb, ln, nln, libm);
    if (!n) return -1;
    for (uint32_t r = 0; r < rows; r++)
        v5_board(n, raw + (size_t)r * V5_ROW_BYTES, cards, P + (size_t)r * V5_D, Jp + (size_t)r * V5_JW);
    v5_free(n);
    return 0;
}

/* Residual block `block` of the trunk, in place on x [rows][HEXES][C]. */
int oracle_v5_block(int mode, const float* w, size_t nw, const float* b, size_t nb, const float* ln, size_t nln,
                    int libm, float* x, uint32_t rows, int block) {
    if (block < 0 || block >= V5_BLOCKS) return -1;
    V5* n = piece_net(mode, w, nw, b, nb, ln, nln, libm);
    if (!n) return -1;
    const size_t cells = (size_t)V5_HEXES * V5_C;
    float* a = (float*)malloc(sizeof(float) * cells);
    float* y = (float*)malloc(sizeof(float) * cells);
    float z[V5_C];
    for (uint32_t r = 0; r < rows; r++) trunk_block(n, block, x + (size_t)r * cells, a, y, z);
    free(a);
    free(y);
    v5_free(n);
    return 0;
}

/* Per config c < ncfg: f [ncfg][D], g [ncfg][POOL] from phi [ncfg][CFEAT], owner [ncfg]. */
int oracle_v5_configs(int mode, const float* w, size_t nw, const float* b, size_t nb, const float* ln, size_t nln,
                      int libm, const float* phi, const uint8_t* owner, uint32_t ncfg, const float* cards, float* f,
                      float* g) {
    V5* n = piece_net(mode, w, nw, b, nb, ln, nln, libm);
    if (!n) return -1;
    for (uint32_t c = 0; c < ncfg; c++)
        v5_config(n, phi + (size_t)c * V5_CFEAT, owner[c], cards, f + (size_t)c * V5_D, g + (size_t)c * V5_POOL);
    v5_free(n);
    return 0;
}

/* Per row r < rows: h [rows][D] for `player`, pooled [rows][2][POOL] (the
 * player's block first). */
int oracle_v5_join(int mode, const float* w, size_t nw, const float* b, size_t nb, const float* ln, size_t nln,
                   int libm, const float* P, const float* Jp, const float* pooled, uint32_t rows, int player,
                   float* h) {
    V5* n = piece_net(mode, w, nw, b, nb, ln, nln, libm);
    if (!n) return -1;
    for (uint32_t r = 0; r < rows; r++)
        v5_join(n, P + (size_t)r * V5_D, Jp + (size_t)r * V5_JW, pooled + (size_t)r * 2 * V5_POOL,
                pooled + (size_t)r * 2 * V5_POOL + V5_POOL, player, h + (size_t)r * V5_D);
    v5_free(n);
    return 0;
}

float oracle_v5_gelu(float x, int libm) {
    V5 n;
    memset(&n, 0, sizeof n);
    n.libm_tanh = libm;
    return v5_gelu(&n, x);
}
