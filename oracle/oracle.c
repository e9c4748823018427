/*
 * ORACLE — test infrastructure only.
 *
 * A plain-C restatement of the reference's CPU subgame solver
 * (engine/src/search.rs) and CPU value net, operating on the WCJ8 job bytes
 * of the reference contract (docs/TREE.md, engine/src/serialize.rs). Only the
 * tests, the smoke check and the benchmark's CPU-baseline leg may load this
 * library, and only as what results are compared against or as the timed CPU
 * baseline: the product path never calls it.
 *
 * Parity status per function (how each part is pinned is recorded in the
 * tests that exercise it):
 *   parse_job            pinned: byte round trip against the product codec, stub KATs
 *   propagate            pinned: tabular world-state CFR brute force, gather replay
 *   backprop (Regret)    pinned: tabular world-state CFR brute force
 *   backprop (Value)     pinned: brute force, zero-sum of terminal-only trees
 *   backprop (BestResp.) pinned: NashConv >= 0 and falling
 *   avg_block/snapshot   pinned: brute force, snapshot_iters closed form
 *   belief_blocks        pinned: numpy float64 restatement
 *   mlp_trunk/values     pinned: numpy float64 restatement
 *   value_under          pinned: brute force
 *   v5 network (v5.c)    pinned: torch float64 restatement of each piece, board
 *                        geometry invariants, special cases (tests/test_v5_pins.py)
 *   carried_beliefs      pinned: brute force (normalised reach under snapshots)
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off: the reference's Rust
 * never contracts a*b+c into an FMA, so neither does this restatement).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "v5.h"

#define NONE 0xffffffffu
#define EPS 1e-6f      /* search.rs:1658 */
#define SMOOTH 1e-30f  /* rebel.rs:359 */

enum { MODEL_V5 = 5, MODEL_MLP = 101, MODEL_TWO_TOWER = 102 };
/* Leaf-net arithmetic models. F32 is the CPU net's float32 loop, bit for
 * bit. The others model a device: operands rounded on entry (and every
 * activation that feeds a layer), exact products, and either a wide (double)
 * sum or, for F16A, a float32 sum in ascending k order -- two equally faithful
 * f16 realizations that differ only in how the f32-level sum is rounded.
 * F16X holds each operand as the f16 pair hi + lo (about 22 significant bits:
 * the compensated mode), F32W keeps float32 operands with a wide sum, BF16A
 * (v5 network only) is F16A with bfloat16 operands. */
enum { NET_EMPTY = 0, NET_F32 = 1, NET_F16 = 2, NET_BF16 = 3, NET_F16A = 4, NET_F16X = 5, NET_F32W = 6, NET_BF16A = 7 };
enum { BACK_REGRET = 0, BACK_VALUE = 1, BACK_BR = 2 };

static __thread char g_err[256];
const char* oracle_last_error(void) { return g_err; }

/* ------------------------------------------------------------------ job */

typedef struct {
    uint32_t n;
    uint32_t* v;
} U32s;
typedef struct {
    uint32_t n;
    float* v;
} F32s;
typedef struct {
    uint32_t n;
    uint8_t* v;
} U8s;

typedef struct {
    uint32_t depth, iters, snapshots;
    float alpha, beta, gamma, predict;
    U32s snap_iters, net_dims;
    uint32_t nodes, ncfg, rows, ncells;
    U8s node_kind, node_player;
    U32s node_child_start, node_child, obs_off, obs_start, obs_act, obs_child;
    U32s legal_row_of, legal_off, legal_action, legal_child, legal_trans, cell_row;
    U32s draw_off, draw_to;
    F32s draw_p;
    U32s draw_row_off, draw_row_start, cfg_off, reach_off, soff, node_parent;
    U32s rev_row_of, rev_start, rev_src, rev_cell, rvd_row_of, rvd_start, rvd_src;
    F32s rvd_p;
    U32s leaf_rows, term_leaves;
    F32s terminal_utility;
    U32s leaf_coff, leaf_cidx, snap_coff;
    U8s leaf_raw;
    F32s card_feat, cphi;
    U8s cplayer;
    U32s bfs_order, level_start;
    F32s root[2];
    uint32_t nroots;
    F32s* carried; /* [2 * nroots]: root r player p at 2r+p */
    /* network shape from net_dims */
    uint32_t kind, in, hidden, layers, heads, pool, priv_in, priv_layers, row_bytes, cfeat;
} Job;

typedef struct {
    const uint8_t* b;
    size_t n, at;
    int ok;
} Rd;

static int rd_take(Rd* r, size_t k, const char* what) {
    if (!r->ok) return 0;
    if (k > r->n - r->at) {
        snprintf(g_err, sizeof g_err, "job truncated reading %s", what);
        r->ok = 0;
        return 0;
    }
    return 1;
}
static uint32_t rd_u32(Rd* r, const char* what) {
    if (!rd_take(r, 4, what)) return 0;
    const uint8_t* p = r->b + r->at;
    r->at += 4;
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
static float rd_f32(Rd* r, const char* what) {
    uint32_t u = rd_u32(r, what);
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static void rd_u8s(Rd* r, U8s* out, const char* what) {
    out->n = rd_u32(r, what);
    out->v = NULL;
    if (!rd_take(r, out->n, what)) return;
    out->v = (uint8_t*)malloc(out->n ? out->n : 1);
    memcpy(out->v, r->b + r->at, out->n);
    r->at += out->n;
}
static void rd_u32s(Rd* r, U32s* out, const char* what) {
    out->n = rd_u32(r, what);
    out->v = NULL;
    if (!rd_take(r, (size_t)out->n * 4, what)) return;
    out->v = (uint32_t*)malloc(((size_t)out->n ? out->n : 1) * 4);
    for (uint32_t i = 0; i < out->n; i++) out->v[i] = rd_u32(r, what);
}
static void rd_f32s(Rd* r, F32s* out, const char* what) {
    out->n = rd_u32(r, what);
    out->v = NULL;
    if (!rd_take(r, (size_t)out->n * 4, what)) return;
    out->v = (float*)malloc(((size_t)out->n ? out->n : 1) * 4);
    for (uint32_t i = 0; i < out->n; i++) out->v[i] = rd_f32(r, what);
}

static void job_free(Job* j) {
    U32s* u32s[] = {&j->snap_iters, &j->net_dims, &j->node_child_start, &j->node_child, &j->obs_off,
                    &j->obs_start, &j->obs_act, &j->obs_child, &j->legal_row_of, &j->legal_off,
                    &j->legal_action, &j->legal_child, &j->legal_trans, &j->cell_row, &j->draw_off,
                    &j->draw_to, &j->draw_row_off, &j->draw_row_start, &j->cfg_off, &j->reach_off,
                    &j->soff, &j->node_parent, &j->rev_row_of, &j->rev_start, &j->rev_src,
                    &j->rev_cell, &j->rvd_row_of, &j->rvd_start, &j->rvd_src, &j->leaf_rows,
                    &j->term_leaves, &j->leaf_coff, &j->leaf_cidx, &j->snap_coff, &j->bfs_order,
                    &j->level_start};
    for (size_t k = 0; k < sizeof u32s / sizeof u32s[0]; k++) free(u32s[k]->v);
    F32s* f32s[] = {&j->draw_p, &j->rvd_p, &j->terminal_utility, &j->card_feat, &j->cphi,
                    &j->root[0], &j->root[1]};
    for (size_t k = 0; k < sizeof f32s / sizeof f32s[0]; k++) free(f32s[k]->v);
    free(j->node_kind.v);
    free(j->node_player.v);
    free(j->leaf_raw.v);
    free(j->cplayer.v);
    if (j->carried) {
        for (uint32_t k = 0; k < 2 * j->nroots; k++) free(j->carried[k].v);
        free(j->carried);
    }
    memset(j, 0, sizeof *j);
}

static int want(uint32_t got, uint64_t expect, const char* what) {
    if (got != expect) {
        snprintf(g_err, sizeof g_err, "job %s: count %u != expected %llu", what, got,
                 (unsigned long long)expect);
        return 0;
    }
    return 1;
}

/* engine/src/serialize.rs:1131-1261, with the payload widths of the network tag. */
static int parse_job(const uint8_t* b, size_t n, Job* j) {
    memset(j, 0, sizeof *j);
    Rd r = {b, n, 0, 1};
    if (rd_u32(&r, "magic") != 0x57434A38u) {
        if (r.ok) snprintf(g_err, sizeof g_err, "job: bad magic");
        return 0;
    }
    if (rd_u32(&r, "version") != 8u) {
        if (r.ok) snprintf(g_err, sizeof g_err, "job: unsupported version");
        return 0;
    }
    j->depth = rd_u32(&r, "depth");
    j->iters = rd_u32(&r, "iters");
    if (rd_take(&r, 1, "snapshots")) j->snapshots = b[r.at++] != 0;
    j->alpha = rd_f32(&r, "alpha");
    j->beta = rd_f32(&r, "beta");
    j->gamma = rd_f32(&r, "gamma");
    j->predict = rd_f32(&r, "predict");
    rd_u32s(&r, &j->snap_iters, "snap_iters");
    rd_u32s(&r, &j->net_dims, "net_dims");
    j->nodes = rd_u32(&r, "nodes");
    j->ncfg = rd_u32(&r, "ncfg");
    j->rows = rd_u32(&r, "rows");
    j->ncells = rd_u32(&r, "ncells");
    rd_u8s(&r, &j->node_kind, "node_kind");
    rd_u8s(&r, &j->node_player, "node_player");
    rd_u32s(&r, &j->node_child_start, "node_child_start");
    rd_u32s(&r, &j->node_child, "node_child");
    rd_u32s(&r, &j->obs_off, "obs_off");
    rd_u32s(&r, &j->obs_start, "obs_start");
    rd_u32s(&r, &j->obs_act, "obs_act");
    rd_u32s(&r, &j->obs_child, "obs_child");
    rd_u32s(&r, &j->legal_row_of, "legal_row_of");
    rd_u32s(&r, &j->legal_off, "legal_off");
    rd_u32s(&r, &j->legal_action, "legal_action");
    rd_u32s(&r, &j->legal_child, "legal_child");
    rd_u32s(&r, &j->legal_trans, "legal_trans");
    rd_u32s(&r, &j->cell_row, "cell_row");
    rd_u32s(&r, &j->draw_off, "draw_off");
    rd_u32s(&r, &j->draw_to, "draw_to");
    rd_f32s(&r, &j->draw_p, "draw_p");
    rd_u32s(&r, &j->draw_row_off, "draw_row_off");
    rd_u32s(&r, &j->draw_row_start, "draw_row_start");
    rd_u32s(&r, &j->cfg_off, "cfg_off");
    rd_u32s(&r, &j->reach_off, "reach_off");
    rd_u32s(&r, &j->soff, "soff");
    rd_u32s(&r, &j->node_parent, "node_parent");
    rd_u32s(&r, &j->rev_row_of, "rev_row_of");
    rd_u32s(&r, &j->rev_start, "rev_start");
    rd_u32s(&r, &j->rev_src, "rev_src");
    rd_u32s(&r, &j->rev_cell, "rev_cell");
    rd_u32s(&r, &j->rvd_row_of, "rvd_row_of");
    rd_u32s(&r, &j->rvd_start, "rvd_start");
    rd_u32s(&r, &j->rvd_src, "rvd_src");
    rd_f32s(&r, &j->rvd_p, "rvd_p");
    rd_u32s(&r, &j->leaf_rows, "leaf_rows");
    rd_u32s(&r, &j->term_leaves, "term_leaves");
    rd_f32s(&r, &j->terminal_utility, "terminal_utility");
    rd_u32s(&r, &j->leaf_coff, "leaf_coff");
    rd_u32s(&r, &j->leaf_cidx, "leaf_cidx");
    rd_u32s(&r, &j->snap_coff, "snap_coff");
    rd_u8s(&r, &j->leaf_raw, "leaf_raw");
    rd_f32s(&r, &j->card_feat, "card_feat");
    rd_f32s(&r, &j->cphi, "cphi");
    rd_u8s(&r, &j->cplayer, "cplayer");
    rd_u32s(&r, &j->bfs_order, "bfs_order");
    rd_u32s(&r, &j->level_start, "level_start");
    rd_f32s(&r, &j->root[0], "root0");
    rd_f32s(&r, &j->root[1], "root1");
    j->nroots = rd_u32(&r, "nroots");
    if (!r.ok) return 0;
    if (j->nroots > (1u << 20)) {
        snprintf(g_err, sizeof g_err, "job: implausible carried-root count");
        return 0;
    }
    j->carried = (F32s*)calloc(2 * (size_t)j->nroots + 1, sizeof(F32s));
    for (uint32_t k = 0; k < j->nroots; k++) {
        rd_f32s(&r, &j->carried[2 * k], "carried0");
        rd_f32s(&r, &j->carried[2 * k + 1], "carried1");
    }
    if (!r.ok) return 0;
    if (r.at != n) {
        snprintf(g_err, sizeof g_err, "job: trailing bytes");
        return 0;
    }
    /* Network payload widths. */
    if (j->net_dims.n < 1) {
        snprintf(g_err, sizeof g_err, "net_dims is empty");
        return 0;
    }
    j->kind = j->net_dims.v[0];
    if (j->kind == MODEL_MLP && j->net_dims.n == 6) {
        j->in = j->net_dims.v[1];
        j->hidden = j->net_dims.v[2];
        j->layers = j->net_dims.v[3];
        j->heads = j->net_dims.v[4];
        j->pool = j->net_dims.v[5];
        j->cfeat = 1 + j->pool;
    } else if (j->kind == MODEL_TWO_TOWER && j->net_dims.n == 7) {
        j->in = j->net_dims.v[1];
        j->hidden = j->net_dims.v[2];
        j->layers = j->net_dims.v[3];
        j->priv_in = j->net_dims.v[4];
        j->priv_layers = j->net_dims.v[5];
        j->pool = j->net_dims.v[6];
        j->cfeat = 1 + j->pool + j->priv_in;
    } else if (j->kind == MODEL_V5 && j->net_dims.n == 1) {
        /* net.rs:41; the join reads both pooled beliefs and the seat */
        j->in = V5_JOIN_IN;
        j->hidden = V5_D;
        j->pool = V5_POOL;
        j->cfeat = V5_CFEAT;
    } else {
        snprintf(g_err, sizeof g_err, "unsupported net_dims");
        return 0;
    }
    if (j->in < 2 * j->pool + 1) {
        snprintf(g_err, sizeof g_err, "net input narrower than the belief block");
        return 0;
    }
    j->row_bytes = j->kind == MODEL_V5 ? V5_ROW_BYTES : j->in - 2 * j->pool - 1;
    uint32_t N = j->nodes;
    if (!want(j->node_kind.n, N, "node_kind") || !want(j->node_player.n, N, "node_player") ||
        !want(j->legal_row_of.n, N, "legal_row_of") ||
        !want(j->node_child_start.n, (uint64_t)N + 1, "node_child_start") ||
        !want(j->obs_off.n, (uint64_t)N + 1, "obs_off") || !want(j->draw_off.n, (uint64_t)N + 1, "draw_off") ||
        !want(j->draw_row_off.n, (uint64_t)N + 1, "draw_row_off") ||
        !want(j->reach_off.n, (uint64_t)N + 1, "reach_off") || !want(j->soff.n, (uint64_t)N + 1, "soff") ||
        !want(j->cfg_off.n, 2 * (uint64_t)N + 1, "cfg_off") ||
        !want(j->cphi.n, (uint64_t)j->ncfg * j->cfeat, "cphi") || !want(j->cplayer.n, j->ncfg, "cplayer") ||
        !want(j->leaf_raw.n, (uint64_t)j->rows * j->row_bytes, "leaf_raw") ||
        !want(j->card_feat.n, j->kind == MODEL_V5 ? (uint64_t)V5_NTYPE * V5_CARD_FEATS : 0, "card_feat") ||
        !want(j->leaf_coff.n, 2 * (uint64_t)j->rows + 1, "leaf_coff") ||
        !want(j->node_parent.n, N, "node_parent") || !want(j->rev_row_of.n, N, "rev_row_of") ||
        !want(j->rvd_row_of.n, N, "rvd_row_of") || !want(j->rev_cell.n, j->rev_src.n, "rev_cell") ||
        !want(j->rvd_p.n, j->rvd_src.n, "rvd_p") || !want(j->legal_action.n, j->ncells, "legal_action") ||
        !want(j->legal_child.n, j->ncells, "legal_child") ||
        !want(j->legal_trans.n, j->ncells, "legal_trans") || !want(j->cell_row.n, j->ncells, "cell_row") ||
        !want(j->leaf_rows.n, j->rows, "rows") ||
        !want(j->snap_coff.n, 2 * ((uint64_t)j->leaf_rows.n + j->term_leaves.n) + 1, "snap_coff") ||
        !want(j->terminal_utility.n, j->term_leaves.n, "terminal_utility"))
        return 0;
    if (N == 0 || j->legal_off.n == 0 || j->legal_off.v[j->legal_off.n - 1] != j->ncells) {
        snprintf(g_err, sizeof g_err, "job: empty tree or legal_off disagrees with ncells");
        return 0;
    }
    return 1;
}

/* ------------------------------------------------------ reduced precision */

/* Round-to-nearest-even float -> IEEE binary16 -> float. */
static float round_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    uint32_t sign = u & 0x80000000u, a = u & 0x7fffffffu;
    uint16_t h;
    if (a >= 0x7f800000u) {
        h = (uint16_t)(a > 0x7f800000u ? 0x7e00 : 0x7c00);
    } else if (a >= 0x477ff000u) { /* rounds to >= 65520: overflow to inf */
        h = 0x7c00;
    } else if (a < 0x38800000u) { /* below the smallest normal half: subnormal or zero */
        /* value = a as float; subnormal half step = 2^-24 */
        float f;
        uint32_t t = a;
        memcpy(&f, &t, 4);
        float q = f * 16777216.0f; /* in units of 2^-24, exact scaling */
        /* round half to even to an integer */
        float fl = floorf(q);
        float rem = q - fl;
        uint32_t m = (uint32_t)fl;
        if (rem > 0.5f || (rem == 0.5f && (m & 1u))) m++;
        h = (uint16_t)m;
    } else {
        uint32_t exp = ((a >> 23) - 112u) << 10;
        uint32_t man = (a >> 13) & 0x3ffu;
        uint32_t rest = a & 0x1fffu;
        uint32_t v = exp | man;
        if (rest > 0x1000u || (rest == 0x1000u && (v & 1u))) v++;
        h = (uint16_t)v;
    }
    h |= (uint16_t)(sign >> 16);
    /* back to float */
    uint32_t hs = (uint32_t)(h & 0x8000u) << 16;
    uint32_t he = (h >> 10) & 0x1fu, hm = h & 0x3ffu;
    uint32_t out;
    if (he == 0) {
        float mag = (float)hm * (1.0f / 16777216.0f);
        memcpy(&out, &mag, 4);
        out |= hs;
    } else if (he == 31) {
        out = hs | 0x7f800000u | (hm << 13);
    } else {
        out = hs | ((he + 112u) << 23) | (hm << 13);
    }
    float f;
    memcpy(&f, &out, 4);
    return f;
}

/* Round-to-nearest-even float -> bfloat16 -> float. */
static float round_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        u |= 0x00400000u;
    } else {
        uint32_t lsb = (u >> 16) & 1u;
        u += 0x7fffu + lsb;
    }
    u &= 0xffff0000u;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float oracle_round_f16(float x) { return round_f16(x); }
float oracle_round_bf16(float x) { return round_bf16(x); }

/* ------------------------------------------------------------------ net */

typedef struct {
    int mode; /* NET_EMPTY / NET_F32 / NET_F16 / NET_BF16 / NET_F16A / NET_F16X / NET_F32W */
    uint32_t kind, in, hidden, layers, heads, pool, priv_in, priv_layers;
    /* MLP: W[0] in x hidden, W[1..layers-1] hidden x hidden, Whead heads x hidden */
    const float* w;
    const float* b;
    float* wq; /* operand copies rounded for the reduced-precision modes */
    const float* W[16];
    const float* B[16];
    const float* Whead;
    const float* bhead;
    /* two-tower */
    const float* PW[16];
    const float* PB[16];
    const float* wread;
    float bread;
    /* v5 (v5.c) */
    V5* v5;
} Net;

/* GELU's tanh in the v5 restatement: its own (0) or the C library's (1). */
static int g_v5_libm_tanh;
void oracle_v5_set_libm_tanh(int on) { g_v5_libm_tanh = on; }

static float q_op(const Net* n, float x) {
    if (n->mode == NET_F16 || n->mode == NET_F16A) return round_f16(x);
    if (n->mode == NET_BF16) return round_bf16(x);
    if (n->mode == NET_F16X) {
        float hi = round_f16(x);
        return hi + round_f16(x - hi);
    }
    return x;
}

/* The model sums in double (every reduced-precision model but F16A, and F32W). */
static int wide_sum(const Net* n) { return n->mode != NET_F32 && n->mode != NET_F16A; }

static int net_init(Net* n, int mode, const uint32_t* dims, uint32_t ndims, const float* w, size_t nw,
                    const float* b, size_t nb, const float* ln, size_t nln) {
    memset(n, 0, sizeof *n);
    n->mode = mode;
    if (mode == NET_EMPTY) return 1;
    if (ndims < 1) {
        snprintf(g_err, sizeof g_err, "net dims empty");
        return 0;
    }
    n->kind = dims[0];
    size_t need_w = 0, need_b = 0;
    if (n->kind == MODEL_V5 && ndims == 1) {
        n->in = V5_JOIN_IN;
        n->hidden = V5_D;
        n->pool = V5_POOL;
        n->v5 = v5_new(mode, w, nw, b, nb, ln, nln, g_v5_libm_tanh, g_err, sizeof g_err);
        return n->v5 != NULL;
    }
    if (mode == NET_BF16A) {
        snprintf(g_err, sizeof g_err, "the BF16A model is the v5 network's only");
        return 0;
    }
    if (n->kind == MODEL_MLP && ndims == 6) {
        n->in = dims[1];
        n->hidden = dims[2];
        n->layers = dims[3];
        n->heads = dims[4];
        n->pool = dims[5];
        if (n->layers == 0 || n->layers > 15) {
            snprintf(g_err, sizeof g_err, "MLP depth out of range");
            return 0;
        }
        need_w = (size_t)n->in * n->hidden + (size_t)(n->layers - 1) * n->hidden * n->hidden +
                 (size_t)n->heads * n->hidden;
        need_b = (size_t)n->layers * n->hidden + n->heads;
    } else if (n->kind == MODEL_TWO_TOWER && ndims == 7) {
        n->in = dims[1];
        n->hidden = dims[2];
        n->layers = dims[3];
        n->priv_in = dims[4];
        n->priv_layers = dims[5];
        n->pool = dims[6];
        if (n->layers == 0 || n->layers > 15 || n->priv_layers == 0 || n->priv_layers > 15) {
            snprintf(g_err, sizeof g_err, "two-tower depth out of range");
            return 0;
        }
        need_w = (size_t)n->in * n->hidden + (size_t)(n->layers - 1) * n->hidden * n->hidden +
                 (size_t)n->priv_in * n->hidden + (size_t)(n->priv_layers - 1) * n->hidden * n->hidden +
                 n->hidden;
        need_b = (size_t)n->layers * n->hidden + (size_t)n->priv_layers * n->hidden + 1;
    } else {
        snprintf(g_err, sizeof g_err, "unsupported net dims");
        return 0;
    }
    if (nw != need_w || nb != need_b) {
        snprintf(g_err, sizeof g_err, "net weights: got %zu/%zu floats, want %zu/%zu", nw, nb, need_w, need_b);
        return 0;
    }
    n->w = w;
    n->b = b;
    const float* ww = w;
    if (mode == NET_F16 || mode == NET_BF16 || mode == NET_F16A || mode == NET_F16X) {
        n->wq = (float*)malloc(nw * sizeof(float));
        for (size_t k = 0; k < nw; k++) n->wq[k] = q_op(n, w[k]);
        ww = n->wq;
    }
    size_t at = 0, bt = 0;
    if (n->kind == MODEL_MLP) {
        n->W[0] = ww;
        at = (size_t)n->in * n->hidden;
        for (uint32_t l = 1; l < n->layers; l++) {
            n->W[l] = ww + at;
            at += (size_t)n->hidden * n->hidden;
        }
        n->Whead = ww + at;
        for (uint32_t l = 0; l < n->layers; l++) {
            n->B[l] = b + bt;
            bt += n->hidden;
        }
        n->bhead = b + bt;
    } else {
        n->W[0] = ww;
        at = (size_t)n->in * n->hidden;
        for (uint32_t l = 1; l < n->layers; l++) {
            n->W[l] = ww + at;
            at += (size_t)n->hidden * n->hidden;
        }
        n->PW[0] = ww + at;
        at += (size_t)n->priv_in * n->hidden;
        for (uint32_t l = 1; l < n->priv_layers; l++) {
            n->PW[l] = ww + at;
            at += (size_t)n->hidden * n->hidden;
        }
        n->wread = ww + at;
        for (uint32_t l = 0; l < n->layers; l++) {
            n->B[l] = b + bt;
            bt += n->hidden;
        }
        for (uint32_t l = 0; l < n->priv_layers; l++) {
            n->PB[l] = b + bt;
            bt += n->hidden;
        }
        n->bread = b[bt];
    }
    return 1;
}

static void net_free(Net* n) {
    free(n->wq);
    n->wq = NULL;
    v5_free(n->v5);
    n->v5 = NULL;
}

/* One dense ReLU layer, y = relu(x W + b), with the row-major `gemm` loop of
 * engine/src/net.rs:102-122: per output, accumulate from zero over ascending
 * inputs, skipping zero inputs, then add the bias. The reduced-precision
 * modes model f16/bf16 operands with a wide accumulator: operands were
 * rounded on entry, products are exact, the sum is taken in double. */
static void dense_relu(const Net* n, const float* x, uint32_t k, const float* W, const float* bias,
                       uint32_t m, float* y) {
    if (!wide_sum(n)) {
        for (uint32_t j = 0; j < m; j++) y[j] = 0.0f;
        for (uint32_t p = 0; p < k; p++) {
            float a = x[p];
            if (a == 0.0f) continue;
            const float* row = W + (size_t)p * m;
            for (uint32_t j = 0; j < m; j++) y[j] += a * row[j];
        }
        for (uint32_t j = 0; j < m; j++) {
            float v = y[j] + bias[j];
            y[j] = v > 0.0f ? v : 0.0f;
        }
        return;
    }
    double* acc = (double*)calloc(m, sizeof(double));
    for (uint32_t p = 0; p < k; p++) {
        double a = (double)x[p];
        if (a == 0.0) continue;
        const float* row = W + (size_t)p * m;
        for (uint32_t j = 0; j < m; j++) acc[j] += a * (double)row[j];
    }
    for (uint32_t j = 0; j < m; j++) {
        float v = (float)acc[j] + bias[j];
        y[j] = v > 0.0f ? v : 0.0f;
    }
    free(acc);
}

/* Trunk: x (in) -> `layers` ReLU layers -> h (hidden). Activations feeding a
 * layer are rounded to the operand precision. */
static void net_trunk(const Net* n, const float* x_in, const float* const* W, const float* const* B,
                      uint32_t in, uint32_t layers, float* h, float* scratch) {
    float* cur = scratch;
    float* nxt = scratch + (in > n->hidden ? in : n->hidden);
    for (uint32_t p = 0; p < in; p++) cur[p] = q_op(n, x_in[p]);
    uint32_t width = in;
    for (uint32_t l = 0; l < layers; l++) {
        dense_relu(n, cur, width, W[l], B[l], n->hidden, nxt);
        width = n->hidden;
        for (uint32_t j = 0; j < width; j++) nxt[j] = q_op(n, nxt[j]);
        float* t = cur;
        cur = nxt;
        nxt = t;
    }
    memcpy(h, cur, (size_t)n->hidden * sizeof(float));
}

/* `Net::values` (engine/src/net.rs:844-853): v = bias, then += row[j] * h[j]. */
static float head_value(const Net* n, const float* h, uint32_t key) {
    const float* row = n->Whead + (size_t)key * n->hidden;
    if (n->mode == NET_F32) {
        float v = n->bhead[key];
        for (uint32_t j = 0; j < n->hidden; j++) v += row[j] * h[j];
        return v;
    }
    if (n->mode == NET_F16A) { /* the product's f32 sum, then the bias, as a GEMM epilogue adds it */
        float v = 0.0f;
        for (uint32_t j = 0; j < n->hidden; j++) v += row[j] * h[j];
        return v + n->bhead[key];
    }
    double v = 0.0;
    for (uint32_t j = 0; j < n->hidden; j++) v += (double)row[j] * (double)h[j];
    return (float)v + n->bhead[key];
}

/* ---------------------------------------------------------------- solver */

typedef struct {
    const Job* j;
    const Net* net;
    uint32_t N;
    uint32_t *nc0, *nc1;
    uint32_t *act_off; /* per node: offset of its action list in obs_act/obs_child */
    uint32_t *na;      /* per node: action count */
    uint32_t *acell_off, *acell; /* per node action-major cell view (node-local cells) */
    uint32_t *aoff;    /* per node: offset into acell_off (na + 1 entries) */
    float *regret, *cur, *sum;
    float *reach;
    float *vals;
    uint32_t* voff;
    uint32_t vals_len;
    float** snaps;
    uint32_t nsnaps, snap_t;
    int avg_touched[2];
    uint32_t steps[2];
    /* leaf batch */
    float* xb; /* [2*rows][pool] pooled beliefs */
    float* h;  /* [rows][hidden] trunk output for the last queried traverser */
    float* xin;
    float* scratch;
    float* wbuf;
    int last_traverser; /* -1 = none */
    int batch_ready;
    /* two-tower: per interned config, the private tower output times the readout weight;
     * v5: f(c) */
    float* fcfg;
    /* v5: the card tokens of both views, per row the board vector and its join
     * projection, per config g(c) */
    float *cards, *P, *Jp, *gcfg;
    /* replay (oracle_solve_replay): the network leaves' values and reach masses
     * of every leaf-net evaluation in schedule order, consumed by readout */
    const float *rp_vals, *rp_mass;
    size_t rp_vn, rp_mn, rp_vpos, rp_mpos;
    int rp_short; /* set when the replay ran out of values */
    /* trace (oracle_solve_trace): the same, recorded from the solver's own net */
    float *tr_vals, *tr_mass, *tr_reach; /* tr_reach optional: each row's reach of both players */
    size_t tr_vpos, tr_mpos, tr_rpos;
} Solver;

static inline uint32_t S_nc(const Solver* s, uint32_t i, int p) { return p ? s->nc1[i] : s->nc0[i]; }
static inline float* reach_of(const Solver* s, uint32_t i, int p) {
    return s->reach + s->j->reach_off.v[i] + (p ? s->nc0[i] : 0);
}

static float cfr_factor(float t, float p) { /* search.rs:185-193 */
    if (isinf(p)) return p > 0.0f ? 1.0f : 0.0f;
    float x = powf(t, p);
    return x / (x + 1.0f);
}
float oracle_factor(float t, float p) { return cfr_factor(t, p); }

/* normalize_weights (engine/src/rebel.rs:1054-1068). */
static void normalize_weights(const float* w, uint32_t n, float* out) {
    float tot = 0.0f;
    for (uint32_t k = 0; k < n; k++) tot += w[k];
    float scale, flat;
    if (tot > SMOOTH) {
        scale = 1.0f / tot;
        flat = 0.0f;
    } else {
        scale = 0.0f;
        flat = 1.0f / (float)(n > 0 ? n : 1);
    }
    for (uint32_t k = 0; k < n; k++) out[k] = w[k] * scale + flat;
}

/* Push reach down the tree under `strat` (engine/src/search.rs:1273-1351). */
static void propagate(Solver* s, const float* strat, const float* root0, const float* root1) {
    const Job* j = s->j;
    memset(s->reach, 0, (size_t)j->reach_off.v[s->N] * sizeof(float));
    float* r0 = s->reach + j->reach_off.v[0];
    memcpy(r0, root0, s->nc0[0] * sizeof(float));
    memcpy(r0 + s->nc0[0], root1, s->nc1[0] * sizeof(float));
    for (uint32_t i = 0; i < s->N; i++) {
        uint8_t kind = j->node_kind.v[i];
        if (kind == 2) continue;
        int me = j->node_player.v[i], op = 1 - me;
        uint32_t nme = S_nc(s, i, me), nop = S_nc(s, i, op);
        const float* src_me = reach_of(s, i, me);
        const float* src_op = reach_of(s, i, op);
        if (kind == 1) {
            uint32_t c = j->node_child.v[j->node_child_start.v[i]];
            float* dst_me = reach_of(s, c, me);
            float* dst_op = reach_of(s, c, op);
            memcpy(dst_op, src_op, nop * sizeof(float));
            uint32_t d0 = j->draw_off.v[i], rb = j->draw_row_off.v[i];
            for (uint32_t ci = 0; ci < nme; ci++) {
                float w = src_me[ci];
                if (w == 0.0f) continue;
                uint32_t lo = j->draw_row_start.v[rb + ci], hi = j->draw_row_start.v[rb + ci + 1];
                for (uint32_t k = lo; k < hi; k++) dst_me[j->draw_to.v[d0 + k]] += w * j->draw_p.v[d0 + k];
            }
            continue;
        }
        const float* cur = strat + j->soff.v[i];
        uint32_t cs0 = j->node_child_start.v[i], cs1 = j->node_child_start.v[i + 1];
        const uint32_t* ostart = j->obs_start.v + j->obs_off.v[i];
        const uint32_t* oact = j->obs_act.v + s->act_off[i];
        for (uint32_t ch = 0; ch < cs1 - cs0; ch++) {
            uint32_t c = j->node_child.v[cs0 + ch];
            float* dst_me = reach_of(s, c, me);
            float* dst_op = reach_of(s, c, op);
            memcpy(dst_op, src_op, nop * sizeof(float));
            for (uint32_t k = ostart[ch]; k < ostart[ch + 1]; k++) {
                uint32_t a = oact[k];
                const uint32_t* ao = s->acell_off + s->aoff[i];
                for (uint32_t x = ao[a]; x < ao[a + 1]; x++) {
                    uint32_t cell = s->acell[x];
                    uint32_t g = j->soff.v[i] + cell;
                    uint32_t t = j->legal_trans.v[g];
                    if (t == NONE) continue;
                    uint32_t ci = j->cell_row.v[g];
                    dst_me[t] += src_me[ci] * cur[cell];
                }
            }
        }
    }
}

static void precompute_reaches(Solver* s) { propagate(s, s->cur, s->j->root[0].v, s->j->root[1].v); }

/* Pooled belief blocks (engine/src/search.rs:1501-1547); `only` < 0 refreshes both. */
static void belief_blocks(Solver* s, int only) {
    const Job* j = s->j;
    uint32_t pool = j->pool;
    for (uint32_t r = 0; r < j->rows; r++) {
        uint32_t i = j->leaf_rows.v[r];
        for (int p = 0; p < 2; p++) {
            if (only >= 0 && only != p) continue;
            uint32_t n = S_nc(s, i, p);
            normalize_weights(reach_of(s, i, p), n, s->wbuf);
            uint32_t q = 2 * r + (uint32_t)p;
            float* out = s->xb + (size_t)q * pool;
            const uint32_t* cidx = j->leaf_cidx.v + j->leaf_coff.v[q];
            /* accumulate (engine/src/net.rs:161-170) */
            for (uint32_t k = 0; k < pool; k++) out[k] = 0.0f;
            for (uint32_t c = 0; c < n; c++) {
                /* the config's pooling vector: g(c) for v5 (search.rs:1525-1545), else the job's embedding */
                const float* row = s->gcfg ? s->gcfg + (size_t)cidx[c] * pool : j->cphi.v + (size_t)cidx[c] * j->cfeat + 1;
                float w = s->wbuf[c];
                for (uint32_t k = 0; k < pool; k++) out[k] += w * row[k];
            }
        }
    }
}

/* The query input of row r for traverser q: both pooled beliefs (traverser's
 * first), the seat, then the row's public features. */
static void query_input(const Solver* s, uint32_t r, int q, float* x) {
    const Job* j = s->j;
    uint32_t pool = j->pool;
    memcpy(x, s->xb + (size_t)(2 * r + (uint32_t)q) * pool, pool * sizeof(float));
    memcpy(x + pool, s->xb + (size_t)(2 * r + (uint32_t)(1 - q)) * pool, pool * sizeof(float));
    x[2 * pool] = q ? 1.0f : -1.0f;
    const uint8_t* raw = j->leaf_raw.v + (size_t)r * j->row_bytes;
    for (uint32_t k = 0; k < j->row_bytes; k++) x[2 * pool + 1 + k] = (float)raw[k] / 255.0f;
}

static void pbs_head(Solver* s, int traverser) {
    const Net* n = s->net;
    if (n->mode == NET_EMPTY) return;
    const Job* j = s->j;
    if (n->v5) { /* Net::join per row (search.rs:1570-1578) */
        for (uint32_t r = 0; r < j->rows; r++)
            v5_join(n->v5, s->P + (size_t)r * V5_D, s->Jp + (size_t)r * V5_JW,
                    s->xb + (size_t)(2 * r + (uint32_t)traverser) * V5_POOL,
                    s->xb + (size_t)(2 * r + 1 - (uint32_t)traverser) * V5_POOL, traverser, s->h + (size_t)r * V5_D);
        return;
    }
    for (uint32_t r = 0; r < j->rows; r++) {
        query_input(s, r, traverser, s->xin);
        net_trunk(n, s->xin, n->W, n->B, n->in, n->layers, s->h + (size_t)r * n->hidden, s->scratch);
    }
}

/* The net's value of network row r's c-th config of player p, from the trunk
 * output of the last pbs_head (engine/src/net.rs:844-853 for the MLP head). */
static float net_value(const Solver* s, uint32_t r, int p, uint32_t c) {
    const Job* j = s->j;
    const Net* n = s->net;
    const uint32_t* cidx = j->leaf_cidx.v + j->leaf_coff.v[2 * r + (uint32_t)p];
    const float* h = s->h + (size_t)r * n->hidden;
    const float* phi = j->cphi.v + (size_t)cidx[c] * j->cfeat;
    if (n->kind == MODEL_MLP) return head_value(n, h, (uint32_t)phi[0]);
    if (n->v5) return v5_value(n->v5, s->fcfg + (size_t)cidx[c] * V5_D, h);
    /* two-tower: <f(c), h> + bias with f(c) = private tower output x readout weight */
    const float* f = s->fcfg + (size_t)cidx[c] * n->hidden;
    if (!wide_sum(n)) {
        float acc = n->bread;
        for (uint32_t k = 0; k < n->hidden; k++) acc += f[k] * h[k];
        return acc;
    }
    double acc = 0.0;
    for (uint32_t k = 0; k < n->hidden; k++) acc += (double)f[k] * (double)h[k];
    return (float)acc + n->bread;
}

/* Leaf counterfactual values for player p (engine/src/search.rs:1587-1636). */
static void readout(Solver* s, int p) {
    const Job* j = s->j;
    const Net* n = s->net;
    int opp = 1 - p;
    for (uint32_t k = 0; k < j->term_leaves.n; k++) {
        uint32_t i = j->term_leaves.v[k];
        float opp_reach = 0.0f;
        const float* ro = reach_of(s, i, opp);
        for (uint32_t c = 0; c < S_nc(s, i, opp); c++) opp_reach += ro[c];
        float u = (int)j->node_player.v[i] == p ? j->terminal_utility.v[k] : -j->terminal_utility.v[k];
        float* v = s->vals + s->voff[i];
        for (uint32_t c = 0; c < S_nc(s, i, p); c++) v[c] = u * opp_reach;
    }
    if (s->rp_vals) { /* replay: the given net values times the given opponent masses */
        size_t need = 0;
        for (uint32_t r = 0; r < j->rows; r++) need += S_nc(s, j->leaf_rows.v[r], p);
        if (s->rp_vpos + need > s->rp_vn || s->rp_mpos + 2 * (size_t)j->rows > s->rp_mn) {
            s->rp_short = 1;
            return;
        }
        const float* rv = s->rp_vals + s->rp_vpos;
        const float* rm = s->rp_mass + s->rp_mpos;
        for (uint32_t r = 0; r < j->rows; r++) {
            uint32_t i = j->leaf_rows.v[r], nn = S_nc(s, i, p);
            float* v = s->vals + s->voff[i];
            for (uint32_t c = 0; c < nn; c++) v[c] = *rv++ * rm[2 * r + (uint32_t)opp];
        }
        s->rp_vpos += need;
        s->rp_mpos += 2 * (size_t)j->rows;
        return;
    }
    for (uint32_t r = 0; r < j->rows; r++) {
        uint32_t i = j->leaf_rows.v[r];
        float opp_reach = 0.0f;
        const float* ro = reach_of(s, i, opp);
        for (uint32_t c = 0; c < S_nc(s, i, opp); c++) opp_reach += ro[c];
        uint32_t nn = S_nc(s, i, p);
        float* v = s->vals + s->voff[i];
        if (n->mode == NET_EMPTY) {
            for (uint32_t c = 0; c < nn; c++) v[c] = 0.0f;
            continue;
        }
        for (uint32_t c = 0; c < nn; c++) v[c] = net_value(s, r, p, c);
        if (s->tr_vals) {
            memcpy(s->tr_vals + s->tr_vpos, v, nn * sizeof(float));
            s->tr_vpos += nn;
            const float* rp = reach_of(s, i, p);
            float own = 0.0f;
            for (uint32_t c = 0; c < nn; c++) own += rp[c];
            s->tr_mass[s->tr_mpos + 2 * r + (uint32_t)p] = own;
            s->tr_mass[s->tr_mpos + 2 * r + (uint32_t)opp] = opp_reach;
        }
        for (uint32_t c = 0; c < nn; c++) v[c] *= opp_reach;
    }
    if (s->tr_vals) s->tr_mpos += 2 * (size_t)j->rows;
    if (s->tr_reach)
        for (uint32_t r = 0; r < j->rows; r++)
            for (int q = 0; q < 2; q++) {
                uint32_t i = j->leaf_rows.v[r], nq = S_nc(s, i, q);
                memcpy(s->tr_reach + s->tr_rpos, reach_of(s, i, q), nq * sizeof(float));
                s->tr_rpos += nq;
            }
}

static void ensure_leaf_batch(Solver* s) {
    if (s->batch_ready) return;
    s->batch_ready = 1;
    const Net* n = s->net;
    const Job* j = s->j;
    if (n->mode == NET_EMPTY) return;
    if (n->v5) { /* search.rs:1463-1498: cards, board, join cache, configs, once per solve */
        s->cards = (float*)malloc(sizeof(float) * 2 * V5_NTYPE * V5_TYPE);
        s->P = (float*)malloc(sizeof(float) * ((size_t)j->rows * V5_D + 1));
        s->Jp = (float*)malloc(sizeof(float) * ((size_t)j->rows * V5_JW + 1));
        s->fcfg = (float*)malloc(sizeof(float) * ((size_t)j->ncfg * V5_D + 1));
        s->gcfg = (float*)malloc(sizeof(float) * ((size_t)j->ncfg * V5_POOL + 1));
        v5_cards(n->v5, j->card_feat.v, s->cards);
        for (uint32_t r = 0; r < j->rows; r++)
            v5_board(n->v5, j->leaf_raw.v + (size_t)r * V5_ROW_BYTES, s->cards, s->P + (size_t)r * V5_D,
                     s->Jp + (size_t)r * V5_JW);
        for (uint32_t c = 0; c < j->ncfg; c++)
            v5_config(n->v5, j->cphi.v + (size_t)c * V5_CFEAT, j->cplayer.v[c], s->cards,
                      s->fcfg + (size_t)c * V5_D, s->gcfg + (size_t)c * V5_POOL);
        return;
    }
    if (n->kind != MODEL_TWO_TOWER) return;
    /* Private tower once per solve, then fold the readout weight in. */
    s->fcfg = (float*)malloc(((size_t)j->ncfg * n->hidden + 1) * sizeof(float));
    float* hbuf = (float*)malloc(n->hidden * sizeof(float));
    for (uint32_t c = 0; c < j->ncfg; c++) {
        const float* phi = j->cphi.v + (size_t)c * j->cfeat + 1 + j->pool;
        net_trunk(n, phi, n->PW, n->PB, n->priv_in, n->priv_layers, hbuf, s->scratch);
        for (uint32_t k = 0; k < n->hidden; k++) {
            float f = hbuf[k] * n->wread[k];
            s->fcfg[(size_t)c * n->hidden + k] = q_op(n, f);
        }
    }
    free(hbuf);
}

static void leaf_values(Solver* s, int traverser) {
    ensure_leaf_batch(s);
    int redo = s->last_traverser;
    s->last_traverser = traverser;
    if (s->net->mode != NET_EMPTY) belief_blocks(s, redo);
    pbs_head(s, traverser);
    readout(s, traverser);
}

static void leaf_beliefs_both(Solver* s) {
    ensure_leaf_batch(s);
    s->last_traverser = -1;
    if (s->net->mode == NET_EMPTY) return;
    belief_blocks(s, -1);
}

/* One value backpropagation for `traverser` (engine/src/search.rs:1654-1803). */
static void backprop(Solver* s, int traverser, const float* strat, int mode) {
    const Job* j = s->j;
    float da = 0, db = 0, dg = 0;
    if (mode == BACK_REGRET) {
        float m = (float)s->steps[traverser] + 1.0f;
        da = cfr_factor(m, j->alpha);
        db = cfr_factor(m, j->beta);
        dg = powf(m / (m + 1.0f), j->gamma);
    }
    for (uint32_t ii = s->N; ii-- > 0;) {
        uint32_t i = ii;
        uint8_t kind = j->node_kind.v[i];
        if (kind == 2) continue;
        int me = j->node_player.v[i];
        uint32_t nc = S_nc(s, i, traverser);
        if (kind == 1) {
            uint32_t ch = j->node_child.v[j->node_child_start.v[i]];
            float* dst = s->vals + s->voff[i];
            const float* src = s->vals + s->voff[ch];
            if (me == traverser) {
                uint32_t d0 = j->draw_off.v[i], rb = j->draw_row_off.v[i];
                for (uint32_t c = 0; c < nc; c++) {
                    uint32_t lo = j->draw_row_start.v[rb + c], hi = j->draw_row_start.v[rb + c + 1];
                    float v = 0.0f;
                    for (uint32_t k = lo; k < hi; k++) v += j->draw_p.v[d0 + k] * src[j->draw_to.v[d0 + k]];
                    dst[c] = v;
                }
            } else {
                memmove(dst, src, nc * sizeof(float));
            }
            continue;
        }
        float* vi = s->vals + s->voff[i];
        int br = mode == BACK_BR && me == traverser;
        for (uint32_t c = 0; c < nc; c++) vi[c] = br ? -INFINITY : 0.0f;
        if (me == traverser) {
            uint32_t so = j->soff.v[i];
            const uint32_t* ochild = j->obs_child.v + s->act_off[i];
            const uint32_t* ao = s->acell_off + s->aoff[i];
            uint32_t cs0 = j->node_child_start.v[i];
            for (uint32_t a = 0; a < s->na[i]; a++) {
                uint32_t ch = j->node_child.v[cs0 + ochild[a]];
                const float* cv = s->vals + s->voff[ch];
                for (uint32_t x = ao[a]; x < ao[a + 1]; x++) {
                    uint32_t cell = s->acell[x];
                    uint32_t t = j->legal_trans.v[so + cell];
                    if (t == NONE) continue;
                    uint32_t c = j->cell_row.v[so + cell];
                    float av = cv[t];
                    if (mode == BACK_REGRET)
                        vi[c] += av * s->cur[so + cell];
                    else if (mode == BACK_VALUE)
                        vi[c] += av * strat[so + cell];
                    else
                        vi[c] = vi[c] > av ? vi[c] : av;
                }
            }
            if (mode == BACK_REGRET) {
                uint32_t row0 = j->legal_row_of.v[i];
                for (uint32_t c = 0; c < nc; c++) {
                    float base = vi[c];
                    uint32_t lo = j->legal_off.v[row0 + c], hi = j->legal_off.v[row0 + c + 1];
                    float sum = 0.0f;
                    for (uint32_t g = lo; g < hi; g++) {
                        float delta = 0.0f;
                        uint32_t t = j->legal_trans.v[g];
                        if (t != NONE) delta += s->vals[s->voff[j->legal_child.v[g]] + t];
                        delta -= base;
                        float old = s->regret[g];
                        float r = old * (old > 0.0f ? da : db) + delta;
                        s->regret[g] = r;
                        float v = fmaxf(r + j->predict * delta, EPS);
                        s->cur[g] = v;
                        sum += v;
                    }
                    if (sum > 0.0f) {
                        float inv = 1.0f / sum;
                        for (uint32_t g = lo; g < hi; g++) s->cur[g] *= inv;
                    }
                }
                for (uint32_t g = j->soff.v[i]; g < j->soff.v[i + 1]; g++) s->sum[g] *= dg;
            } else if (mode == BACK_BR) {
                for (uint32_t c = 0; c < nc; c++)
                    if (vi[c] == -INFINITY) vi[c] = 0.0f;
            }
        } else {
            for (uint32_t k = j->node_child_start.v[i]; k < j->node_child_start.v[i + 1]; k++) {
                const float* cv = s->vals + s->voff[j->node_child.v[k]];
                for (uint32_t c = 0; c < nc; c++) vi[c] += cv[c];
            }
        }
    }
}

/* avg_block (engine/src/search.rs:1818-1835). */
static void avg_block(Solver* s, int traverser) {
    const Job* j = s->j;
    s->avg_touched[traverser] = 1;
    for (uint32_t i = 0; i < s->N; i++) {
        if (j->node_kind.v[i] != 0 || (int)j->node_player.v[i] != traverser) continue;
        uint32_t row0 = j->legal_row_of.v[i];
        const float* r = reach_of(s, i, traverser);
        for (uint32_t c = 0; c < S_nc(s, i, traverser); c++)
            for (uint32_t g = j->legal_off.v[row0 + c]; g < j->legal_off.v[row0 + c + 1]; g++)
                s->sum[g] += r[c] * s->cur[g];
    }
}

static int snap_kept(const Solver* s, uint32_t t) {
    const Job* j = s->j;
    if (j->snapshots) {
        for (uint32_t k = 0; k < j->snap_iters.n; k++)
            if (j->snap_iters.v[k] == t) return 1;
        return 0;
    }
    return t == j->iters;
}

/* snapshot (engine/src/search.rs:899-938). */
static void snapshot(Solver* s) {
    const Job* j = s->j;
    uint32_t t = s->snap_t++;
    if (!snap_kept(s, t)) return;
    float* snap = (float*)malloc(((size_t)j->ncells + 1) * sizeof(float));
    memcpy(snap, s->cur, (size_t)j->ncells * sizeof(float));
    for (uint32_t i = 0; i < s->N; i++) {
        if (j->node_kind.v[i] != 0 || !s->avg_touched[j->node_player.v[i]]) continue;
        int me = j->node_player.v[i];
        uint32_t row0 = j->legal_row_of.v[i];
        for (uint32_t c = 0; c < S_nc(s, i, me); c++) {
            uint32_t lo = j->legal_off.v[row0 + c], hi = j->legal_off.v[row0 + c + 1];
            float sum = 0.0f;
            for (uint32_t g = lo; g < hi; g++) sum += s->sum[g];
            float k = (float)(hi > lo ? hi - lo : 1);
            for (uint32_t g = lo; g < hi; g++) snap[g] = sum > 0.0f ? s->sum[g] / sum : 1.0f / k;
        }
    }
    s->snaps[s->nsnaps++] = snap;
}

static void solver_free(Solver* s) {
    free(s->nc0);
    free(s->nc1);
    free(s->act_off);
    free(s->na);
    free(s->acell_off);
    free(s->acell);
    free(s->aoff);
    free(s->regret);
    free(s->cur);
    free(s->sum);
    free(s->reach);
    free(s->vals);
    free(s->voff);
    if (s->snaps)
        for (uint32_t k = 0; k < s->nsnaps; k++) free(s->snaps[k]);
    free(s->snaps);
    free(s->xb);
    free(s->h);
    free(s->xin);
    free(s->scratch);
    free(s->wbuf);
    free(s->fcfg);
    free(s->cards);
    free(s->P);
    free(s->Jp);
    free(s->gcfg);
    memset(s, 0, sizeof *s);
}

/* Solver::new's arena set-up (engine/src/search.rs:796-876). */
static int solver_init(Solver* s, const Job* j, const Net* net) {
    memset(s, 0, sizeof *s);
    s->j = j;
    s->net = net;
    uint32_t N = s->N = j->nodes;
    if (net->mode != NET_EMPTY) {
        if (net->kind != j->kind || net->in != j->in || net->hidden != j->hidden || net->pool != j->pool ||
            (net->kind == MODEL_MLP && net->heads != j->heads)) {
            snprintf(g_err, sizeof g_err, "network shape disagrees with the job's net_dims");
            return 0;
        }
    }
    s->nc0 = (uint32_t*)malloc(N * sizeof(uint32_t));
    s->nc1 = (uint32_t*)malloc(N * sizeof(uint32_t));
    s->act_off = (uint32_t*)calloc(N + 1, sizeof(uint32_t));
    s->na = (uint32_t*)calloc(N + 1, sizeof(uint32_t));
    s->voff = (uint32_t*)malloc((N + 1) * sizeof(uint32_t));
    s->aoff = (uint32_t*)calloc(N + 1, sizeof(uint32_t));
    uint32_t maxnc = 1, acts = 0, vl = 0, aoffs = 0;
    for (uint32_t i = 0; i < N; i++) {
        s->nc0[i] = j->cfg_off.v[2 * i + 1] - j->cfg_off.v[2 * i];
        s->nc1[i] = j->cfg_off.v[2 * i + 2] - j->cfg_off.v[2 * i + 1];
        if (s->nc0[i] > maxnc) maxnc = s->nc0[i];
        if (s->nc1[i] > maxnc) maxnc = s->nc1[i];
        s->voff[i] = vl;
        vl += s->nc0[i] > s->nc1[i] ? s->nc0[i] : s->nc1[i];
        s->act_off[i] = acts;
        s->aoff[i] = aoffs;
        if (j->node_kind.v[i] == 0) {
            uint32_t o0 = j->obs_off.v[i], o1 = j->obs_off.v[i + 1];
            if (o1 <= o0) {
                snprintf(g_err, sizeof g_err, "decision node %u has no observation rows", i);
                return 0;
            }
            s->na[i] = j->obs_start.v[o1 - 1];
            acts += s->na[i];
            aoffs += s->na[i] + 1;
        }
    }
    s->voff[N] = vl;
    s->vals_len = vl;
    if (acts != j->obs_act.n || acts != j->obs_child.n) {
        snprintf(g_err, sizeof g_err, "observation arrays disagree with action counts");
        return 0;
    }
    /* Action-major cell view, as the reference keeps per node (search.rs:1093-1107). */
    s->acell_off = (uint32_t*)calloc((size_t)aoffs + 1, sizeof(uint32_t));
    s->acell = (uint32_t*)calloc((size_t)j->ncells + 1, sizeof(uint32_t));
    for (uint32_t i = 0; i < N; i++) {
        if (j->node_kind.v[i] != 0) continue;
        uint32_t so = j->soff.v[i], ncl = j->soff.v[i + 1] - so, na = s->na[i];
        uint32_t* ao = s->acell_off + s->aoff[i];
        for (uint32_t x = 0; x < ncl; x++) {
            uint32_t a = j->legal_action.v[so + x];
            if (a >= na) {
                snprintf(g_err, sizeof g_err, "legal_action out of range at node %u", i);
                return 0;
            }
            ao[a + 1]++;
        }
        for (uint32_t a = 0; a < na; a++) ao[a + 1] += ao[a];
        uint32_t* fill = (uint32_t*)malloc((na + 1) * sizeof(uint32_t));
        memcpy(fill, ao, (na + 1) * sizeof(uint32_t));
        for (uint32_t x = 0; x < ncl; x++) s->acell[so + fill[j->legal_action.v[so + x]]++] = x;
        for (uint32_t a = 0; a <= na; a++) ao[a] += so; /* absolute index into acell */
        free(fill);
    }
    size_t nc = j->ncells;
    s->regret = (float*)calloc(nc + 1, sizeof(float));
    s->cur = (float*)calloc(nc + 1, sizeof(float));
    s->sum = (float*)calloc(nc + 1, sizeof(float));
    s->reach = (float*)calloc((size_t)j->reach_off.v[N] + 1, sizeof(float));
    s->vals = (float*)calloc((size_t)vl + 1, sizeof(float));
    s->snaps = (float**)calloc(j->iters + 2, sizeof(float*));
    uint32_t pool = j->pool ? j->pool : 1;
    s->xb = (float*)calloc(2 * (size_t)j->rows * pool + 1, sizeof(float));
    uint32_t hid = net->hidden ? net->hidden : 1;
    s->h = (float*)calloc((size_t)j->rows * hid + 1, sizeof(float));
    uint32_t wide = j->in > hid ? j->in : hid;
    if (net->priv_in > wide) wide = net->priv_in;
    s->xin = (float*)calloc(wide + 1, sizeof(float));
    s->scratch = (float*)calloc(2 * (size_t)wide + 2, sizeof(float));
    s->wbuf = (float*)calloc(maxnc + 1, sizeof(float));
    s->last_traverser = -1;
    if (j->root[0].n != s->nc0[0] || j->root[1].n != s->nc1[0]) {
        snprintf(g_err, sizeof g_err, "root belief length != root support");
        return 0;
    }
    /* Uniform current strategy over each row's legal cells. */
    for (uint32_t i = 0; i < N; i++) {
        if (j->node_kind.v[i] != 0) continue;
        int me = j->node_player.v[i];
        uint32_t row0 = j->legal_row_of.v[i];
        for (uint32_t c = 0; c < S_nc(s, i, me); c++) {
            uint32_t lo = j->legal_off.v[row0 + c], hi = j->legal_off.v[row0 + c + 1];
            float k = (float)(hi - lo);
            for (uint32_t g = lo; g < hi; g++) s->cur[g] = 1.0f / k;
        }
    }
    precompute_reaches(s);
    /* Seed the sums with one reach-weighted uniform strategy. */
    for (uint32_t i = 0; i < N; i++) {
        if (j->node_kind.v[i] != 0 || j->soff.v[i + 1] == j->soff.v[i]) continue;
        int me = j->node_player.v[i];
        uint32_t row0 = j->legal_row_of.v[i];
        const float* r = reach_of(s, i, me);
        for (uint32_t c = 0; c < S_nc(s, i, me); c++)
            for (uint32_t g = j->legal_off.v[row0 + c]; g < j->legal_off.v[row0 + c + 1]; g++)
                s->sum[g] += r[c] * s->cur[g];
    }
    /* snapshot_initial */
    s->snap_t = 1;
    if (j->snapshots || j->iters == 0) {
        float* snap = (float*)malloc((nc + 1) * sizeof(float));
        memcpy(snap, s->cur, nc * sizeof(float));
        s->snaps[s->nsnaps++] = snap;
    }
    return 1;
}

static void step(Solver* s, int traverser) { /* search.rs:1805-1814 */
    leaf_values(s, traverser);
    backprop(s, traverser, NULL, BACK_REGRET);
    precompute_reaches(s);
    avg_block(s, traverser);
    snapshot(s);
    s->steps[traverser] += 1;
}

/* value_under for every carried root (engine/src/search.rs:1851-1871). */
static void value_under(Solver* s, float* out) {
    const Job* j = s->j;
    const float* ref = s->snaps[s->nsnaps - 1];
    uint32_t n0 = s->nc0[0], n1 = s->nc1[0];
    for (uint32_t r = 0; r < j->nroots; r++) {
        propagate(s, ref, j->carried[2 * r].v, j->carried[2 * r + 1].v);
        leaf_beliefs_both(s);
        for (int p = 0; p < 2; p++) {
            pbs_head(s, p);
            readout(s, p);
            backprop(s, p, ref, BACK_VALUE);
            uint32_t n = p ? n1 : n0;
            memcpy(out + (size_t)r * (n0 + n1) + (p ? n0 : 0), s->vals + s->voff[0], n * sizeof(float));
        }
    }
    precompute_reaches(s);
    s->last_traverser = -1;
}

/* carried_beliefs for every exit and every kept snapshot but the last
 * (engine/src/search.rs:1937-1956), laid out like the device carry store:
 * out[slot * snapshot_configs + snap_coff[2 * exit + p] + c]. */
static void carried_beliefs(Solver* s, float* out) {
    const Job* j = s->j;
    uint32_t nexit = j->leaf_rows.n + j->term_leaves.n;
    uint32_t total = j->snap_coff.v[2 * nexit];
    for (uint32_t k = 0; k + 1 < s->nsnaps; k++) {
        propagate(s, s->snaps[k], j->root[0].v, j->root[1].v);
        for (uint32_t e = 0; e < nexit; e++) {
            uint32_t leaf = e < j->leaf_rows.n ? j->leaf_rows.v[e] : j->term_leaves.v[e - j->leaf_rows.n];
            for (int p = 0; p < 2; p++)
                normalize_weights(reach_of(s, leaf, p), S_nc(s, leaf, p),
                                  out + (size_t)k * total + j->snap_coff.v[2 * e + (uint32_t)p]);
        }
    }
    precompute_reaches(s);
}

/* nash_conv (engine/src/search.rs:1884-1906). */
static void nash_conv(Solver* s, float* nash_out, float* zero_sum_out) {
    const Job* j = s->j;
    const float* ref = s->snaps[s->nsnaps - 1];
    propagate(s, ref, j->root[0].v, j->root[1].v);
    leaf_beliefs_both(s);
    float nash = 0.0f, zs = 0.0f;
    for (int p = 0; p < 2; p++) {
        pbs_head(s, p);
        readout(s, p);
        uint32_t nc = S_nc(s, 0, p);
        const float* root = j->root[p].v;
        backprop(s, p, ref, BACK_VALUE);
        float v = 0.0f;
        for (uint32_t c = 0; c < nc; c++) v += root[c] * s->vals[s->voff[0] + c];
        backprop(s, p, ref, BACK_BR);
        float b = 0.0f;
        for (uint32_t c = 0; c < nc; c++) b += root[c] * s->vals[s->voff[0] + c];
        nash += b - v;
        zs += v;
    }
    precompute_reaches(s);
    s->last_traverser = -1;
    *nash_out = nash;
    *zero_sum_out = zs;
}

/* -------------------------------------------------------------- exports */

typedef struct {
    uint32_t nodes, ncells, rows, nterm, ncfg, reach_len, nroots, root_n0, root_n1, snapshot_configs,
        carry_slots, iters, nlevels, decision_nodes, chance_nodes, leaves;
} OracleShape;

int oracle_job_shape(const uint8_t* b, size_t n, OracleShape* out) {
    Job j;
    if (!parse_job(b, n, &j)) {
        job_free(&j);
        return -1;
    }
    memset(out, 0, sizeof *out);
    out->nodes = j.nodes;
    out->ncells = j.ncells;
    out->rows = j.rows;
    out->nterm = j.term_leaves.n;
    out->ncfg = j.ncfg;
    out->reach_len = j.reach_off.v[j.nodes];
    out->nroots = j.nroots;
    out->root_n0 = j.root[0].n;
    out->root_n1 = j.root[1].n;
    out->snapshot_configs = j.snap_coff.v[j.snap_coff.n - 1];
    out->carry_slots = j.snapshots && j.snap_iters.n > 0 ? j.snap_iters.n - 1 : 0;
    out->iters = j.iters;
    out->nlevels = j.level_start.n ? j.level_start.n - 1 : 0;
    for (uint32_t i = 0; i < j.nodes; i++) {
        if (j.node_kind.v[i] == 0) out->decision_nodes++;
        if (j.node_kind.v[i] == 1) out->chance_nodes++;
        if (j.node_kind.v[i] == 2) out->leaves++;
    }
    job_free(&j);
    return 0;
}

/* Solve one job the way the reference CPU path does: Solver::new, multistep(iters),
 * then value_under(carried) and carried_beliefs. Outputs may be NULL.
 * strategy: [ncells]; roots: [nroots * (n0 + n1)]; carries: [carry_slots * snapshot_configs];
 * conv: [2] = (nash_conv, zero_sum) of the final average (computed only if non-NULL). */
int oracle_solve(const uint8_t* b, size_t n, int net_mode, const uint32_t* dims, uint32_t ndims,
                 const float* w, size_t nw, const float* bias, size_t nb, const float* ln, size_t nln,
                 float* strategy, float* roots, float* carries, float* conv) {
    Job j;
    Net net;
    Solver s;
    int rc = -1;
    memset(&s, 0, sizeof s);
    memset(&net, 0, sizeof net);
    if (!parse_job(b, n, &j)) goto out;
    if (!net_init(&net, net_mode, dims, ndims, w, nw, bias, nb, ln, nln)) goto out;
    if (!solver_init(&s, &j, &net)) goto out;
    for (uint32_t t = 0; t < j.iters; t++) step(&s, (int)(t % 2));
    if (strategy) memcpy(strategy, s.snaps[s.nsnaps - 1], (size_t)j.ncells * sizeof(float));
    if (roots) value_under(&s, roots);
    if (carries && j.snapshots) carried_beliefs(&s, carries);
    if (conv) nash_conv(&s, &conv[0], &conv[1]);
    rc = 0;
out:
    solver_free(&s);
    net_free(&net);
    job_free(&j);
    return rc;
}

/* The leaf net's values at the initial reach (Solver::new: uniform strategy,
 * the root beliefs) for traverser p: for each network row in order, the net's
 * value of each of the row's configs of player p, in the row's config order
 * (values: the sum over rows of nc_p floats, *count receives it; nothing is
 * written when it exceeds cap), and every row's reach masses of both players
 * (mass: rows x 2, config-order sums). */
int oracle_leaf_probe(const uint8_t* b, size_t n, int net_mode, const uint32_t* dims, uint32_t ndims,
                      const float* w, size_t nw, const float* bias, size_t nb, const float* ln, size_t nln,
                      int traverser, float* values, size_t cap, size_t* count, float* mass) {
    Job j;
    Net net;
    Solver s;
    int rc = -1;
    memset(&s, 0, sizeof s);
    memset(&net, 0, sizeof net);
    if (!parse_job(b, n, &j)) goto out;
    if (!net_init(&net, net_mode, dims, ndims, w, nw, bias, nb, ln, nln)) goto out;
    if (net_mode == NET_EMPTY || traverser < 0 || traverser > 1) {
        snprintf(g_err, sizeof g_err, "leaf probe needs a network and a traverser 0 or 1");
        goto out;
    }
    if (!solver_init(&s, &j, &net)) goto out;
    leaf_beliefs_both(&s);
    pbs_head(&s, traverser);
    size_t k = 0;
    for (uint32_t r = 0; r < j.rows; r++) k += S_nc(&s, j.leaf_rows.v[r], traverser);
    *count = k;
    if (k > cap) {
        rc = 0;
        goto out;
    }
    k = 0;
    for (uint32_t r = 0; r < j.rows; r++) {
        uint32_t i = j.leaf_rows.v[r];
        for (uint32_t c = 0; c < S_nc(&s, i, traverser); c++) values[k++] = net_value(&s, r, traverser, c);
        for (int p = 0; p < 2; p++) {
            const float* ro = reach_of(&s, i, p);
            float tot = 0.0f;
            for (uint32_t c = 0; c < S_nc(&s, i, p); c++) tot += ro[c];
            if (mass) mass[2 * r + (uint32_t)p] = tot;
        }
    }
    rc = 0;
out:
    solver_free(&s);
    net_free(&net);
    job_free(&j);
    return rc;
}

/* Per network row, how many floats the leaf evaluations below take and give:
 * out[0] / out[1] the values of traverser 0 / 1 (the sum over rows of nc_p),
 * out[2] the rows, out[3] the rows' reach (the sum of nc_0 + nc_1). */
int oracle_leaf_counts(const uint8_t* b, size_t n, size_t* out) {
    Job j;
    if (!parse_job(b, n, &j)) {
        job_free(&j);
        return -1;
    }
    out[0] = out[1] = out[3] = 0;
    out[2] = j.rows;
    for (uint32_t r = 0; r < j.rows; r++) {
        uint32_t i = j.leaf_rows.v[r];
        size_t a = j.cfg_off.v[2 * i + 1] - j.cfg_off.v[2 * i], c = j.cfg_off.v[2 * i + 2] - j.cfg_off.v[2 * i + 1];
        out[0] += a;
        out[1] += c;
        out[3] += a + c;
    }
    job_free(&j);
    return 0;
}

/* The leaf net's values for traverser p at a given reach: the leaf rows'
 * reach is set from `reach` (per row in order, player 0's configs then player
 * 1's) and the leaf input and net run as belief_blocks + pbs_head do. values
 * (out[traverser] floats of oracle_leaf_counts) and mass (rows x 2, the
 * config-order sums of the given reach) as oracle_leaf_probe gives them. */
int oracle_leaf_eval(const uint8_t* b, size_t n, int net_mode, const uint32_t* dims, uint32_t ndims, const float* w,
                     size_t nw, const float* bias, size_t nb, const float* ln, size_t nln, int traverser,
                     const float* reach, float* values, float* mass) {
    Job j;
    Net net;
    Solver s;
    int rc = -1;
    memset(&s, 0, sizeof s);
    memset(&net, 0, sizeof net);
    if (!parse_job(b, n, &j)) goto out;
    if (!net_init(&net, net_mode, dims, ndims, w, nw, bias, nb, ln, nln)) goto out;
    if (net_mode == NET_EMPTY || traverser < 0 || traverser > 1) {
        snprintf(g_err, sizeof g_err, "leaf evaluation needs a network and a traverser 0 or 1");
        goto out;
    }
    if (!solver_init(&s, &j, &net)) goto out;
    {
        const float* rr = reach;
        for (uint32_t r = 0; r < j.rows; r++) {
            uint32_t i = j.leaf_rows.v[r];
            for (int p = 0; p < 2; p++) {
                float* ro = reach_of(&s, i, p);
                float tot = 0.0f;
                for (uint32_t c = 0; c < S_nc(&s, i, p); c++) {
                    ro[c] = *rr++;
                    tot += ro[c];
                }
                if (mass) mass[2 * r + (uint32_t)p] = tot;
            }
        }
    }
    leaf_beliefs_both(&s);
    pbs_head(&s, traverser);
    {
        size_t k = 0;
        for (uint32_t r = 0; r < j.rows; r++)
            for (uint32_t c = 0; c < S_nc(&s, j.leaf_rows.v[r], traverser); c++)
                values[k++] = net_value(&s, r, traverser, c);
    }
    rc = 0;
out:
    solver_free(&s);
    net_free(&net);
    job_free(&j);
    return rc;
}

/* oracle_solve recording every leaf-net evaluation in the layout
 * oracle_solve_replay takes: vals and mass must hold the sum over the
 * evaluations (iterations 0 .. iters-1, then per carried root players 0 and 1)
 * of each one's values (the rows' configs of its player) and 2 * rows masses;
 * reach (may be NULL) per evaluation each row's reach of both players, as
 * oracle_leaf_eval takes it. */
int oracle_solve_trace(const uint8_t* b, size_t n, int net_mode, const uint32_t* dims, uint32_t ndims,
                       const float* w, size_t nw, const float* bias, size_t nb, const float* ln, size_t nln,
                       float* vals, float* mass, float* reach, float* strategy, float* roots) {
    Job j;
    Net net;
    Solver s;
    int rc = -1;
    memset(&s, 0, sizeof s);
    memset(&net, 0, sizeof net);
    if (!parse_job(b, n, &j)) goto out;
    if (!net_init(&net, net_mode, dims, ndims, w, nw, bias, nb, ln, nln)) goto out;
    if (net_mode == NET_EMPTY) {
        snprintf(g_err, sizeof g_err, "a trace needs a network");
        goto out;
    }
    if (!solver_init(&s, &j, &net)) goto out;
    s.tr_vals = vals;
    s.tr_mass = mass;
    s.tr_reach = reach;
    for (uint32_t t = 0; t < j.iters; t++) step(&s, (int)(t % 2));
    if (strategy) memcpy(strategy, s.snaps[s.nsnaps - 1], (size_t)j.ncells * sizeof(float));
    if (roots) value_under(&s, roots);
    rc = 0;
out:
    solver_free(&s);
    net_free(&net);
    job_free(&j);
    return rc;
}

/* oracle_solve with every network leaf's value given instead of computed:
 * `vals` holds, for each leaf-net evaluation in schedule order (iterations
 * 0 .. iters-1 with traverser t % 2, then per carried root players 0 and 1),
 * each network row's values of that evaluation's player (row order, row config
 * order), and `mass` the rows' reach masses of that evaluation (rows x 2); a
 * network leaf's counterfactual value is its given value times the given mass
 * of the opponent. Everything else (terminals, backprop, regret matching, the
 * average, Phase 2, carries) is the solver's own. With the values and masses a
 * device's leaf net produced inside its own solve, the outputs equal that
 * device's bit for bit exactly when its CFR arithmetic is the solver's. */
int oracle_solve_replay(const uint8_t* b, size_t n, const float* vals, size_t nvals, const float* mass, size_t nmass,
                        float* strategy, float* roots, float* carries) {
    Job j;
    Net net;
    Solver s;
    int rc = -1;
    memset(&s, 0, sizeof s);
    memset(&net, 0, sizeof net);
    if (!parse_job(b, n, &j)) goto out;
    if (!net_init(&net, NET_EMPTY, NULL, 0, NULL, 0, NULL, 0, NULL, 0)) goto out;
    if (!solver_init(&s, &j, &net)) goto out;
    s.rp_vals = vals;
    s.rp_mass = mass;
    s.rp_vn = nvals;
    s.rp_mn = nmass;
    for (uint32_t t = 0; t < j.iters; t++) step(&s, (int)(t % 2));
    if (strategy) memcpy(strategy, s.snaps[s.nsnaps - 1], (size_t)j.ncells * sizeof(float));
    if (roots) value_under(&s, roots);
    if (carries && j.snapshots) carried_beliefs(&s, carries);
    if (s.rp_short) {
        snprintf(g_err, sizeof g_err, "the replay holds fewer leaf values than the schedule evaluates");
        goto out;
    }
    if (s.rp_vpos != nvals || s.rp_mpos != nmass) {
        snprintf(g_err, sizeof g_err, "the replay holds more leaf values than the schedule evaluates");
        goto out;
    }
    rc = 0;
out:
    solver_free(&s);
    net_free(&net);
    job_free(&j);
    return rc;
}

/* Run the MLP trunk + per-key head on dense inputs: x [rows x in], keys [rows x nk]
 * (head rows to read per query), out [rows x nk]; h_out (optional) [rows x hidden]. */
int oracle_mlp(uint32_t rows, const float* x, uint32_t nk, const uint32_t* keys, int net_mode,
               const uint32_t* dims, uint32_t ndims, const float* w, size_t nw, const float* bias, size_t nb,
               float* out, float* h_out) {
    Net net;
    if (!net_init(&net, net_mode, dims, ndims, w, nw, bias, nb, NULL, 0)) return -1;
    if (net.kind != MODEL_MLP) {
        snprintf(g_err, sizeof g_err, "oracle_mlp needs an MLP tag");
        net_free(&net);
        return -1;
    }
    uint32_t wide = net.in > net.hidden ? net.in : net.hidden;
    float* scratch = (float*)malloc((2 * (size_t)wide + 2) * sizeof(float));
    float* h = (float*)malloc(((size_t)net.hidden + 1) * sizeof(float));
    for (uint32_t r = 0; r < rows; r++) {
        net_trunk(&net, x + (size_t)r * net.in, net.W, net.B, net.in, net.layers, h, scratch);
        if (h_out) memcpy(h_out + (size_t)r * net.hidden, h, net.hidden * sizeof(float));
        for (uint32_t k = 0; k < nk; k++) out[(size_t)r * nk + k] = head_value(&net, h, keys[(size_t)r * nk + k]);
    }
    free(scratch);
    free(h);
    net_free(&net);
    return 0;
}

/* ------------------------------------------------- threaded CPU baseline */

typedef struct {
    const uint8_t* const* jobs;
    const size_t* lens;
    uint32_t njobs;
    int net_mode;
    const uint32_t* dims;
    uint32_t ndims;
    const float *w, *b, *ln;
    size_t nw, nb, nln;
    volatile uint32_t next;
    volatile int failed;
    uint64_t node_iters;
    uint64_t leaf_queries;
    pthread_mutex_t mu;
} Batch;

static void* batch_worker(void* arg) {
    Batch* bt = (Batch*)arg;
    for (;;) {
        uint32_t k = __atomic_fetch_add(&bt->next, 1u, __ATOMIC_RELAXED);
        if (k >= bt->njobs) break;
        Job j;
        Net net;
        Solver s;
        memset(&s, 0, sizeof s);
        memset(&net, 0, sizeof net);
        int ok = parse_job(bt->jobs[k], bt->lens[k], &j) &&
                 net_init(&net, bt->net_mode, bt->dims, bt->ndims, bt->w, bt->nw, bt->b, bt->nb, bt->ln, bt->nln) &&
                 solver_init(&s, &j, &net);
        if (ok) {
            for (uint32_t t = 0; t < j.iters; t++) step(&s, (int)(t % 2));
            size_t nr = (size_t)j.nroots * (j.root[0].n + j.root[1].n);
            float* roots = (float*)malloc((nr + 1) * sizeof(float));
            value_under(&s, roots);
            free(roots);
            pthread_mutex_lock(&bt->mu);
            bt->node_iters += (uint64_t)j.nodes * j.iters;
            bt->leaf_queries += (uint64_t)j.rows * (j.iters + 2ull * j.nroots);
            pthread_mutex_unlock(&bt->mu);
        } else {
            bt->failed = 1;
        }
        solver_free(&s);
        net_free(&net);
        job_free(&j);
    }
    return NULL;
}

/* Solve `njobs` jobs, one job per thread at a time, on `threads` threads (the
 * reference parallelises across solves, engine/src/selfplay.rs:1426-1428).
 * Returns wall seconds, or a negative value on failure. */
double oracle_solve_batch(uint32_t njobs, const uint8_t* const* jobs, const size_t* lens, uint32_t threads,
                          int net_mode, const uint32_t* dims, uint32_t ndims, const float* w, size_t nw,
                          const float* bias, size_t nb, const float* ln, size_t nln, uint64_t* node_iters,
                          uint64_t* leaf_queries) {
    Batch bt;
    memset(&bt, 0, sizeof bt);
    bt.jobs = jobs;
    bt.lens = lens;
    bt.njobs = njobs;
    bt.net_mode = net_mode;
    bt.dims = dims;
    bt.ndims = ndims;
    bt.w = w;
    bt.b = bias;
    bt.nw = nw;
    bt.nb = nb;
    bt.ln = ln;
    bt.nln = nln;
    pthread_mutex_init(&bt.mu, NULL);
    if (threads < 1) threads = 1;
    pthread_t* th = (pthread_t*)malloc(threads * sizeof(pthread_t));
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (uint32_t k = 0; k < threads; k++) pthread_create(&th[k], NULL, batch_worker, &bt);
    for (uint32_t k = 0; k < threads; k++) pthread_join(th[k], NULL);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    free(th);
    pthread_mutex_destroy(&bt.mu);
    if (node_iters) *node_iters = bt.node_iters;
    if (leaf_queries) *leaf_queries = bt.leaf_queries;
    if (bt.failed) return -1.0;
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

typedef struct {
    const float* x;
    uint32_t rows, nk;
    const uint32_t* keys;
    Net* net;
    float* out;
    volatile uint32_t next;
} MlpBatch;

static void* mlp_worker(void* arg) {
    MlpBatch* m = (MlpBatch*)arg;
    Net* n = m->net;
    uint32_t wide = n->in > n->hidden ? n->in : n->hidden;
    float* scratch = (float*)malloc((2 * (size_t)wide + 2) * sizeof(float));
    float* h = (float*)malloc(((size_t)n->hidden + 1) * sizeof(float));
    for (;;) {
        uint32_t r0 = __atomic_fetch_add(&m->next, 64u, __ATOMIC_RELAXED);
        if (r0 >= m->rows) break;
        uint32_t r1 = r0 + 64 < m->rows ? r0 + 64 : m->rows;
        for (uint32_t r = r0; r < r1; r++) {
            net_trunk(n, m->x + (size_t)r * n->in, n->W, n->B, n->in, n->layers, h, scratch);
            for (uint32_t k = 0; k < m->nk; k++)
                m->out[(size_t)r * m->nk + k] = head_value(n, h, m->keys ? m->keys[(size_t)r * m->nk + k] : k);
        }
    }
    free(scratch);
    free(h);
    return NULL;
}

/* Dense MLP over `rows` queries on `threads` threads; head rows 0..nk-1 (keys NULL)
 * or the given keys. Returns wall seconds. */
double oracle_mlp_batch(uint32_t rows, const float* x, uint32_t nk, const uint32_t* keys, uint32_t threads,
                        int net_mode, const uint32_t* dims, uint32_t ndims, const float* w, size_t nw,
                        const float* bias, size_t nb, float* out) {
    Net net;
    if (!net_init(&net, net_mode, dims, ndims, w, nw, bias, nb, NULL, 0)) return -1.0;
    MlpBatch m = {x, rows, nk, keys, &net, out, 0};
    if (threads < 1) threads = 1;
    pthread_t* th = (pthread_t*)malloc(threads * sizeof(pthread_t));
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (uint32_t k = 0; k < threads; k++) pthread_create(&th[k], NULL, mlp_worker, &m);
    for (uint32_t k = 0; k < threads; k++) pthread_join(th[k], NULL);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    free(th);
    net_free(&net);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}
