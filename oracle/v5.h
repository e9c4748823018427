/*
 * ORACLE — test infrastructure only (see oracle.c's header).
 *
 * The reference's production leaf network, the v5 model (net_dims [5]):
 * engine/src/net.rs restated in C, in the CPU loop order of net.rs, on the
 * GPU job contract's inputs (the per-row public bytes of
 * engine/src/rebel.rs:966-986 and the per-job card table).
 */
#pragma once

#include <stddef.h>
#include <stdint.h>

/* engine/src/net.rs:22-39 */
enum { V5_TYPE = 64, V5_C = 96, V5_BLOCKS = 8, V5_D = 256, V5_POOL = 64, V5_CFGH = 128, V5_JW = 128,
       V5_JBLOCKS = 3, V5_JOIN_IN = 2 * V5_POOL + 1 };
/* engine/src/board.rs:8, rebel.rs:61,891,903-923, units.rs:71 */
enum { V5_HEXES = 37, V5_NSLOT = 5, V5_NTYPE = 10, V5_HEX_FACTS = 6, V5_PILE_COUNTS = 4, V5_CARD_FEATS = 25,
       V5_CFEAT = 15, V5_LOOSE = 15 };
/* GPU public row (engine/src/rebel.rs:973-986) */
enum { V5_ROW_BYTES = 201 };
/* Norms in application order (net.rs:415-419): two per trunk block, the
 * trunk's, the config encoder's, one per join block, the join output's, h's. */
enum { V5_NORMS = 2 * V5_BLOCKS + 1 + 1 + V5_JBLOCKS + 1 + 1 };

/* Flat blob sizes of the v5 model (net.rs:233-316). */
void v5_sizes(size_t* nw, size_t* nb, size_t* nln);

typedef struct V5 V5;
/* mode: the oracle's NET_* arithmetic model; libm_tanh selects the C
 * library's tanhf inside GELU instead of the restatement's own (see v5.c). */
V5* v5_new(int mode, const float* w, size_t nw, const float* b, size_t nb, const float* ln, size_t nln,
           int libm_tanh, char* err, size_t errlen);
void v5_free(V5* n);

/* Net::cards for both seat views: cards[v][t][TYPE] from the job's card table
 * (NTYPE x CARD_FEATS, physical coin-type order). */
void v5_cards(const V5* n, const float* card_feat, float* cards);
/* Net::board + Net::join_cache for one network row: P (D) and Jp (JW). */
void v5_board(const V5* n, const uint8_t* raw, const float* cards, float* P, float* Jp);
/* Net::configs for one config: f (D) and g (POOL). */
void v5_config(const V5* n, const float* phi, int owner, const float* cards, float* f, float* g);
/* Net::join for one row and player: h (D). */
void v5_join(const V5* n, const float* P, const float* Jp, const float* pooled_me, const float* pooled_opp,
             int player, float* h);
/* Net::values for one config: <f, h> + value_bias. */
float v5_value(const V5* n, const float* f, const float* h);
/* The GELU the restatement uses (for the pins). */
float v5_gelu(const V5* n, float x);
