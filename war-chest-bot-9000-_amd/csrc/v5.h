// The reference's production leaf network (net_dims [5], engine/src/net.rs):
// shapes, the flat weight blob's layout, the board geometry, and the device
// entry points the executor drives.
//
// Per wave (once per upload and weight bank): the card tokens of both seat
// views and their count-weighted bag rows per job, the board trunk of every
// network row (stem, 8 pre-activation residual blocks over the hex
// adjacency, the pooled board vector P and its join projection Jp), and the
// config encoder's f(c) and g(c) per interned config. Per iteration: the
// pooled beliefs sum_c beta(c) g(c) (the shared leaf-input kernel), the join
// (129 -> 128, three residual blocks, 128 -> 256 plus P, LayerNorm) per row,
// and the readout <f(c), h(row)> + value_bias per leaf slot (the shared
// readout-block kernels).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace wc {

namespace v5 {

// engine/src/net.rs:22-39
constexpr uint32_t TYPE = 64, C = 96, BLOCKS = 8, D = 256, POOL = 64, CFGH = 128, JW = 128, JBLOCKS = 3,
                   JOIN_IN = 2 * POOL + 1;
// engine/src/board.rs:8; rebel.rs:61,891,903-923; units.rs:71
constexpr uint32_t HEXES = 37, NSLOT = 5, NTYPE = 10, HEX_FACTS = 6, PILE_COUNTS = 4, CARD_FEATS = 25, CFEAT = 15,
                   LOOSE = 15;
// The GPU public row (engine/src/rebel.rs:973-986).
constexpr uint32_t GR_HEX_OWNER = 0, GR_HEX_SLOT = GR_HEX_OWNER + HEXES, GR_HEX_HEIGHT = GR_HEX_SLOT + HEXES,
                   GR_HEX_MARKER = GR_HEX_HEIGHT + HEXES, GR_PILES = GR_HEX_MARKER + HEXES,
                   GR_MARKERS = GR_PILES + NTYPE * PILE_COUNTS, GR_HAND = GR_MARKERS + 2, GR_FD = GR_HAND + 2,
                   GR_BAG = GR_FD + 2, GR_INITIATIVE = GR_BAG + 2, GR_INIT_MOVED = GR_INITIATIVE + 1,
                   GR_TO_ACT = GR_INIT_MOVED + 1, GR_PLIES = GR_TO_ACT + 1, ROW_BYTES = GR_PLIES + 2;
static_assert(ROW_BYTES == 201, "GPU_ROW_BYTES");
// Norms in application order (net.rs:214-219,233-242).
constexpr uint32_t NORMS = 2 * BLOCKS + 1 + 1 + JBLOCKS + 1 + 1;
constexpr uint32_t LN_TRUNK = 2 * BLOCKS, LN_CFG = LN_TRUNK + 1, LN_JOIN = LN_CFG + 1, LN_JOUT = LN_JOIN + JBLOCKS,
                   LN_H = LN_JOUT + 1;
// Join input as a 16-bit GEMM operand: the 129 columns padded to whole 32-column k steps.
constexpr uint32_t JOIN_IN_PAD = 160;

// One linear layer in the flat blob: matrix [i x o] row-major at w, bias at b.
struct Span {
    uint32_t w = 0, b = 0, i = 0, o = 0;
    bool bias = false;
};

// NetLayout::new (net.rs:272-316): offsets in blob order.
struct Layout {
    Span card[2], pile;
    uint32_t seat = 0;
    Span hex_stem, tok_stem;
    uint32_t pos = 0;
    Span glob_stem;
    Span mix[BLOCKS], pool[BLOCKS], out[BLOCKS];
    Span board_out, cfg1, cfg_f, cfg_g, cfg_m, join_p, join_b, join_w[JBLOCKS], join_out;
    uint32_t value_bias = 0;
    uint32_t norm_g[NORMS] = {}, norm_b[NORMS] = {}, norm_width[NORMS] = {};
    uint32_t w_len = 0, b_len = 0, ln_len = 0;
};
Layout layout();

// Hex h's neighbour in each of the six axial directions of board.rs:14
// (HEXES when off the board), and whether h is a location.
struct Board {
    uint8_t nb[HEXES][6];
    uint8_t loc[HEXES];
};
Board board();

// The 16-bit GEMMs of the fast path (the ones the reference runs on tensor
// cores, device.rs gemm()), in one enumeration: the bank stores each as the
// B operand (one K-contiguous row per output, fragment-major, K padded to a
// multiple of 32, rows padded to GEMM_ROWS).
enum Mat : uint32_t {
    M_CARD0 = 0, M_CARD1, M_CFG_M, M_MIX0, M_POOL0 = M_MIX0 + BLOCKS, M_OUT0 = M_POOL0 + BLOCKS,
    M_BOARD = M_OUT0 + BLOCKS, M_JOIN_P, M_CFG1, M_CFG_F, M_CFG_G, M_JOIN_B, M_JOIN_W0, M_JOIN_OUT = M_JOIN_W0 + JBLOCKS,
    M_COUNT
};
Span mat_span(const Layout& L, uint32_t m);
inline uint32_t kpad(uint32_t k) { return (k + 31) / 32 * 32; }

// Device view of a published v5 bank: the f32 blob (every matrix, bias and
// norm), and for the 16-bit path each GEMM's operand copy.
struct Net {
    const float* w = nullptr;
    const float* b = nullptr;
    const float* ln = nullptr;
    const uint8_t* nb = nullptr;   // Board::nb, HEXES x 6
    const uint8_t* loc = nullptr;  // Board::loc
    const uint16_t* m16[M_COUNT] = {};
    float value_bias = 0.0f;
};

// Per-wave inputs and outputs.
struct WaveIn {
    uint32_t jobs = 0, rows = 0, ncfg = 0;
    const float* card_feat = nullptr;  // [jobs][NTYPE * CARD_FEATS], physical order
    const uint8_t* raw = nullptr;      // [rows][ROW_BYTES]
    const uint32_t* row_job = nullptr; // [rows]
    const float* phi = nullptr;        // [ncfg][CFEAT]
    const uint32_t* cfg_job = nullptr; // [ncfg]
    const uint8_t* cfg_owner = nullptr;  // [ncfg]
};
struct WaveOut {
    float* cards = nullptr;  // [jobs][2][NTYPE][TYPE]
    float* bag = nullptr;    // [jobs][2][NTYPE][3 * POOL]
    float* P = nullptr;      // [rows][D]
    float* Jp = nullptr;     // [rows][JW]
    float* G = nullptr;      // [ncfg][POOL] (the pooling vectors, f32)
    void* F = nullptr;       // [ncfg][D]: f32 (exact) or 16-bit row-major (readout operand)
};

// The per-wave build. precision: WC_PRECISE (float32 in the CPU loop order)
// or WC_F16 / WC_BF16 (16-bit operands on the matrix cores for the GEMMs
// above, float32 elsewhere).
void launch_build(int precision, const Net& net, const WaveIn& in, const WaveOut& out, hipStream_t s);
// The join for one traverser: X the pooled query input (precise: [rows][JOIN_IN]
// f32; 16-bit: fragment-major, K = JOIN_IN_PAD), H the readout operand
// (precise: [rows][D] f32; 16-bit: fragment-major, K = D). xf: rows x JOIN_IN
// floats of scratch for the 16-bit path.
void launch_join(int precision, const Net& net, uint32_t rows, const void* X, const float* P, const float* Jp,
                 void* H, float* xf, hipStream_t s);

}  // namespace v5
}  // namespace wc
