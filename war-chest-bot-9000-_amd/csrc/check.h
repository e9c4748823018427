// Element checks of an uploaded wave on the device.
//
// The kernels follow the indices of a packed wave with no bounds checks of
// their own. A wave packed from jobs that each passed validation at submit
// (the service's) skips the host's deep check, whose element scans cost as
// much host time as the packing itself; its upload instead runs the host's
// structural checks (validate_shape) and then these kernels, which read the
// element tables once from HBM (a fraction of a millisecond) and report the
// first failing condition before any kernel of the schedule is launched.
//
// They cover every element table the schedule reads: the node slots, the
// cells' value slots, the network rows and their config lists, the pool
// groups (bounds, shared lists, every row in exactly one group), every row
// record and the elements it names, the two-tower blocks' rows, and each
// subtree unit's windows (its rows write and read inside them; a reach row
// reads a window slot only after a shallower level wrote it). The lists only
// the host reads (node CSR, task lists) are not uploaded and not checked here.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"
#include "wave.h"

namespace wc {

// Failing conditions, numbered in the order validate_deep checks them on the
// host, so that the device reports the same first failure for one bad entry.
enum CheckCode : uint32_t {
    CK_OK = 0,
    CK_NODE_META,
    CK_REACH_SLOT,
    CK_VALUE_SLOT,
    CK_LEGAL_VALUE,
    CK_ROW_NODE,
    CK_ROW_CONFIGS,
    CK_ROW_CFG,
    CK_POOL_GROUP,
    CK_POOL_REACH,
    CK_POOL_ROW,
    CK_POOL_LIST,
    CK_POOL_COVER,
    CK_BACK_REC,
    CK_TOP_BACK_REC,
    CK_REACH_REC,
    CK_TOP_REACH_REC,
    CK_ACC_REC,
    CK_LEAF_REC,
    CK_TOWER_CONFIGS,
    CK_UNIT_RWIN,
    CK_UNIT_UNWRITTEN,
    CK_UNIT_WRITES_OUT,
    CK_UNIT_LEAF_OUT,
    CK_UNIT_TERM_OUT,
    CK_UNIT_ROW_OUT,
    CK_UNIT_ROW_READS_OUT,
    CK_COUNT
};
// validate_deep's message for the condition ("wave bounds: " + it); null for
// a code out of range.
const char* check_message(uint32_t code);

// The flag word holds CHECK_BASE - code of the lowest failing code (an atomic
// max), or 0 when every check passed.
constexpr uint32_t CHECK_BASE = 0x10000;
// The widest unit reach window the unit check's LDS bitmap covers (64 KB of
// bits); a wave with a wider one is checked on the host.
constexpr uint32_t CHECK_RWIN_MAX = 64u * 1024u * 8u;

struct CheckArgs {
    WaveDev w;  // the uploaded tables (pointers and counts)
    const BackRec* top_back[2];
    const ReachRec* top_reach[2];
    uint32_t* flag;   // one word, zero before the checks
    uint32_t* cover;  // 2 * rows counters, zero before the checks: pool-group rows per (player, row)
    uint64_t nodes, ncells, reach_len, vals_len, rows, ncfg, row_cfg_n, draw_to_n, rev_n, rvd_n, heads_end, term_n;
    uint64_t child_vb_n[2], nback[2], ntop_back[2], nreach[2], ntop_reach[2], nacc[2];
    uint32_t max_rwin;
    uint32_t tower;  // 1: a readout net's blocks (their rows' configs are checked)
};

// The sizes of the host wave `h` whose tables `w` holds on the device; flag
// and cover point at device words the caller zeroes first.
CheckArgs check_args(const WaveHost& h, const WaveDev& w, const BackRec* const top_back[2],
                     const ReachRec* const top_reach[2], uint32_t* flag, uint32_t* cover);
// Enqueues every element check on stream s (requires h.max_rwin <= CHECK_RWIN_MAX).
void launch_check(const CheckArgs& a, hipStream_t s);

}  // namespace wc
