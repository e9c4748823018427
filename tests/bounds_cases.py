"""Single-fault edits of a packed wave's tables (wc_wave_poke), each with the
condition the host's deep check (validate_deep) reports first for it. The
host-check tests (CPU) and the device-check tests (GPU) share them: the
device must name the same condition.

Each edit breaks one condition and no earlier one: a node that is a decision
node and no exit (its slots feed no exit or row check), a reach row of a
unit's deepest level (no deeper row of the unit reads its slot), and so on.
"""
import numpy as np

import workloads as W

NONE = 0xFFFFFFFF
UNIT_WORDS, REC_WORDS, GROUP_WORDS = 24, 4, 36
# UnitDev word offsets
U_NLEVELS, U_LVL0, U_VWIN0, U_VWIN_N0, U_LEAF0_0, U_LEAF1_0, U_RWIN0, U_RWIN_N0 = 0, 1, 12, 14, 16, 18, 20, 22
# PoolGroup word offsets
G_NROWS, G_RBASE0 = 2, 18
# A unit budget small enough that these trees get top regions (swept per depth).
UNIT_SLOTS = "256"


def jobs():
    """Four 150-300-node subgames: 247 units and 8 top depths at UNIT_SLOTS."""
    return W.jobs("wave256", trees=4, nodes_lo=150, nodes_hi=300, seed=81)


def cases(wave):
    """(table, word index, value, the message after "wave bounds: ")."""
    st = wave.stats()
    a = wave.array
    n_nodes, reach_len, vals_len, ncells = st["nodes"], st["reach_len"], st["vals_len"], st["cells"]
    meta, nc = a("node_meta"), a("node_nc")
    exits = set(a("exit_node").tolist())
    node = next(i for i in range(n_nodes) if nc[2 * i] > 0 and (meta[i] & 3) == 0 and i not in exits)
    cell = int(np.flatnonzero(a("legal_value") != NONE)[0])
    out = [
        ("node_meta", node, 0xFF, "node_meta"),
        ("reach_base", 2 * node, reach_len, "reach slot"),
        ("vals_base", 2 * node, vals_len, "value slot"),
        ("legal_value", cell, vals_len + 7, "legal_value"),
        ("row_node", 0, n_nodes + 5, "row_node"),
        ("row_cfg", 0, 0xFFFFFFF0, "row_cfg"),
        ("row_cfg_off", 0, 0xFFFFFFFD, "row_cfg_off"),  # a first offset near 2^32: row 0's list would wrap
        ("exit_coff", 0, 0xFFFFFFFD, "exit_coff"),
        ("pool_grp0", G_NROWS, 0, "pool group"),
        ("pool_grp0", G_RBASE0, int(a("pool_grp0")[G_RBASE0]) + 1, "pool group reach"),
        ("back_rec0", 0, vals_len, "back record"),
        ("top_back_rec0", 0, vals_len, "top back record"),
        ("reach_rec1", 0, reach_len + 3, "reach record"),
        ("top_reach_rec1", 0, reach_len + 3, "top reach record"),
        ("acc_rec0", 1, ncells, "accumulation record"),
        ("leaf_rec0", 1, 0xFFFFFFF0, "leaf record"),
        ("units", U_RWIN_N0, reach_len + 1, "unit window size"),  # wider than the wave's widest window
        ("units", U_RWIN0, reach_len + 1, "unit reach window"),  # a window past the reach table
        ("top_back_run0", 0, st["top_levels"] + 3, "top back runs"),  # a depth the wave does not have
        ("top_back_chunk0", 1, 0, "top back chunks"),  # a chunk bound before the depth's first row
        ("top_back_chunk0", 0, int(a("top_back_chunk0")[0]) + 1, "top back chunks"),  # skips the first row
        ("top_reach_run1", 0, 0, "top reach runs"),  # the root depth, which has no reach rows
        ("top_reach_chunk1", 0, int(a("top_reach_chunk1")[0]) + 1, "top reach chunks"),
        ("top_reach_par1", 0, 0xFFFFFFF0, "top reach parents"),  # a parent row past the top rows
    ]
    # Window conditions, on a unit with reach rows at its deepest level, value
    # rows and network leaves: a slot just outside the window, inside the table.
    units = a("units").reshape(-1, UNIT_WORDS)
    rl, bl = a("reach_lvl0"), a("back_lvl0")
    for k, u in enumerate(units):
        nl, l0 = int(u[U_NLEVELS]), int(u[U_LVL0])
        if nl == 0 or rl[l0 + nl] == rl[l0 + nl - 1] or bl[l0 + nl] == bl[l0] or u[U_LEAF1_0] == u[U_LEAF0_0]:
            continue
        rwin, rn, vwin, vn = (int(u[i]) for i in (U_RWIN0, U_RWIN_N0, U_VWIN0, U_VWIN_N0))
        r_out = rwin + rn if rwin + rn < reach_len else rwin - 1
        v_out = vwin + vn if vwin + vn < vals_len else vwin - 1
        out += [
            ("reach_rec0", REC_WORDS * int(rl[l0 + nl - 1]), r_out, "unit reach row writes outside its reach window"),
            ("back_rec0", REC_WORDS * int(bl[l0]), v_out, "unit row outside its value window"),
            ("leaf_rec0", REC_WORDS * int(u[U_LEAF0_0]), v_out, "unit leaf outside its value window"),
        ]
        break
    else:
        raise AssertionError("no unit has reach rows at its deepest level, value rows and leaves")
    return out
