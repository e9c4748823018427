"""The service's view of a job, restated independently from the WCJ8 bytes.

`PackedJob::work` (engine/src/serialize.rs:394-431), `job_cost`
(engine/src/gpu/client.rs:282-291), `cost_class`
(engine/src/gpu/service.rs:967-991) and the route predicates
(serialize.rs:174-201) are recomputed here in Python from tests/wcj8.py's
decoding and compared with the library's (wc_job_work). The device arena
(`mutable_bytes`) is this executor's own layout, so it is checked for its
bounds rather than restated.
"""
import numpy as np
import pytest

import warchest_wave as ww
import wcj8
import workloads as W

U32_FIELDS = [
    "node_child_start", "node_child", "obs_off", "obs_start", "obs_act", "obs_child", "legal_row_of", "legal_off",
    "legal_action", "legal_child", "legal_trans", "cell_row", "draw_off", "draw_to", "draw_row_off",
    "draw_row_start", "cfg_off", "reach_off", "soff", "node_parent", "rev_row_of", "rev_start", "rev_src",
    "rev_cell", "rvd_row_of", "rvd_start", "rvd_src", "leaf_rows", "term_leaves", "leaf_coff", "leaf_cidx",
    "snap_coff", "bfs_order", "level_start"]
F32_FIELDS = ["draw_p", "rvd_p", "terminal_utility", "card_feat", "cphi"]
U8_FIELDS = ["node_kind", "node_player", "leaf_raw", "cplayer"]


def restated_work(d):
    nodes = d["nodes"]
    cfg = d["cfg_off"].astype(np.int64)
    nc = lambda i, p: int(cfg[2 * i + p + 1] - cfg[2 * i + p])  # noqa: E731
    reach = nc(0, 0) + nc(0, 1) + sum(nc(i, int(d["node_player"][d["node_parent"][i]])) for i in range(1, nodes))
    owned = sum(len(d[f]) for f in U8_FIELDS) + 4 * (sum(len(d[f]) for f in U32_FIELDS) +
                                                     sum(len(d[f]) for f in F32_FIELDS))
    root_configs = int(cfg[2] - cfg[0])
    nroots = len(d["carried"])
    table = owned + max(2 * nodes - len(d["reach_off"]), 0) * 4 + 4 * (len(d["root"][0]) + len(d["root"][1])) \
        + 4 * nroots * root_configs
    snap_cfgs = int(d["snap_coff"][-1]) if len(d["snap_coff"]) else 0
    carried_out = (d["ncells"] + nroots * root_configs) * 4 + max(len(d["snap_iters"]) - 1, 0) * snap_cfgs * 2
    return dict(network_rows=d["rows"], legal_cells=d["ncells"], reach_slots=reach,
                reverse_nonzeros=len(d["rev_src"]) + len(d["rvd_src"]), table_bytes=table,
                carried_output_bytes=carried_out, levels=max(len(d["level_start"]) - 1, 0))


def restated_cost(w, iters):
    it = max(iters, 1)
    return max(w["network_rows"] * it * 16 + w["legal_cells"] * it + w["reach_slots"] * it + w["table_bytes"] // 16, 1)


def next_pow2(x):
    return 1 if x <= 1 else 1 << (int(x) - 1).bit_length()


def restated_class(w, shift, unit):
    byts = w["table_bytes"] + w["mutable_bytes"] + w["carried_output_bytes"]
    reserved = w["mutable_bytes"] + next_pow2(w["table_bytes"])
    if reserved >= 4 * unit or w["legal_cells"] >= 8_000_000:
        return 31
    work = max(w["network_rows"], w["legal_cells"] // 8, w["reach_slots"] // 16, w["reverse_nonzeros"] // 16, 1)
    if byts >= 512 << 20 or work >= 4_000_000:
        c = 3
    elif byts >= 64 << 20 or work >= 500_000:
        c = 2
    elif byts >= 16 << 20 or work >= 125_000:
        c = 1
    else:
        c = 0
    return c >> min(shift, 2)


@pytest.mark.parametrize("family", ["tree48", "wave64", "wave256", "wave512w"])
def test_work_vector_cost_and_class(family):
    jobs = W.jobs(family, trees=3) if family != "tree48" else W.jobs(family)
    for job in jobs:
        d = wcj8.decode(job)
        want = restated_work(d)
        for prec in (ww.WC_PRECISE, ww.WC_F16):
            got = ww.job_work(job, prec)
            for k, v in want.items():
                assert got[k] == v, (family, k)
            assert got["cost"] == restated_cost(got, int(d["iters"]))
            assert got["reserved_bytes"] == got["mutable_bytes"] + next_pow2(got["table_bytes"])
            # the arena holds at least the CFR state, reach and the query inputs
            assert got["mutable_bytes"] >= 16 * d["ncells"] + 8 * want["reach_slots"]
            for shift in (0, 1, 2):
                assert ww.job_work(job, prec, class_shift=shift)["cost_class"] == restated_class(got, shift, 1 << 30)


def test_route_predicates_follow_the_reservation():
    """Exclusive at >= 4 units of reservation, card-exclusive at >= 6, arena guard
    at >= 4 units of arena when not card-exclusive (serialize.rs:174-201)."""
    [job] = W.jobs("wave256", trees=1)
    base = ww.job_work(job, ww.WC_F16)
    assert not (base["exclusive_route"] or base["arena_guard_route"] or base["card_exclusive_route"])
    assert base["cost_class"] != 31
    reserved, mutable = base["reserved_bytes"], base["mutable_bytes"]
    for unit in (reserved // 7 + 1, reserved // 5 + 1, reserved // 4, mutable // 4, reserved // 3 + 1):
        w = ww.job_work(job, ww.WC_F16, route_unit=unit)
        assert w["exclusive_route"] == int(reserved >= 4 * unit)
        assert w["card_exclusive_route"] == int(reserved >= 6 * unit)
        assert w["arena_guard_route"] == int(mutable >= 4 * unit and not reserved >= 6 * unit)
        assert (w["cost_class"] == 31) == bool(w["exclusive_route"])


def test_prepared_job_carries_the_jobs_cost():
    """wc_prepare (PreparedJob::new, engine/src/gpu/client.rs:165-181) costs a job once:
    its cost is job_cost of the work vector restated above, for each precision; bytes
    that do not decode, or decode to an invalid job, are refused."""
    jobs = W.jobs("wave64")[:3] + W.jobs("wave512w", trees=4)[:2]
    for j in jobs:
        d = wcj8.decode(j)
        for prec in (ww.WC_PRECISE, ww.WC_F16, ww.WC_BF16):
            p = ww.PreparedJob(j, prec)
            assert p.cost == ww.job_work(j, prec)["cost"]
            assert p.cost == restated_cost({**restated_work(d), "mutable_bytes": 0}, d["iters"])
            p.close()
    with pytest.raises(ww.WaveError):
        ww.PreparedJob(jobs[0][:-9], ww.WC_F16)
    with pytest.raises(ww.WaveError):
        ww.PreparedJob(jobs[0], 17)
