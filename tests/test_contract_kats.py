"""Known-answer tests of the job contract and the wave layout, from the
reference's own unit tests, plus a cross-check of the C++ WCJ8 codec against
the independent Python reader/writer (tests/wcj8.py)."""
import numpy as np
import pytest

import warchest_wave as ww
import wcj8
import workloads as W

NONE = 0xFFFFFFFF
SMALL_MLP = [101, 64, 32, 1, 4, 8]  # in 64, hidden 32, 1 layer, 4 heads, pool 8: 47 raw bytes per row


def stub_job():
    """The reference's smallest well-formed job (engine/src/serialize.rs:1263-1324):
    one network leaf with one config per player. The reference's stub shares
    one interned config between the players; the contract here interns one per
    player (cplayer must name the owning player)."""
    raw, cphi = wcj8.mlp_payload(SMALL_MLP, rows=1, ncfg=2)
    return dict(
        depth=2, iters=4, snapshots=True, alpha=1.5, beta=0.0, gamma=2.0, predict=0.0,
        snap_iters=[0, 1, 2, 4], net_dims=SMALL_MLP,
        nodes=1, ncfg=2, rows=1, ncells=0,
        node_kind=[2], node_player=[0], node_child_start=[0, 0], node_child=[],
        obs_off=[0, 0], obs_start=[0], obs_act=[], obs_child=[],
        legal_row_of=[NONE], legal_off=[0], legal_action=[], legal_child=[], legal_trans=[], cell_row=[],
        draw_off=[0, 0], draw_to=[], draw_p=[], draw_row_off=[0, 0], draw_row_start=[],
        cfg_off=[0, 1, 2], reach_off=[0, 2], soff=[0, 0], node_parent=[NONE],
        rev_row_of=[NONE], rev_start=[0], rev_src=[], rev_cell=[],
        rvd_row_of=[NONE], rvd_start=[0], rvd_src=[], rvd_p=[],
        leaf_rows=[0], term_leaves=[], terminal_utility=[],
        leaf_coff=[0, 1, 2], leaf_cidx=[0, 1], snap_coff=[0, 1, 2],
        leaf_raw=np.zeros(raw, np.uint8), card_feat=[], cphi=np.zeros(cphi, np.float32), cplayer=[0, 1],
        bfs_order=[0], level_start=[0, 1],
        root=[[1.0], [1.0]], carried=[],
    )


def test_stub_job_is_valid_and_round_trips():
    b = wcj8.encode(stub_job())
    ww.job_validate(b)
    assert ww.job_roundtrip(b) == b


def test_stub_wave_patches_every_space():
    """engine/src/gpu/wave.rs:747-762: two stubs packed into one wave."""
    b = wcj8.encode(stub_job())
    w = ww.Wave([b, b])
    st = w.stats()
    assert st["jobs"] == 2 and st["nodes"] == 2
    assert list(w.array("row_node")) == [0, 1]
    assert list(w.array("reach_base")) == [0, 1, 2, 3]
    assert st["reach_len"] == 4
    assert list(w.array("exit_node")) == [0, 1]
    assert list(w.array("exit_coff")) == [0, 1, 2, 3, 4]
    assert st["snapshot_configs"] == 4
    assert st["rows"] == 2


def alias_job():
    """A chance node of player 0 over one leaf (engine/src/serialize.rs:1392-1408):
    cfg_off [0,1,2,4,5] gives the chance node one config per player and the
    leaf two configs for player 0 and one for player 1."""
    j = stub_job()
    raw, cphi = wcj8.mlp_payload(SMALL_MLP, rows=1, ncfg=3)
    j.update(
        nodes=2, ncfg=3, rows=1, ncells=0,
        node_kind=[1, 2], node_player=[0, 0], node_child_start=[0, 1, 1], node_child=[1],
        obs_off=[0, 0, 0], legal_row_of=[NONE, NONE],
        draw_off=[0, 2, 2], draw_to=[0, 1], draw_p=[0.5, 0.5], draw_row_off=[0, 2, 2], draw_row_start=[0, 2],
        cfg_off=[0, 1, 2, 4, 5], reach_off=[0, 2, 5], soff=[0, 0, 0], node_parent=[NONE, 0],
        rev_row_of=[NONE, NONE], rev_start=[0], rvd_row_of=[NONE, 0], rvd_start=[0, 1, 2], rvd_src=[0, 0],
        rvd_p=[0.5, 0.5],
        leaf_rows=[1], leaf_coff=[0, 2, 3], leaf_cidx=[0, 1, 2], snap_coff=[0, 2, 3],
        leaf_raw=np.zeros(raw, np.uint8), cphi=np.zeros(cphi, np.float32), cplayer=[0, 0, 1],
        bfs_order=[0, 1], level_start=[0, 1, 2],
    )
    return j


def test_opponent_chance_values_alias_the_child():
    """device_value_layout KAT: base[p][node] = [[2, 0], [0, 0]], length 3."""
    b = wcj8.encode(alias_job())
    ww.job_validate(b)
    w = ww.Wave([b])
    vb = w.array("vals_base").reshape(2, 2)  # [node, player]
    assert list(vb[:, 0]) == [2, 0]
    assert list(vb[:, 1]) == [0, 0]
    assert w.stats()["vals_len"] == 3


def test_cpp_codec_agrees_with_python_codec():
    for name, kw in (("tree48", {}), ("wave64", {"trees": 3}), ("wave256", {"trees": 2, "nodes_lo": 60, "nodes_hi": 90,
                                                                "terminal_p": 0.2, "nroots": 3})):
        for b in W.jobs(name, **kw):
            d = wcj8.decode(b)
            assert wcj8.encode(d) == b
            assert d["ncells"] == len(d["legal_action"]) and d["nodes"] == len(d["node_kind"])


@pytest.mark.parametrize("field", ["legal_trans", "rev_src", "draw_to", "leaf_cidx"])
def test_out_of_range_indices_are_rejected(field):
    [b] = W.jobs("wave256", trees=1, nodes_lo=40, nodes_hi=60, seed=5)
    d = wcj8.decode(b)
    arr = np.array(d[field], np.uint32)
    assert arr.size
    arr[arr != NONE] = 10 ** 6
    d[field] = arr
    with pytest.raises(ww.WaveError):
        ww.job_validate(wcj8.encode(d))
