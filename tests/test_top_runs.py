"""Fused top-depth value launches (WaveHost::top_back_run, csrc/wave.cpp
plan_top_back), checked on the host against a restatement of what each row
reads.

The top regions' value rows run one depth per launch, deepest first
(engine/src/gpu/wave.rs:559-610 walks the same depths bottom-up, one level
task list per launch). A pair of consecutive non-empty depths may share one
launch when its rows are dealt into chunks such that every value a shallower
row reads from the deeper depth is written in the same chunk: the workgroup
runs the chunk's deeper rows, then, after a block barrier, its shallower rows.
These tests hold the packer's plan to that rule, independently of it:

- every non-empty depth is launched once, deepest first, a fused pair being
  two consecutive non-empty depths;
- each fused pair's chunk bounds run through both depths' rows in order;
- every slot a shallower row reads (its legal cells, draw outcomes or
  children, restated from the record kinds) that a deeper row of the pair
  writes is written by a row of the same chunk;
- the rows of each depth are the same tasks as an unfused packing's, and
  each record still belongs to its task (out = the node's value base + the
  config);
- with WC_TOP_FUSE=0 every depth is its own launch.

The device results of fused waves are bit-identical to the oracle's in the
float32 GPU parity tests, which pack with fusion, while the service's lanes
pack without it.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import warchest_wave as ww
import workloads as W

NONE = 0xFFFFFFFF
BACK_OWN, BACK_DRAW, BACK_OPP = 0, 1, 2


def reads(tables, p, rec):
    """The value slots a list of top back records reads (wave.h BackRec), as
    (reader index, slot) arrays."""
    start, kn, arg = rec[:, 2].astype(np.int64), rec[:, 3].astype(np.int64), rec[:, 1].astype(np.int64)
    kind, n = kn >> 30, kn & 0x1FFFFFFF
    reader = np.repeat(np.arange(len(rec)), n)
    first = np.repeat(np.cumsum(n) - n, n)
    idx = np.repeat(start, n) + (np.arange(int(n.sum())) - first)
    k = np.repeat(kind, n)
    slot = np.full(len(idx), -1, dtype=np.int64)
    own, draw, opp = k == BACK_OWN, k == BACK_DRAW, k == BACK_OPP
    slot[own] = tables["legal_value"][idx[own]]
    slot[own & (slot == NONE)] = -1  # an illegal cell reads nothing
    slot[draw] = np.repeat(arg, n)[draw] + tables["draw_to"][idx[draw]]
    slot[opp] = tables[f"child_vb{p}"][idx[opp]] + np.repeat(arg, n)[opp]
    keep = slot >= 0
    return reader[keep], slot[keep]


def check_plan(wave):
    a = wave.array
    tables = {n: a(n).astype(np.int64) for n in ("legal_value", "draw_to", "child_vb0", "child_vb1")}
    top_levels = wave.stats()["top_levels"]
    vb = a("vals_base")
    fused = 0
    for p in (0, 1):
        lvl = a(f"top_back_lvl{p}")
        rec = a(f"top_back_rec{p}").reshape(-1, 4)
        task = a(f"top_back{p}").reshape(-1, 2)
        runs = a(f"top_back_run{p}").reshape(-1, 4)
        off = a(f"top_back_chunk{p}").astype(np.int64)
        # records belong to their tasks
        np.testing.assert_array_equal(rec[:, 0], vb[2 * task[:, 0].astype(np.int64) + p] + task[:, 1])
        depths = [d for d in range(top_levels - 1, -1, -1) if lvl[d + 1] > lvl[d]]
        launched = []
        for d, e, at, nch in (tuple(int(x) for x in r) for r in runs):
            launched.append(d)
            if e == NONE:
                continue
            launched.append(e)
            fused += 1
            assert depths.index(e) == depths.index(d) + 1, "a fused pair is two consecutive non-empty depths"
            oa, ob = off[at:at + nch + 1], off[at + nch + 1:at + 2 * nch + 2]
            assert oa[0] == lvl[d] and oa[-1] == lvl[d + 1] and ob[0] == lvl[e] and ob[-1] == lvl[e + 1]
            assert np.all(np.diff(oa) >= 0) and np.all(np.diff(ob) >= 0)
            # the chunk of every deeper row, by its output slot
            deep = rec[lvl[d]:lvl[d + 1]]
            deep_chunk = np.searchsorted(oa, np.arange(lvl[d], lvl[d + 1]), side="right") - 1
            order = np.argsort(deep[:, 0])
            outs, outs_chunk = deep[order, 0].astype(np.int64), deep_chunk[order]
            assert np.all(np.diff(outs) > 0), "each deeper row writes its own slot"
            # every read of a deeper row's slot comes from the same chunk
            shallow = rec[lvl[e]:lvl[e + 1]]
            shallow_chunk = np.searchsorted(ob, np.arange(lvl[e], lvl[e + 1]), side="right") - 1
            reader, slot = reads(tables, p, shallow)
            at_slot = np.searchsorted(outs, slot)
            hit = (at_slot < len(outs)) & (outs[np.minimum(at_slot, len(outs) - 1)] == slot)
            assert hit.any(), "the shallower rows read the deeper ones"
            np.testing.assert_array_equal(outs_chunk[at_slot[hit]], shallow_chunk[reader[hit]])
        assert launched == depths, "every non-empty depth once, deepest first"
    return fused


def tasks_by_depth(wave):
    a = wave.array
    out = {}
    for p in (0, 1):
        lvl = a(f"top_back_lvl{p}")
        task = a(f"top_back{p}").reshape(-1, 2)
        for d in range(len(lvl) - 1):
            rows = task[lvl[d]:lvl[d + 1]]
            out[f"{p}/{d}"] = sorted(map(tuple, rows.tolist()))
    return out


FAMILIES = [("wave256", dict(trees=6, nodes_lo=150, nodes_hi=300, seed=81)),
            ("wave256v5", dict(trees=4, nodes_lo=150, nodes_hi=300, seed=82)),
            ("wave512w", dict(trees=4, nodes_lo=150, nodes_hi=300, seed=83))]


@pytest.mark.parametrize("family,spec", FAMILIES, ids=[f for f, _ in FAMILIES])
def test_fused_chunks_hold_the_rows_they_read(family, spec, monkeypatch):
    monkeypatch.setenv("WC_UNIT_SLOTS", "256")  # small units: several top depths per tree
    wave = ww.Wave(W.jobs(family, **spec))
    assert check_plan(wave) >= 2
    wave.check()


def test_the_benchmarked_wave_fuses_its_draw_pairs():
    wave = ww.Wave(W.jobs("wave256"))
    assert check_plan(wave) == 7  # four pairs of player 0's depths, three of player 1's


def test_fused_rows_are_the_unfused_rows_reordered(tmp_path, monkeypatch):
    monkeypatch.setenv("WC_UNIT_SLOTS", "256")
    jobs = W.jobs("wave256", trees=6, nodes_lo=150, nodes_hi=300, seed=81)
    fused = tasks_by_depth(ww.Wave(jobs))
    # The switch is read once per process: the unfused packing runs in a child.
    path = tmp_path / "jobs.bin"
    path.write_bytes(b"".join(len(j).to_bytes(8, "little") + j for j in jobs))
    here = os.path.dirname(os.path.abspath(__file__))
    code = (
        "import json, sys\n"
        "import warchest_wave as ww\n"
        "sys.path.insert(0, %r)\n"
        "from test_top_runs import tasks_by_depth\n"
        "raw = open(%r, 'rb').read(); jobs = []; i = 0\n"
        "while i < len(raw):\n"
        "    n = int.from_bytes(raw[i:i + 8], 'little'); jobs.append(raw[i + 8:i + 8 + n]); i += 8 + n\n"
        "w = ww.Wave(jobs)\n"
        "runs = [w.array('top_back_run%%d' %% p).reshape(-1, 4)[:, 1].tolist() for p in (0, 1)]\n"
        "print(json.dumps({'runs': runs, 'tasks': tasks_by_depth(w)}))\n" % (here, str(path)))
    env = dict(os.environ, WC_TOP_FUSE="0", PYTHONPATH=os.pathsep.join(sys.path))
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr
    plain = json.loads(res.stdout)
    assert all(e == NONE for runs in plain["runs"] for e in runs), "WC_TOP_FUSE=0: one depth per launch"
    assert {k: [list(t) for t in v] for k, v in fused.items()} == plain["tasks"]


def test_a_row_moved_out_of_its_chunk_is_caught(monkeypatch):
    """The plan check itself: swap a deeper row that a shallower row reads
    with a deeper row of another chunk (task and record together, so each
    record still belongs to its task) and the check must name the chunk."""
    monkeypatch.setenv("WC_UNIT_SLOTS", "256")
    wave = ww.Wave(W.jobs("wave256", trees=6, nodes_lo=150, nodes_hi=300, seed=81))
    a = wave.array
    tables = {n: a(n).astype(np.int64) for n in ("legal_value", "draw_to", "child_vb0", "child_vb1")}
    d, e, at, nch = (int(x) for x in a("top_back_run0").reshape(-1, 4)[[
        i for i, r in enumerate(a("top_back_run0").reshape(-1, 4)) if r[1] != NONE][0]])
    off = a("top_back_chunk0").astype(np.int64)
    oa, ob = off[at:at + nch + 1], off[at + nch + 1:at + 2 * nch + 2]
    rec = a("top_back_rec0").reshape(-1, 4)
    # a deeper row of chunk 0 that one of chunk 0's shallower rows reads
    _, slot = reads(tables, 0, rec[ob[0]:ob[1]])
    r1 = next(r for r in range(oa[0], oa[1]) if int(rec[r][0]) in set(slot.tolist()))
    r2 = int(oa[1])  # the first deeper row of chunk 1
    for name, words in (("top_back_rec0", 4), ("top_back0", 2)):
        t = a(name)
        x, y = t[words * r1:words * r1 + words].copy(), t[words * r2:words * r2 + words].copy()
        for k in range(words):
            wave.poke(name, words * r1 + k, int(y[k]))
            wave.poke(name, words * r2 + k, int(x[k]))
    with pytest.raises(AssertionError, match="not equal"):  # the chunk comparison, not an earlier check
        check_plan(wave)


def reach_reads(tables, rec):
    """The reach slots a list of top reach records reads (wave.h ReachRec:
    the parent's slots pbase + rev_src or rvd_src entries), as (reader
    index, slot) arrays."""
    pbase, start, kn = rec[:, 1].astype(np.int64), rec[:, 2].astype(np.int64), rec[:, 3].astype(np.int64)
    rev, n = (kn >> 31) == 0, kn & 0x1FFFFFFF
    reader = np.repeat(np.arange(len(rec)), n)
    idx = np.repeat(start, n) + (np.arange(int(n.sum())) - np.repeat(np.cumsum(n) - n, n))
    use_rev = np.repeat(rev, n)
    src = np.where(use_rev, tables["rev_src"][np.where(use_rev, idx, 0)], tables["rvd_src"][np.where(use_rev, 0, idx)])
    return reader, np.repeat(pbase, n) + src


def check_reach_plan(wave):
    """The reach pass's runs (WaveHost::top_reach_run): every non-empty depth
    once, top-down; in a fused pair every shallower row is computed by some
    chunk, and each chunk computes every shallower row its deeper rows read."""
    a = wave.array
    tables = {n: a(n).astype(np.int64) for n in ("rev_src", "rvd_src")}
    top_levels = wave.stats()["top_levels"]
    fused = 0
    for p in (0, 1):
        lvl = a(f"top_reach_lvl{p}")
        rec = a(f"top_reach_rec{p}").reshape(-1, 4)
        runs = a(f"top_reach_run{p}").reshape(-1, 4)
        off = a(f"top_reach_chunk{p}").astype(np.int64)
        par = a(f"top_reach_par{p}").astype(np.int64)
        depths = [d for d in range(top_levels) if lvl[d + 1] > lvl[d]]
        launched = []
        for d, e, at, nch in (tuple(int(x) for x in r) for r in runs):
            launched.append(d)
            if e == NONE:
                continue
            launched.append(e)
            fused += 1
            assert depths.index(e) == depths.index(d) + 1
            ob, oq = off[at:at + nch + 1], off[at + nch + 1:at + 2 * nch + 2]
            assert ob[0] == lvl[e] and ob[-1] == lvl[e + 1] and np.all(np.diff(ob) >= 0) and np.all(np.diff(oq) >= 0)
            names = par[oq[0]:oq[-1]]
            assert np.all((names >= lvl[d]) & (names < lvl[d + 1]))
            assert set(names.tolist()) == set(range(lvl[d], lvl[d + 1])), "every shallower row is computed"
            # (chunk, shallower row) pairs the plan computes, and those the deeper rows read
            chunk_of_name = np.searchsorted(oq, np.arange(oq[0], oq[-1]), side="right") - 1
            have = set((chunk_of_name * (1 << 32) + names).tolist())
            shallow = rec[lvl[d]:lvl[d + 1]]
            order = np.argsort(shallow[:, 0])
            outs = shallow[order, 0].astype(np.int64)
            reader, slot = reach_reads(tables, rec[lvl[e]:lvl[e + 1]])
            at_slot = np.searchsorted(outs, slot)
            hit = (at_slot < len(outs)) & (outs[np.minimum(at_slot, len(outs) - 1)] == slot)
            assert hit.any()
            row = lvl[d] + order[at_slot[hit]]
            chunk = np.searchsorted(ob, lvl[e] + reader[hit], side="right") - 1
            need = set((chunk * (1 << 32) + row).tolist())
            assert need <= have, "a deeper row reads a shallower row its chunk does not compute"
        assert launched == depths
    return fused


@pytest.mark.parametrize("family,spec", FAMILIES, ids=[f for f, _ in FAMILIES])
def test_fused_reach_chunks_compute_what_they_read(family, spec, monkeypatch):
    monkeypatch.setenv("WC_UNIT_SLOTS", "256")
    wave = ww.Wave(W.jobs(family, **spec))
    assert check_reach_plan(wave) >= 2
    wave.check()


def test_the_benchmarked_wave_fuses_its_reach_pairs():
    assert check_reach_plan(ww.Wave(W.jobs("wave256"))) == 6  # three pairs of each player's depths


def test_a_parent_left_out_of_its_chunk_is_caught(monkeypatch):
    monkeypatch.setenv("WC_UNIT_SLOTS", "256")
    wave = ww.Wave(W.jobs("wave256", trees=6, nodes_lo=150, nodes_hi=300, seed=81))
    check_reach_plan(wave)
    a = wave.array
    d, e, at, nch = (int(x) for x in next(r for r in a("top_reach_run0").reshape(-1, 4) if r[1] != NONE))
    off = a("top_reach_chunk0")
    first = int(off[at + nch + 1])  # chunk 0's first named shallower row, which its deeper rows read
    assert off[at + 1] > off[at]  # chunk 0 has deeper rows
    wave.poke("top_reach_par0", first, int(a("top_reach_par0")[first]) ^ 1)
    with pytest.raises(AssertionError):
        check_reach_plan(wave)
