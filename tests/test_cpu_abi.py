"""CPU checks of the C ABI: the library loads, exports what the header declares,
and its host-only entry points (job codec, validation, synthesis, packing) work
without a GPU."""
import os
import re

import numpy as np
import pytest

import warchest_wave as ww
import workloads as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "wc_wave.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wc_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    L = ww.lib()
    syms = header_symbols()
    assert len(syms) >= 30
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    assert set(syms) == set(ww.EXPORTS)


def test_job_roundtrip_is_byte_identical():
    for name in ("tree48", "wave64"):
        for j in W.jobs(name, trees=3) if name == "wave64" else W.jobs(name):
            assert ww.job_roundtrip(j) == j
            ww.job_validate(j)


def test_truncated_and_corrupt_jobs_are_rejected():
    j = W.jobs("tree48")[0]
    for cut in (0, 3, 8, len(j) // 2, len(j) - 1):
        with pytest.raises(ww.WaveError):
            ww.job_validate(j[:cut])
    bad = bytearray(j)
    bad[0] ^= 0xFF  # magic
    with pytest.raises(ww.WaveError, match="magic"):
        ww.job_validate(bytes(bad))
    with pytest.raises(ww.WaveError):
        ww.job_validate(j + b"\0")


@pytest.mark.parametrize("family", ["wave256", "wave512w", "wave256v5"])
def test_edited_jobs_are_refused_or_pack_into_checked_waves(family):
    """Random byte edits of WCJ8 jobs (bit flips, bytes, whole words, truncation):
    parsing and validation accept or refuse them, and an accepted job packs into a
    wave that passes the deep bounds check (wc_wave_pack runs it), as the service
    relies on for jobs validated at submit. Edits like these found, in validation:
    row ranges running backwards (rev_start, rvd_start), offsets checked one step
    at a time while being read (draw_off, node_child_start), a draw bound that
    overflowed 32 bits, carry layouts (snap_coff) and snapshot iterations that
    only the packer noticed, a leaf listed twice among the network and terminal
    leaves, child lists naming a node twice, and head rows converted before
    their range was checked."""
    import random

    jobs = W.jobs(family, trees=3, nodes_lo=60, nodes_hi=150, seed=91,
                  **({"whale_frac": 0.0} if family == "wave512w" else {}))
    rng = random.Random(7)
    accepted = 0
    for _ in range(1500):
        b = bytearray(rng.choice(jobs))
        for _ in range(rng.randint(1, 4)):
            at = rng.randrange(len(b))
            kind = rng.randrange(4)
            if kind == 0:
                b[at] ^= 1 << rng.randrange(8)
            elif kind == 1:
                b[at] = rng.randrange(256)
            elif kind == 2:
                w = at & ~3
                if w + 4 <= len(b):
                    b[w:w + 4] = (0xFFFFFFFF if rng.randrange(4) == 0 else rng.randrange(1024)).to_bytes(4, "little")
            else:
                del b[at + 1:]
        try:
            ww.job_validate(bytes(b))
        except ww.WaveError:
            continue
        accepted += 1
        ww.Wave([bytes(b)]).close()  # raises if the packed wave fails its bounds check
    assert accepted > 100


def test_wave_pack_names_the_first_bad_job():
    # Jobs parse on several threads; the error still names the first bad one.
    jobs = W.jobs("wave64", trees=5)
    bad = bytearray(jobs[1])
    bad[0] ^= 0xFF  # magic
    jobs[1] = bytes(bad)
    jobs[3] = jobs[3][: len(jobs[3]) // 2]
    with pytest.raises(ww.WaveError, match="job 1: .*magic"):
        ww.Wave(jobs)


def test_wave_pack_rejects_mixed_schedules():
    a = W.jobs("tree48")[0]
    b = W.jobs("tree48", iters=8)[0]
    with pytest.raises(ww.WaveError, match="schedule"):
        ww.Wave([a, b])


def test_wave_counts_add_up():
    jobs = W.jobs("wave64", trees=5)
    st = ww.Wave(jobs).stats()
    parts = [ww.Wave([j]).stats() for j in jobs]
    for k in ("nodes", "cells", "rows", "rev_nnz", "reach_len", "vals_len", "snapshot_configs"):
        assert st[k] == sum(p[k] for p in parts), k
    assert st["jobs"] == 5
    assert st["cfr_bytes_per_iter"][0] == sum(p["cfr_bytes_per_iter"][0] for p in parts)


@pytest.mark.parametrize("family", ["wave256", "wave256v5"])
def test_wave_lists_are_the_jobs_lists_shifted(family):
    # The packer lays the jobs out in parallel and writes each at its offset
    # into every wave list; the result must be the jobs' own lists (each job
    # packed alone) appended in job order, every index shifted by the lists
    # before it: nodes, children, cells, legal rows, reach and value slots,
    # snapshot configs.
    jobs = W.jobs(family, trees=9, nodes_lo=60, nodes_hi=400)
    NONE = 0xFFFFFFFF
    names = ("child_start", "child", "legal_off", "legal_value", "reach_base", "vals_base", "row_node",
             "exit_node", "exit_coff")
    whole = ww.Wave(jobs)
    F = {k: whole.array(k).astype(np.int64) for k in names}
    node0 = child0 = cell0 = lrow0 = row0 = exit0 = reach_at = vals_at = cfg_at = 0
    for j in jobs:
        one = ww.Wave([j])
        S = {k: one.array(k).astype(np.int64) for k in names}
        st = one.stats()
        one.close()
        n, kids, cells = len(S["child_start"]) - 1, len(S["child"]), len(S["legal_value"])
        lrows, rows, exits = len(S["legal_off"]) - 1, len(S["row_node"]), len(S["exit_node"])
        np.testing.assert_array_equal(F["child_start"][node0:node0 + n + 1], S["child_start"] + child0)
        np.testing.assert_array_equal(F["child"][child0:child0 + kids], S["child"] + node0)
        np.testing.assert_array_equal(F["legal_off"][lrow0:lrow0 + lrows + 1], S["legal_off"] + cell0)
        np.testing.assert_array_equal(F["row_node"][row0:row0 + rows], S["row_node"] + node0)
        np.testing.assert_array_equal(F["exit_node"][exit0:exit0 + exits], S["exit_node"] + node0)
        ecfg0 = F["exit_coff"][2 * exit0]
        assert ecfg0 == cfg_at
        np.testing.assert_array_equal(F["exit_coff"][2 * exit0:2 * (exit0 + exits) + 1], S["exit_coff"] + ecfg0)
        reach0 = F["reach_base"][2 * node0] - S["reach_base"][0]
        assert reach0 == reach_at
        np.testing.assert_array_equal(F["reach_base"][2 * node0:2 * (node0 + n)], S["reach_base"] + reach0)
        vals0 = F["vals_base"][2 * node0] - S["vals_base"][0]
        assert vals0 == vals_at
        np.testing.assert_array_equal(F["vals_base"][2 * node0:2 * (node0 + n)], S["vals_base"] + vals0)
        lv = S["legal_value"]
        np.testing.assert_array_equal(F["legal_value"][cell0:cell0 + cells], np.where(lv == NONE, NONE, lv + vals0))
        node0, child0, cell0, lrow0, row0, exit0 = node0 + n, child0 + kids, cell0 + cells, lrow0 + lrows, \
            row0 + rows, exit0 + exits
        reach_at, vals_at, cfg_at = reach_at + st["reach_len"], vals_at + st["vals_len"], \
            cfg_at + st["snapshot_configs"]
    assert node0 == len(F["child_start"]) - 1 and cell0 == len(F["legal_value"]) and row0 == len(F["row_node"])
    whole.close()


@pytest.mark.parametrize("budget", [256, 1024, None])
def test_unit_windows_fit_the_budget(budget, monkeypatch):
    # A unit is a run of sibling subtrees; its value slots form one window no
    # wider than the slot budget, so the sweep can stage every unit in LDS.
    if budget is not None:
        monkeypatch.setenv("WC_UNIT_SLOTS", str(budget))
    st = ww.Wave(W.jobs("wave256", trees=12)).stats()
    assert st["units"] > 12 and st["top_levels"] > 0
    assert 0 < st["max_window"] <= (budget or 4096)


@pytest.mark.parametrize("family", ["wave256", "wave512w"])
@pytest.mark.parametrize("budget", [64, 300, 8192])
def test_parity_waves_pack_and_validate(budget, family, monkeypatch):
    # The GPU parity suite's waves (chance nodes, terminals, 3 carried roots;
    # MLP and two-tower nets) at its unit budgets: packing runs the full
    # host-side validation.
    monkeypatch.setenv("WC_UNIT_SLOTS", str(budget))
    jobs = W.jobs(family, trees=8, nodes_lo=30, nodes_hi=90, chance=1, terminal_p=0.15, notrans_p=0.05,
                  nroots=3, iters=8, info_median=6.0, info_p99=40.0, info_cap=40, seed=13, whale_frac=0.0)
    st = ww.Wave(jobs).stats()
    assert st["terminals"] > 0 and st["chance_nodes"] > 0
    if budget == 64:
        assert st["top_levels"] > 0


def test_service_style_mixed_waves_pass_the_deep_check():
    """The service buckets whatever compatible jobs its queue holds (one schedule,
    any sizes, carried-root counts and tree shapes) and packs them from jobs
    validated at submit, skipping the packed wave's deep bounds check
    (validate_deep). The packer's output does not depend on that flag, so every
    mix it can form must pass the check: 30 random mixes of 1..24 jobs from a
    pool of differently shaped jobs with one schedule (small and full-size
    trees, terminals, no-successor cells, 1..3 carried roots, a whale), packed
    through wc_wave_pack, which runs the deep check."""
    spec = dict(iters=8, info_median=6.0, info_p99=40.0, info_cap=40)
    pool = (W.jobs("wave256", trees=6, nodes_lo=30, nodes_hi=90, chance=1, terminal_p=0.15, notrans_p=0.05,
                   nroots=2, seed=71, **spec)
            + W.jobs("wave256", trees=4, nodes_lo=200, nodes_hi=400, nroots=1, seed=72, **spec)
            + W.jobs("wave256", trees=4, nodes_lo=40, nodes_hi=120, chance=1, terminal_p=0.3, nroots=3, seed=73,
                     **spec)
            + W.jobs("wave256", trees=2, nodes_lo=200, nodes_hi=300, whale_frac=1.0, whale_nodes=600,
                     whale_info=120, nroots=1, seed=74, iters=8))
    rng = np.random.default_rng(5)
    for m in range(30):
        pick = rng.choice(len(pool), size=int(rng.integers(1, 25)), replace=True)
        wave = ww.Wave([pool[k] for k in pick])  # raises on any failed bound
        st = wave.stats()
        assert st["jobs"] == len(pick)
        wave.close()


def test_host_check_names_the_first_failing_condition(monkeypatch):
    """wc_wave_check on the host (the check wc_wave_pack runs) against single-
    fault edits of a packed wave (wc_wave_poke): each edit is refused with the
    condition it breaks, and the wave passes again once the word is restored.
    The device check (GPU tests) must name the same conditions."""
    import bounds_cases as B

    monkeypatch.setenv("WC_UNIT_SLOTS", B.UNIT_SLOTS)
    wave = ww.Wave(B.jobs())
    assert wave.stats()["top_levels"] > 0
    wave.check()
    cases = B.cases(wave)
    assert len(cases) == 27
    for name, index, value, msg in cases:
        old = int(wave.array(name)[index])
        wave.poke(name, index, value)
        with pytest.raises(ww.WaveError, match="^wave bounds: " + re.escape(msg) + "$"):
            wave.check()
        wave.poke(name, index, old)
        wave.check()
    with pytest.raises(ww.WaveError, match="index beyond"):
        wave.poke("row_node", wave.stats()["rows"], 0)
    with pytest.raises(ww.WaveError, match="unknown array"):
        wave.poke("no_such_table", 0, 0)
    # an empty table is a table of no words, not an unknown one
    plain = ww.Wave(W.jobs("wave256", trees=2, nodes_lo=60, nodes_hi=90))
    assert plain.stats()["terminals"] == 0 and len(plain.array("term_node")) == 0
    with pytest.raises(ww.WaveError, match="unknown array"):
        plain.array("no_such_table")


def test_host_check_survives_random_single_word_edits(monkeypatch):
    """Random single-word edits of every table wc_wave_array names: the host
    check accepts the wave or refuses it with "wave bounds: ...", and never
    reads outside a table itself (a child node's check once read its parent's
    actor before the parent's own check had bounded it)."""
    import random

    import bounds_cases as B

    monkeypatch.setenv("WC_UNIT_SLOTS", B.UNIT_SLOTS)
    wave = ww.Wave(B.jobs())
    names = ["row_node", "reach_base", "vals_base", "exit_node", "exit_coff", "legal_value", "child_start", "child",
             "legal_off", "node_meta", "node_nc", "row_cfg", "row_cfg_off", "draw_to", "rev_src", "rvd_src",
             "term_node", "unit_term", "units", "trees"]
    names += [f"{k}{p}" for k in ("back_rec", "top_back_rec", "reach_rec", "top_reach_rec", "acc_rec", "leaf_rec",
                                  "pool_grp", "child_vb", "back_lvl", "reach_lvl", "top_back", "top_reach",
                                  "top_back_lvl", "top_reach_lvl", "top_back_run", "top_back_chunk", "top_reach_run",
                                  "top_reach_chunk", "top_reach_par", "head_rb_n")
              for p in (0, 1)]
    tables = {n: wave.array(n) for n in names}
    rng = random.Random(5)
    refused = 0
    for _ in range(800):
        name = rng.choice([n for n in names if len(tables[n])])
        i = rng.randrange(len(tables[name]))
        old = int(tables[name][i])
        value = rng.choice([0, 1, old + 1, (old - 1) & 0xFFFFFFFF, 0xFFFFFFFF, 0x7FFFFFFF, rng.getrandbits(32)])
        wave.poke(name, i, value)
        try:
            wave.check()
        except ww.WaveError as e:
            assert str(e).startswith("wave bounds: "), (name, i, value, str(e))
            refused += 1
        wave.poke(name, i, old)
    wave.check()
    assert refused > 200


def test_repacking_a_wave_equals_packing_it_fresh():
    """A reused wave (wc_wave_repack, the service lanes' path) keeps the
    lengths and old contents of the lists the packer overwrites whole, so a
    list entry the packer missed would keep the previous wave's value. Packing
    mixes of differently shaped jobs one after another into one wave must give
    every list and count exactly as a fresh pack does (wc_wave_digest), also
    after a larger wave and after a smaller one."""
    spec = dict(iters=8, info_median=6.0, info_p99=40.0, info_cap=40)
    pool = (W.jobs("wave256", trees=6, nodes_lo=30, nodes_hi=90, chance=1, terminal_p=0.15, notrans_p=0.05,
                   nroots=2, seed=81, **spec)
            + W.jobs("wave256", trees=4, nodes_lo=200, nodes_hi=400, nroots=1, seed=82, **spec)
            + W.jobs("wave256", trees=4, nodes_lo=40, nodes_hi=120, chance=1, terminal_p=0.3, nroots=3, seed=83,
                     **spec))
    rng = np.random.default_rng(8)
    mixes = [[pool[k] for k in rng.choice(len(pool), size=int(rng.integers(1, 25)), replace=True)]
             for _ in range(12)]
    fresh = []
    for mix in mixes:
        w = ww.Wave(mix)
        fresh.append(w.digest())
        w.close()
    reused = ww.Wave(pool)  # the largest wave first
    for mix, want in zip(mixes, fresh):
        reused.repack(mix)
        assert reused.digest() == want
        assert reused.stats()["jobs"] == len(mix)
    # jobs that do not parse leave the wave as it was; a failed pack leaves it unusable
    with pytest.raises(ww.WaveError):
        reused.repack([b"not a job"])
    assert reused.digest() == fresh[-1]
    with pytest.raises(ww.WaveError):
        reused.repack([W.jobs("wave64", trees=1)[0], W.jobs("wave256", trees=1)[0]])  # two schedules
    with pytest.raises(ww.WaveError, match="no packed jobs"):
        reused.digest()
    with pytest.raises(ww.WaveError, match="no packed jobs"):
        reused.stats()
    reused.repack(mixes[0])
    assert reused.digest() == fresh[0]
    reused.close()


def test_synthesis_is_seeded_and_prefix_stable():
    a = W.jobs("wave64", trees=4)
    b = W.jobs("wave64", trees=6)
    assert a == b[:4]
    assert W.jobs("wave64", trees=2, seed=99) != a[:2]


def test_weights_and_features_are_seeded():
    n1 = W.net_for("mlp65k")
    n2 = W.net_for("mlp65k")
    np.testing.assert_array_equal(n1.w, n2.w)
    x = W.mlp65k_inputs(rows=64)
    assert x.shape == (64, 512)
    assert x.min() >= 0.0 and x.max() <= 1.0
    # Kaiming-normal: first-layer std ~ sqrt(2 / 512)
    w1 = n1.w[: 512 * 384]
    assert abs(w1.std() - np.sqrt(2 / 512)) < 0.003


def test_value_net_plan_covers_every_block_once():
    # 65,536 queries with 64 heads on 256 CUs: 4,096 blocks of one width, so
    # every pass is a full eight-block pass, two per CU.
    plan = ww.value_net_plan(4096, 256, heads=64)
    assert len(plan) == 512
    assert all(c == 64 and len(b) == 8 for c, b in plan)
    assert sorted(x for _, b in plan for x in b) == list(range(4096))


def test_value_net_plan_keeps_wide_passes_short():
    # A wave's spread of head widths: most blocks need a few 16-column steps,
    # some all 567 columns. Widest blocks come first, each pass's width covers
    # its blocks, and passes of 567-column blocks hold fewer blocks than
    # passes of 64-column blocks (their estimated cost is capped).
    rng = np.random.default_rng(5)
    cols = rng.choice([16, 32, 64, 128, 256, 567], size=3086, p=[0.3, 0.25, 0.2, 0.12, 0.08, 0.05])
    cols = cols.astype(np.uint32)
    plan = ww.value_net_plan(cols, 256, heads=567)
    seen = sorted(x for _, b in plan for x in b)
    assert seen == list(range(len(cols)))
    for c, b in plan:
        assert 1 <= len(b) <= 8
        assert c == max(int(cols[x]) for x in b)
    wide = [len(b) for c, b in plan if c == 567]
    narrow = [len(b) for c, b in plan if c == 64]
    assert wide and narrow and max(wide) < max(narrow) == 8
    assert plan[0][0] == 567  # the longest passes start first
    assert len(plan) >= 256  # at least one pass per CU


def test_value_net_plan_rejects_null_output():
    n = ww.C.c_size_t(7)
    assert ww.lib().wc_value_net_plan(None, 4, 64, 256, None, 4, ww.C.byref(n)) == -1  # WC_ERR_INVALID
    assert n.value == 0
    assert ww.lib().wc_value_net_plan(None, 4, 64, 256, None, 0, None) == -1  # WC_ERR_INVALID


def test_tape_refuses_bad_arguments_and_files(tmp_path):
    """wc_tape (the service's throughput tape) is built beside the library; it
    refuses a wrong argument count or zero waves (status 2) and a truncated
    tape file (status 1, naming the file) before it touches a device."""
    import struct
    import subprocess

    tape = os.path.join(ROOT, "war-chest-bot-9000-_amd", "wc_tape")
    assert os.path.exists(tape), "build first: python __graft_entry__.py"
    assert subprocess.run([tape], capture_output=True).returncode == 2
    bad = tmp_path / "bad.tape"
    bad.write_bytes(b"WCTP" + struct.pack("<I", 3) + struct.pack("<Q", 10) + b"short")
    r = subprocess.run([tape, str(bad), "0", "1", "1", "1"], capture_output=True, text=True)
    assert r.returncode == 2
    r = subprocess.run([tape, str(bad), "1", "1", "1", "1"], capture_output=True, text=True)
    assert r.returncode == 1 and "malformed tape file" in r.stderr
