"""The leaf net checked at the reach the solve itself reaches, and the CFR
arithmetic of reduced-precision solves checked bit for bit (through the C ABI).

wc_wave_leaf_trace captures, inside one whole schedule, what the leaf-input and
value-net kernels produced right after the net ran at chosen schedule points
(iterations; Phase 2's evaluations per carried root and player): each network
row's values, the rows' reach masses, and the reach that fed them.

- float32: the device's trace equals the oracle's own trace bit for bit
  (values, masses, reach) at every probed point;
- 16-bit nets: at iterations 0, 1, 2, 31, 63 and Phase 2 (both traversers), the
  device's values are held to the oracle's model of the same operand rounding
  evaluated at the device's own reach (oracle_leaf_eval), as tightly as the
  initial-reach probes: the per-iteration single-player pooling, the Phase-2
  pooling under the final average and the fixed-column product reused across
  iterations are all inside this check;
- replay: the oracle solver run with the device's own leaf values and masses of
  every evaluation (oracle_solve_replay) gives the device's strategy, root
  values and carries bit for bit. So everything a reduced-precision solve adds
  to the float32 solve's error comes through leaf values that the checks above
  bound; how far 64 DCFR iterations carry such a difference is the conditioning
  of the subgame (tests/test_conditioning.py), not a device error.
"""
import os
import sys
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle as O
import warchest_wave as ww
import workloads as W

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)
NAMES = {ww.WC_PRECISE: "float32", ww.WC_F16: "f16", ww.WC_BF16: "bf16", ww.WC_F16X: "compensated f16"}


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def pmap(fn, items):
    with ThreadPoolExecutor(THREADS) as pool:
        return list(pool.map(fn, items))


_EX = {}


def executor(precision):
    if precision not in _EX:
        _EX[precision] = ww.Executor(0, precision)
    return _EX[precision]


def probe_points(iters, nroots):
    pts = sorted({t for t in (0, 1, 2, 31, 63) if t < iters} | {iters - 1})
    return pts + [ww.phase2_point(r, p) for r in {0, nroots - 1} for p in (0, 1)]


def all_points(iters, nroots):
    return list(range(iters)) + [ww.phase2_point(r, p) for r in range(nroots) for p in (0, 1)]


def traverser(pt):
    return pt & 1 if pt >= 0 else (-pt - 1) & 1


def split(trace, counts):
    """Per job, per point: (values, mass [rows, 2], reach) of the wave trace."""
    out = []
    for pt in trace:
        p = pt["traverser"]
        v0 = m0 = r0 = 0
        per = []
        for n0, n1, rows, nreach in counts:
            nv = n1 if p else n0
            per.append((pt["values"][v0:v0 + nv], pt["mass"][m0:m0 + rows],
                        None if pt["reach"] is None else pt["reach"][r0:r0 + nreach]))
            v0, m0, r0 = v0 + nv, m0 + rows, r0 + nreach
        assert v0 == len(pt["values"]) and m0 == len(pt["mass"])
        out.append(per)
    return out


def device_trace(precision, jobs, net, points, reach=True):
    ex = executor(precision)
    v = ex.publish(net)
    wave = ww.Wave(jobs)
    try:
        return ex.leaf_trace(wave, v, points, reach=reach)
    finally:
        wave.close()


def assert_tracks(got, want, tol, tag, median=0.05):
    """|got - want| <= tol * max |want|, the median far below it (the probes' criterion)."""
    assert got.shape == want.shape, tag
    scale = float(np.abs(want).max())
    err = np.abs(got.astype(np.float64) - want)
    say(f"{tag}: {got.size} values, max error {err.max() / scale:.2e}, median {np.median(err) / scale:.2e} "
        f"of the largest |value|")
    assert err.max() <= tol * scale, tag
    assert np.median(err) <= median * tol * scale, tag


def test_trace_float32_is_the_oracles_trace():
    jobs = W.jobs("wave64")
    net = W.net_for("wave64")
    s0 = O.shape(jobs[0])
    pts = probe_points(s0.iters, s0.nroots)
    say(f"case trace float32: wave64, all {len(jobs)} subgames, points {pts}")
    got = split(device_trace(ww.WC_PRECISE, jobs, net, pts), [O.leaf_counts(j) for j in jobs])
    refs = pmap(lambda j: O.solve_trace(j, net, O.NET_F32), jobs)
    for k, (job, ref) in enumerate(zip(jobs, refs)):
        s = O.shape(job)
        n0, n1, rows, nreach = O.leaf_counts(job)
        evals = all_points(s.iters, s.nroots)
        voff = np.cumsum([0] + [n1 if traverser(e) else n0 for e in evals])
        for i, pt in enumerate(pts):
            e = evals.index(pt)
            vals, mass, reach = got[i][k]
            np.testing.assert_array_equal(vals, ref["vals"][voff[e]:voff[e + 1]], err_msg=f"tree {k} point {pt}")
            np.testing.assert_array_equal(mass.reshape(-1), ref["mass"][2 * rows * e:2 * rows * (e + 1)],
                                          err_msg=f"tree {k} point {pt}")
            np.testing.assert_array_equal(reach, ref["reach"][nreach * e:nreach * (e + 1)],
                                          err_msg=f"tree {k} point {pt}")


# Subgames whose whole 16-bit solves land outside the emulations' envelope
# (tests/envelope.py): reported one by one at every probed point.
WATCH = {"wave64": (8, 15, 24, 37, 53, 57), "wave256": (6,)}


def check_trace_against_model(precision, mode, tol, jobs, net, tag, median=0.05):
    s0 = O.shape(jobs[0])
    pts = probe_points(s0.iters, max(O.shape(j).nroots for j in jobs))
    say(f"case trace {NAMES[precision]}: {tag}, {len(jobs)} subgames, points {pts}")
    counts = [O.leaf_counts(j) for j in jobs]
    per = split(device_trace(precision, jobs, net, pts), counts)
    for i, pt in enumerate(pts):
        p = traverser(pt)
        live = [k for k, j in enumerate(jobs) if pt >= 0 or (-pt - 1) // 2 < O.shape(j).nroots]
        want = pmap(lambda k: O.leaf_eval(jobs[k], net, mode, p, per[i][k][2]), live)
        got = np.concatenate([per[i][k][0] for k in live])
        assert_tracks(got, np.concatenate([w for w, _ in want]), tol, f"{tag} point {pt}", median)
        scale = float(max(np.abs(w).max() for w, _ in want if w.size))
        for k in WATCH.get(tag, ()):
            if k in live and per[i][k][0].size:
                e = np.abs(per[i][k][0].astype(np.float64) - want[live.index(k)][0]) / scale
                say(f"{tag} point {pt} subgame {k}: max error {e.max():.2e}, median {np.median(e):.2e}")
        # masses: the device's reach summed in another order. Any two orders of
        # a sum of n positive float32 terms agree within 2 (n - 1) 2^-24 of it;
        # lists hold up to 567 configs.
        np.testing.assert_allclose(np.concatenate([per[i][k][1] for k in live]),
                                   np.concatenate([m for _, m in want]), rtol=2 * 566 * 2.0 ** -24, atol=1e-30)


@pytest.mark.parametrize("precision,mode,tol", [(ww.WC_F16, O.NET_F16, 2e-3), (ww.WC_BF16, O.NET_BF16, 1e-2),
                                                (ww.WC_F16X, O.NET_F16X, 1e-5)])
def test_trace_wave64_tracks_the_operand_model_at_the_solves_reach(precision, mode, tol):
    """f16 and bf16 against their operand models; compensated f16 (hi + lo operand
    pairs) against its own model, to a few float32 roundings (measured: max 6e-7,
    median 8e-8 of the largest value at every probed point)."""
    check_trace_against_model(precision, mode, tol, W.jobs("wave64"), W.net_for("wave64"), "wave64")


def test_trace_wave256_tracks_the_operand_model_at_the_solves_reach():
    """The whole benchmarked wave: 256 subgames, 49,371 rows, 567 heads, the
    fixed-column split reused across iterations."""
    check_trace_against_model(ww.WC_F16, O.NET_F16, 2e-3, W.jobs("wave256"), W.net_for("wave256"), "wave256")


def whales():
    jobs = W.jobs("wave512w", trees=40)
    big = [j for j in jobs if O.shape(j).nodes >= 1500][:2]
    small = [j for j in jobs if O.shape(j).nodes < 1500][:2]
    return big + small


def test_trace_whales_bf16_two_tower_tracks_the_operand_model():
    check_trace_against_model(ww.WC_BF16, O.NET_BF16, 1e-2, whales(), W.net_for("wave512w"), "wave512w whales")


def replay_and_compare(precision, jobs, net, tag):
    """Device solve, then a trace of every leaf evaluation; each job's replay in the
    oracle must give the device's outputs bit for bit."""
    ex = executor(precision)
    v = ex.publish(net)
    wave = ww.Wave(jobs)
    try:
        got = ex.solve(wave, v)
        again = ex.solve(wave, v)
        nroots = max(O.shape(j).nroots for j in jobs)
        iters = O.shape(jobs[0]).iters
        pts = all_points(iters, nroots)
        trace = ex.leaf_trace(wave, v, pts, reach=False)
    finally:
        wave.close()
    for k, (a, b) in enumerate(zip(got, again)):
        np.testing.assert_array_equal(a.strategy, b.strategy, err_msg=f"{tag} tree {k}: repeat")
        np.testing.assert_array_equal(a.root_values, b.root_values, err_msg=f"{tag} tree {k}: repeat")
    per = split(trace, [O.leaf_counts(j) for j in jobs])

    def replay(k):
        s = O.shape(jobs[k])
        use = [i for i, pt in enumerate(pts) if pt >= 0 or (-pt - 1) // 2 < s.nroots]
        vals = np.concatenate([per[i][k][0] for i in use])
        mass = np.concatenate([per[i][k][1].reshape(-1) for i in use])
        return O.solve_replay(jobs[k], vals, mass)

    refs = pmap(replay, range(len(jobs)))
    for k, (g, r) in enumerate(zip(got, refs)):
        np.testing.assert_array_equal(g.strategy, r["strategy"], err_msg=f"{tag} tree {k}: strategy")
        np.testing.assert_array_equal(g.root_values, r["roots"], err_msg=f"{tag} tree {k}: root values")
        np.testing.assert_array_equal(g.carries, r["carries"].astype(np.float16), err_msg=f"{tag} tree {k}: carries")
    say(f"{tag}: {len(jobs)} subgames, the oracle's replay of the device's leaf values is the device's solve "
        f"bit for bit")


@pytest.mark.parametrize("precision", [ww.WC_F16, ww.WC_BF16, ww.WC_F16X])
def test_replay_wave64_reduced_precision_solves_bit_exact(precision):
    say(f"case replay {NAMES[precision]}: wave64, all 64 subgames, every leaf evaluation")
    replay_and_compare(precision, W.jobs("wave64"), W.net_for("wave64"), f"wave64 {NAMES[precision]}")


def test_replay_wave256_full_shape_f16_bit_exact():
    say("case replay f16: wave256, 16 full-shape subgames, every leaf evaluation")
    replay_and_compare(ww.WC_F16, W.jobs("wave256")[:16], W.net_for("wave256"), "wave256 f16")


@pytest.mark.timeout(400)
def test_replay_whales_bf16_bit_exact():
    say("case replay bf16 two-tower: whales, every leaf evaluation (128 iterations)")
    replay_and_compare(ww.WC_BF16, whales(), W.net_for("wave512w"), "wave512w whales bf16")
