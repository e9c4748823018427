"""The v5 leaf network on the GPU (the reference's device path:
engine/src/gpu/device.rs:836-1106 per wave, 1218-1305 per iteration), through
the C ABI, against the oracle's restatement of engine/src/net.rs:

- float32: the leaf values at the initial reach (wc_wave_leaf_probe: cards,
  trunk, join cache, config encoder, pooled beliefs, join, readout) and whole
  solves (strategies, root values, carries) bit-identical to the oracle;
- the zero network: every leaf valued at value_bias;
- 16-bit operands: the leaf values track the oracle's model of the same
  operand rounding;
- jobs tagged [5] through the service boundary, bit-identical in float32;
- whole f16 solves held to the reference's own gate for its fast tensor-core
  head (engine/src/gpu/tests.rs:393-446) on its own test network and
  schedule: root values within 1e-2 + 2e-3 |x| of the float32 solve, mean
  strategy error <= 5e-3, strategy entries within 0.4 + 0.1 |x|; bf16 solves
  near float32;
- inside the benchmarked wave's full-shape solves (random-init network, 64
  iterations), at iterations 0, 1, 2, 31, 63 and Phase 2, the leaf values
  against the 16-bit operand model at the device's own reach, and the
  oracle's replay of the device's own leaf values equal to the device's solve
  bit for bit.
"""
import os
import sys
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle as O
import warchest_wave as ww

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def pmap(fn, items):
    with ThreadPoolExecutor(THREADS) as pool:
        return list(pool.map(fn, items))


def v5_jobs(trees=8, seed=31, **kw):
    spec = dict(seed=seed, trees=trees, nodes_lo=30, nodes_hi=90, chance=1, terminal_p=0.1, notrans_p=0.05,
                info_median=6.0, info_p99=40.0, info_cap=40, iters=16, nroots=2, dirichlet=1, depth=2, act_lo=3,
                act_hi=8)
    spec.update(kw)
    return ww.synth_jobs(ww.V5_DIMS, **spec)


_EX = {}


def executor(precision):
    if precision not in _EX:
        _EX[precision] = ww.Executor(0, precision)
    return _EX[precision]


def device_probe(ex, jobs, net, p):
    v = ex.publish(net)
    wave = ww.Wave(jobs)
    try:
        return ex.leaf_probe(wave, v, p)
    finally:
        wave.close()


def oracle_probe(jobs, net, mode, p):
    out = pmap(lambda j: O.leaf_probe(j, net, mode, p), jobs)
    return np.concatenate([v for v, _ in out]), np.concatenate([m for _, m in out])


def test_v5_leaf_probe_float32_bit_exact():
    jobs = v5_jobs()
    net = ww.synth_weights(ww.V5_DIMS, 1)
    ex = executor(ww.WC_PRECISE)
    for p in (0, 1):
        say(f"case v5 leaf probe float32: {len(jobs)} subgames, traverser {p}")
        got, mass = device_probe(ex, jobs, net, p)
        want, want_mass = oracle_probe(jobs, net, O.NET_F32, p)
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(mass, want_mass)


def test_v5_zero_network():
    jobs = v5_jobs(trees=4, seed=33)
    net = ww.synth_weights(ww.V5_DIMS, 1)
    w = np.zeros_like(net.w)
    b = np.zeros_like(net.b)
    b[-1] = 0.375  # value_bias
    zero = ww.Net(list(net.dims), w, b, net.ln)
    for precision in (ww.WC_PRECISE, ww.WC_F16):
        say(f"case v5 zero network: precision {precision}")
        got, _ = device_probe(executor(precision), jobs, zero, 0)
        assert got.size and np.all(got == np.float32(0.375))


def test_v5_solve_float32_bit_exact():
    jobs = v5_jobs(trees=6, seed=35)
    net = ww.synth_weights(ww.V5_DIMS, 2)
    say(f"case v5 solve float32: {len(jobs)} subgames, 16 iterations, 2 carried roots")
    ex = executor(ww.WC_PRECISE)
    v = ex.publish(net)
    wave = ww.Wave(jobs)
    got = ex.solve(wave, v)
    wave.close()
    refs = pmap(lambda j: O.solve(j, net, O.NET_F32), jobs)
    for k, (g, o) in enumerate(zip(got, refs)):
        np.testing.assert_array_equal(g.strategy, o["strategy"], err_msg=f"tree {k}: strategy")
        np.testing.assert_array_equal(g.root_values, o["roots"], err_msg=f"tree {k}: root values")
        np.testing.assert_array_equal(g.carries, o["carries"].astype(np.float16), err_msg=f"tree {k}: carries")


def test_v5_jobs_through_the_service():
    """Jobs tagged [5] submitted through the service (wc_submit / wc_wait:
    two lanes, waves of at most three jobs, the v5 bank published at spawn)
    come back bit-identical to the oracle's float32 solves, with their tags."""
    jobs = v5_jobs(trees=7, seed=47)
    net = ww.synth_weights(ww.V5_DIMS, 3)
    say(f"case v5 service: {len(jobs)} subgames, 2 lanes, waves of at most 3")
    with ww.spawn(0, net, ww.WC_PRECISE, lanes=2, wave_jobs=3, window_us=500) as client:
        handles = [client.submit(j, tag=500 + k) for k, j in enumerate(jobs)]
        got = [h.wait() for h in handles]
        assert client.queued_work() == 0
    refs = pmap(lambda j: O.solve(j, net, O.NET_F32), jobs)
    for k, (g, o) in enumerate(zip(got, refs)):
        assert g.tag == 500 + k
        np.testing.assert_array_equal(g.strategy, o["strategy"], err_msg=f"tree {k}: strategy")
        np.testing.assert_array_equal(g.root_values, o["roots"], err_msg=f"tree {k}: root values")
        np.testing.assert_array_equal(g.carries, o["carries"].astype(np.float16), err_msg=f"tree {k}: carries")


@pytest.mark.parametrize("precision,mode,tol", [(ww.WC_F16, O.NET_F16A, 3e-3), (ww.WC_BF16, O.NET_BF16A, 3e-2)])
def test_v5_leaf_probe_16bit_tracks_the_operand_model(precision, mode, tol):
    """16-bit leaf values against the oracle's model of the same operand
    rounding (max within tol of the largest value, median within tol / 6),
    and no further from the float32 values than the model is (their median
    distance within 1.5x the model's): through eight residual blocks a
    different summation order moves activations across 16-bit rounding
    boundaries, so two faithful 16-bit evaluations differ by about as much as
    each differs from float32."""
    jobs = v5_jobs(seed=37)
    net = ww.synth_weights(ww.V5_DIMS, 1)
    ex = executor(precision)
    for p in (0, 1):
        say(f"case v5 leaf probe precision {precision}: traverser {p}")
        got, mass = device_probe(ex, jobs, net, p)
        want, want_mass = oracle_probe(jobs, net, mode, p)
        exact, _ = oracle_probe(jobs, net, O.NET_F32, p)
        scale = float(np.abs(exact).max())
        err = np.abs(got.astype(np.float64) - want)
        dev32 = float(np.median(np.abs(got.astype(np.float64) - exact)))
        emu32 = float(np.median(np.abs(want.astype(np.float64) - exact)))
        say(f"against the model: max {err.max() / scale:.2e}, median {np.median(err) / scale:.2e}; median distance "
            f"to float32: device {dev32 / scale:.2e}, model {emu32 / scale:.2e} of the largest |value|")
        assert err.max() <= tol * scale
        assert np.median(err) <= tol / 6 * scale
        assert dev32 <= 1.5 * emu32 + 1e-6 * scale
        np.testing.assert_allclose(mass, want_mass, rtol=2e-6, atol=1e-30)


@pytest.mark.parametrize("precision,mode", [(ww.WC_F16, O.NET_F16A), (ww.WC_BF16, O.NET_BF16A)])
def test_v5_matrix_cores_track_the_scalar_path(precision, mode):
    """The trunk and the join on the matrix cores (the default 16-bit path)
    against the same operands summed in ascending float32 order
    (WC_V5_SCALAR=1, the oracle model's order): the MFMA's own summation
    order, the LayerNorm statistics' order and the hardware-exponential GELU
    only, within the 16-bit bounds above."""
    jobs = v5_jobs(seed=39)
    net = ww.synth_weights(ww.V5_DIMS, 1)
    os.environ["WC_V5_SCALAR"] = "1"
    try:
        scalar = ww.Executor(0, precision)
    finally:
        del os.environ["WC_V5_SCALAR"]
    tol = 3e-3 if precision == ww.WC_F16 else 3e-2
    try:
        for p in (0, 1):
            say(f"case v5 matrix cores precision {precision}: traverser {p}")
            got, _ = device_probe(executor(precision), jobs, net, p)
            ref, _ = device_probe(scalar, jobs, net, p)
            want, _ = oracle_probe(jobs, net, mode, p)
            scale = float(np.abs(want).max())
            # the scalar path is the oracle's model, bit for bit up to the readout's MFMA
            np.testing.assert_allclose(ref, want, rtol=0, atol=1e-3 * scale)
            err = np.abs(got.astype(np.float64) - ref)
            say(f"matrix cores against the scalar path: max {err.max() / scale:.2e}, median "
                f"{np.median(err) / scale:.2e} of the largest |value|")
            assert err.max() <= tol * scale
            assert np.median(err) <= tol / 6 * scale
    finally:
        scalar.close()


def test_v5_trunk_partial_workgroups():
    """The matrix-core trunk takes four network rows per workgroup (two
    groups of two): waves whose row count leaves the last workgroup one, two
    or three rows (an empty or half-empty group) still match the scalar path
    on every row."""
    net = ww.synth_weights(ww.V5_DIMS, 1)
    os.environ["WC_V5_SCALAR"] = "1"
    try:
        scalar = ww.Executor(0, ww.WC_F16)
    finally:
        del os.environ["WC_V5_SCALAR"]
    seen = set()
    try:
        for trees in range(1, 9):
            jobs = v5_jobs(trees=trees, seed=41 + trees)
            wave = ww.Wave(jobs)
            rows = wave.stats()["rows"]
            wave.close()
            if rows % 4 == 0 or rows % 4 in seen:
                continue
            seen.add(rows % 4)
            say(f"case v5 partial workgroups: {trees} trees, {rows} rows")
            got, _ = device_probe(executor(ww.WC_F16), jobs, net, 0)
            ref, _ = device_probe(scalar, jobs, net, 0)
            scale = float(np.abs(ref).max())
            assert np.abs(got.astype(np.float64) - ref).max() <= 3e-3 * scale
    finally:
        scalar.close()
    assert seen == {1, 2, 3}, seen


def reference_test_weights():
    """The reference's GPU-test network (engine/src/gpu/tests.rs:34-46): every weight
    (next_u64 / u64::MAX - 0.5) * 0.1 in float32 from its xorshift64* stream
    (engine/src/rng.rs:8-21) seeded 0xD15EA5E, biases zero, LayerNorm gains one and
    shifts zero."""
    nw, nb = ww.net_sizes(ww.V5_DIMS)
    nln = ww.net_norms(ww.V5_DIMS)
    m = (1 << 64) - 1
    x = 0xD15EA5E ^ 0x9E3779B97F4A7C15
    raw = np.empty(nw, np.uint64)
    for k in range(nw):
        x ^= x >> 12
        x ^= (x << 25) & m
        x ^= x >> 27
        raw[k] = (x * 0x2545F4914F6CDD1D) & m
    w = (raw.astype(np.float32) / np.float32(m) - np.float32(0.5)) * np.float32(0.1)
    ln = np.zeros(nln, np.float32)
    at = 0
    # per norm, its gains then its shifts (net.rs:272-316 order): 16 trunk-block
    # norms of 96, the trunk's 96, the config encoder's 128, three join-block
    # norms of 128, the join output's 128, the head's 256
    for width in [96] * 16 + [96, 128] + [128] * 3 + [128, 256]:
        ln[at:at + width] = 1.0
        at += 2 * width
    assert at == nln
    return ww.Net(list(ww.V5_DIMS), w, np.zeros(nb, np.float32), ln)


LINEAR = dict(alpha=1.0, beta=1.0, gamma=1.0, predict=0.0)  # Cfr::LINEAR, engine/src/search.rs:141-146


def gate_ratios(g, o):
    """engine/src/gpu/tests.rs:413-444: cmp(a, b, atol, rtol) is |a - b| <= atol + rtol
    max(|a|, |b|) elementwise; roots at (1e-2, 2e-3), strategy entries at (0.4, 0.1)."""
    def ratio(a, b, atol, rtol):
        a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
        return np.abs(a - b) / (atol + rtol * np.maximum(np.abs(a), np.abs(b)))

    pw = ratio(g.strategy, o["strategy"], 0.4, 0.1)
    return (float(ratio(g.root_values, o["roots"], 1e-2, 2e-3).max()), float(np.abs(g.strategy - o["strategy"]).mean()),
            float(pw.max()), float((pw > 1.0).mean()))


def v5_full_shape(trees=8, **kw):
    import workloads as W
    return W.jobs("wave256v5", **kw)[:trees]


@pytest.mark.parametrize("shape", ["small", "full"])
def test_v5_f16_solves_meet_the_references_gate(shape):
    """Whole f16 v5 solves against the float32 solver under the reference's gate for
    its fast tensor-core head (engine/src/gpu/tests.rs:393-446), on the reference's
    own test network and schedule (8 linear-CFR iterations, depth 2): root values
    within 1e-2 + 2e-3 |x|, mean strategy error <= 5e-3, and every strategy entry
    within 0.4 + 0.1 |x|. Eight small subgames and eight subgames of the benchmarked
    v5 wave at full shape (200..800 nodes, infostates up to 567). On the full-shape
    ones a near-tie flips single strategy entries under any f16 evaluation (the
    oracle's f16 model itself exceeds the pointwise guard on one of them), so there
    at most 1 in 1,000 entries may lie outside the guard; with the random-init
    network of the v5 workloads and 64 iterations the gate is out of reach of any
    16-bit evaluation (tests/test_gpu_trace.py and the replay below judge those)."""
    net = reference_test_weights()
    jobs = v5_jobs(trees=8, seed=43, iters=8, **LINEAR) if shape == "small" else \
        v5_full_shape(iters=8, **LINEAR)
    say(f"case v5 f16 reference gate: {len(jobs)} {shape} subgames, the reference's test network")
    ex = executor(ww.WC_F16)
    v = ex.publish(net)
    wave = ww.Wave(jobs)
    got = ex.solve(wave, v)
    wave.close()
    refs = pmap(lambda j: O.solve(j, net, O.NET_F32), jobs)
    for k, (g, o) in enumerate(zip(got, refs)):
        rr, ms, pw, out = gate_ratios(g, o)
        say(f"v5 {shape} tree {k}: roots {rr:.2f} of the gate, mean strategy error {ms:.1e}, pointwise {pw:.2f} of "
            f"the guard ({out:.1e} of the entries outside)")
        assert rr <= 1.0 and ms <= 5e-3, f"tree {k}"
        assert (pw <= 1.0) if shape == "small" else (out <= 1e-3), f"tree {k}"


def test_v5_bf16_solves_track_float32():
    """bf16 v5 solves (the reference gates only its f16 mode) on the same network and
    schedule, judged by what bf16 operands do by themselves: per subgame the root
    error within max(5e-2, 3x the oracle's bf16 model's), mean strategy error
    <= 1.5e-2 (the bf16 whales' bounds); the median root error within 2x the
    model's."""
    net = reference_test_weights()
    jobs = v5_jobs(trees=8, seed=43, iters=8, **LINEAR) + v5_full_shape(trees=4, iters=8, **LINEAR)
    say(f"case v5 bf16: {len(jobs)} subgames, the reference's test network")
    ex = executor(ww.WC_BF16)
    v = ex.publish(net)
    wave = ww.Wave(jobs)
    got = ex.solve(wave, v)
    wave.close()
    refs = pmap(lambda j: O.solve(j, net, O.NET_F32), jobs)
    emus = pmap(lambda j: O.solve(j, net, O.NET_BF16A), jobs)
    devs, models = [], []
    for k, (g, o, e) in enumerate(zip(got, refs, emus)):
        scale = float(np.abs(o["roots"]).max())
        rel = float(np.abs(g.root_values - o["roots"]).max()) / scale
        emu = float(np.abs(e["roots"] - o["roots"]).max()) / scale
        ms = float(np.abs(g.strategy - o["strategy"]).mean())
        say(f"v5 bf16 tree {k}: root error {rel:.1e} of the largest root value (bf16 model {emu:.1e}), mean "
            f"strategy error {ms:.1e}")
        assert rel <= max(5e-2, 3 * emu) and ms <= 1.5e-2, f"tree {k}"
        devs.append(rel)
        models.append(emu)
    assert np.median(devs) <= 2 * np.median(models) + 1e-4


@pytest.mark.parametrize("precision,mode,tol", [(ww.WC_F16, O.NET_F16A, 3e-3), (ww.WC_BF16, O.NET_BF16A, 3e-2)])
def test_v5_trace_tracks_the_operand_model_at_the_solves_reach(precision, mode, tol):
    """The v5 leaf values inside the full-shape solves (the per-iteration pooling of
    g(c), the join and the readout on the device's own reach) against the 16-bit
    model, with the initial-reach probe's bounds (median within tol / 6)."""
    from test_gpu_trace import check_trace_against_model
    check_trace_against_model(precision, mode, tol, v5_full_shape(), ww.synth_weights(ww.V5_DIMS, 1),
                              "wave256v5 full shape", median=1 / 6)


@pytest.mark.parametrize("precision", [ww.WC_F16, ww.WC_BF16])
def test_v5_replay_of_16bit_solves_bit_exact(precision):
    from test_gpu_trace import replay_and_compare
    say(f"case v5 replay precision {precision}: full-shape subgames, every leaf evaluation")
    replay_and_compare(precision, v5_full_shape(), ww.synth_weights(ww.V5_DIMS, 1), f"wave256v5 {precision}")
