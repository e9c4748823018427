"""Pins of the oracle's leaf trace, leaf evaluation and replay (CPU only).

These three functions let the GPU tests separate a device error from the
conditioning of a reduced-precision solve:

- oracle_leaf_eval computes the leaf net's values at a reach the caller gives
  (the reach a device solve actually reached), so one well-conditioned network
  evaluation can be held to the operand model at every iteration;
- oracle_solve_replay runs the CPU solver with every network leaf's value and
  reach mass given (the values the device's own leaf net produced inside its
  solve), so the device's CFR arithmetic can be compared bit for bit whatever
  its leaf net's precision.

Pins, none of which shares code with the functions pinned:
- the solver's own trace replayed is the solve, bit for bit (strategy, roots,
  carries), in float32 and under an f16 operand model;
- planted mistakes in a replay (one Phase-2 evaluation scaled by 1e-3, one
  iteration's values scaled, the players' masses swapped at one iteration,
  one evaluation short) change the result or are refused;
- oracle_leaf_eval at the reach the solver reached at an evaluation gives that
  evaluation's values and masses bit for bit, and at the initial reach it is
  oracle_leaf_probe.
"""
import numpy as np
import pytest

import oracle as O
import workloads as W


def cases():
    return [("tree48", 0), ("wave64", 5), ("wave64", 57)]


def job_net(name, k):
    return W.jobs(name)[k], W.net_for(name)


def evaluations(job):
    s = O.shape(job)
    n0, n1, rows, nreach = O.leaf_counts(job)
    trav = [t % 2 for t in range(s.iters)] + [p for _ in range(s.nroots) for p in (0, 1)]
    voff, v = [], 0
    for p in trav:
        voff.append(v)
        v += n1 if p else n0
    return trav, voff, rows, nreach, (n0, n1)


@pytest.mark.parametrize("name,k", cases())
@pytest.mark.parametrize("mode", [O.NET_F32, O.NET_F16])
def test_replay_of_the_solvers_own_trace_is_the_solve(name, k, mode):
    job, net = job_net(name, k)
    want = O.solve(job, net, mode)
    tr = O.solve_trace(job, net, mode)
    np.testing.assert_array_equal(tr["strategy"], want["strategy"])
    np.testing.assert_array_equal(tr["roots"], want["roots"])
    got = O.solve_replay(job, tr["vals"], tr["mass"])
    np.testing.assert_array_equal(got["strategy"], want["strategy"])
    np.testing.assert_array_equal(got["roots"], want["roots"])
    np.testing.assert_array_equal(got["carries"], want["carries"])


@pytest.mark.parametrize("name,k", cases()[1:])
def test_planted_replay_mistakes_are_seen(name, k):
    job, net = job_net(name, k)
    tr = O.solve_trace(job, net, O.NET_F32)
    base = O.solve_replay(job, tr["vals"], tr["mass"])
    trav, voff, rows, _, n = evaluations(job)
    it = O.shape(job).iters
    # the last Phase-2 evaluation (player 1 of the last carried root) scaled by 1e-3
    v = tr["vals"].copy()
    v[voff[-1]:] *= 1.001
    got = O.solve_replay(job, v, tr["mass"])
    np.testing.assert_array_equal(got["strategy"], base["strategy"])
    assert np.abs(got["roots"] - base["roots"]).max() > 1e-6 * np.abs(base["roots"]).max()
    # every value of iteration 2 scaled by 1e-2
    v = tr["vals"].copy()
    v[voff[2]:voff[3]] *= 1.01
    got = O.solve_replay(job, v, tr["mass"])
    assert np.abs(got["strategy"] - base["strategy"]).max() > 1e-6
    # the players' masses swapped at iteration 1
    m = tr["mass"].copy().reshape(-1, rows, 2)
    m[1] = m[1][:, ::-1]
    got = O.solve_replay(job, tr["vals"], m.reshape(-1))
    assert np.abs(got["strategy"] - base["strategy"]).max() > 1e-6
    # one evaluation short, or one too many
    with pytest.raises(ValueError, match="fewer"):
        O.solve_replay(job, tr["vals"][: voff[-1]], tr["mass"][: 2 * rows * (len(trav) - 1)])
    with pytest.raises(ValueError, match="more"):
        O.solve_replay(job, np.concatenate([tr["vals"], tr["vals"][: n[0]]]),
                       np.concatenate([tr["mass"], tr["mass"][: 2 * rows]]))
    assert it == 64


@pytest.mark.parametrize("name,k", cases())
@pytest.mark.parametrize("mode", [O.NET_F32, O.NET_F16, O.NET_BF16])
def test_leaf_eval_at_the_solvers_reach_is_its_evaluation(name, k, mode):
    job, net = job_net(name, k)
    tr = O.solve_trace(job, net, mode)
    trav, voff, rows, nreach, n = evaluations(job)
    voff.append(len(tr["vals"]))
    it = O.shape(job).iters
    for e in sorted({0, 1, 2, it // 2 - 1, it - 1, len(trav) - 2, len(trav) - 1}):
        p = trav[e]
        vals, mass = O.leaf_eval(job, net, mode, p, tr["reach"][e * nreach:(e + 1) * nreach])
        np.testing.assert_array_equal(vals, tr["vals"][voff[e]:voff[e + 1]], err_msg=f"evaluation {e}")
        np.testing.assert_array_equal(mass.reshape(-1), tr["mass"][e * 2 * rows:(e + 1) * 2 * rows],
                                      err_msg=f"evaluation {e}")


@pytest.mark.parametrize("mode", [O.NET_F32, O.NET_F16])
def test_leaf_eval_at_the_initial_reach_is_the_leaf_probe(mode):
    job, net = job_net("wave64", 5)
    tr = O.solve_trace(job, net, mode)
    nreach = O.leaf_counts(job)[3]
    for p in (0, 1):
        want, want_mass = O.leaf_probe(job, net, mode, p)
        # evaluation 0 runs at the initial reach; its reach is traverser-independent
        got, mass = O.leaf_eval(job, net, mode, p, tr["reach"][:nreach])
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(mass, want_mass)
