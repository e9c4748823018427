"""Pins of the oracle (oracle/oracle.c) against checks that do not share its code.

- game value: textbook vanilla CFR over world states (tests/brute_cfr.py),
  for every CFR variant the reference names (engine/src/search.rs:141-179),
  as the reference checks its own solver (engine/tests/rebel_solver.rs:166-280);
- the iterate itself: average strategy and Phase 2 root values after 1..6
  iterations against a float64 world-state discounted-CFR restatement
  (tests/tabular_dcfr.py), which fixes the discount schedule (which update
  count feeds each factor, when the sums are seeded and discounted);
- zero-sum root values and NashConv >= 0 and falling (rebel_solver.rs:239-263);
- reverse gathers: reach replayed through the rev/rvd tables equals the
  forward scatter of search.rs:1273-1351 (pattern of serialize.rs:1411-1508),
  and the oracle's carried beliefs equal that reach, normalised;
- closed forms: DCFR factors (search.rs:185-193), snapshot iterations
  (search.rs:102-110, rebel_solver.rs:578-602), the belief fallback
  (rebel.rs:1054-1068), f16/bf16 round-to-nearest-even;
- the leaf MLP against a numpy float64 evaluation;
- the zero network (the principle of engine/src/gpu/tests.rs:274-325).
"""
import math

import numpy as np
import pytest

import brute_cfr as B
import oracle as O
import wcj8
import workloads as W

NONE = 0xFFFFFFFF
VARIANTS = {  # engine/src/search.rs:141-179
    "linear": (1.0, 1.0, 1.0, 0.0),
    "plus": (math.inf, -math.inf, 2.0, 0.0),
    "dcfr": (1.5, 0.0, 2.0, 0.0),
    "pcfr": (math.inf, -math.inf, 2.0, 1.0),
    "sapcfr": (math.inf, -math.inf, 2.0, np.float32(1.0 / 3.0)),
}


def tiny_terminal_tree(seed, variant="dcfr", iters=500, notrans=0.0, chance=1):
    a, b, g, p = VARIANTS[variant]
    [j] = W.jobs("wave256", trees=1, seed=seed, nodes_lo=8, nodes_hi=24, act_lo=2, act_hi=4, chance=chance, draw_lo=2,
                 draw_hi=3, info_fixed=3, terminal_p=1.0, notrans_p=notrans, collapse=0.3, iters=iters, dirichlet=1,
                 nroots=1, alpha=a, beta=b, gamma=g, predict=float(p))
    return j


def root_values(job, out):
    d = wcj8.decode(job)
    n0 = len(d["root"][0])
    v0 = float(np.dot(d["root"][0].astype(np.float64), out["roots"][0][:n0]))
    v1 = float(np.dot(d["root"][1].astype(np.float64), out["roots"][0][n0:]))
    return v0, v1


def with_iters(job, iters):
    d = wcj8.decode(job)
    snaps = [t for t in range(iters + 1) if t == 0 or (t & (t - 1)) == 0 or t == iters]
    return wcj8.encode(dict(d, iters=iters, snap_iters=np.array(snaps, np.uint32)))


@pytest.mark.parametrize("variant", sorted(VARIANTS))
def test_solver_matches_tabular_cfr(variant):
    checked = 0
    for seed in range(200, 206):
        job = tiny_terminal_tree(seed, variant)
        d = wcj8.decode(job)
        if d["nodes"] < 9 or len(set(np.round(d["terminal_utility"], 4))) < 2:
            continue
        exact = B.game_value(d, iters=200)
        late = O.solve(job, None, O.NET_EMPTY, conv=True)
        v0, v1 = root_values(job, late)
        assert abs(v0 + v1) < 1e-4, f"seed {seed}: root values not zero-sum: {v0} + {v1}"
        # The reference holds its solver to 0.03 of tabular CFR; these tiny trees
        # converge far closer.
        assert abs(v0 - exact) < 5e-3, f"seed {seed} {variant}: solver {v0:.5f} vs tabular CFR {exact:.5f}"
        early = O.solve(with_iters(job, 2), None, O.NET_EMPTY, conv=True)
        assert late["conv"][0] > -1e-3, f"seed {seed}: NashConv negative"
        assert late["conv"][0] < max(early["conv"][0], 1e-3), "NashConv did not fall"
        checked += 1
    assert checked >= 3


def test_no_successor_cells_keep_the_game_value():
    """A legal cell with no successor config is worth 0 (search.rs:1720-1740); the
    game value still matches tabular CFR, which scores such a world 0. The
    reference's best response skips those cells, so NashConv is only bounded on
    trees without them."""
    for seed in (300, 301, 302):
        job = tiny_terminal_tree(seed, "dcfr", notrans=0.1)
        d = wcj8.decode(job)
        assert (d["legal_trans"] == NONE).any() or d["nodes"] < 6
        exact = B.game_value(d, iters=200)
        v0, v1 = root_values(job, O.solve(job, None, O.NET_EMPTY))
        assert abs(v0 - exact) < 5e-3 and abs(v0 + v1) < 1e-4


# ------------------------------------------------------------- reverse gathers

def uniform_cur(d):
    cur = np.zeros(d["ncells"], np.float64)
    for i in range(d["nodes"]):
        if d["node_kind"][i] != 0:
            continue
        me = int(d["node_player"][i])
        r0 = int(d["legal_row_of"][i])
        nc = int(d["cfg_off"][2 * i + me + 1] - d["cfg_off"][2 * i + me])
        for c in range(nc):
            lo, hi = int(d["legal_off"][r0 + c]), int(d["legal_off"][r0 + c + 1])
            cur[lo:hi] = 1.0 / (hi - lo)
    return cur


def nc_of(d, i, p):
    return int(d["cfg_off"][2 * i + p + 1] - d["cfg_off"][2 * i + p])


def forward_reach(d, cur):
    """Forward scatter in float64, search.rs:1273-1351 restated on the tables."""
    N = d["nodes"]
    reach = [[np.zeros(nc_of(d, i, 0)), np.zeros(nc_of(d, i, 1))] for i in range(N)]
    reach[0] = [d["root"][0].astype(np.float64), d["root"][1].astype(np.float64)]
    act_base = 0
    for i in range(N):
        kind, me = int(d["node_kind"][i]), int(d["node_player"][i])
        op = 1 - me
        cs0, cs1 = int(d["node_child_start"][i]), int(d["node_child_start"][i + 1])
        if kind == 2:
            continue
        if kind == 1:
            c = int(d["node_child"][cs0])
            reach[c][op] = reach[i][op].copy()
            d0, rb = int(d["draw_off"][i]), int(d["draw_row_off"][i])
            for ci in range(nc_of(d, i, me)):
                lo, hi = int(d["draw_row_start"][rb + ci]), int(d["draw_row_start"][rb + ci + 1])
                for x in range(lo, hi):
                    reach[c][me][d["draw_to"][d0 + x]] += reach[i][me][ci] * d["draw_p"][d0 + x]
            continue
        so, se = int(d["soff"][i]), int(d["soff"][i + 1])
        o0 = int(d["obs_off"][i])
        na = int(d["obs_start"][int(d["obs_off"][i + 1]) - 1])
        oact = d["obs_act"][act_base:act_base + na]
        act_base += na
        for ch in range(cs1 - cs0):
            c = int(d["node_child"][cs0 + ch])
            reach[c][op] = reach[i][op].copy()
            for k in range(int(d["obs_start"][o0 + ch]), int(d["obs_start"][o0 + ch + 1])):
                a = int(oact[k])
                for g in range(so, se):
                    if d["legal_action"][g] != a or d["legal_trans"][g] == NONE:
                        continue
                    reach[c][me][d["legal_trans"][g]] += reach[i][me][d["cell_row"][g]] * cur[g]
    return reach


def gathered_reach(d, cur):
    """The same reach through the reverse tables alone (rev: decision parent, rvd: chance parent)."""
    N = d["nodes"]
    reach = [None] * N
    reach[0] = [d["root"][0].astype(np.float64), d["root"][1].astype(np.float64)]
    for i in range(1, N):
        par = int(d["node_parent"][i])
        me = int(d["node_player"][par])
        r = [None, None]
        r[1 - me] = reach[par][1 - me].copy()
        mine = np.zeros(nc_of(d, i, me))
        if d["rev_row_of"][i] != NONE:
            r0 = int(d["rev_row_of"][i])
            for t in range(len(mine)):
                for x in range(int(d["rev_start"][r0 + t]), int(d["rev_start"][r0 + t + 1])):
                    mine[t] += reach[par][me][d["rev_src"][x]] * cur[d["rev_cell"][x]]
        else:
            r0 = int(d["rvd_row_of"][i])
            for t in range(len(mine)):
                for x in range(int(d["rvd_start"][r0 + t]), int(d["rvd_start"][r0 + t + 1])):
                    mine[t] += reach[par][me][d["rvd_src"][x]] * d["rvd_p"][x]
        r[me] = mine
        reach[i] = r
    return reach


def test_reverse_gathers_replay_the_forward_scatter():
    jobs = W.jobs("wave256", trees=3, seed=17, nodes_lo=40, nodes_hi=90, chance=1, notrans_p=0.05, collapse=0.5,
                  info_median=6.0, info_p99=30.0, info_cap=30, terminal_p=0.1, iters=4)
    for job in jobs:
        d = wcj8.decode(job)
        cur = uniform_cur(d)
        fwd, rev = forward_reach(d, cur), gathered_reach(d, cur)
        for i in range(d["nodes"]):
            for p in (0, 1):
                np.testing.assert_allclose(rev[i][p], fwd[i][p], rtol=1e-12, atol=1e-15)
        # Snapshot 0 is the uniform strategy; its carried beliefs are the
        # normalised reach at every exit (search.rs:1937-1956).
        o = O.solve(job, None, O.NET_EMPTY)
        exits = list(d["leaf_rows"]) + list(d["term_leaves"])
        for e, node in enumerate(exits):
            for p in (0, 1):
                w = fwd[node][p]
                want = w / w.sum() if w.sum() > 1e-30 else np.full(len(w), 1.0 / max(len(w), 1))
                lo, hi = int(d["snap_coff"][2 * e + p]), int(d["snap_coff"][2 * e + p + 1])
                got = o["carries"][0][lo:hi]
                assert np.all(np.abs(got - want) <= 1e-6 + 1e-5 * np.abs(want))


def test_belief_fallback_is_uniform():
    """normalize_weights: a reach vector summing to <= 1e-30 becomes uniform 1/n."""
    [job] = W.jobs("wave256", trees=1, seed=23, nodes_lo=30, nodes_hi=50, chance=1, info_fixed=5, iters=2,
                   terminal_p=0.2)
    d = wcj8.decode(job)
    d["root"][1] = np.zeros_like(d["root"][1])
    o = O.solve(wcj8.encode(d), None, O.NET_EMPTY)
    exits = list(d["leaf_rows"]) + list(d["term_leaves"])
    for e, node in enumerate(exits):
        lo, hi = int(d["snap_coff"][2 * e + 1]), int(d["snap_coff"][2 * e + 2])
        n = hi - lo
        assert np.all(o["carries"][0][lo:hi] == np.float32(1.0) / np.float32(n))


# ------------------------------------------------------------------ closed forms

def test_dcfr_factors():
    for m in range(1, 70):
        for p in (1.5, 1.0, 2.0, 0.5):
            want = m ** p / (m ** p + 1.0)
            assert abs(O.factor(m, p) - want) <= 2e-7 * want
        assert O.factor(m, 0.0) == 0.5
        assert O.factor(m, math.inf) == 1.0
        assert O.factor(m, -math.inf) == 0.0


@pytest.mark.parametrize("iters", [1, 2, 8, 16, 64, 100])
def test_snapshot_iterations_are_log_spaced_plus_final(iters):
    [job] = W.jobs("tree48", iters=iters)
    got = list(wcj8.decode(job)["snap_iters"])
    want = [t for t in range(iters + 1) if t == 0 or (t & (t - 1)) == 0 or t == iters]
    assert got == want
    assert O.shape(job).carry_slots == len(want) - 1


def test_f16_rounding_is_ieee_nearest_even():
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.standard_normal(4000) * 10.0 ** rng.integers(-9, 5, 4000),
        np.array([0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 7e4, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 1e-9]),
        (np.arange(1, 200) + 0.5) * 2.0 ** -24,  # ties among subnormals
        1.0 + (np.arange(0, 64) * 2 + 1) * 2.0 ** -11,  # ties at 1.0
    ]).astype(np.float32)
    for x in vals:
        with np.errstate(over="ignore"):
            want = np.float32(np.float16(x))
        got = np.float32(O.round_f16(float(x)))
        assert got == want or (np.isnan(got) and np.isnan(want)), (x, got, want)


def test_bf16_rounding_is_nearest_even():
    rng = np.random.default_rng(4)
    vals = np.concatenate([rng.standard_normal(4000) * 10.0 ** rng.integers(-20, 20, 4000),
                           1.0 + (np.arange(0, 64) * 2 + 1) * 2.0 ** -8]).astype(np.float32)
    for x in vals:
        m, e = np.frexp(np.float64(x))
        want = np.float32(np.ldexp(np.round(m * 256.0), e - 8))  # 8 significant bits, ties to even
        assert np.float32(O.round_bf16(float(x))) == want, x


# ------------------------------------------------------------------------ net

def test_mlp_matches_float64_numpy():
    net = W.net_for("mlp65k")
    dims = net.dims
    inp, hid, layers, heads = dims[1], dims[2], dims[3], dims[4]
    x = W.mlp65k_inputs(rows=96, seed=12)
    w = net.w.astype(np.float64)
    b = net.b.astype(np.float64)
    h = x.astype(np.float64)
    at, bt, k = 0, 0, inp
    for _ in range(layers):
        Wl = w[at:at + k * hid].reshape(k, hid)
        h = np.maximum(h @ Wl + b[bt:bt + hid], 0.0)
        at += k * hid
        bt += hid
        k = hid
    Wh = w[at:at + heads * hid].reshape(heads, hid)
    want = h @ Wh.T + b[bt:bt + heads]
    keys = np.tile(np.arange(heads, dtype=np.uint32), (x.shape[0], 1))
    got = O.mlp(x, keys, net, O.NET_F32)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    # Keyed head reads pick the requested head rows.
    perm = np.ascontiguousarray(keys[:, ::-1])
    np.testing.assert_array_equal(O.mlp(x, perm, net, O.NET_F32), got[:, ::-1])


def test_zero_network_keeps_every_value_zero():
    [job] = W.jobs("tree48")
    net = W.net_for("tree48")
    zero = type(net)(net.dims, np.zeros_like(net.w), np.zeros_like(net.b))
    o = O.solve(job, zero, O.NET_F32)
    assert np.all(o["roots"] == 0.0)
    d = wcj8.decode(job)
    np.testing.assert_allclose(o["strategy"], uniform_cur(d), rtol=2e-6)


def numpy_leaf_net(d, net, reach):
    """The leaf net in float64 at a given reach: pooled beliefs (search.rs:1501-1547),
    the query input, the MLP or two-tower net. Returns values(r, p): the net's
    value of each of network row r's configs of traverser p."""
    dims = [int(x) for x in net.dims]
    w, b = net.w.astype(np.float64), net.b.astype(np.float64)

    def tower(at, k, layers, hid):
        mats = []
        for _ in range(layers):
            mats.append(w[at:at + k * hid].reshape(k, hid))
            at += k * hid
            k = hid
        return mats, at

    if dims[0] == 101:  # MLP: [101, in, hidden, layers, heads, pool]
        inp, hid, layers, heads, pool = dims[1:6]
        cfeat = 1 + pool
        mats, at = tower(0, inp, layers, hid)
        Wh = w[at:at + heads * hid].reshape(heads, hid)
    else:  # two-tower: [102, in, width, pub_layers, priv_in, priv_layers, pool]
        inp, hid, layers, priv_in, priv_layers, pool = dims[1:7]
        cfeat = 1 + pool + priv_in
        mats, at = tower(0, inp, layers, hid)
        pmats, at = tower(at, priv_in, priv_layers, hid)
        wread = w[at:at + hid]
        pb = b[layers * hid:(layers + priv_layers) * hid]
        bread = b[(layers + priv_layers) * hid]
    cphi = d["cphi"].astype(np.float64).reshape(-1, cfeat)
    rb = len(d["leaf_raw"]) // max(d["rows"], 1)
    pooled = {}
    for r, leaf in enumerate(d["leaf_rows"]):
        for p in (0, 1):
            wv = reach[leaf][p]
            beta = wv / wv.sum() if wv.sum() > 1e-30 else np.full(len(wv), 1.0 / max(len(wv), 1))
            cid = d["leaf_cidx"][d["leaf_coff"][2 * r + p]:d["leaf_coff"][2 * r + p + 1]]
            pooled[(r, p)] = beta @ cphi[cid, 1:1 + pool] if len(cid) else np.zeros(pool)

    def values(r, p):
        raw = d["leaf_raw"][r * rb:(r + 1) * rb].astype(np.float64) / 255.0
        h = np.concatenate([pooled[(r, p)], pooled[(r, 1 - p)], [1.0 if p else -1.0], raw])
        for l in range(layers):
            h = np.maximum(h @ mats[l] + b[l * hid:(l + 1) * hid], 0.0)
        cid = d["leaf_cidx"][d["leaf_coff"][2 * r + p]:d["leaf_coff"][2 * r + p + 1]]
        if dims[0] == 101:
            keys = cphi[cid, 0].astype(int)
            return Wh[keys] @ h + b[layers * hid + keys]
        v = np.zeros(len(cid))  # <w_read * private_tower(features(c)), public_tower(query)> + b_read
        for x, c in enumerate(cid):
            f = cphi[c, 1 + pool:]
            for l in range(priv_layers):
                f = np.maximum(f @ pmats[l] + pb[l * hid:(l + 1) * hid], 0.0)
            v[x] = (wread * f) @ h + bread
        return v

    return values


def numpy_value_under(d, net, root):
    """value_under (search.rs:1851-1871) in float64 under the uniform strategy:
    propagate, the leaf net, leaf readout (search.rs:1587-1636) and the Value
    backprop (search.rs:1654-1803)."""
    cur = uniform_cur(d)
    dd = dict(d, root=[np.asarray(root[0]), np.asarray(root[1])])
    reach = forward_reach(dd, cur)
    leaf_net = numpy_leaf_net(d, net, reach)
    out = []
    for p in (0, 1):
        vals = {}
        for k, leaf in enumerate(d["term_leaves"]):
            u = d["terminal_utility"][k] if d["node_player"][leaf] == p else -d["terminal_utility"][k]
            vals[int(leaf)] = np.full(nc_of(d, leaf, p), float(u) * reach[leaf][1 - p].sum())
        for r, leaf in enumerate(d["leaf_rows"]):
            vals[int(leaf)] = leaf_net(r, p) * reach[leaf][1 - p].sum()
        for i in range(d["nodes"] - 1, -1, -1):
            kind, me = int(d["node_kind"][i]), int(d["node_player"][i])
            if kind == 2:
                continue
            cs0, cs1 = int(d["node_child_start"][i]), int(d["node_child_start"][i + 1])
            n = nc_of(d, i, p)
            if kind == 1:
                ch = int(d["node_child"][cs0])
                if me != p:
                    vals[i] = vals[ch].copy()
                    continue
                d0, rb0 = int(d["draw_off"][i]), int(d["draw_row_off"][i])
                v = np.zeros(n)
                for c in range(n):
                    for x in range(int(d["draw_row_start"][rb0 + c]), int(d["draw_row_start"][rb0 + c + 1])):
                        v[c] += d["draw_p"][d0 + x] * vals[ch][d["draw_to"][d0 + x]]
                vals[i] = v
            elif me == p:
                v = np.zeros(n)
                for g in range(int(d["soff"][i]), int(d["soff"][i + 1])):
                    t = d["legal_trans"][g]
                    if t != NONE:
                        v[d["cell_row"][g]] += vals[int(d["legal_child"][g])][t] * cur[g]
                vals[i] = v
            else:
                vals[i] = sum(vals[int(d["node_child"][x])] for x in range(cs0, cs1))
        out.append(vals[0])
    return np.concatenate(out)


@pytest.mark.parametrize("family", ["wave256", "wave512w"])
def test_value_under_matches_float64_restatement(family):
    """Pins belief_blocks, the query input, readout and the Value backprop, for
    the MLP and for the two-tower net: a zero-iteration solve is value_under
    under the uniform strategy."""
    net = W.net_for(family)
    jobs = W.jobs(family, trees=2, seed=29, nodes_lo=30, nodes_hi=60, chance=1, terminal_p=0.2, notrans_p=0.05,
                  info_median=5.0, info_p99=20.0, info_cap=20, iters=0, nroots=2, whale_frac=0.0)
    for job in jobs:
        d = wcj8.decode(job)
        o = O.solve(job, net, O.NET_F32)
        for r, (c0, c1) in enumerate(d["carried"]):
            want = numpy_value_under(d, net, (c0, c1))
            got = o["roots"][r].astype(np.float64)
            assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max() + 1e-7, r


@pytest.mark.parametrize("family", ["wave256", "wave512w"])
def test_leaf_probe_matches_float64_restatement(family):
    """Pins oracle_leaf_probe (the leaf net's values and the reach masses at the
    initial reach, the reference for the device's own leaf probe) against the
    float64 restatement, for both traversers."""
    net = W.net_for(family)
    jobs = W.jobs(family, trees=2, seed=23, nodes_lo=30, nodes_hi=70, chance=1, terminal_p=0.15, notrans_p=0.05,
                  info_median=6.0, info_p99=30.0, info_cap=30, iters=4, nroots=1, whale_frac=0.0)
    for job in jobs:
        d = wcj8.decode(job)
        reach = forward_reach(d, uniform_cur(d))
        leaf_net = numpy_leaf_net(d, net, reach)
        for p in (0, 1):
            want = np.concatenate([leaf_net(r, p) for r in range(d["rows"])])
            got, mass = O.leaf_probe(job, net, O.NET_F32, p)
            assert got.shape == want.shape
            assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max() + 1e-7
            for mode in (O.NET_F32W, O.NET_F16X):  # near-float32 models stay near float32
                other, _ = O.leaf_probe(job, net, mode, p)
                assert np.abs(other - want).max() <= 1e-4 * np.abs(want).max()
        want_mass = np.array([[reach[leaf][q].sum() for q in (0, 1)] for leaf in d["leaf_rows"]])
        np.testing.assert_allclose(mass, want_mass, rtol=1e-6, atol=1e-30)


def f16_round(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def test_reduced_precision_models_match_numpy():
    """The MLP's arithmetic models (oracle.c): F16A is f16-rounded operands and
    activations with a float32 sum in ascending k (zero inputs skipped), the
    bias added after the sum; F16 / F32W / F16X sum wide (float64) over f16,
    float32 and hi + lo pair operands."""
    dims = [101, 64, 32, 2, 10, 8]
    import warchest_wave as ww
    net = ww.synth_weights(dims, seed=5)
    x = ww.synth_features(40, 64, seed=6)
    keys = np.tile(np.arange(10, dtype=np.uint32), (40, 1))
    inp, hid, layers, heads = 64, 32, 2, 10
    w, b = net.w, net.b

    def mats(q):
        out, at, k = [], 0, inp
        for _ in range(layers):
            out.append(q(w[at:at + k * hid]).reshape(k, hid))
            at += k * hid
            k = hid
        return out, q(w[at:at + heads * hid]).reshape(heads, hid)

    # F16A: float32 products and sums, one k at a time
    M, Wh = mats(f16_round)
    h = f16_round(x)
    for l in range(layers):
        acc = np.zeros((h.shape[0], hid), np.float32)
        for k in range(h.shape[1]):
            acc = np.where(h[:, k:k + 1] != 0, acc + h[:, k:k + 1] * M[l][k][None, :], acc).astype(np.float32)
        h = f16_round(np.maximum(acc + b[l * hid:(l + 1) * hid], 0))
    acc = np.zeros((h.shape[0], heads), np.float32)
    for k in range(hid):
        acc = (acc + h[:, k:k + 1] * Wh[:, k][None, :]).astype(np.float32)
    want = (acc + b[layers * hid:layers * hid + heads]).astype(np.float32)
    np.testing.assert_array_equal(O.mlp(x, keys, net, O.NET_F16A), want)

    def wide(q):
        M, Wh = mats(q)
        h = q(x).astype(np.float64)
        for l in range(layers):
            pre = (h @ M[l].astype(np.float64)).astype(np.float32) + b[l * hid:(l + 1) * hid]
            h = q(np.maximum(pre, 0)).astype(np.float64)
        return (h @ Wh.astype(np.float64).T).astype(np.float32) + b[layers * hid:layers * hid + heads]

    def pair(a):
        hi = f16_round(a)
        return hi + f16_round(np.asarray(a, np.float32) - hi)

    for mode, q in ((O.NET_F16, f16_round), (O.NET_F32W, lambda a: np.asarray(a, np.float32)), (O.NET_F16X, pair)):
        got = O.mlp(x, keys, net, mode)
        ref = wide(q)
        assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max(), mode


@pytest.mark.parametrize("variant", sorted(VARIANTS))
def test_solver_trajectory_matches_tabular_dcfr(variant):
    """The iterate itself, not only where it converges: after 1, 2, 3 and 6
    alternating iterations the oracle's average strategy and its Phase 2 root
    values equal a float64 world-state restatement of discounted CFR
    (tests/tabular_dcfr.py) to float32 rounding. Trees with and without
    no-successor cells, both players drawing."""
    import tabular_dcfr as TD
    checked = 0
    for notrans in (0.0, 0.3):
        for seed in range(200, 206):
            job = tiny_terminal_tree(seed, variant, iters=6, notrans=notrans)
            for iters in (1, 2, 3, 6):
                j = with_iters(job, iters)
                got = O.solve(j, None, O.NET_EMPTY)
                strat, roots = TD.solve(wcj8.decode(j))
                ds = float(np.abs(got["strategy"] - strat).max())
                dr = float(np.abs(got["roots"] - roots).max() / max(np.abs(roots).max(), 1e-9))
                assert ds < 5e-6 and dr < 5e-6, f"seed {seed} notrans {notrans} iters {iters}: {ds:.2e} {dr:.2e}"
                checked += 1
    assert checked == 48


def test_trajectory_pin_sees_schedule_mistakes():
    """The restatement with a mistake planted in its schedule departs from the
    oracle by far more than the tolerance above: the discount factors of the
    next update (m + 1 instead of m), no seeding of the average sums, and
    average weights from the reach under the strategy before the update."""
    import tabular_dcfr as TD

    class LateFactors(TD.Solver):
        def step(self, p):
            self.steps[p] += 1
            super().step(p)
            self.steps[p] -= 1

    class Unseeded(TD.Solver):
        def _add_average(self, p):
            if self.steps != [0, 0]:
                super()._add_average(p)

    class StaleReach(TD.Solver):
        def step(self, p):
            self.before = self.sigma.copy()
            super().step(p)

        def _add_average(self, p):
            sigma = getattr(self, "before", self.sigma)
            reach = TD.own_reach(self.t, sigma, self.prior[p], p)
            for i, c, row in self.decision_rows(p):
                for g, _, _ in row:
                    self.sum[g] += reach[i][c] * self.sigma[g]

    worst = {}
    for seed in range(200, 206):
        j = with_iters(tiny_terminal_tree(seed, "dcfr", iters=6), 3)
        got = O.solve(j, None, O.NET_EMPTY)["strategy"]
        d = wcj8.decode(j)
        for cls in (LateFactors, Unseeded, StaleReach):
            s = cls(d)
            for it in range(3):
                s.step(it % 2)
            worst[cls.__name__] = max(worst.get(cls.__name__, 0.0), float(np.abs(s.average() - got).max()))
    assert min(worst.values()) > 1e-2, worst
