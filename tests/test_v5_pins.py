"""Pins of the oracle's v5 network (oracle/v5.c, engine/src/net.rs) against
checks that do not share its code:

- the blob sizes, from net.rs's layer list counted here;
- the board geometry's invariants (37 hexes, 90 edges, opposite directions,
  19 interior hexes, 10 locations: board.rs);
- every piece (cards, board trunk, join cache, config encoder, join,
  readout) against a float64 torch restatement (tests/v5_torch.py) on
  synthetic jobs' own inputs;
- GELU against its closed form; the restatement's own tanh against the C
  library's, and what that difference does to whole solves (below the float32
  tolerance);
- special cases: a network with every matrix and bias zero values every leaf
  at value_bias; the config encoder does not depend on the order of a
  config's coin slots (net.rs:751-757: a sum over slot tokens);
- the 16-bit models (NET_F16 / NET_F16A / NET_BF16 / NET_BF16A) against the
  torch restatement with the operands of exactly the tensor-core products
  rounded, piece by piece, and with any one of them left unrounded (a planted
  mistake, which the comparison must see).
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
import v5_torch as T
import warchest_wave as ww
import wcj8

torch.set_default_dtype(torch.float64)


def v5_jobs(trees=3, seed=11, **kw):
    spec = dict(seed=seed, trees=trees, nodes_lo=30, nodes_hi=60, chance=1, info_median=6.0, info_p99=30.0,
                info_cap=30, iters=8, nroots=1, dirichlet=1, depth=2, act_lo=3, act_hi=6)
    spec.update(kw)
    return ww.synth_jobs(ww.V5_DIMS, **spec)


@pytest.fixture(scope="module")
def net():
    return ww.synth_weights(ww.V5_DIMS, 1)


def test_blob_sizes_follow_net_rs():
    TYPE, C, BLOCKS, D, POOL, CFGH, JW, JB = 64, 96, 8, 256, 64, 128, 128, 3
    mats = [(25, TYPE), (TYPE, TYPE), (4, TYPE), (6, C), (TYPE, C), (15, C)] + [(2 * C, C), (2 * C, C), (C, C)] * BLOCKS
    mats += [(2 * C + 15, D), (3 + TYPE, CFGH), (CFGH, D), (CFGH, POOL), (TYPE, 3 * POOL), (D, JW), (2 * POOL + 1, JW)]
    mats += [(JW, JW)] * JB + [(JW, D)]
    nw = sum(i * o for i, o in mats) + 2 * TYPE + 37 * C  # + seat and position embeddings
    biased = [TYPE, TYPE, C] + [C, C, C] * BLOCKS + [D, CFGH, D, POOL, JW] + [JW] * JB + [D]
    nb = sum(biased) + 1  # + value_bias
    nln = 2 * (2 * BLOCKS * C + C + CFGH + JB * JW + JW + D)
    assert O.v5_sizes() == (nw, nb, nln)
    assert ww.net_sizes(ww.V5_DIMS) == (nw, nb) and ww.net_norms(ww.V5_DIMS) == nln


def test_board_geometry():
    nb, loc = O.v5_board_geometry()
    assert nb.shape == (37, 6)
    edges = {(min(a, b), max(a, b)) for a in range(37) for b in nb[a] if b >= 0}
    assert len(edges) == 90  # a radius-3 hexagon: 3 n (3 n + 1) edges
    opposite = {0: 1, 1: 0, 2: 3, 3: 2, 4: 5, 5: 4}  # board.rs:14 direction pairs
    for a in range(37):
        for d in range(6):
            b = nb[a, d]
            if b >= 0:
                assert nb[b, opposite[d]] == a
    assert int((nb >= 0).all(axis=1).sum()) == 19  # the radius-2 interior
    assert loc.sum() == 10
    tnb, tloc = T.board()
    np.testing.assert_array_equal(np.where(nb < 0, 37, nb), tnb)
    np.testing.assert_array_equal(loc, tloc)


def test_gelu_closed_form_and_tanh():
    xs = np.concatenate([np.linspace(-12, 12, 4001), [0.0, 1e-6, -1e-6, 30.0, -30.0]]).astype(np.float32)
    own = np.array([O.v5_gelu(x) for x in xs])
    libm = np.array([O.v5_gelu(x, libm=True) for x in xs])
    exact = np.array([0.5 * float(x) * (1.0 + math.tanh(math.sqrt(2.0 / math.pi) * (float(x) + 0.044715 * float(x) ** 3)))
                      for x in xs])
    # float32 evaluation of 0.5 x (1 + tanh u): about one rounding of (1 + tanh u), times |x| / 2
    scale = np.maximum(np.abs(xs.astype(np.float64)), 1.0)
    assert np.max(np.abs(own - exact) / scale) < 2e-7
    assert np.max(np.abs(libm - exact) / scale) < 2e-7
    # the two tanh evaluations differ by a few units of float32 rounding at most
    assert np.max(np.abs(own - libm) / scale) < 2e-7


def piece_inputs(job):
    d = wcj8.decode(job)
    return d["card_feat"], d["leaf_raw"].reshape(-1, 201), d["cphi"].reshape(-1, 15), d["cplayer"]


def close(got, want, tol, tag):
    want = np.asarray(want, np.float64)
    scale = max(float(np.abs(want).max()), 1.0)
    err = float(np.abs(np.asarray(got, np.float64) - want).max()) / scale
    print(f"{tag}: max error {err:.2e} of the largest magnitude")
    assert err < tol, tag


def test_pieces_match_the_torch_float64_restatement(net):
    blob = T.Blob(net)
    for job in v5_jobs(trees=2):
        cf, raw, phi, owner = piece_inputs(job)
        crd = O.v5_cards(net, cf)
        tcrd = T.cards(blob, cf)
        close(crd, tcrd.numpy(), 1e-5, "cards")
        P, Jp = O.v5_board(net, raw, crd)
        tP, tJp = T.board_vectors(blob, raw, tcrd)
        close(P, tP.numpy(), 1e-4, "board vector P")
        close(Jp, tJp.numpy(), 1e-4, "join cache Jp")
        f, g = O.v5_configs(net, phi, owner, crd)
        tf, tg = T.configs(blob, phi, owner, tcrd)
        close(f, tf.numpy(), 1e-5, "config f")
        close(g, tg.numpy(), 1e-5, "config g")
        rng = np.random.default_rng(5)
        pooled = rng.random((P.shape[0], 2, 64)).astype(np.float32)
        for player in (0, 1):
            h = O.v5_join(net, P, Jp, pooled, player)
            th = T.join(blob, P, Jp, pooled, player)
            close(h, th.numpy(), 1e-4, f"join h (player {player})")
            v = T.values(blob, f, h).numpy()
            ov = np.array([[np.float32(blob.value_bias) + np.dot(f[c].astype(np.float64), h[r].astype(np.float64))
                            for c in range(len(f))] for r in range(len(h))])
            close(ov, v, 1e-6, "readout")


def test_zero_network_values_every_leaf_at_value_bias(net):
    w = np.zeros_like(net.w)
    b = np.zeros_like(net.b)
    b[-1] = 0.375  # value_bias, the blob's last bias
    zero = ww.Net(list(net.dims), w, b, net.ln)
    for job in v5_jobs(trees=2, seed=13):
        for p in (0, 1):
            vals, _ = O.leaf_probe(job, zero, O.NET_F32, p)
            assert vals.size and np.all(vals == np.float32(0.375))


def test_config_encoder_ignores_slot_order(net):
    [job] = v5_jobs(trees=1, seed=17)
    cf, _, phi, owner = piece_inputs(job)
    crd = O.v5_cards(net, cf)
    f, g = O.v5_configs(net, phi, owner, crd)
    perm = np.array([3, 0, 4, 1, 2])
    # permute each seat's coin slots: the card table (physical types p*5 + k)
    # and every config's counts together
    cf2 = cf.reshape(10, 25).copy()
    for p in (0, 1):
        cf2[p * 5:(p + 1) * 5] = cf.reshape(10, 25)[p * 5 + perm]
    phi2 = phi.reshape(-1, 3, 5)[:, :, perm].reshape(-1, 15)
    crd2 = O.v5_cards(net, cf2.reshape(-1))
    f2, g2 = O.v5_configs(net, phi2, owner, crd2)
    close(f2, f, 1e-5, "f under a slot permutation")
    close(g2, g, 1e-5, "g under a slot permutation")


def test_own_tanh_against_the_c_librarys(net):
    """The restatement's tanh against the C library's tanhf (what the
    reference's CPU net calls through f32::tanh; its value is itself a
    property of the platform's libm). Leaf values agree within 1e-5 of the
    largest (a few float32 roundings, carried through eight residual blocks
    and their norms); over a 16-iteration solve the root values stay within 1e-5 of
    the largest, and the strategies within 1e-3: regret matching turns a
    last-bit change of a leaf value into a visible change of a strategy entry
    where two actions' regrets nearly tie."""
    for job in v5_jobs(trees=2, seed=19, iters=16):
        for p in (0, 1):
            own, _ = O.leaf_probe(job, net, O.NET_F32, p)
            with O.libm_tanh():
                ref, _ = O.leaf_probe(job, net, O.NET_F32, p)
            dv = float(np.abs(own - ref).max() / np.abs(ref).max())
            assert dv <= 1e-5, dv
        own = O.solve(job, net, O.NET_F32)
        with O.libm_tanh():
            ref = O.solve(job, net, O.NET_F32)
        ds = float(np.abs(own["strategy"] - ref["strategy"]).max())
        dr = float(np.abs(own["roots"] - ref["roots"]).max() / max(np.abs(ref["roots"]).max(), 1e-30))
        print(f"own vs libm tanh: leaf values {dv:.2e}, strategy {ds:.2e}, roots {dr:.2e}")
        assert ds <= 1e-3 and dr <= 1e-5


def test_reduced_models_track_float32(net):
    """The 16-bit operand models (what the device's fast path is held to) stay
    near float32 at the leaves: f16 within 1e-2 of the largest value, bf16
    within 5e-2."""
    [job] = v5_jobs(trees=1, seed=23)
    exact, _ = O.leaf_probe(job, net, O.NET_F32, 0)
    scale = float(np.abs(exact).max())
    for mode, tol in ((O.NET_F16, 1e-2), (O.NET_F16A, 1e-2), (O.NET_BF16, 5e-2)):
        got, _ = O.leaf_probe(job, net, mode, 0)
        err = float(np.abs(got - exact).max()) / scale
        print(f"mode {mode}: {err:.2e}")
        assert err < tol


def _median_rel(got, want):
    want = np.asarray(want, np.float64)
    return float(np.median(np.abs(np.asarray(got, np.float64) - want)) / max(float(np.abs(want).max()), 1e-30))


@pytest.mark.parametrize("kind,mode", [("f16", O.NET_F16), ("f16", O.NET_F16A), ("bf16", O.NET_BF16),
                                       ("bf16", O.NET_BF16A)])
def test_16bit_models_round_exactly_the_fast_products(net, kind, mode):
    """The oracle's 16-bit v5 models (what the device's fast path is held to)
    round the operands of exactly the products the reference runs on tensor
    cores (T.FAST): piece by piece, each model agrees with the float64 torch
    restatement that rounds those products' operands to a median of a few
    float32 roundings (<= 2e-7 of the largest value), while the same
    restatement with any one of those products left unrounded, the planted
    mistake, moves the piece it feeds by a median >= 5e-6 (measured 1.7e-5 ..
    7e-4). One trunk block is compared alone, on float32 inputs: through eight
    blocks a single activation that rounds to the neighbouring 16-bit value
    spreads to the level of the whole rounding effect."""
    [job] = v5_jobs(trees=1, seed=11)
    cf, raw, phi, owner = piece_inputs(job)
    crd32 = O.v5_cards(net, cf)
    P, Jp = O.v5_board(net, raw, crd32)
    pooled = np.random.default_rng(5).random((P.shape[0], 2, 64)).astype(np.float32)
    b32 = T.Blob(net)
    x = T.stem(b32, raw, T.cards(b32, cf))[0]
    for i in range(3):
        x = T.block(b32, i, x)
    x32 = x.numpy().astype(np.float32)
    tx = torch.tensor(x32.astype(np.float64))

    def pieces(blob):
        tf, tg = T.configs(blob, phi, owner, torch.tensor(crd32.astype(np.float64)))
        return {"cards": T.cards(blob, cf).numpy(), "f": tf.numpy(), "g": tg.numpy(),
                "block": T.block(blob, 3, tx).numpy(), "h": T.join(blob, P, Jp, pooled, 1).numpy()}

    f, g = O.v5_configs(net, phi, owner, crd32, mode)
    got = {"cards": O.v5_cards(net, cf, mode), "f": f, "g": g, "block": O.v5_block(net, x32, 3, mode),
           "h": O.v5_join(net, P, Jp, pooled, 1, mode)}
    want = pieces(T.Blob(net).round(kind))
    for k in got:
        e = _median_rel(got[k], want[k])
        print(f"{kind} model {mode}, {k}: median {e:.1e} of the largest value")
        assert e <= 2e-7, k
    feeds = {"card": ["cards"], "cfg1": ["f", "g"], "cfg_f": ["f"], "cfg_g": ["g"], "cfg_m": ["g"], "mix": ["block"],
             "out": ["block"], "poolm": ["block"], "join_b": ["h"], "join_w": ["h"], "join_out": ["h"]}
    for name, hit in feeds.items():
        planted = pieces(T.Blob(net).round(kind, T.FAST - {name}))
        for k in hit:
            e = _median_rel(got[k], planted[k])
            print(f"{kind} model {mode}, {name} left unrounded: {k} median {e:.1e}")
            assert e >= 5e-6, (name, k)
