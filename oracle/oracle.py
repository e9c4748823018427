"""ctypes loader for the oracle (test infrastructure; see oracle.c's header).

Only tests, the smoke check and the benchmark's CPU-baseline leg import this.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")

NET_EMPTY, NET_F32, NET_F16, NET_BF16 = 0, 1, 2, 3
# Further arithmetic models of the leaf net (oracle.c): f16 operands with a
# float32 sum in ascending k order; compensated f16 operand pairs (hi + lo);
# float32 operands with a wide sum.
NET_F16A, NET_F16X, NET_F32W = 4, 5, 6
# bfloat16 operands with float32 ascending sums (the v5 network only).
NET_BF16A = 7

_lib = None


class Shape(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "nodes", "ncells", "rows", "nterm", "ncfg", "reach_len", "nroots", "root_n0", "root_n1",
        "snapshot_configs", "carry_slots", "iters", "nlevels", "decision_nodes", "chance_nodes",
        "leaves")]


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = C.CDLL(LIB)
        u8p, f32p, u32p = C.POINTER(C.c_uint8), C.POINTER(C.c_float), C.POINTER(C.c_uint32)
        L.oracle_last_error.restype = C.c_char_p
        L.oracle_job_shape.argtypes = [u8p, C.c_size_t, C.POINTER(Shape)]
        L.oracle_solve.argtypes = [u8p, C.c_size_t, C.c_int, u32p, C.c_uint32, f32p, C.c_size_t, f32p,
                                   C.c_size_t, f32p, C.c_size_t, f32p, f32p, f32p, f32p]
        L.oracle_mlp.argtypes = [C.c_uint32, f32p, C.c_uint32, u32p, C.c_int, u32p, C.c_uint32, f32p,
                                 C.c_size_t, f32p, C.c_size_t, f32p, f32p]
        L.oracle_solve_batch.argtypes = [C.c_uint32, C.POINTER(u8p), C.POINTER(C.c_size_t), C.c_uint32,
                                         C.c_int, u32p, C.c_uint32, f32p, C.c_size_t, f32p, C.c_size_t,
                                         f32p, C.c_size_t, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
        L.oracle_solve_batch.restype = C.c_double
        L.oracle_mlp_batch.argtypes = [C.c_uint32, f32p, C.c_uint32, u32p, C.c_uint32, C.c_int, u32p,
                                       C.c_uint32, f32p, C.c_size_t, f32p, C.c_size_t, f32p]
        L.oracle_mlp_batch.restype = C.c_double
        L.oracle_leaf_probe.argtypes = [u8p, C.c_size_t, C.c_int, u32p, C.c_uint32, f32p, C.c_size_t, f32p,
                                        C.c_size_t, f32p, C.c_size_t, C.c_int, f32p, C.c_size_t,
                                        C.POINTER(C.c_size_t), f32p]
        L.oracle_leaf_counts.argtypes = [u8p, C.c_size_t, C.POINTER(C.c_size_t)]
        L.oracle_leaf_eval.argtypes = [u8p, C.c_size_t, C.c_int, u32p, C.c_uint32, f32p, C.c_size_t, f32p,
                                       C.c_size_t, f32p, C.c_size_t, C.c_int, f32p, f32p, f32p]
        L.oracle_solve_trace.argtypes = [u8p, C.c_size_t, C.c_int, u32p, C.c_uint32, f32p, C.c_size_t, f32p,
                                         C.c_size_t, f32p, C.c_size_t, f32p, f32p, f32p, f32p, f32p]
        L.oracle_solve_replay.argtypes = [u8p, C.c_size_t, f32p, C.c_size_t, f32p, C.c_size_t, f32p, f32p, f32p]
        net5 = [C.c_int, f32p, C.c_size_t, f32p, C.c_size_t, f32p, C.c_size_t, C.c_int]
        L.oracle_v5_sizes.argtypes = [C.POINTER(C.c_size_t)] * 3
        L.oracle_v5_cards.argtypes = net5 + [f32p, f32p]
        L.oracle_v5_board.argtypes = net5 + [u8p, C.c_uint32, f32p, f32p, f32p]
        L.oracle_v5_configs.argtypes = net5 + [f32p, u8p, C.c_uint32, f32p, f32p, f32p]
        L.oracle_v5_join.argtypes = net5 + [f32p, f32p, f32p, C.c_uint32, C.c_int, f32p]
        L.oracle_v5_block.argtypes = net5 + [f32p, C.c_uint32, C.c_int]
        L.oracle_v5_gelu.argtypes = [C.c_float, C.c_int]
        L.oracle_v5_gelu.restype = C.c_float
        L.oracle_v5_set_libm_tanh.argtypes = [C.c_int]
        L.oracle_v5_board_geometry.argtypes = [C.POINTER(C.c_int32), f32p]
        L.oracle_factor.argtypes = [C.c_float, C.c_float]
        L.oracle_factor.restype = C.c_float
        L.oracle_round_f16.argtypes = [C.c_float]
        L.oracle_round_f16.restype = C.c_float
        L.oracle_round_bf16.argtypes = [C.c_float]
        L.oracle_round_bf16.restype = C.c_float
        _lib = L
    return _lib


def _p(a, ctype):
    return a.ctypes.data_as(C.POINTER(ctype))


def _err():
    return lib().oracle_last_error().decode(errors="replace")


def shape(job: bytes) -> Shape:
    s = Shape()
    buf = (C.c_uint8 * len(job)).from_buffer_copy(job)
    if lib().oracle_job_shape(buf, len(job), C.byref(s)) != 0:
        raise ValueError(_err())
    return s


def _net_args(net, mode):
    if net is None or mode == NET_EMPTY:
        z = np.zeros(1, np.float32)
        d = np.zeros(1, np.uint32)
        return d, 0, z, 0, z, 0
    d = np.ascontiguousarray(net.dims, np.uint32)
    w = np.ascontiguousarray(net.w, np.float32)
    b = np.ascontiguousarray(net.b, np.float32)
    return d, len(d), w, w.size, b, b.size


def _ln_args(net, mode):
    ln = getattr(net, "ln", None) if net is not None and mode != NET_EMPTY else None
    if ln is None or len(ln) == 0:
        return None, 0
    ln = np.ascontiguousarray(ln, np.float32)
    return ln, ln.size


def solve(job: bytes, net=None, mode=NET_F32, conv=False):
    """Solve one job on the CPU: returns dict(strategy, roots [nroots, n0+n1], carries
    [slots, snapshot_configs], conv (nash, zero_sum) or None)."""
    s = shape(job)
    strategy = np.zeros(max(s.ncells, 1), np.float32)
    roots = np.zeros(max(s.nroots * (s.root_n0 + s.root_n1), 1), np.float32)
    carries = np.zeros(max(s.carry_slots * s.snapshot_configs, 1), np.float32)
    cv = np.zeros(2, np.float32)
    d, nd, w, nw, b, nb = _net_args(net, mode)
    ln, nln = _ln_args(net, mode)
    buf = (C.c_uint8 * len(job)).from_buffer_copy(job)
    rc = lib().oracle_solve(buf, len(job), mode, _p(d, C.c_uint32), nd, _p(w, C.c_float), nw,
                            _p(b, C.c_float), nb, _p(ln, C.c_float) if nln else None, nln,
                            _p(strategy, C.c_float), _p(roots, C.c_float),
                            _p(carries, C.c_float), _p(cv, C.c_float) if conv else None)
    if rc != 0:
        raise ValueError(_err())
    return {
        "strategy": strategy[: s.ncells],
        "roots": roots[: s.nroots * (s.root_n0 + s.root_n1)].reshape(s.nroots, s.root_n0 + s.root_n1),
        "carries": carries[: s.carry_slots * s.snapshot_configs].reshape(s.carry_slots, s.snapshot_configs),
        "conv": (float(cv[0]), float(cv[1])) if conv else None,
        "shape": s,
    }


def leaf_probe(job: bytes, net, mode, traverser):
    """The leaf net's values at the initial reach for `traverser` (oracle_leaf_probe):
    (values: each network row's configs of the traverser in row order, concatenated;
    mass: [rows, 2] reach masses)."""
    s = shape(job)
    d, nd, w, nw, b, nb = _net_args(net, mode)
    ln, nln = _ln_args(net, mode)
    lnp = _p(ln, C.c_float) if nln else None
    buf = (C.c_uint8 * len(job)).from_buffer_copy(job)
    count = C.c_size_t()
    mass = np.zeros((max(s.rows, 1), 2), np.float32)
    rc = lib().oracle_leaf_probe(buf, len(job), mode, _p(d, C.c_uint32), nd, _p(w, C.c_float), nw,
                                 _p(b, C.c_float), nb, lnp, nln, traverser, None, 0, C.byref(count), None)
    if rc != 0:
        raise ValueError(_err())
    vals = np.zeros(max(count.value, 1), np.float32)
    rc = lib().oracle_leaf_probe(buf, len(job), mode, _p(d, C.c_uint32), nd, _p(w, C.c_float), nw,
                                 _p(b, C.c_float), nb, lnp, nln, traverser, _p(vals, C.c_float), vals.size,
                                 C.byref(count), _p(mass, C.c_float))
    if rc != 0:
        raise ValueError(_err())
    return vals[: count.value], mass[: s.rows]


def mlp(x: np.ndarray, keys: np.ndarray, net, mode=NET_F32, want_h=False):
    x = np.ascontiguousarray(x, np.float32)
    keys = np.ascontiguousarray(keys, np.uint32)
    rows, nk = keys.shape
    out = np.zeros((rows, nk), np.float32)
    hidden = net.dims[2]
    h = np.zeros((rows, hidden), np.float32) if want_h else None
    d, nd, w, nw, b, nb = _net_args(net, mode)
    rc = lib().oracle_mlp(rows, _p(x, C.c_float), nk, _p(keys, C.c_uint32), mode, _p(d, C.c_uint32), nd,
                          _p(w, C.c_float), nw, _p(b, C.c_float), nb, _p(out, C.c_float),
                          _p(h, C.c_float) if want_h else None)
    if rc != 0:
        raise ValueError(_err())
    return (out, h) if want_h else out


def solve_batch(jobs, net, mode=NET_F32, threads=1):
    """Time `jobs` solved one per thread on `threads` threads: (seconds, node_iters, leaf_queries)."""
    bufs = [(C.c_uint8 * len(j)).from_buffer_copy(j) for j in jobs]
    u8p = C.POINTER(C.c_uint8)
    ptrs = (u8p * len(jobs))(*[C.cast(b, u8p) for b in bufs])
    lens = (C.c_size_t * len(jobs))(*[len(j) for j in jobs])
    d, nd, w, nw, b, nb = _net_args(net, mode)
    ln, nln = _ln_args(net, mode)
    ni, lq = C.c_uint64(), C.c_uint64()
    sec = lib().oracle_solve_batch(len(jobs), ptrs, lens, threads, mode, _p(d, C.c_uint32), nd,
                                   _p(w, C.c_float), nw, _p(b, C.c_float), nb, _p(ln, C.c_float) if nln else None,
                                   nln, C.byref(ni), C.byref(lq))
    if sec < 0:
        raise ValueError(_err())
    return sec, ni.value, lq.value


def mlp_batch(x, heads, net, mode=NET_F32, threads=1):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros((x.shape[0], heads), np.float32)
    d, nd, w, nw, b, nb = _net_args(net, mode)
    sec = lib().oracle_mlp_batch(x.shape[0], _p(x, C.c_float), heads, None, threads, mode,
                                 _p(d, C.c_uint32), nd, _p(w, C.c_float), nw, _p(b, C.c_float), nb,
                                 _p(out, C.c_float))
    if sec < 0:
        raise ValueError(_err())
    return sec, out


def factor(t, p):
    return lib().oracle_factor(t, p)


def round_f16(x):
    return lib().oracle_round_f16(x)


def round_bf16(x):
    return lib().oracle_round_bf16(x)


# ------------------------------------------------------------ the v5 network

V5 = dict(TYPE=64, C=96, BLOCKS=8, D=256, POOL=64, CFGH=128, JW=128, JBLOCKS=3, JOIN_IN=129, HEXES=37, NSLOT=5,
          NTYPE=10, HEX_FACTS=6, PILE_COUNTS=4, CARD_FEATS=25, CFEAT=15, LOOSE=15, ROW_BYTES=201)


def v5_sizes():
    n = [C.c_size_t() for _ in range(3)]
    lib().oracle_v5_sizes(*[C.byref(x) for x in n])
    return tuple(x.value for x in n)


def _v5_net(net, mode, libm):
    w = np.ascontiguousarray(net.w, np.float32)
    b = np.ascontiguousarray(net.b, np.float32)
    ln = np.ascontiguousarray(net.ln, np.float32)
    keep = (w, b, ln)
    return keep, [mode, _p(w, C.c_float), w.size, _p(b, C.c_float), b.size, _p(ln, C.c_float), ln.size, int(libm)]


def v5_cards(net, card_feat, mode=NET_F32, libm=False):
    """Net::cards for both seat views: [2, NTYPE, TYPE]."""
    keep, a = _v5_net(net, mode, libm)
    cf = np.ascontiguousarray(card_feat, np.float32)
    out = np.zeros((2, V5["NTYPE"], V5["TYPE"]), np.float32)
    if lib().oracle_v5_cards(*a, _p(cf, C.c_float), _p(out, C.c_float)) != 0:
        raise ValueError("v5 cards")
    return out


def v5_board(net, raw, cards, mode=NET_F32, libm=False):
    """Net::board + join_cache per row: (P [rows, D], Jp [rows, JW])."""
    keep, a = _v5_net(net, mode, libm)
    raw = np.ascontiguousarray(raw, np.uint8).reshape(-1, V5["ROW_BYTES"])
    cards = np.ascontiguousarray(cards, np.float32)
    P = np.zeros((raw.shape[0], V5["D"]), np.float32)
    Jp = np.zeros((raw.shape[0], V5["JW"]), np.float32)
    if lib().oracle_v5_board(*a, _p(raw, C.c_uint8), raw.shape[0], _p(cards, C.c_float), _p(P, C.c_float),
                             _p(Jp, C.c_float)) != 0:
        raise ValueError("v5 board")
    return P, Jp


def v5_configs(net, phi, owner, cards, mode=NET_F32, libm=False):
    """Net::configs: (f [ncfg, D], g [ncfg, POOL])."""
    keep, a = _v5_net(net, mode, libm)
    phi = np.ascontiguousarray(phi, np.float32).reshape(-1, V5["CFEAT"])
    owner = np.ascontiguousarray(owner, np.uint8)
    cards = np.ascontiguousarray(cards, np.float32)
    f = np.zeros((phi.shape[0], V5["D"]), np.float32)
    g = np.zeros((phi.shape[0], V5["POOL"]), np.float32)
    if lib().oracle_v5_configs(*a, _p(phi, C.c_float), _p(owner, C.c_uint8), phi.shape[0], _p(cards, C.c_float),
                               _p(f, C.c_float), _p(g, C.c_float)) != 0:
        raise ValueError("v5 configs")
    return f, g


def v5_join(net, P, Jp, pooled, player, mode=NET_F32, libm=False):
    """Net::join per row: h [rows, D]; pooled [rows, 2, POOL] with the player's block first."""
    keep, a = _v5_net(net, mode, libm)
    P = np.ascontiguousarray(P, np.float32)
    Jp = np.ascontiguousarray(Jp, np.float32)
    pooled = np.ascontiguousarray(pooled, np.float32)
    h = np.zeros((P.shape[0], V5["D"]), np.float32)
    if lib().oracle_v5_join(*a, _p(P, C.c_float), _p(Jp, C.c_float), _p(pooled, C.c_float), P.shape[0], player,
                            _p(h, C.c_float)) != 0:
        raise ValueError("v5 join")
    return h


def v5_block(net, x, block, mode=NET_F32, libm=False):
    """One residual block of the board trunk on x [rows, 37, 96]: the block's output."""
    keep, a = _v5_net(net, mode, libm)
    out = np.array(x, np.float32, copy=True, order="C")
    if lib().oracle_v5_block(*a, _p(out, C.c_float), out.shape[0], int(block)) != 0:
        raise ValueError("v5 block")
    return out


def v5_gelu(x, libm=False):
    return lib().oracle_v5_gelu(float(x), int(libm))


def v5_board_geometry():
    nb = np.zeros(37 * 6, np.int32)
    loc = np.zeros(37, np.float32)
    lib().oracle_v5_board_geometry(nb.ctypes.data_as(C.POINTER(C.c_int32)), _p(loc, C.c_float))
    return nb.reshape(37, 6), loc


class libm_tanh:
    """Context manager: the v5 restatement's GELU calls the C library's tanhf."""

    def __enter__(self):
        lib().oracle_v5_set_libm_tanh(1)

    def __exit__(self, *a):
        lib().oracle_v5_set_libm_tanh(0)


def leaf_counts(job: bytes):
    """(values of traverser 0, values of traverser 1, network rows, reach floats) that
    one leaf evaluation of this job takes or gives (oracle_leaf_counts)."""
    out = (C.c_size_t * 4)()
    buf = (C.c_uint8 * len(job)).from_buffer_copy(job)
    if lib().oracle_leaf_counts(buf, len(job), out) != 0:
        raise ValueError(_err())
    return int(out[0]), int(out[1]), int(out[2]), int(out[3])


def leaf_eval(job: bytes, net, mode, traverser, reach):
    """The leaf net's values for `traverser` at a given reach of the job's network rows
    (per row, player 0's configs then player 1's), and the rows' masses [rows, 2]."""
    n0, n1, rows, nreach = leaf_counts(job)
    reach = np.ascontiguousarray(reach, np.float32)
    if reach.size != nreach:
        raise ValueError(f"reach holds {reach.size} floats, the job's rows take {nreach}")
    vals = np.zeros(max(n1 if traverser else n0, 1), np.float32)
    mass = np.zeros(max(2 * rows, 1), np.float32)
    d, nd, w, nw, b, nb = _net_args(net, mode)
    ln, nln = _ln_args(net, mode)
    buf = (C.c_uint8 * len(job)).from_buffer_copy(job)
    rc = lib().oracle_leaf_eval(buf, len(job), mode, _p(d, C.c_uint32), nd, _p(w, C.c_float), nw,
                                _p(b, C.c_float), nb, _p(ln, C.c_float) if nln else None, nln, traverser,
                                _p(reach if reach.size else np.zeros(1, np.float32), C.c_float),
                                _p(vals, C.c_float), _p(mass, C.c_float))
    if rc != 0:
        raise ValueError(_err())
    return vals[: n1 if traverser else n0], mass[: 2 * rows].reshape(rows, 2)


def solve_replay(job: bytes, vals, mass):
    """oracle_solve with every network leaf's value given (oracle_solve_replay): vals
    and mass concatenated over the job's leaf-net evaluations in schedule order
    (iterations, then per carried root players 0 and 1)."""
    s = shape(job)
    vals = np.ascontiguousarray(vals, np.float32)
    mass = np.ascontiguousarray(mass, np.float32)
    strategy = np.zeros(max(s.ncells, 1), np.float32)
    roots = np.zeros(max(s.nroots * (s.root_n0 + s.root_n1), 1), np.float32)
    carries = np.zeros(max(s.carry_slots * s.snapshot_configs, 1), np.float32)
    buf = (C.c_uint8 * len(job)).from_buffer_copy(job)
    one = np.zeros(1, np.float32)
    rc = lib().oracle_solve_replay(buf, len(job), _p(vals if vals.size else one, C.c_float), vals.size,
                                   _p(mass if mass.size else one, C.c_float), mass.size,
                                   _p(strategy, C.c_float), _p(roots, C.c_float), _p(carries, C.c_float))
    if rc != 0:
        raise ValueError(_err())
    return {
        "strategy": strategy[: s.ncells],
        "roots": roots[: s.nroots * (s.root_n0 + s.root_n1)].reshape(s.nroots, s.root_n0 + s.root_n1),
        "carries": carries[: s.carry_slots * s.snapshot_configs].reshape(s.carry_slots, s.snapshot_configs),
        "shape": s,
    }


def replay_sizes(job: bytes):
    """(values, masses) a replay of this job takes: per leaf-net evaluation in
    schedule order (iterations, then per carried root players 0 and 1)."""
    s = shape(job)
    n0, n1, rows, _ = leaf_counts(job)
    trav = [t % 2 for t in range(s.iters)] + [p for _ in range(s.nroots) for p in (0, 1)]
    return sum(n1 if p else n0 for p in trav), 2 * rows * len(trav)


def solve_trace(job: bytes, net, mode=NET_F32):
    """oracle_solve recording every leaf-net evaluation's values and masses in the
    layout solve_replay takes, and the reach that fed each one (per evaluation, per
    row, player 0's configs then player 1's): dict(vals, mass, reach, strategy, roots)."""
    s = shape(job)
    nv, nm = replay_sizes(job)
    nreach = leaf_counts(job)[3] * (s.iters + 2 * s.nroots)
    vals = np.zeros(max(nv, 1), np.float32)
    mass = np.zeros(max(nm, 1), np.float32)
    reach = np.zeros(max(nreach, 1), np.float32)
    strategy = np.zeros(max(s.ncells, 1), np.float32)
    roots = np.zeros(max(s.nroots * (s.root_n0 + s.root_n1), 1), np.float32)
    d, nd, w, nw, b, nb = _net_args(net, mode)
    ln, nln = _ln_args(net, mode)
    buf = (C.c_uint8 * len(job)).from_buffer_copy(job)
    rc = lib().oracle_solve_trace(buf, len(job), mode, _p(d, C.c_uint32), nd, _p(w, C.c_float), nw,
                                  _p(b, C.c_float), nb, _p(ln, C.c_float) if nln else None, nln,
                                  _p(vals, C.c_float), _p(mass, C.c_float), _p(reach, C.c_float),
                                  _p(strategy, C.c_float), _p(roots, C.c_float))
    if rc != 0:
        raise ValueError(_err())
    return {"vals": vals[:nv], "mass": mass[:nm], "reach": reach[:nreach], "strategy": strategy[: s.ncells],
            "roots": roots[: s.nroots * (s.root_n0 + s.root_n1)].reshape(s.nroots, s.root_n0 + s.root_n1)}
