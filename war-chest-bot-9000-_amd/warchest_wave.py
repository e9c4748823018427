"""Python host binding of the MI355X wave executor's C ABI (include/wc_wave.h).

The names mirror the reference client surface (engine/src/gpu/client.rs,
service.rs): `spawn` returns a `GpuClient` with `submit`, `submit_tagged`,
`set_weights`, `queued_work`; `SolveHandle.wait()` returns a `SolveResult`.
Lower-level `Executor` / `Wave` objects mirror `Executor` and `Wave::pack`
(engine/src/gpu/device.rs:515-831, wave.rs:127-221) for tests and benchmarks.

Nothing here computes: every call goes through the native library, and loading
fails loudly when it is missing (build it with `python build.py`).
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libwcwave.so")

WC_PRECISE, WC_F16, WC_BF16, WC_F16X = 0, 1, 2, 3
MODEL_V5, MODEL_MLP, MODEL_TWO_TOWER = 5, 101, 102

_lib = None


def phase2_point(root: int, p: int) -> int:
    """The schedule point of Phase 2's leaf-net evaluation for carried root `root`
    and player p (Executor.leaf_trace)."""
    return -(1 + 2 * root + p)


class WaveError(RuntimeError):
    pass


def lib():
    """Load the native library (once). Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise WaveError(f"native library missing: {LIB_PATH} (run build.py)")
    L = C.CDLL(LIB_PATH)
    _declare(L)
    _lib = L
    return L


class NetDesc(C.Structure):
    _fields_ = [
        ("dims", C.POINTER(C.c_uint32)), ("ndims", C.c_uint32),
        ("w", C.POINTER(C.c_float)), ("nw", C.c_size_t),
        ("b", C.POINTER(C.c_float)), ("nb", C.c_size_t),
        ("ln", C.POINTER(C.c_float)), ("nln", C.c_size_t),
    ]


class ServiceOpts(C.Structure):
    _fields_ = [("lanes", C.c_uint32), ("wave_jobs", C.c_uint32),
                ("wave_rows", C.c_uint32), ("window_us", C.c_uint32),
                ("whale_lanes", C.c_uint32), ("class_shift", C.c_uint32), ("route_unit", C.c_uint64)]


class WorkVectorC(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "network_rows", "legal_cells", "reach_slots", "reverse_nonzeros", "table_bytes", "mutable_bytes",
        "carried_output_bytes", "levels", "reserved_bytes")] + [
        (n, C.c_uint32) for n in ("exclusive_route", "arena_guard_route", "card_exclusive_route")]


class SynthSpecC(C.Structure):
    _fields_ = [
        ("seed", C.c_uint64), ("trees", C.c_uint32),
        ("nodes_lo", C.c_uint32), ("nodes_hi", C.c_uint32),
        ("exact_decisions", C.c_uint32), ("exact_leaves", C.c_uint32),
        ("act_lo", C.c_uint32), ("act_hi", C.c_uint32),
        ("collapse", C.c_float), ("chance", C.c_uint32),
        ("draw_lo", C.c_uint32), ("draw_hi", C.c_uint32),
        ("info_fixed", C.c_uint32), ("info_median", C.c_float), ("info_p99", C.c_float),
        ("info_cap", C.c_uint32),
        ("legal_p", C.c_float), ("shift_p", C.c_float), ("notrans_p", C.c_float),
        ("terminal_p", C.c_float),
        ("dirichlet", C.c_uint32), ("nroots", C.c_uint32),
        ("whale_frac", C.c_float), ("whale_nodes", C.c_uint32), ("whale_info", C.c_uint32),
        ("depth", C.c_uint32), ("iters", C.c_uint32), ("snapshots", C.c_uint32),
        ("alpha", C.c_float), ("beta", C.c_float), ("gamma", C.c_float), ("predict", C.c_float),
        ("net_dims", C.POINTER(C.c_uint32)), ("n_net_dims", C.c_uint32),
    ]


class WaveStats(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "jobs", "nodes", "decision_nodes", "chance_nodes", "leaves", "rows", "terminals",
        "levels", "iters", "nroots_max", "carry_slots", "units", "top_levels", "max_window")] + [(n, C.c_uint64) for n in (
        "cells", "reach_slots", "reach_len", "vals_len", "rev_nnz", "rvd_nnz", "draw_nnz",
        "snapshot_configs", "table_bytes", "arena_bytes")] + [
        ("cfr_bytes_per_iter", C.c_uint64 * 2), ("cfr_bytes_by_kernel", (C.c_uint64 * 4) * 2),
        ("mlp_flops_per_query", C.c_uint64), ("mlp_flops_executed", C.c_uint64),
        ("mlp_flops_algorithmic", C.c_uint64), ("leaf_input_bytes", C.c_uint64 * 2)]

    def as_dict(self):
        out = {}
        for name, _ in self._fields_:
            v = getattr(self, name)
            if name in ("cfr_bytes_per_iter", "leaf_input_bytes"):
                out[name] = list(v)
            elif name == "cfr_bytes_by_kernel":
                out[name] = [list(r) for r in v]
            else:
                out[name] = int(v)
        return out


# Symbols every build must export (checked by the CPU test suite).
EXPORTS = [
    "wc_last_error", "wc_net_sizes", "wc_net_norms",
    "wc_service_create", "wc_service_destroy", "wc_set_weights", "wc_queued_work",
    "wc_submit", "wc_wait", "wc_poll", "wc_ticket_free", "wc_service_stats", "wc_job_work",
    "wc_prepare", "wc_prepared_cost", "wc_prepared_free", "wc_submit_prepared",
    "wc_result_tag", "wc_result_weight_version", "wc_result_strategy", "wc_result_root_values",
    "wc_result_carries", "wc_result_routes", "wc_result_free",
    "wc_executor_create", "wc_executor_destroy", "wc_executor_publish",
    "wc_wave_pack", "wc_wave_repack", "wc_wave_digest", "wc_wave_free", "wc_wave_stats_get", "wc_wave_array",
    "wc_wave_poke", "wc_wave_check", "wc_value_net_plan", "wc_solve_wave",
    "wc_launch", "wc_inflight_ready", "wc_collect", "wc_wave_leaf_probe", "wc_wave_leaf_trace",
    "wc_time_wave", "wc_peak_probe",
    "wc_mlp_forward", "wc_mlp_forward_noalloc", "wc_time_mlp",
    "wc_job_roundtrip", "wc_job_validate",
    "wc_synth_spec_default", "wc_synth", "wc_jobset_count", "wc_jobset_job", "wc_jobset_free",
    "wc_synth_weights", "wc_synth_norms", "wc_synth_features",
]

_u8p = C.POINTER(C.c_uint8)
_f32p = C.POINTER(C.c_float)
_u32p = C.POINTER(C.c_uint32)
_u16p = C.POINTER(C.c_uint16)


def _declare(L):
    L.wc_last_error.restype = C.c_char_p
    L.wc_net_sizes.argtypes = [_u32p, C.c_uint32, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    L.wc_net_norms.argtypes = [_u32p, C.c_uint32, C.POINTER(C.c_size_t)]
    L.wc_service_create.argtypes = [C.c_int, C.POINTER(NetDesc), C.c_int, C.POINTER(ServiceOpts),
                                    C.POINTER(C.c_void_p)]
    L.wc_service_destroy.argtypes = [C.c_void_p]
    L.wc_service_destroy.restype = None
    L.wc_set_weights.argtypes = [C.c_void_p, C.POINTER(NetDesc)]
    L.wc_set_weights.restype = C.c_uint64
    L.wc_queued_work.argtypes = [C.c_void_p]
    L.wc_queued_work.restype = C.c_uint64
    L.wc_submit.argtypes = [C.c_void_p, _u8p, C.c_size_t, C.c_uint64, C.POINTER(C.c_void_p)]
    L.wc_wait.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    L.wc_prepare.argtypes = [_u8p, C.c_size_t, C.c_int, C.POINTER(C.c_void_p)]
    L.wc_prepared_cost.argtypes = [C.c_void_p]
    L.wc_prepared_cost.restype = C.c_uint64
    L.wc_prepared_free.argtypes = [C.c_void_p]
    L.wc_prepared_free.restype = None
    L.wc_submit_prepared.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.POINTER(C.c_void_p)]
    L.wc_poll.argtypes = [C.c_void_p]
    L.wc_ticket_free.argtypes = [C.c_void_p]
    L.wc_ticket_free.restype = None
    L.wc_service_stats.argtypes = [C.c_void_p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
    L.wc_job_work.argtypes = [_u8p, C.c_size_t, C.c_int, C.c_uint64, C.c_uint32, C.POINTER(WorkVectorC),
                              C.POINTER(C.c_uint64), C.POINTER(C.c_uint32)]
    L.wc_result_routes.argtypes = [C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_int)]
    L.wc_launch.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.POINTER(C.c_void_p)]
    L.wc_inflight_ready.argtypes = [C.c_void_p, C.c_void_p]
    L.wc_collect.argtypes = [C.c_void_p, C.c_void_p, C.POINTER(C.c_void_p)]
    L.wc_wave_leaf_probe.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_int, _f32p, C.c_size_t,
                                     C.POINTER(C.c_size_t), _f32p]
    L.wc_wave_leaf_trace.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.POINTER(C.c_int32), C.c_size_t,
                                     _f32p, C.c_size_t, _f32p, C.c_size_t, _f32p, C.c_size_t,
                                     C.POINTER(C.c_size_t)]
    L.wc_result_tag.argtypes = [C.c_void_p]
    L.wc_result_tag.restype = C.c_uint64
    L.wc_result_weight_version.argtypes = [C.c_void_p]
    L.wc_result_weight_version.restype = C.c_uint64
    L.wc_result_strategy.argtypes = [C.c_void_p, C.POINTER(C.c_size_t)]
    L.wc_result_strategy.restype = _f32p
    L.wc_result_root_values.argtypes = [C.c_void_p, _u32p, _u32p, _u32p]
    L.wc_result_root_values.restype = _f32p
    L.wc_result_carries.argtypes = [C.c_void_p, _u32p, _u32p]
    L.wc_result_carries.restype = _u16p
    L.wc_result_free.argtypes = [C.c_void_p]
    L.wc_result_free.restype = None
    L.wc_executor_create.argtypes = [C.c_int, C.c_int, C.POINTER(C.c_void_p)]
    L.wc_executor_destroy.argtypes = [C.c_void_p]
    L.wc_executor_destroy.restype = None
    L.wc_executor_publish.argtypes = [C.c_void_p, C.POINTER(NetDesc)]
    L.wc_executor_publish.restype = C.c_uint64
    L.wc_wave_pack.argtypes = [C.POINTER(_u8p), C.POINTER(C.c_size_t), C.c_uint32, C.POINTER(C.c_void_p)]
    L.wc_wave_repack.argtypes = [C.c_void_p, C.POINTER(_u8p), C.POINTER(C.c_size_t), C.c_uint32]
    L.wc_wave_digest.argtypes = [C.c_void_p, C.POINTER(C.c_uint64)]
    L.wc_wave_free.argtypes = [C.c_void_p]
    L.wc_wave_free.restype = None
    L.wc_wave_stats_get.argtypes = [C.c_void_p, C.POINTER(WaveStats)]
    L.wc_wave_array.argtypes = [C.c_void_p, C.c_char_p, C.POINTER(C.c_size_t)]
    L.wc_wave_array.restype = _u32p
    L.wc_wave_poke.argtypes = [C.c_void_p, C.c_char_p, C.c_size_t, C.c_uint32]
    L.wc_wave_check.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64]
    L.wc_value_net_plan.argtypes = [C.POINTER(C.c_uint32), C.c_uint32, C.c_uint32, C.c_uint32,
                                    C.POINTER(C.c_uint32), C.c_size_t, C.POINTER(C.c_size_t)]
    L.wc_solve_wave.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.POINTER(C.c_void_p)]
    L.wc_time_wave.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint32, C.c_uint32,
                               C.POINTER(C.c_double), C.POINTER(C.c_double)]
    L.wc_peak_probe.argtypes = [C.c_int, C.c_size_t] + [C.POINTER(C.c_double)] * 4
    L.wc_mlp_forward.argtypes = [C.c_void_p, C.c_uint64, C.c_uint32, _f32p, _f32p]
    L.wc_mlp_forward_noalloc.argtypes = [C.c_void_p, C.c_uint64, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p]
    L.wc_time_mlp.argtypes = [C.c_void_p, C.c_uint64, C.c_uint32, _f32p, C.c_uint32,
                              C.POINTER(C.c_double), C.POINTER(C.c_double)]
    L.wc_job_roundtrip.argtypes = [_u8p, C.c_size_t, _u8p, C.c_size_t, C.POINTER(C.c_size_t)]
    L.wc_job_validate.argtypes = [_u8p, C.c_size_t]
    L.wc_synth_spec_default.argtypes = [C.POINTER(SynthSpecC)]
    L.wc_synth_spec_default.restype = None
    L.wc_synth.argtypes = [C.POINTER(SynthSpecC), C.POINTER(C.c_void_p)]
    L.wc_jobset_count.argtypes = [C.c_void_p]
    L.wc_jobset_count.restype = C.c_uint32
    L.wc_jobset_job.argtypes = [C.c_void_p, C.c_uint32, C.POINTER(C.c_size_t)]
    L.wc_jobset_job.restype = _u8p
    L.wc_jobset_free.argtypes = [C.c_void_p]
    L.wc_jobset_free.restype = None
    L.wc_synth_weights.argtypes = [_u32p, C.c_uint32, C.c_uint64, _f32p, C.c_size_t, _f32p, C.c_size_t]
    L.wc_synth_norms.argtypes = [_u32p, C.c_uint32, C.c_uint64, _f32p, C.c_size_t]
    L.wc_synth_features.argtypes = [C.c_uint32, C.c_uint32, C.c_uint64, _f32p]


def _check(rc):
    if rc != 0:
        raise WaveError(lib().wc_last_error().decode(errors="replace") or f"error {rc}")


def _bytes_ptr(b):
    """A uint8 pointer to the bytes of `b` and the object that keeps them alive.
    An immutable `bytes` is passed in place (the library copies what it keeps
    during the call); other buffers are copied first."""
    if isinstance(b, bytes):
        return b, C.cast(C.c_char_p(b), _u8p)
    buf = (C.c_uint8 * len(b)).from_buffer_copy(b)
    return buf, C.cast(buf, _u8p)


def _arr(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    ctype = {np.float32: C.c_float, np.uint32: C.c_uint32}[dtype]
    return a, a.ctypes.data_as(C.POINTER(ctype))


# ------------------------------------------------------------------ networks

def value_net_plan(cols, cus, heads=None):
    """The fused value net's passes (wc_value_net_plan) for 16-row blocks of
    head widths `cols` (or, with cols an int, that many blocks of width
    `heads`) on `cus` compute units: a list of (head columns, [blocks]) in
    launch order."""
    if isinstance(cols, int):
        nrb, cp = cols, None
    else:
        a = np.ascontiguousarray(cols, dtype=np.uint32)
        nrb, cp = len(a), a.ctypes.data_as(C.POINTER(C.c_uint32))
        heads = int(a.max()) if heads is None and nrb else (heads or 0)
    n = C.c_size_t(0)
    _check(lib().wc_value_net_plan(cp, nrb, heads, cus, None, 0, C.byref(n)))
    out = np.zeros((max(n.value, 1), 10), dtype=np.uint32)
    _check(lib().wc_value_net_plan(cp, nrb, heads, cus, out.ctypes.data_as(C.POINTER(C.c_uint32)), n.value,
                                   C.byref(n)))
    return [(int(r[1]), [int(b) for b in r[2:2 + r[0]]]) for r in out[:n.value]]


def peak_probe(device=0, nbytes=1 << 30):
    """What the device sustains (wc_peak_probe): HBM copy and read GB/s over buffers of
    nbytes, and f16 MFMA TFLOP/s on register operands (32x32x16, and the 16x16x32
    instruction the fused value net issues)."""
    c, r, m, m16 = C.c_double(), C.c_double(), C.c_double(), C.c_double()
    _check(lib().wc_peak_probe(device, nbytes, C.byref(c), C.byref(r), C.byref(m), C.byref(m16)))
    return {"hbm_copy_gbs": c.value, "hbm_read_gbs": r.value, "mfma_f16_tflops": m.value,
            "mfma_f16_16x16x32_tflops": m16.value}


def mlp_dims(inputs=512, hidden=384, layers=3, heads=22, pool=64):
    return [MODEL_MLP, inputs, hidden, layers, heads, pool]


def two_tower_dims(inputs=512, width=512, pub_layers=2, priv_in=96, priv_layers=2, pool=64):
    return [MODEL_TWO_TOWER, inputs, width, pub_layers, priv_in, priv_layers, pool]


# The reference's production network (engine/src/net.rs:41 MODEL_TAG).
V5_DIMS = [MODEL_V5]


def net_sizes(dims):
    d, dp = _arr(dims, np.uint32)
    nw, nb = C.c_size_t(), C.c_size_t()
    _check(lib().wc_net_sizes(dp, len(d), C.byref(nw), C.byref(nb)))
    return nw.value, nb.value


def net_norms(dims):
    d, dp = _arr(dims, np.uint32)
    n = C.c_size_t()
    _check(lib().wc_net_norms(dp, len(d), C.byref(n)))
    return n.value


@dataclass
class Net:
    dims: list
    w: np.ndarray
    b: np.ndarray
    ln: np.ndarray = None  # v5: LayerNorm (gain, shift) pairs in application order

    def desc(self):
        """A NetDesc whose pointers stay valid while this object lives."""
        self._d, dp = _arr(self.dims, np.uint32)
        self._w, wp = _arr(self.w, np.float32)
        self._b, bp = _arr(self.b, np.float32)
        if self.ln is None or len(self.ln) == 0:
            return NetDesc(dp, len(self._d), wp, self._w.size, bp, self._b.size, None, 0)
        self._ln, lp = _arr(self.ln, np.float32)
        return NetDesc(dp, len(self._d), wp, self._w.size, bp, self._b.size, lp, self._ln.size)


def synth_weights(dims, seed=1):
    nw, nb = net_sizes(dims)
    w = np.zeros(nw, np.float32)
    b = np.zeros(nb, np.float32)
    d, dp = _arr(dims, np.uint32)
    _check(lib().wc_synth_weights(dp, len(d), seed, w.ctypes.data_as(_f32p), nw, b.ctypes.data_as(_f32p), nb))
    nln = net_norms(dims)
    if not nln:
        return Net(list(dims), w, b)
    ln = np.zeros(nln, np.float32)
    _check(lib().wc_synth_norms(dp, len(d), seed, ln.ctypes.data_as(_f32p), nln))
    return Net(list(dims), w, b, ln)


def synth_features(rows, width, seed=7):
    x = np.zeros((rows, width), np.float32)
    _check(lib().wc_synth_features(rows, width, seed, x.ctypes.data_as(_f32p)))
    return x


# ------------------------------------------------------------------ workloads

def default_spec(**kw):
    s = SynthSpecC()
    lib().wc_synth_spec_default(C.byref(s))
    for k, v in kw.items():
        if k == "net_dims":
            continue
        if not hasattr(s, k):
            raise KeyError(k)
        setattr(s, k, v)
    return s


def synth_jobs(net_dims, **kw) -> list:
    """Seeded synthetic jobs as WCJ8 bytes, one per tree."""
    s = default_spec(**kw)
    d, dp = _arr(net_dims, np.uint32)
    s.net_dims = dp
    s.n_net_dims = len(d)
    h = C.c_void_p()
    _check(lib().wc_synth(C.byref(s), C.byref(h)))
    try:
        out = []
        for k in range(lib().wc_jobset_count(h)):
            n = C.c_size_t()
            p = lib().wc_jobset_job(h, k, C.byref(n))
            out.append(C.string_at(p, n.value))
        return out
    finally:
        lib().wc_jobset_free(h)


def job_roundtrip(b: bytes) -> bytes:
    buf, p = _bytes_ptr(b)
    n = C.c_size_t()
    _check(lib().wc_job_roundtrip(p, len(b), None, 0, C.byref(n)))
    out = (C.c_uint8 * n.value)()
    _check(lib().wc_job_roundtrip(p, len(b), out, n.value, C.byref(n)))
    return bytes(out)


def job_validate(b: bytes):
    buf, p = _bytes_ptr(b)
    _check(lib().wc_job_validate(p, len(b)))


def job_work(b: bytes, precision=WC_PRECISE, route_unit=0, class_shift=0) -> dict:
    """`PackedJob::work`, `job_cost` and `cost_class` of one job (wc_job_work): the work
    vector's fields, `reserved_bytes`, the three route predicates, `cost` and `cost_class`."""
    buf, p = _bytes_ptr(b)
    w = WorkVectorC()
    cost, cls = C.c_uint64(), C.c_uint32()
    _check(lib().wc_job_work(p, len(b), precision, route_unit, class_shift, C.byref(w), C.byref(cost),
                             C.byref(cls)))
    out = {name: int(getattr(w, name)) for name, _ in w._fields_}
    out["cost"] = int(cost.value)
    out["cost_class"] = int(cls.value)
    return out


# ------------------------------------------------------------------ results

@dataclass
class SolveResult:
    """`SolveResult` (engine/src/gpu/client.rs:113-122), copied out of the native result."""
    tag: int
    weight_version: int
    strategy: np.ndarray
    root_values: np.ndarray  # [nroots, n0 + n1]
    root_n: tuple
    carries: np.ndarray      # [slots, snapshot_configs] float16
    oversize_route: bool = False
    card_exclusive_route: bool = False

    @staticmethod
    def take(ptr) -> "SolveResult":
        L = lib()
        n = C.c_size_t()
        sp = L.wc_result_strategy(ptr, C.byref(n))
        strategy = np.ctypeslib.as_array(sp, (n.value,)).copy() if n.value else np.zeros(0, np.float32)
        nr, n0, n1 = C.c_uint32(), C.c_uint32(), C.c_uint32()
        rp = L.wc_result_root_values(ptr, C.byref(nr), C.byref(n0), C.byref(n1))
        k = nr.value * (n0.value + n1.value)
        roots = (np.ctypeslib.as_array(rp, (k,)).copy() if k else np.zeros(0, np.float32)).reshape(
            nr.value, n0.value + n1.value)
        slots, cfgs = C.c_uint32(), C.c_uint32()
        cp = L.wc_result_carries(ptr, C.byref(slots), C.byref(cfgs))
        k = slots.value * cfgs.value
        carries = (np.ctypeslib.as_array(cp, (k,)).copy() if k else np.zeros(0, np.uint16)).view(
            np.float16).reshape(slots.value, cfgs.value)
        ov, card = C.c_int(), C.c_int()
        _check(L.wc_result_routes(ptr, C.byref(ov), C.byref(card)))
        r = SolveResult(int(L.wc_result_tag(ptr)), int(L.wc_result_weight_version(ptr)), strategy, roots,
                        (n0.value, n1.value), carries, bool(ov.value), bool(card.value))
        L.wc_result_free(ptr)
        return r


# ------------------------------------------------------------------ executor

class Wave:
    """`Wave::pack` over WCJ8 jobs."""

    def __init__(self, jobs: Sequence[bytes]):
        held, ptrs, lens = Wave._marshal(jobs)  # the library parses the jobs during the call
        h = C.c_void_p()
        _check(lib().wc_wave_pack(ptrs, lens, len(jobs), C.byref(h)))
        self.h = h
        self.njobs = len(jobs)

    @staticmethod
    def _marshal(jobs):
        held = [_bytes_ptr(j) for j in jobs]
        ptrs = (_u8p * len(jobs))(*[p for _, p in held])
        lens = (C.c_size_t * len(jobs))(*[len(j) for j in jobs])
        return held, ptrs, lens

    def repack(self, jobs: Sequence[bytes]):
        """Pack other jobs into this wave's host buffers (wc_wave_repack)."""
        held, ptrs, lens = Wave._marshal(jobs)
        _check(lib().wc_wave_repack(self.h, ptrs, lens, len(jobs)))
        self.njobs = len(jobs)

    def digest(self) -> int:
        """A digest of every packed list and count (wc_wave_digest)."""
        d = C.c_uint64()
        _check(lib().wc_wave_digest(self.h, C.byref(d)))
        return int(d.value)

    def stats(self) -> dict:
        s = WaveStats()
        _check(lib().wc_wave_stats_get(self.h, C.byref(s)))
        return s.as_dict()

    def array(self, name: str) -> np.ndarray:
        """A copy of one packed index array (wc_wave_array)."""
        n = C.c_size_t()
        p = lib().wc_wave_array(self.h, name.encode(), C.byref(n))
        if not p:
            _check(-1)
        return np.ctypeslib.as_array(p, (n.value,)).copy() if n.value else np.zeros(0, np.uint32)

    def poke(self, name: str, index: int, value: int):
        """Overwrite one word of a packed table (wc_wave_poke; test support): the
        wave then counts as unchecked."""
        _check(lib().wc_wave_poke(self.h, name.encode(), index, value & 0xFFFFFFFF))

    def check(self, executor: "Executor" = None, version: int = 0):
        """Check every index the kernels follow (wc_wave_check): on the host, or
        with an executor on its device. Raises WaveError with "wave bounds: ..."."""
        _check(lib().wc_wave_check(self.h, executor.h if executor is not None else None, version))

    def close(self):
        if self.h:
            lib().wc_wave_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Executor:
    """One device, one stream: `Executor::{new, publish, solve}`."""

    def __init__(self, device=0, precision=WC_PRECISE):
        h = C.c_void_p()
        _check(lib().wc_executor_create(device, precision, C.byref(h)))
        self.h = h

    def publish(self, net: Net) -> int:
        d = net.desc()
        v = lib().wc_executor_publish(self.h, C.byref(d))
        if v == 0:
            _check(-1)
        return int(v)

    def solve(self, wave: Wave, version: int) -> list:
        res = (C.c_void_p * wave.njobs)()
        _check(lib().wc_solve_wave(self.h, wave.h, version, res))
        return [SolveResult.take(res[k]) for k in range(wave.njobs)]

    def launch(self, wave: Wave, version: int) -> "InFlight":
        """`Executor::launch`: queue the wave and return at once; `collect` the record later."""
        f = C.c_void_p()
        _check(lib().wc_launch(self.h, wave.h, version, C.byref(f)))
        return InFlight(self, f, wave.njobs)

    def leaf_probe(self, wave: Wave, version: int, traverser: int):
        """The leaf net's values at the initial reach for `traverser`, from the wave's own
        kernels (wc_wave_leaf_probe): (values in row order, each row's configs of the
        traverser; mass [rows, 2])."""
        rows = wave.stats()["rows"]
        n = C.c_size_t()
        mass = np.zeros((max(rows, 1), 2), np.float32)
        _check(lib().wc_wave_leaf_probe(self.h, wave.h, version, traverser, None, 0, C.byref(n), None))
        vals = np.zeros(max(n.value, 1), np.float32)
        _check(lib().wc_wave_leaf_probe(self.h, wave.h, version, traverser, vals.ctypes.data_as(_f32p), vals.size,
                                        C.byref(n), mass.ctypes.data_as(_f32p)))
        return vals[: n.value], mass[:rows]

    def leaf_trace(self, wave: Wave, version: int, points, reach=True):
        """The leaf net's values captured inside one whole schedule right after the
        net runs at each schedule point (wc_wave_leaf_trace): t >= 0 is iteration t
        (traverser t & 1), phase2_point(root, p) Phase 2's evaluation. One dict per
        point: traverser, values (row order, each row's configs of the traverser),
        mass [rows, 2], reach (each row's reach over its configs, player 0's then
        player 1's; None with reach=False)."""
        pts = (C.c_int32 * max(len(points), 1))(*points)
        counts = (C.c_size_t * 4)()
        _check(lib().wc_wave_leaf_trace(self.h, wave.h, version, pts, len(points), None, 0, None, 0, None, 0,
                                        counts))
        nval, rows, nreach = (counts[0], counts[1]), counts[2], counts[3]
        trav = [pt & 1 if pt >= 0 else (-pt - 1) & 1 for pt in points]
        vals = np.zeros(max(sum(nval[p] for p in trav), 1), np.float32)
        mass = np.zeros(max(len(points) * 2 * rows, 1), np.float32)
        rbuf = np.zeros(max(len(points) * nreach, 1), np.float32) if reach else None
        _check(lib().wc_wave_leaf_trace(self.h, wave.h, version, pts, len(points), vals.ctypes.data_as(_f32p),
                                        vals.size, mass.ctypes.data_as(_f32p), mass.size,
                                        rbuf.ctypes.data_as(_f32p) if reach else None,
                                        rbuf.size if reach else 0, counts))
        out, v0 = [], 0
        for k, (pt, p) in enumerate(zip(points, trav)):
            out.append({"point": pt, "traverser": p, "values": vals[v0:v0 + nval[p]].copy(),
                        "mass": mass[k * 2 * rows:(k + 1) * 2 * rows].reshape(rows, 2).copy(),
                        "reach": rbuf[k * nreach:(k + 1) * nreach].copy() if reach else None})
            v0 += nval[p]
        return out

    def time_wave(self, wave: Wave, version: int, reps: int, warmup: int = 1):
        """Mean device ms per wave over `reps` timed schedules after `warmup` untimed
        ones, and one profiled schedule's [cfr, leaf net, leaf input, other, mean CFR iteration,
        mean subtree sweep, mean top sweep, mean subtree reach, graph build (host), the leaf
        net's per-wave work, the v5 joins] ms."""
        ms = C.c_double()
        parts = (C.c_double * 11)()
        _check(lib().wc_time_wave(self.h, wave.h, version, warmup, reps, C.byref(ms), parts))
        return ms.value, list(parts)

    def mlp(self, version: int, x: np.ndarray, heads: int) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros((x.shape[0], heads), np.float32)
        _check(lib().wc_mlp_forward(self.h, version, x.shape[0], x.ctypes.data_as(_f32p),
                                    out.ctypes.data_as(_f32p)))
        return out

    def mlp_noalloc(self, version: int, rows: int, x_dev: int, out_dev: int, stream: int = 0):
        """wc_mlp_forward_noalloc on device buffers (addresses as ints): x_dev rows x in f32,
        out_dev rows x heads f32. stream 0 waits on the executor's stream."""
        _check(lib().wc_mlp_forward_noalloc(self.h, version, rows, C.c_void_p(x_dev), C.c_void_p(out_dev),
                                            C.c_void_p(stream) if stream else None))

    def time_mlp(self, version: int, x: np.ndarray, reps: int):
        x = np.ascontiguousarray(x, np.float32)
        ms = C.c_double()
        layers = (C.c_double * 8)()
        _check(lib().wc_time_mlp(self.h, version, x.shape[0], x.ctypes.data_as(_f32p), reps,
                                 C.byref(ms), layers))
        return ms.value, list(layers)

    def close(self):
        if self.h:
            lib().wc_executor_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class InFlight:
    """A launched wave (`InFlight`, engine/src/gpu/device.rs:596-757)."""

    def __init__(self, ex: Executor, handle, njobs: int):
        self.ex, self.h, self.njobs = ex, handle, njobs

    def ready(self) -> bool:
        return bool(self.h) and bool(lib().wc_inflight_ready(self.ex.h, self.h))

    def collect(self) -> list:
        if not self.h:
            raise WaveError("already collected")
        res = (C.c_void_p * self.njobs)()
        h, self.h = self.h, None
        _check(lib().wc_collect(self.ex.h, h, res))
        return [SolveResult.take(res[k]) for k in range(self.njobs)]


# ------------------------------------------------------------------ service

class SolveHandle:
    def __init__(self, ticket):
        self._t = ticket

    def ready(self) -> bool:
        return bool(lib().wc_poll(self._t))

    def wait(self) -> SolveResult:
        out = C.c_void_p()
        t, self._t = self._t, None
        if t is None:
            raise WaveError("handle already waited on")
        _check(lib().wc_wait(t, C.byref(out)))
        return SolveResult.take(out)

    def __del__(self):
        # a handle dropped without wait frees its ticket (the solve's result is discarded)
        t, self._t = getattr(self, "_t", None), None
        if t is not None:
            try:
                lib().wc_ticket_free(t)
            except Exception:
                pass


class PreparedJob:
    """`PreparedJob` (engine/src/gpu/client.rs:165-181): a WCJ8 job parsed, validated
    and costed once for a service precision (wc_prepare); submit it any number of
    times with GpuClient.submit_prepared."""

    def __init__(self, job: bytes, precision=WC_PRECISE):
        buf, p = _bytes_ptr(job)
        h = C.c_void_p()
        _check(lib().wc_prepare(p, len(job), precision, C.byref(h)))
        self.h = h

    @property
    def cost(self) -> int:
        return int(lib().wc_prepared_cost(self.h))

    def close(self):
        if self.h:
            lib().wc_prepared_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GpuClient:
    """`GpuClient` (engine/src/gpu/client.rs:196-313) over the native service."""

    def __init__(self, handle):
        self.h = handle

    def submit(self, job: bytes, tag: int = 0) -> SolveHandle:
        buf, p = _bytes_ptr(job)
        t = C.c_void_p()
        _check(lib().wc_submit(self.h, p, len(job), tag, C.byref(t)))
        return SolveHandle(t)

    def submit_prepared(self, job: PreparedJob, tag: int = 0) -> SolveHandle:
        t = C.c_void_p()
        _check(lib().wc_submit_prepared(self.h, job.h, tag, C.byref(t)))
        return SolveHandle(t)

    def set_weights(self, net: Net) -> int:
        d = net.desc()
        v = lib().wc_set_weights(self.h, C.byref(d))
        if v == 0:
            _check(-1)
        return int(v)

    def queued_work(self) -> int:
        return int(lib().wc_queued_work(self.h))

    def stats(self) -> dict:
        """Waves launched and guarded routes taken so far."""
        w, g = C.c_uint64(), C.c_uint64()
        _check(lib().wc_service_stats(self.h, C.byref(w), C.byref(g)))
        return {"waves": int(w.value), "guarded_routes": int(g.value)}

    def close(self):
        if self.h:
            lib().wc_service_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


def spawn(device: int, net: Net, precision=WC_PRECISE, lanes=2, wave_jobs=64, wave_rows=49152,
          window_us=800, whale_lanes=1, class_shift=0, route_unit=0) -> GpuClient:
    """`service::spawn` (engine/src/gpu/service.rs:55-82)."""
    d = net.desc()
    opts = ServiceOpts(lanes, wave_jobs, wave_rows, window_us, whale_lanes, class_shift, route_unit)
    h = C.c_void_p()
    _check(lib().wc_service_create(device, C.byref(d), precision, C.byref(opts), C.byref(h)))
    return GpuClient(h)
