"""The allocation-free value-net entry point (wc_mlp_forward_noalloc) against
wc_mlp_forward, through the C ABI, on device-resident buffers.

Two calls in a row, the second with fewer rows (the shared scratch keeps the
first call's contents), in f16 (the fused net), float32 (the exact net) and
compensated f16 (layer by layer): outputs bit-identical to wc_mlp_forward's.
Rows beyond the scratch are refused with an error naming it. The same two calls
queued on a stream the caller created (the call returns at once; the caller
synchronizes that stream) give the same outputs.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import warchest_wave as ww
import workloads as W

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class Hip:
    """The few HIP runtime calls the test needs for device buffers."""

    def __init__(self):
        self.L = C.CDLL("libamdhip64.so")
        self.L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.L.hipFree.argtypes = [C.c_void_p]
        self.L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.L.hipDeviceSynchronize.argtypes = []
        self.L.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.L.hipStreamSynchronize.argtypes = [C.c_void_p]
        self.L.hipStreamDestroy.argtypes = [C.c_void_p]
        for f in (self.L.hipMalloc, self.L.hipFree, self.L.hipMemcpy, self.L.hipDeviceSynchronize,
                  self.L.hipStreamCreate, self.L.hipStreamSynchronize, self.L.hipStreamDestroy):
            f.restype = C.c_int

    def stream(self):
        s = C.c_void_p()
        assert self.L.hipStreamCreate(C.byref(s)) == 0  # default flags and priority
        return s.value

    def sync(self, s):
        assert self.L.hipStreamSynchronize(C.c_void_p(s)) == 0

    def destroy(self, s):
        assert self.L.hipStreamDestroy(C.c_void_p(s)) == 0

    def alloc(self, nbytes):
        p = C.c_void_p()
        assert self.L.hipMalloc(C.byref(p), nbytes) == 0
        return p.value

    def to_dev(self, dst, a):
        assert self.L.hipMemcpy(C.c_void_p(dst), a.ctypes.data_as(C.c_void_p), a.nbytes, 1) == 0  # host to device

    def to_host(self, a, src):
        assert self.L.hipMemcpy(a.ctypes.data_as(C.c_void_p), C.c_void_p(src), a.nbytes, 2) == 0  # device to host

    def free(self, p):
        assert self.L.hipFree(C.c_void_p(p)) == 0


@pytest.mark.parametrize("precision", [ww.WC_F16, ww.WC_PRECISE, ww.WC_F16X])
def test_noalloc_matches_mlp_forward_twice(precision):
    hip = Hip()
    net = W.net_for("mlp65k")
    heads = net.dims[4]
    ex = ww.Executor(0, precision)
    v = ex.publish(net)
    sizes = (4000, 1000) if precision != ww.WC_PRECISE else (2000, 600)
    xd = hip.alloc(sizes[0] * 512 * 4)
    od = hip.alloc(sizes[0] * heads * 4)
    try:
        for call, rows in enumerate(sizes):
            say(f"case no-alloc precision {precision}: call {call + 1}, {rows} rows")
            x = W.mlp65k_inputs(rows=rows, seed=40 + call)
            hip.to_dev(xd, x)
            ex.mlp_noalloc(v, rows, xd, od)
            got = np.zeros((rows, heads), np.float32)
            hip.to_host(got, od)
            want = ex.mlp(v, x, heads=heads)
            np.testing.assert_array_equal(got, want)
    finally:
        hip.free(xd)
        hip.free(od)
        ex.close()


@pytest.mark.parametrize("precision", [ww.WC_F16, ww.WC_PRECISE])
def test_noalloc_on_a_caller_stream(precision):
    """Queued on the caller's own stream (the plan kernel and the net run there):
    the call returns at once, and after the caller synchronizes that stream the
    outputs equal wc_mlp_forward's, on two calls in a row, the second smaller."""
    hip = Hip()
    net = W.net_for("mlp65k")
    heads = net.dims[4]
    ex = ww.Executor(0, precision)
    v = ex.publish(net)
    sizes = (3000, 700) if precision != ww.WC_PRECISE else (1500, 500)
    xd = hip.alloc(sizes[0] * 512 * 4)
    od = hip.alloc(sizes[0] * heads * 4)
    st = hip.stream()
    try:
        for call, rows in enumerate(sizes):
            say(f"case no-alloc on a caller stream, precision {precision}: call {call + 1}, {rows} rows")
            x = W.mlp65k_inputs(rows=rows, seed=60 + call)
            hip.to_dev(xd, x)
            ex.mlp_noalloc(v, rows, xd, od, stream=st)
            hip.sync(st)
            got = np.zeros((rows, heads), np.float32)
            hip.to_host(got, od)
            want = ex.mlp(v, x, heads=heads)
            np.testing.assert_array_equal(got, want)
    finally:
        hip.sync(st)
        hip.destroy(st)
        hip.free(xd)
        hip.free(od)
        ex.close()


def test_noalloc_refuses_rows_beyond_the_scratch():
    net = W.net_for("mlp65k")
    ex = ww.Executor(0, ww.WC_F16)
    v = ex.publish(net)
    say("case no-alloc: 65,536 rows, beyond the scratch")
    # the size check runs before any device work: the buffers are never touched
    with pytest.raises(ww.WaveError, match="scratch"):
        ex.mlp_noalloc(v, 65536, 1 << 20, 1 << 20)
    ex.close()
