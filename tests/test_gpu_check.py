"""The device bounds check of a packed wave (csrc/check.hip), through the C ABI.

A service wave packed from jobs validated at submit skips the host's deep
check; its upload runs the structural checks on the host and then checks the
element tables on the device before any kernel of the schedule runs. These
tests hold the device check to the host's (validate_deep):

- waves of each network family pass both, with and without top regions;
- each single-fault edit of a packed wave (tests/bounds_cases.py) is refused
  on the device with the condition the host names, and the restored wave
  passes again;
- an edited wave given to wc_solve_wave is refused before its schedule runs,
  and the executor then solves a good wave as before.

The check kernels read only what their own index comparisons allow, so an
edited table makes them report, never fault.
"""
import sys

import numpy as np
import pytest

import bounds_cases as B
import oracle as O
import warchest_wave as ww
import workloads as W

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def executor_for(family):
    ex = ww.Executor(0, ww.WC_BF16 if family == "wave512w" else ww.WC_F16)
    return ex, ex.publish(W.net_for(family))


@pytest.mark.parametrize("slots", ["4096", B.UNIT_SLOTS])
@pytest.mark.parametrize("family", ["wave256", "wave256v5", "wave512w"])
def test_device_check_passes_packed_waves(family, slots, monkeypatch):
    monkeypatch.setenv("WC_UNIT_SLOTS", slots)
    wave = ww.Wave(W.jobs(family, trees=4, nodes_lo=100, nodes_hi=250, seed=83))
    ex, v = executor_for(family)
    say(f"[check] {family} unit slots {slots}: {wave.stats()['top_levels']} top depths")
    wave.check()
    wave.check(ex, v)


def test_device_check_names_what_the_host_names(monkeypatch):
    monkeypatch.setenv("WC_UNIT_SLOTS", B.UNIT_SLOTS)
    wave = ww.Wave(B.jobs())
    ex, v = executor_for("wave256")
    wave.check(ex, v)
    for name, index, value, msg in B.cases(wave):
        say(f"[check] {name}[{index}] = {value}: expect {msg!r}")
        old = int(wave.array(name)[index])
        wave.poke(name, index, value)
        with pytest.raises(ww.WaveError, match=r"^wave bounds: (.*)$") as host:
            wave.check()
        with pytest.raises(ww.WaveError, match=r"^wave bounds: (.*)$") as dev:
            wave.check(ex, v)
        assert str(host.value) == "wave bounds: " + msg
        assert str(dev.value) == str(host.value), name
        wave.poke(name, index, old)
        wave.check(ex, v)


def test_an_edited_wave_is_refused_before_its_schedule(monkeypatch):
    monkeypatch.setenv("WC_UNIT_SLOTS", B.UNIT_SLOTS)
    jobs = B.jobs()[:2]
    net = W.net_for("wave256")
    ex = ww.Executor(0, ww.WC_PRECISE)
    v = ex.publish(net)
    wave = ww.Wave(jobs)
    st = wave.stats()
    say("[check] solve with a value row written past the value table")
    wave.poke("back_rec0", 0, st["vals_len"])
    with pytest.raises(ww.WaveError, match="^wave bounds: back record$"):
        ex.solve(wave, v)
    say("[check] solve with a pool group's row count zero")
    good = ww.Wave(jobs)
    good.poke("pool_grp1", B.G_NROWS, 0)
    with pytest.raises(ww.WaveError, match="^wave bounds: pool group$"):
        ex.solve(good, v)
    say("[check] the same executor solves the unedited wave")
    got = ex.solve(ww.Wave(jobs), v)
    for j, r in zip(jobs, got):
        o = O.solve(j, net, O.NET_F32)
        np.testing.assert_array_equal(r.strategy, o["strategy"])
        np.testing.assert_array_equal(r.root_values, o["roots"])
