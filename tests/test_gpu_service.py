"""The service and the executor's launch/collect split on the GPU, through the C ABI.

Every result is compared bit for bit with the float32 CPU solver (the oracle),
not with another run of the device.

- queued_work (engine/src/gpu/client.rs:274-291) is the sum of the queued
  jobs' job_cost while they wait, and drains to zero;
- several lanes and several submitting threads return every job's result
  bit-identical to the oracle's solve of that job (the reference's lanes,
  engine/src/gpu/service.rs:546-742);
- wc_launch / wc_collect (engine/src/gpu/device.rs:596-831): two waves in
  flight on one executor, the packed wave freed while its wave runs, and a
  wave repacked (wc_wave_repack) while its solve is in flight;
- cost classes and guarded routes (service.rs:452-532,967-991): exclusive
  jobs run in one-job waves, guarded jobs after every lane has drained and
  trimmed, and the results carry their route flags (client.rs:119-121);
- the service's waves are bounds-checked at upload on the device by default,
  and on the host with WC_DEEP_CHECK=1 (a child process).
"""
import os
import sys
import threading
from concurrent.futures import ThreadPoolExecutor
from types import SimpleNamespace

import numpy as np
import pytest

import oracle as O
import warchest_wave as ww
import workloads as W

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def small_jobs(trees, seed, **kw):
    spec = dict(trees=trees, nodes_lo=30, nodes_hi=90, chance=1, terminal_p=0.15, notrans_p=0.05, nroots=2, iters=8,
                info_median=6.0, info_p99=40.0, info_cap=40, seed=seed)
    spec.update(kw)
    return W.jobs("wave256", **spec)


def alone(jobs, net):
    """Each job solved by the float32 CPU solver (the oracle), carries rounded to
    f16 as the result store keeps them."""
    def one(j):
        o = O.solve(j, net, O.NET_F32)
        return SimpleNamespace(strategy=o["strategy"], root_values=o["roots"],
                               carries=o["carries"].astype(np.float16))

    with ThreadPoolExecutor(min(16, os.cpu_count() or 1)) as pool:
        return list(pool.map(one, jobs))


def same(g, r, tag):
    np.testing.assert_array_equal(g.strategy, r.strategy, err_msg=tag)
    np.testing.assert_array_equal(g.root_values, r.root_values, err_msg=tag)
    np.testing.assert_array_equal(g.carries, r.carries, err_msg=tag)


def test_queued_work_is_the_sum_of_job_costs_and_drains():
    jobs = small_jobs(6, 51)
    net = W.net_for("wave256")
    costs = [ww.job_work(j, ww.WC_PRECISE)["cost"] for j in jobs]
    say(f"case queued work: 6 jobs, costs {costs}")
    # A 3-second bucket window: the lane holds the wave open while every job
    # is submitted, so nothing is answered before the check.
    with ww.spawn(0, net, ww.WC_PRECISE, lanes=1, wave_jobs=64, window_us=3_000_000) as client:
        handles = [client.submit(j, tag=k) for k, j in enumerate(jobs)]
        assert client.queued_work() == sum(costs)
        got = [h.wait() for h in handles]
        assert client.queued_work() == 0
    for k, (g, r) in enumerate(zip(got, alone(jobs, net))):
        same(g, r, f"job {k}")


def test_lanes_and_submitting_threads():
    jobs = small_jobs(20, 53)
    net = W.net_for("wave256")
    ref = alone(jobs, net)
    say("case lanes: 3 lanes, 4 submitting threads, 20 jobs, waves of at most 3")
    results = {}
    errors = []
    with ww.spawn(0, net, ww.WC_PRECISE, lanes=3, wave_jobs=3, window_us=500) as client:
        def submitter(t):
            try:
                mine = list(range(t, len(jobs), 4))
                handles = [(k, client.submit(jobs[k], tag=1000 + k)) for k in mine]
                for k, h in handles:
                    results[k] = h.wait()
            except Exception as e:  # reported after the join
                errors.append(e)

        threads = [threading.Thread(target=submitter, args=(t,)) for t in range(4)]
        for th in threads:
            th.start()
        for th in threads:
            th.join()
        stats = client.stats()
        assert client.queued_work() == 0
    assert not errors, errors
    say(f"{stats['waves']} waves")
    assert stats["waves"] >= 7
    for k in range(len(jobs)):
        assert results[k].tag == 1000 + k
        same(results[k], ref[k], f"job {k}")


def test_launch_collect_two_waves_in_flight():
    jobs = small_jobs(7, 57)
    net = W.net_for("wave256")
    ref = alone(jobs, net)
    say("case launch/collect: waves of 4 and 3 jobs in flight together on one executor")
    ex = ww.Executor(0, ww.WC_PRECISE)
    v = ex.publish(net)
    a, b = ww.Wave(jobs[:4]), ww.Wave(jobs[4:])
    fa = ex.launch(a, v)
    a.close()  # the packed wave may go as soon as launch returns
    fb = ex.launch(b, v)
    c = ww.Wave(jobs[:1])
    with pytest.raises(ww.WaveError):
        ex.launch(c, v)  # a third wave before a collect
    got = fa.collect() + fb.collect()
    assert fb.ready() is False  # collected
    fc = ex.launch(c, v)
    got_c = fc.collect()
    b.close()
    c.close()
    ex.close()
    for k, (g, r) in enumerate(zip(got, ref)):
        same(g, r, f"job {k}")
    same(got_c[0], ref[0], "relaunch")


def test_mixed_schedules_are_bucketed_apart():
    """Jobs of different schedules submitted interleaved (DCFR and linear CFR,
    8 and 5 iterations) share no wave: the service buckets only jobs with the
    same schedule metadata (engine/src/gpu/service.rs:621-637). Every result
    bit-identical to the oracle's solve of its own job."""
    net = W.net_for("wave256")
    groups = [small_jobs(4, 63), small_jobs(4, 65, alpha=1.0, beta=1.0, gamma=1.0),
              small_jobs(4, 67, iters=5)]
    jobs = [j for trio in zip(*groups) for j in trio]  # interleaved
    ref = alone(jobs, net)
    say("case mixed schedules: 12 jobs of three schedules interleaved, 2 lanes, waves of up to 64")
    with ww.spawn(0, net, ww.WC_PRECISE, lanes=2, wave_jobs=64, window_us=200_000) as client:
        handles = [client.submit(j, tag=k) for k, j in enumerate(jobs)]
        got = [h.wait() for h in handles]
        stats = client.stats()
    say(f"{stats['waves']} waves")
    assert stats["waves"] >= 3
    for k, (g, r) in enumerate(zip(got, ref)):
        assert g.tag == k
        same(g, r, f"job {k}")


def test_repack_while_the_wave_is_in_flight():
    """wc_wave_repack into a wave whose solve is still in flight (the service's
    lanes repack their wave right after launching it): the wave in flight keeps
    what it was launched with, and the repacked wave, launched next on the same
    executor, solves its own jobs. Both bit-identical to the oracle, with waves
    of different sizes so the reused lists shrink and grow."""
    jobs = small_jobs(9, 59)
    net = W.net_for("wave256")
    ref = alone(jobs, net)
    say("case repack in flight: waves of 6, 3 and 6 jobs through one reused wave on one executor")
    ex = ww.Executor(0, ww.WC_PRECISE)
    v = ex.publish(net)
    w = ww.Wave(jobs[:6])
    f1 = ex.launch(w, v)
    w.repack(jobs[6:])  # smaller, while the first solve runs
    f2 = ex.launch(w, v)
    got1 = f1.collect()
    w.repack(jobs[:6])  # larger again, while the second solve runs
    got2 = f2.collect()
    f3 = ex.launch(w, v)
    got3 = f3.collect()
    w.close()
    ex.close()
    for k, g in enumerate(got1):
        same(g, ref[k], f"first wave, job {k}")
    for k, g in enumerate(got2):
        same(g, ref[6 + k], f"repacked wave, job {k}")
    for k, g in enumerate(got3):
        same(g, ref[k], f"repacked again, job {k}")


def test_cost_classes_and_guarded_routes():
    """With the route unit lowered so that the larger of these jobs need one-job
    waves, arena guards or the whole device (the reference's 4 / 6 GiB
    thresholds scaled down), results stay bit-exact and carry their routes."""
    jobs = small_jobs(6, 59) + small_jobs(4, 61, nodes_lo=150, nodes_hi=260, info_median=12.0, info_p99=80.0,
                                          info_cap=80)
    net = W.net_for("wave256")
    ref = alone(jobs, net)
    work = [ww.job_work(j, ww.WC_PRECISE) for j in jobs]
    reserved = sorted(w["reserved_bytes"] for w in work)
    chosen = None
    for unit in sorted({max(r // 6, 1) for r in reserved} | {max(r // 4, 1) for r in reserved}):
        ws = [ww.job_work(j, ww.WC_PRECISE, route_unit=unit) for j in jobs]
        ex = sum(w["exclusive_route"] for w in ws)
        card = sum(w["card_exclusive_route"] for w in ws)
        guard = sum(w["arena_guard_route"] for w in ws)
        if 1 <= card and 1 <= guard + card and ex < len(jobs) - 2:
            chosen, work = unit, ws
            break
    assert chosen, "no route unit splits these jobs into ordinary, exclusive and card-exclusive"
    guarded = sum(1 for w in work if w["arena_guard_route"] or w["card_exclusive_route"])
    say(f"case routes: unit {chosen} bytes; exclusive {[w['exclusive_route'] for w in work]}, "
        f"card {[w['card_exclusive_route'] for w in work]}, guard {[w['arena_guard_route'] for w in work]}")
    with ww.spawn(0, net, ww.WC_PRECISE, lanes=2, wave_jobs=8, window_us=1000, route_unit=chosen) as client:
        handles = [client.submit(j, tag=k) for k, j in enumerate(jobs)]
        got = [h.wait() for h in handles]
        stats = client.stats()
        assert client.queued_work() == 0
    assert stats["guarded_routes"] == guarded
    exclusive = sum(w["exclusive_route"] for w in work)
    assert stats["waves"] >= exclusive + 1
    for k, (g, r, w) in enumerate(zip(got, ref, work)):
        same(g, r, f"job {k}")
        assert g.oversize_route == bool(w["exclusive_route"])
        assert g.card_exclusive_route == bool(w["card_exclusive_route"])


def test_dropped_handle_frees_its_ticket():
    jobs = small_jobs(3, 63)
    net = W.net_for("wave256")
    say("case dropped handle: a job submitted and never waited on")
    with ww.spawn(0, net, ww.WC_PRECISE, lanes=1, wave_jobs=1, window_us=0) as client:
        h = client.submit(jobs[0], tag=1)
        del h
        rest = [client.submit(j, tag=2 + k) for k, j in enumerate(jobs[1:])]
        got = [h.wait() for h in rest]
    for g, r in zip(got, alone(jobs[1:], net)):
        same(g, r, "after a dropped handle")


def test_prepared_jobs_submitted_again_and_again():
    """GpuClient::submit_prepared (engine/src/gpu/client.rs:212-255): jobs prepared once
    and submitted three times each from several threads, interleaved with the same
    jobs as WCJ8 bytes, all return the oracle's results; a job prepared for another
    precision is refused; queued work drains to zero."""
    jobs = small_jobs(6, 65)
    net = W.net_for("wave256")
    ref = alone(jobs, net)
    say("case prepared jobs: 6 jobs x 3 prepared submissions + 6 byte submissions, 2 lanes")
    prepared = [ww.PreparedJob(j, ww.WC_PRECISE) for j in jobs]
    with ww.spawn(0, net, ww.WC_PRECISE, lanes=2, wave_jobs=4, window_us=500) as client:
        with pytest.raises(ww.WaveError, match="precision"):
            client.submit_prepared(ww.PreparedJob(jobs[0], ww.WC_F16))
        items = [(k, r) for r in range(3) for k in range(len(jobs))]
        with ThreadPoolExecutor(4) as pool:
            handles = list(pool.map(lambda kr: (kr[0], client.submit_prepared(prepared[kr[0]], tag=10 * kr[0] + kr[1])),
                                    items))
        raw = [(k, client.submit(j, tag=900 + k)) for k, j in enumerate(jobs)]
        for p in prepared:
            p.close()  # queued submissions keep their job
        got = [(k, h.wait()) for k, h in handles + raw]
        assert client.queued_work() == 0
    for k, g in got:
        same(g, ref[k], f"job {k}")


def test_two_tower_service_waves():
    """Service waves of the two-tower net: their readout blocks are checked at
    upload on the device too; every result bit-identical to the oracle."""
    jobs = W.jobs("wave512w", trees=4, nodes_lo=40, nodes_hi=120, whale_frac=0.0, info_median=6.0, info_p99=40.0,
                  info_cap=40, iters=8, nroots=2, seed=59)
    net = W.net_for("wave512w")
    say("case two-tower service: 4 jobs, 2 lanes, waves of at most 2")
    with ww.spawn(0, net, ww.WC_PRECISE, lanes=2, wave_jobs=2, window_us=500) as client:
        got = [h.wait() for h in [client.submit(j, tag=k) for k, j in enumerate(jobs)]]
    for k, (g, r) in enumerate(zip(got, alone(jobs, net))):
        same(g, r, f"job {k}")


_HOST_CHECKED_CHILD = r"""
import sys
import numpy as np
sys.path[:0] = sys.argv[1:]
import oracle as O
import warchest_wave as ww
import workloads as W
jobs = W.jobs("wave256", trees=4, nodes_lo=30, nodes_hi=90, chance=1, terminal_p=0.15, nroots=2, iters=8, seed=57)
net = W.net_for("wave256")
with ww.spawn(0, net, ww.WC_PRECISE, lanes=2, wave_jobs=2, window_us=500) as client:
    got = [h.wait() for h in [client.submit(j, tag=k) for k, j in enumerate(jobs)]]
for k, (g, j) in enumerate(zip(got, jobs)):
    o = O.solve(j, net, O.NET_F32)
    np.testing.assert_array_equal(g.strategy, o["strategy"], err_msg=f"job {k}")
    np.testing.assert_array_equal(g.root_values, o["roots"], err_msg=f"job {k}")
print("host-checked service waves: 4 jobs bit-identical", flush=True)
"""


def test_service_with_host_checks():
    """WC_DEEP_CHECK=1 makes the service check its waves on the host
    (validate_deep) instead of at upload on the device; the setting is read
    once per process, so a child process runs the service with it."""
    import subprocess

    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    paths = [os.path.join(root, "war-chest-bot-9000-_amd"), os.path.join(root, "oracle"), here]
    env = dict(os.environ, WC_DEEP_CHECK="1")
    say("case host-checked service: a child process, 4 jobs, 2 lanes")
    run = subprocess.run([sys.executable, "-c", _HOST_CHECKED_CHILD, *paths], env=env, capture_output=True,
                         text=True, timeout=240)
    assert run.returncode == 0, run.stderr[-3000:]
    say(run.stdout.strip())


_FUSED_CHILD = r"""
import sys
import numpy as np
sys.path[:0] = sys.argv[1:]
import oracle as O
import warchest_wave as ww
import workloads as W
NONE = 0xFFFFFFFF
def fused(w, name):
    return any(r[1] != NONE for p in (0, 1) for r in w.array(name + str(p)).reshape(-1, 4))
jobs = []
for j in W.jobs("wave256")[:96]:  # trees whose own top regions fuse value and reach pairs
    w = ww.Wave([j])
    if fused(w, "top_back_run") and fused(w, "top_reach_run"):
        jobs.append(j)
    w.close()
    if len(jobs) == 3:
        break
assert len(jobs) == 3, len(jobs)
net = W.net_for("wave256")
with ww.spawn(0, net, ww.WC_PRECISE, lanes=2, wave_jobs=3, window_us=20000) as client:
    got = [h.wait() for h in [client.submit(j, tag=k) for k, j in enumerate(jobs)]]
for k, (g, j) in enumerate(zip(got, jobs)):
    o = O.solve(j, net, O.NET_F32)
    np.testing.assert_array_equal(g.strategy, o["strategy"], err_msg=f"job {k}")
    np.testing.assert_array_equal(g.root_values, o["roots"], err_msg=f"job {k}")
print("service waves with fused top launches: 3 jobs bit-identical", flush=True)
"""


def test_service_with_fused_top_launches():
    """WC_TOP_FUSE=1 makes the service's lanes plan fused top-depth launches
    (value pairs and reach pairs), whose run, chunk and parent tables the
    upload's structural checks bound; by default the lanes pack one depth per
    launch. The setting is read once per process, so a child process runs the
    service with it, on full-size subgames whose top regions fuse both."""
    import subprocess

    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    paths = [os.path.join(root, "war-chest-bot-9000-_amd"), os.path.join(root, "oracle"), here]
    env = dict(os.environ, WC_TOP_FUSE="1")
    say("case fused-top service: a child process, 3 full-size jobs, 2 lanes")
    run = subprocess.run([sys.executable, "-c", _FUSED_CHILD, *paths], env=env, capture_output=True, text=True,
                         timeout=240)
    assert run.returncode == 0, run.stderr[-3000:]
    say(run.stdout.strip())
