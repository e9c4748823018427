"""Throughput of the MI355X wave executor on one GPU.

One step = one wave solved end to end on the device: 256 seeded depth-2 DCFR
subgames (200..800 public nodes, chance nodes with 2..6 outcomes, lognormal
infostates with median 22 and p99 567), 64 DCFR(1.5, 0, 2) iterations with an
f16 512 -> 3x384 -> 567 value-net call per iteration, then Phase 2 (root
values under the final average strategy). Tables, weights and state are
resident in HBM before the timed region; device time comes from HIP events
on the executor's stream.

Printed as one JSON line: CFR node-iterations/s (`value`), leaf queries/s,
the roofline of the dominant kernel, the value-net GEMM chain alone on
65,536 queries (512 -> 3x384 -> 64) against the MFMA roofline, and the CPU
oracle timed on a bounded sample of the same wave on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "war-chest-bot-9000-_amd"), os.path.join(ROOT, "oracle")]

HBM_PEAK_GBS = 8000.0     # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16/bf16


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def measured_traffic(workload, kernel):
    """HBM bytes per dispatch of `kernel` from the committed rocprofv3 counter
    summary of this workload (FETCH_SIZE + WRITE_SIZE, copy-calibrated), or None."""
    path = os.path.join(ROOT, "profiles", f"{workload}_hbm_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) == 5 and cells[0] == f"`{kernel}`":
                    return int(cells[4])
    except OSError:
        pass
    return None


def host_cpu():
    """The host's CPU model and core counts, from lscpu."""
    import subprocess

    info = {}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in txt.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    model = info.get("Model name", "unknown")
    sockets = info.get("Socket(s)", "?")
    cores = info.get("Core(s) per socket", "?")
    tpc = info.get("Thread(s) per core", "?")
    return f"{model}; {sockets} socket(s) x {cores} cores x {tpc} threads = {os.cpu_count()} logical CPUs"


def cpu_share():
    """Threads for the CPU baseline: the CPUs this process may run on, bounded by
    the cgroup's CPU quota and by the share the environment states
    (OMP_NUM_THREADS), and a description of where the number came from."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    why = [f"{n} CPUs in the affinity mask"]
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            q = max(1, int(int(quota) // int(period)))
            why.append(f"cgroup quota {q} CPUs")
            n = min(n, q)
    except (OSError, ValueError):
        pass
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        why.append(f"OMP_NUM_THREADS={omp}")
        n = min(n, int(omp))
    return max(1, n), ", ".join(why)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--workload", default="wave256", choices=["wave64", "wave256", "wave512w"],
                    help="wave256: 256 depth-2 subgames, f16 MLP (the headline); wave512w: 512 subgames with 10%% "
                         "whales, 128 iterations, bf16 two-tower net")
    ap.add_argument("--cpu-trees", type=int, default=0, help="trees in the CPU-baseline sample (0 = 2 per thread)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-mlp", action="store_true", help="skip the GEMM-chain-alone leg")
    ap.add_argument("--no-host", action="store_true", help="skip the host-path (PCIe-inclusive) leg")
    ap.add_argument("--no-v5", action="store_true", help="skip the v5-network wave leg")
    ap.add_argument("--service", type=int, default=48, metavar="WAVES",
                    help="stream WAVES copies of the wave's subgames through the service and report the end-to-end "
                         "rate: prepared jobs (wc_prepare once, wc_submit_prepared per wave, as the reference's "
                         "throughput tape does) and, beside it, WCJ8 bytes per submission (wc_submit); 0 skips it")
    ap.add_argument("--service-lanes", type=int, default=8, help="executor lanes of the service leg")
    ap.add_argument("--graph-compare", action="store_true",
                    help="also time the schedule captured into one HIP graph and replayed")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="after the run, copy MIB MiB device to device 3 times (calibrates HBM counters)")
    ap.add_argument("--no-peaks", action="store_true",
                    help="skip measuring the device's HBM and MFMA peaks (the fractions then use the datasheet only)")
    ap.add_argument("--no-accuracy", action="store_true",
                    help="skip comparing the timed wave's first subgames with the float32 CPU solver")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the wave executor shards whole trees across devices with no exchange, "
              f"and this build runs on a single MI355X (got --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)

    import numpy as np

    import warchest_wave as ww
    import workloads as W

    t0 = time.time()
    jobs = W.jobs(args.workload)
    net = W.net_for(args.workload)
    log(f"[bench] generated {len(jobs)} subgames in {time.time() - t0:.1f}s")
    wave = ww.Wave(jobs)
    st = wave.stats()
    log(f"[bench] wave: {st['nodes']} nodes, {st['cells']} cells, {st['rows']} leaf rows, {st['levels']} levels")

    pk = None
    if not args.no_peaks:
        # What this device sustains (HIP events), measured first, on an idle device:
        # a 16-byte copy and read over 1 GiB buffers and the f16 MFMA on register
        # operands. Every fraction is also given against these measured peaks.
        pk = ww.peak_probe(0, 1 << 30)
        hbm_meas = max(pk["hbm_copy_gbs"], pk["hbm_read_gbs"])
        mfma_meas = pk["mfma_f16_tflops"]
        peaks = {"hbm_copy_gbs": round(pk["hbm_copy_gbs"], 1), "hbm_read_gbs": round(pk["hbm_read_gbs"], 1),
                 "mfma_f16_tflops": round(mfma_meas, 1),
                 "mfma_f16_16x16x32_tflops": round(pk["mfma_f16_16x16x32_tflops"], 1),
                 "datasheet_hbm_gbs": HBM_PEAK_GBS, "datasheet_mfma_f16_tflops": MFMA_F16_PEAK_TFLOPS,
                 "note": "measured on this device with wc_peak_probe before the timed work (MFMA: the 32x32x16 "
                         "instruction; the 16x16x32 one the value net issues beside it); `peak` fields are the "
                         "datasheet's, `frac_measured` fields divide by the measured peak (HBM: the larger of "
                         "copy and read)"}
        log(f"[bench] peaks: HBM copy {pk['hbm_copy_gbs']:.0f} GB/s, read {pk['hbm_read_gbs']:.0f} GB/s, "
            f"f16 MFMA {mfma_meas:.0f} TFLOP/s (16x16x32: {pk['mfma_f16_16x16x32_tflops']:.0f})")
    tower = args.workload == "wave512w"
    ex = ww.Executor(0, ww.WC_BF16 if tower else ww.WC_F16)
    ver = ex.publish(net)
    wave_ms, parts = ex.time_wave(wave, ver, reps=args.steps, warmup=args.warmup)
    log(f"[bench] {args.steps} timed waves: {wave_ms:.3f} ms/wave; per class {parts}")

    iters = st["iters"]
    node_iters = st["nodes"] * iters
    queries = st["rows"] * (iters + 2 * st["nroots_max"])
    value = node_iters / (wave_ms * 1e-3)
    cfr_ms, mlp_ms, leaf_ms, other_ms, iter_ms, back_ms, top_ms, reach_ms = parts[:8]
    # Algorithmic bytes of one launch of each CFR kernel, averaged over the two traversers.
    kernels = {"k_sweep<regret>": (0, back_ms), "top-region launches (k_back_rows, k_back_pair, k_reach_rows, k_reach_pair)": (1, top_ms),
               "k_reach": (2, reach_ms)}
    by_kernel = {}
    for name, (k, ms) in kernels.items():
        nbytes = 0.5 * (st["cfr_bytes_by_kernel"][0][k] + st["cfr_bytes_by_kernel"][1][k])
        gbs = nbytes / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
        by_kernel[name] = {"launch_ms": round(ms, 5), "bytes_per_launch": int(nbytes), "achieved_gbs": round(gbs, 2),
                           "frac": round(gbs / HBM_PEAK_GBS, 5)}
    # The iteration's CFR launches (sweep, tops, reach). The average-strategy
    # accumulation runs inside the leaf-input launch and is timed with it.
    bk = st["cfr_bytes_by_kernel"]
    bytes_per_iter = 0.5 * sum(bk[0][k] + bk[1][k] for k in range(3))
    acc_bytes = 0.5 * (bk[0][3] + bk[1][3])
    iter_gbs = bytes_per_iter / (iter_ms * 1e-3) / 1e9
    passes = iters + 2 * st["nroots_max"]  # leaf-net passes per wave
    # The fused f16 net takes the first layer's product over the fixed query
    # columns (seat, public features) once per traverser per wave, then only
    # the pooled columns per pass: count each part as often as it runs.
    dims = W.SPECS[args.workload]["net_dims"]
    fixed = 0
    if not tower:  # the executor splits when the fused kernel takes the net (chain_fits) and the
        _, n_in, hidden, layers, _, pool = dims  # pooled columns are whole 32-column steps
        fused = n_in % 32 == 0 and n_in <= 512 and hidden % 32 == 0 and hidden <= 384 and 1 <= layers <= 8
        if fused and 0 < 2 * pool < n_in and (2 * pool) % 32 == 0:
            fixed = st["rows"] * 2 * (n_in - 2 * pool) * hidden
    pass_flops = st["mlp_flops_algorithmic"] - fixed
    mlp_flops_wave = pass_flops * passes + 2 * fixed
    mlp_tflops_in_wave = mlp_flops_wave / (mlp_ms * 1e-3) / 1e12 if mlp_ms > 0 else 0.0
    mlp_exec_tflops = ((st["mlp_flops_executed"] - fixed) * passes + 2 * fixed) / (mlp_ms * 1e-3) / 1e12 \
        if mlp_ms > 0 else 0.0
    # The roofline names one kernel: the one with the most device time per wave
    # among the subtree sweep, the subtree reach and the value net.
    net_name = "two-tower net (k_gemm layers + k_tower_dense)" if tower else "k_chain"
    per_wave = {"k_sweep<regret>": back_ms * iters, "k_reach": reach_ms * iters, net_name: mlp_ms}
    dominant = max(per_wave, key=per_wave.get)
    if dominant == net_name:
        launch_ms = mlp_ms / passes
        flops = mlp_flops_wave / passes  # mean per launch, the fixed-column product included once per traverser
        tf = flops / (launch_ms * 1e-3) / 1e12
        trace_name = "wc::k_chain<1, 1>" if fixed else "wc::k_chain<1, 0>"
        roofline = {"bound": "mfma", "kernel": dominant, "achieved": round(tf, 2), "peak": MFMA_F16_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 5), "flops_per_launch": round(flops),
                    "launch_ms": round(launch_ms, 5)}
        if not tower:
            # Algorithmic bytes of one pass launch: the pooled input columns
            # (16-bit), the first layer's fixed-column partial products (float32
            # accumulator tiles, when split), every weight matrix once, and one
            # float32 head output per (row, traverser config).
            _, n_in, hidden, layers, heads_n, pool = dims
            trunk_flops = 2 * (n_in * hidden + (layers - 1) * hidden * hidden)
            head_cols = (st["mlp_flops_algorithmic"] - st["rows"] * trunk_flops) // (2 * hidden)
            in_cols = 2 * pool if fixed else n_in
            weights = 2 * (n_in * hidden + (layers - 1) * hidden * hidden + heads_n * hidden) + \
                4 * (layers * hidden + heads_n)
            roofline["algorithmic_bytes"] = int(st["rows"] * in_cols * 2 + (st["rows"] * hidden * 4 if fixed else 0)
                                                + weights + head_cols * 4)
    else:
        d = by_kernel[dominant]
        trace_name = {"k_sweep<regret>": "wc::k_sweep<0, %s>" % ("true" if st["max_window"] * 4 <= 65536 else "false"),
                      "k_reach": "wc::k_reach"}[dominant]
        roofline = {"bound": "hbm", "kernel": dominant, "achieved": d["achieved_gbs"], "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": d["frac"], "bytes_per_launch": d["bytes_per_launch"],
                    "launch_ms": d["launch_ms"]}
    traffic = measured_traffic(args.workload, trace_name) if not tower else None
    roofline["traffic"] = traffic
    roofline["traffic_source"] = f"profiles/{args.workload}_hbm_traffic.md ({trace_name})" if traffic else None
    roofline["ms_per_wave"] = round(per_wave[dominant], 4)

    out = {
        "metric": "CFR node-iters/sec + value-net leaf queries/sec on 1 MI355X; % HBM/MFMA peak",
        "value": round(value, 1),
        "unit": "node-iters/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wave_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 CFR state, %s leaf-net operands (f32 accumulate)" % ("bf16" if tower else "f16"),
        "data": "synthetic (seeded subgames and Kaiming-normal random-init value net)",
        "config": {
            "workload": (f"wave of {st['jobs']} depth-2 DCFR subgames (10% whales: 2,000 nodes, 567 infostates), "
                         f"{iters} iterations, bf16 two-tower value net 512->2x512 public, 96->2x512 private "
                         f"({args.workload})") if tower else
                        (f"wave of {st['jobs']} depth-2 DCFR subgames, {iters} iterations, 512->3x384->567 f16 "
                         f"value net ({args.workload})"),
            "trees": st["jobs"], "nodes": st["nodes"], "legal_cells": st["cells"], "leaf_rows": st["rows"],
            "iters": iters, "sweep_units": st["units"], "top_levels": st["top_levels"],
            "parallelism": "1 GPU; subgames cut into subtree units, one workgroup per unit",
        },
        "leaf_queries_per_s": round(queries / (wave_ms * 1e-3), 1),
        "ms_by_class": {"cfr": round(cfr_ms, 4), "mlp": round(mlp_ms, 4), "leaf_input": round(leaf_ms, 4),
                        "other": round(other_ms, 4)},
        "roofline": roofline,
        "roofline_cfr_iteration": {"bound": "hbm", "kernels": by_kernel, "achieved": round(iter_gbs, 2),
                                   "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(iter_gbs / HBM_PEAK_GBS, 5),
                                   "bytes_per_iter": int(bytes_per_iter), "iter_ms": round(iter_ms, 5),
                                   "accumulation_bytes_per_iter": int(acc_bytes),
                                   "note": "sweep + top regions + reach; the average accumulation runs in the "
                                           "leaf-input launch (k_pool_mfma) and is timed with the leaf input"},
        "roofline_mlp_in_wave": {"bound": "mfma", "achieved": round(mlp_tflops_in_wave, 2),
                                 "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                 "frac": round(mlp_tflops_in_wave / MFMA_F16_PEAK_TFLOPS, 5),
                                 "flops_per_pass": pass_flops, "flops_fixed_per_wave": 2 * fixed,
                                 "executed_tflops": round(mlp_exec_tflops, 2),
                                 "note": "public tower + one readout per (row, config) of the traverser" if tower
                                 else "algorithmic = trunk + one head row per traverser config"},
    }

    # The leaf-input launches: per iteration the traverser's pooling (its rows'
    # pooled beliefs into both query inputs) with the traverser's average-strategy
    # accumulation beside it, and in Phase 2 both players' pooling per carried root.
    lib_bytes = st["leaf_input_bytes"]
    acc = [bk[0][3], bk[1][3]]
    leaf_launches = iters + st["nroots_max"]
    leaf_total = sum(lib_bytes[t & 1] + acc[t & 1] for t in range(iters)) + \
        st["nroots_max"] * (lib_bytes[0] + lib_bytes[1])
    leaf_gbs = leaf_total / (leaf_ms * 1e-3) / 1e9 if leaf_ms > 0 else 0.0
    out["roofline_leaf_input"] = {
        "bound": "hbm", "kernel": "k_pool_mfma<1>" if not tower else "k_pool_mfma<2>",
        "achieved": round(leaf_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(leaf_gbs / HBM_PEAK_GBS, 5),
        "bytes_per_launch": int(leaf_total / leaf_launches), "launch_ms": round(leaf_ms / leaf_launches, 5),
        "note": "pooling: each row's reach and outputs, each distinct config list and embedding once; plus the "
                "traverser's average-strategy accumulation (12 B per cell + 4 B per row) in the same launch"}

    if args.graph_compare:
        # The same schedule captured once into a HIP graph and replayed.
        os.environ["WC_GRAPH"] = "1"
        gex = ww.Executor(0, ww.WC_BF16 if tower else ww.WC_F16)
        del os.environ["WC_GRAPH"]
        gv = gex.publish(net)
        g_ms, g_parts = gex.time_wave(wave, gv, reps=args.steps, warmup=args.warmup)
        gex.close()
        out["graph"] = {"ms_per_wave": round(g_ms, 4), "eager_ms_per_wave": round(wave_ms, 4),
                        "build_ms": round(g_parts[8], 2),
                        "note": "the whole schedule (one wave) captured into one hipGraph, instantiated once, replayed"}
        log(f"[bench] graph replay: {g_ms:.3f} ms/wave (eager {wave_ms:.3f}); capture + instantiate "
            f"{g_parts[8]:.1f} ms on the host")

    if not args.no_mlp:
        mnet = W.net_for("mlp65k")
        x = W.mlp65k_inputs()
        mex = ww.Executor(0, ww.WC_F16)
        mv = mex.publish(mnet)
        chain_ms, layer_ms = mex.time_mlp(mv, x, reps=20)
        flops = x.shape[0] * 2 * (512 * 384 + 2 * 384 * 384 + 384 * 64)
        tf = flops / (chain_ms * 1e-3) / 1e12
        out["mlp_alone"] = {"workload": "65,536 queries, 512->384->384->384->64, f16 operands, f32 accumulate",
                            "queries_per_s": round(x.shape[0] / (chain_ms * 1e-3), 1),
                            "ms": round(chain_ms, 5), "layer_ms": [round(v, 5) for v in layer_ms[:4]],
                            "achieved": round(tf, 2), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                            "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 5)}
        mex.close()
        log(f"[bench] GEMM chain alone: {chain_ms:.4f} ms, {tf:.1f} TFLOP/s")

    if not args.no_v5:
        # The reference's production leaf network (net_dims [5]) on the same
        # 256 trees: per wave the card tokens, the board trunk of every
        # network row and the config encoder; per iteration the pooled
        # beliefs, the join and the readout (16-bit operands on the matrix cores).
        vjobs = W.jobs("wave256v5")
        vnet = W.net_for("wave256v5")
        vex = ww.Executor(0, ww.WC_F16)
        vv = vex.publish(vnet)
        vwave = ww.Wave(vjobs)
        vst = vwave.stats()
        v_ms, v_parts = vex.time_wave(vwave, vv, reps=args.steps, warmup=args.warmup)
        vwave.close()
        vex.close()
        v_ni = vst["nodes"] * vst["iters"]
        vrows = vst["rows"]
        vpasses = vst["iters"] + 2 * vst["nroots_max"]
        # algorithmic FLOPs: the trunk per row (8 blocks of mix 192->96 and out 96->96 over
        # 37 hexes, the pool bias 192->96, the board 207->256, the join cache 256->128) and the
        # join per row and pass (129->128, 3 x 128->128, 128->256)
        trunk = 8 * 37 * 2 * (192 * 96 + 96 * 96) + 8 * 2 * 192 * 96 + 2 * 207 * 256 + 2 * 256 * 128
        join = 2 * (129 * 128 + 3 * 128 * 128 + 128 * 256)
        build_ms, join_ms = v_parts[9], v_parts[10]
        # the per-wave build is the cards, the trunk and the config encoder: its
        # fraction counts the trunk's FLOPs only (a lower bound for the trunk kernel)
        build_tf = vrows * trunk / (build_ms * 1e-3) / 1e12 if build_ms > 0 else 0.0
        join_tf = vrows * join * vpasses / (join_ms * 1e-3) / 1e12 if join_ms > 0 else 0.0
        out["v5_wave"] = {"workload": "wave256v5: the 256 depth-2 trees with the v5 leaf network, f16 operands",
                          "ms_per_wave": round(v_ms, 3), "node_iters_per_s": round(v_ni / (v_ms * 1e-3), 1),
                          "rows": vrows, "net_ms": round(v_parts[1], 3), "cfr_ms": round(v_parts[0], 3),
                          "trunk_gflop_per_wave": round(vrows * trunk / 1e9, 2),
                          "join_gflop_per_pass": round(vrows * join / 1e9, 3),
                          "build_ms": round(build_ms, 3), "join_ms_per_pass": round(join_ms / vpasses, 4),
                          "trunk_mfma": {"achieved": round(build_tf, 2), "unit": "TFLOP/s",
                                         "frac": round(build_tf / MFMA_F16_PEAK_TFLOPS, 5),
                                         "note": "trunk FLOPs over the whole per-wave build (cards, trunk, configs)"},
                          "join_mfma": {"achieved": round(join_tf, 2), "unit": "TFLOP/s",
                                        "frac": round(join_tf / MFMA_F16_PEAK_TFLOPS, 5)},
                          "note": "net_ms = the per-wave build (cards, trunk, configs) + every join and readout"}
        log(f"[bench] v5 wave: {v_ms:.2f} ms/wave ({v_parts[1]:.2f} ms in the network)")

    dev_results = None
    if not args.no_host:
        # The boundary takes host buffers: the same wave through wc_solve_wave
        # (pinned upload of the packed tables, the schedule, collection and the
        # per-job unpack), and the packing itself. Reported beside `value`, never as it.
        t = time.time()
        ww.Wave(jobs).close()
        pack_s = time.time() - t
        ex.solve(wave, ver)  # sizes the pinned staging
        reps = 3
        t = time.time()
        for _ in range(reps):
            dev_results = ex.solve(wave, ver)
        solve_ms = (time.time() - t) / reps * 1e3
        out["host_path"] = {
            "solve_ms_per_wave": round(solve_ms, 3),
            "solve_node_iters_per_s": round(node_iters / (solve_ms * 1e-3), 1),
            "pack_ms_per_wave": round(pack_s * 1e3, 1),
            "table_bytes": st["table_bytes"],
            "note": "wc_solve_wave on a packed wave: pinned H2D of the tables, the schedule, D2H and unpack; "
                    "pack = parse + validate + wc_wave_pack on the host",
        }
        log(f"[bench] host path: solve {solve_ms:.1f} ms per wave, pack {pack_s * 1e3:.0f} ms")
    if args.service:
        # The drop-in's own throughput, as the reference measures it with its
        # throughput tape (engine/examples/wave_tape.rs:80-99): jobs prepared once
        # and submitted wave after wave by several threads, results waited on.
        # A native caller of the C ABI does it (wc_tape, built beside the
        # library), in a child process: the figure is the library's, not the
        # Python binding's.
        import struct
        import subprocess
        import tempfile

        lanes, subs = args.service_lanes, 8
        prec = ww.WC_BF16 if tower else ww.WC_F16
        tape_bin = os.path.join(ROOT, "war-chest-bot-9000-_amd", "wc_tape")
        if not os.path.exists(tape_bin):
            raise SystemExit(f"{tape_bin} is missing: build first (python __graft_entry__.py)")
        with tempfile.NamedTemporaryFile(prefix="wc_", suffix=".tape", delete=False) as f:
            f.write(b"WCTP" + struct.pack("<I", len(jobs)))
            for j in jobs:
                f.write(struct.pack("<Q", len(j)) + j)
            dims = np.asarray(net.dims, np.uint32)
            f.write(struct.pack("<I", dims.size) + dims.tobytes())
            for arr in (net.w, net.b, net.ln if net.ln is not None else np.zeros(0, np.float32)):
                a = np.ascontiguousarray(arr, np.float32)
                f.write(struct.pack("<Q", a.size) + a.tobytes())
            tape_file = f.name
        try:
            run = subprocess.run([tape_bin, tape_file, str(args.service), str(lanes), str(subs), str(prec)],
                                 capture_output=True, text=True, timeout=900)
        finally:
            os.unlink(tape_file)
        if run.returncode != 0:
            raise SystemExit(f"wc_tape failed ({run.returncode}): {run.stderr[-2000:]}")
        sv = json.loads(run.stdout.strip().splitlines()[-1])
        dt = sv["ms_per_wave"] * args.service / 1e3
        out["service"] = {"waves": args.service, "lanes": lanes, "submit_threads": subs,
                          "ms_per_wave": round(sv["ms_per_wave"], 2),
                          "node_iters_per_s": round(args.service * node_iters / dt, 1),
                          "solves_per_s": round(args.service * len(jobs) / dt, 1),
                          "prepare_ms_once": sv["prepare_ms_once"],
                          "bytes_ms_per_wave": round(sv["bytes_ms_per_wave"], 2),
                          "device_waves": sv["device_waves"],
                          "bytes_device_waves": sv["bytes_device_waves"],
                          "driver": "wc_tape (csrc/wave_tape.cpp), a native caller of the C ABI, in a child process",
                          "note": "end to end through the C ABI: jobs prepared once (parse, validate, cost) and "
                                  "submitted per wave from several threads, every result waited on and read; lanes "
                                  "pack over one shared host thread pool, pinned transfers, lanes overlap on their "
                                  "own streams; the service forms its own device waves (one cost class each, at "
                                  "most 256 jobs and 48k network rows, an 800 us fill window from the oldest job: "
                                  "device_waves per WAVES). bytes_ms_per_wave: WCJ8 bytes per submission (parsed and "
                                  "validated every time). After full-size warm-up waves of both kinds, the two kinds "
                                  "are timed alternately, twice each (the means)"}
        log(f"[bench] service: {sv['ms_per_wave']:.1f} ms per wave end to end with prepared jobs, "
            f"{sv['bytes_ms_per_wave']:.1f} ms with bytes per submission "
            f"({sv['device_waves']:.1f} and {sv['bytes_device_waves']:.1f} device waves per {args.service}; native driver)")

    if not args.no_cpu:
        import oracle as O

        threads, share = cpu_share()
        n = args.cpu_trees or min(len(jobs), 2 * threads)
        sample = jobs[:n]
        host = host_cpu()
        log(f"[bench] CPU oracle: {n} trees on {threads} threads ({share}; host: {host}) ...")
        sec, ni, lq = O.solve_batch(sample, net, O.NET_F32, threads=threads)
        out["cpu_baseline"] = {"value": round(ni / sec, 1), "unit": "node-iters/s", "cores": threads,
                               "kind": "port", "leaf_queries_per_s": round(lq / sec, 1),
                               "sample": f"first {n} of the {len(jobs)} subgames, all {iters} iterations + Phase 2, "
                                         f"one subgame per thread at a time, f32 net, {sec:.1f} s wall",
                               "cpu": host, "cpu_share": share}
        log(f"[bench] CPU oracle: {sec:.1f}s, {ni / sec:.0f} node-iters/s")

        if not args.no_accuracy:
            # The timed wave's results on the sampled subgames against the float32
            # CPU solver: root errors relative to each subgame's largest root value,
            # the reference's gate for its fast head (engine/src/gpu/tests.rs:413-444),
            # and mean strategy errors. Outside the timed region.
            from concurrent.futures import ThreadPoolExecutor

            if dev_results is None:
                dev_results = ex.solve(wave, ver)
            with ThreadPoolExecutor(threads) as pool:
                refs = list(pool.map(lambda j: O.solve(j, net, O.NET_F32), sample))
            rel, gate, ms_err = [], [], []
            for g, o in zip(dev_results, refs):
                a, b = g.root_values.astype(np.float64), o["roots"].astype(np.float64)
                rel.append(float(np.abs(a - b).max() / np.abs(b).max()))
                gate.append(float((np.abs(a - b) / (1e-2 + 2e-3 * np.maximum(np.abs(a), np.abs(b)))).max()))
                ms_err.append(float(np.abs(g.strategy - o["strategy"]).mean()))
            rel = np.array(rel)
            out["accuracy"] = {
                "against": f"float32 CPU solver (the oracle), first {n} of the {len(jobs)} subgames",
                "root_rel_err_median": float(np.median(rel)), "root_rel_err_max": float(rel.max()),
                "subgames_within_2e-3": int((rel <= 2e-3).sum()), "subgames": n,
                "root_gate_ratio_max": round(max(gate), 4), "mean_strategy_err_max": float(max(ms_err)),
                "note": "root errors relative to each subgame's largest |root value|; root_gate_ratio = |d| / "
                        "(1e-2 + 2e-3 |x|), the reference's bound for its fast head (<= 1 passes)"}
            log(f"[bench] accuracy: root error median {np.median(rel):.2e}, max {rel.max():.2e}, "
                f"{int((rel <= 2e-3).sum())} of {n} within 2e-3, gate ratio {max(gate):.2f}")

    ex.close()
    if pk is not None:
        out["peaks"] = peaks
        for r in (out.get("roofline"), out.get("roofline_cfr_iteration"), out.get("roofline_mlp_in_wave"),
                  out.get("roofline_leaf_input"), out.get("mlp_alone"), out.get("v5_wave", {}).get("trunk_mfma"),
                  out.get("v5_wave", {}).get("join_mfma")):
            if r:
                r["frac_measured"] = round(r["achieved"] / (mfma_meas if r.get("unit") == "TFLOP/s" else hbm_meas), 5)
        for d in out["roofline_cfr_iteration"]["kernels"].values():
            d["frac_measured"] = round(d["achieved_gbs"] / hbm_meas, 5)
    if args.copy_probe:
        # A plain device-to-device copy through the HIP runtime's blit kernel:
        # the reference point that scales the HBM byte counters.
        import ctypes

        hip = ctypes.CDLL("libamdhip64.so")
        # every call's signature declared: no argument goes through ctypes' default int conversion
        hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        hip.hipFree.argtypes = [ctypes.c_void_p]
        hip.hipDeviceSynchronize.argtypes = []
        for f in (hip.hipMalloc, hip.hipMemcpy, hip.hipFree, hip.hipDeviceSynchronize):
            f.restype = ctypes.c_int
        n = args.copy_probe << 20
        src, dst = ctypes.c_void_p(), ctypes.c_void_p()
        assert hip.hipMalloc(ctypes.byref(src), ctypes.c_size_t(n)) == 0
        assert hip.hipMalloc(ctypes.byref(dst), ctypes.c_size_t(n)) == 0
        for _ in range(3):
            assert hip.hipMemcpy(dst, src, ctypes.c_size_t(n), 3) == 0  # hipMemcpyDeviceToDevice
        assert hip.hipDeviceSynchronize() == 0
        hip.hipFree(src)
        hip.hipFree(dst)
        log(f"[bench] copy probe: 3 x {n} bytes read and written")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
