"""The five synthetic workloads of the wave executor, as generator specs.

Each maps one benchmark/parity configuration onto the job contract:
  tree48    one depth-1 subgame from seed 0: 48 decision nodes, 64 leaves, branching
      (private actions) U{3..12}, 22 infostates per player with uniform beliefs,
      f32 MLP 512 -> 3x384 -> 22 heads, DCFR(1.5, 0, 2) for 16 iterations.
  mlp65k    the leaf MLP alone: 65,536 queries, 512 -> 384 -> 384 -> 384 -> 64.
  wave64    64 depth-1 subgames: 32..128 public nodes, branching 3..12, lognormal
      infostates (median 22, p99 567, cap 567), Dirichlet(1) beliefs, f16 MLP,
      64 iterations.
  wave256   256 depth-2 subgames: 200..800 public nodes, chance nodes (2..6 uniform
      outcomes) after every decision ply, lognormal infostates, f16 MLP with one
      head row per infostate (567), 64 iterations.
  wave512w  512 depth-2 subgames, 10% whales (2,000 nodes, 567 infostates), 128
      iterations, two-tower bf16 net (512 -> 2x512 public, 96 -> 2x512 private).
  wave256v5 the 256-subgame wave's trees with the reference's production v5 leaf
      network (net_dims [5]): per-row public bytes (the GPU row format), per-job
      card tables, per-config hand / face-down / bag counts.
"""
from __future__ import annotations

import warchest_wave as ww

DCFR = dict(alpha=1.5, beta=0.0, gamma=2.0, predict=0.0)

MLP_TREE48 = ww.mlp_dims(inputs=512, hidden=384, layers=3, heads=22, pool=64)
MLP_65K = ww.mlp_dims(inputs=512, hidden=384, layers=3, heads=64, pool=64)
MLP_WAVE = ww.mlp_dims(inputs=512, hidden=384, layers=3, heads=567, pool=64)
TWO_TOWER = ww.two_tower_dims(inputs=512, width=512, pub_layers=2, priv_in=96, priv_layers=2, pool=64)

NET_SEED = 1
FEATURE_SEED = 7
MLP65K_ROWS = 65536

SPECS = {
    "tree48": dict(net_dims=MLP_TREE48, seed=0, trees=1, exact_decisions=48, exact_leaves=64, act_lo=3, act_hi=12,
               chance=0, info_fixed=22, dirichlet=0, iters=16, depth=1, snapshots=1, nroots=1, **DCFR),
    "wave64": dict(net_dims=MLP_WAVE, seed=3, trees=64, nodes_lo=32, nodes_hi=128, act_lo=3, act_hi=12,
               collapse=0.6, chance=0, info_median=22.0, info_p99=567.0, info_cap=567, dirichlet=1,
               iters=64, depth=1, snapshots=1, nroots=1, **DCFR),
    "wave256": dict(net_dims=MLP_WAVE, seed=4, trees=256, nodes_lo=200, nodes_hi=800, act_lo=3, act_hi=12,
               collapse=0.6, chance=1, draw_lo=2, draw_hi=6, info_median=22.0, info_p99=567.0, info_cap=567,
               dirichlet=1, iters=64, depth=2, snapshots=1, nroots=1, **DCFR),
    "wave512w": dict(net_dims=TWO_TOWER, seed=5, trees=512, nodes_lo=200, nodes_hi=800, act_lo=3, act_hi=12,
               collapse=0.6, chance=1, draw_lo=2, draw_hi=6, info_median=22.0, info_p99=567.0, info_cap=567,
               dirichlet=1, whale_frac=0.1, whale_nodes=2000, whale_info=567, iters=128, depth=2,
               snapshots=1, nroots=1, **DCFR),
    "wave256v5": dict(net_dims=ww.V5_DIMS, seed=4, trees=256, nodes_lo=200, nodes_hi=800, act_lo=3, act_hi=12,
               collapse=0.6, chance=1, draw_lo=2, draw_hi=6, info_median=22.0, info_p99=567.0, info_cap=567,
               dirichlet=1, iters=64, depth=2, snapshots=1, nroots=1, **DCFR),
}


def jobs(name: str, **overrides) -> list:
    spec = dict(SPECS[name])
    spec.update(overrides)
    dims = spec.pop("net_dims")
    return ww.synth_jobs(dims, **spec)


def net_for(name: str, seed: int = NET_SEED) -> ww.Net:
    dims = MLP_65K if name == "mlp65k" else SPECS[name]["net_dims"]
    return ww.synth_weights(dims, seed)


def mlp65k_inputs(rows: int = MLP65K_ROWS, seed: int = FEATURE_SEED):
    return ww.synth_features(rows, MLP_65K[1], seed)
