"""Bounds for whole reduced-precision solves against the float32 CPU solver.

A 64-iteration DCFR solve of these subgames amplifies a one-ulp change of a
single f16-rounded activation into root-value changes of the same size as the
whole f16 rounding effect (tests/test_conditioning.py): two equally faithful
f16 emulations differ per subgame by up to 2.5e-2 of the largest root value,
and a device is a third realization. Per subgame, only the envelope that the
emulations draw is meaningful; across a wave the device must follow the same
distribution:

- on at least `frac` of the subgames, the root error is within
  max(2e-3, 1.5 e + 2e-4), e the larger of the emulations' own errors;
- the median root error is within 2x the emulations' median (+1e-4);
- every subgame's mean strategy error is within `mean_strategy`;
- no subgame goes unbounded: every root error is within max(cap, 3 e). For
  plain f16 the cap is F16_CAP, the worst root error either f16 emulation
  shows on the 64-subgame wave (the pinned fixture
  tests/golden/wave64_conditioning.json): a device bug confined to a few jobs
  of a wave (a wrong offset for the last jobs, say) moves their roots by the
  roots' own size, far beyond it.

Why a subgame outside its envelope is conditioning and not a device error is
shown per evaluation in tests/test_gpu_trace.py: the oracle's solver fed the
device's own leaf values reproduces the device's solve bit for bit, and those
leaf values track the operand model at the device's own reach.

A device error in the leaf values themselves is caught tightly by the leaf
probes (tests/test_gpu_waves.py), which compare one network evaluation, a
well-conditioned quantity, against the oracle's model of the operand rounding.
"""
import json
import os

import numpy as np

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "wave64_conditioning.json")


def _worst(*models):
    with open(FIXTURE) as f:
        doc = json.load(f)
    return float(max(max(doc["models"][m]["root"]) for m in models))


# The worst root error a faithful f16 emulation (wide or float32-ascending sums)
# shows on any of the 64-subgame wave's subgames: 5.7e-2.
F16_CAP = _worst("F16", "F16A")


def check(dev, emu, mean_strategy, mean_strategy_bound, say, tag, frac=0.85, cap=F16_CAP):
    dev, emu, ms = np.asarray(dev, np.float64), np.asarray(emu, np.float64), np.asarray(mean_strategy)
    bound = np.maximum(2e-3, 1.5 * emu + 2e-4)
    hard = np.maximum(cap, 3.0 * emu)
    inside = dev <= bound
    for k in range(len(dev)):
        say(f"{tag} tree {k}: root error {dev[k]:.2e} (emulations {emu[k]:.2e}, envelope {bound[k]:.2e}"
            f"{'' if inside[k] else ', OUTSIDE'}, cap {hard[k]:.2e}), mean strategy error {ms[k]:.2e}")
    worst = int(np.argmax(dev / hard))
    assert (dev <= hard).all(), f"{tag}: tree {worst} root error {dev[worst]:.2e} beyond its cap {hard[worst]:.2e}"
    say(f"{tag}: {int(inside.sum())} of {len(dev)} inside their envelope; median root error device "
        f"{np.median(dev):.2e} vs emulations {np.median(emu):.2e}; within 2e-3: device {int((dev <= 2e-3).sum())}, "
        f"emulations {int((emu <= 2e-3).sum())}")
    assert (ms <= mean_strategy_bound).all(), f"{tag}: mean strategy error {ms.max():.2e}"
    assert inside.mean() >= frac, f"{tag}: only {int(inside.sum())} of {len(dev)} subgames inside the envelope"
    assert np.median(dev) <= 2.0 * np.median(emu) + 1e-4, f"{tag}: median root error"
