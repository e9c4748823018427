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
- every subgame's mean strategy error is within `mean_strategy`.

A device error in the leaf values themselves is caught tightly by the leaf
probes (tests/test_gpu_waves.py), which compare one network evaluation, a
well-conditioned quantity, against the oracle's model of the operand rounding.
"""
import numpy as np


def check(dev, emu, mean_strategy, mean_strategy_bound, say, tag, frac=0.85):
    dev, emu, ms = np.asarray(dev, np.float64), np.asarray(emu, np.float64), np.asarray(mean_strategy)
    bound = np.maximum(2e-3, 1.5 * emu + 2e-4)
    inside = dev <= bound
    for k in range(len(dev)):
        say(f"{tag} tree {k}: root error {dev[k]:.2e} (emulations {emu[k]:.2e}, envelope {bound[k]:.2e}"
            f"{'' if inside[k] else ', OUTSIDE'}), mean strategy error {ms[k]:.2e}")
    say(f"{tag}: {int(inside.sum())} of {len(dev)} inside their envelope; median root error device "
        f"{np.median(dev):.2e} vs emulations {np.median(emu):.2e}; within 2e-3: device {int((dev <= 2e-3).sum())}, "
        f"emulations {int((emu <= 2e-3).sum())}")
    assert (ms <= mean_strategy_bound).all(), f"{tag}: mean strategy error {ms.max():.2e}"
    assert inside.mean() >= frac, f"{tag}: only {int(inside.sum())} of {len(dev)} subgames inside the envelope"
    assert np.median(dev) <= 2.0 * np.median(emu) + 1e-4, f"{tag}: median root error"
