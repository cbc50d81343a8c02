"""A seeded sweep of shapes through the path bench.py times (the forward, then
mxfa_run_bwd_ws: the one launch for bf16, in its two-wave form on grids the
three-wave kernel holds at once, with the GQA split where the shape has one;
two launches for fp32) against the oracle, at the BASELINE tolerances.

The shapes come from a fixed generator, so every run checks the same ones:
batch 1-3, query heads per KV head 1-8, 1-2 KV heads, ragged lengths 1-700,
d = 64 and 128, causal and not, bf16 and fp32 (d = 64), the default softmax
scale and a general one. They cover combinations the named tests do not:
groups of 3 and 5 split over work-groups, lengths that end inside a 64-row
stage, one-row heads under the split.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_helpers import TOL_BF16, TOL_F32, gpu_fwd_bwd_timed, make_inputs, oracle_fwd_bwd, parity

pytestmark = pytest.mark.gpu


def _cases(n=24, seed=20261202):
    rng = np.random.RandomState(seed)
    cases = []
    for i in range(n):
        bf16 = bool(rng.rand() < 0.75)
        d = int(rng.choice([64, 128])) if bf16 else 64
        B = int(rng.randint(1, 4))
        hkv = int(rng.randint(1, 3))
        group = int(rng.choice([1, 2, 3, 5, 7, 8]))
        N = int(rng.choice([1, 17, 63, 64, 65, 127, 129, 200, 333, 511, 640, 700]))
        causal = bool(rng.rand() < 0.6)
        scale = 0.1 if rng.rand() < 0.3 else 0.0
        cases.append((B, hkv * group, hkv, N, d, causal, bf16, scale, 100 + 4 * i))
    return cases


# One-row heads (N = 1: dQ and dK cancel to exactly zero in the oracle, and the
# GPU's rounding is measured against the size of what cancels, cancel_scale),
# with wide groups and a large scale, where that rounding is largest: the first
# is a shape a wider seeded sweep found over the fixed 1e-2 floor
ONE_ROW = [
    (2, 12, 1, 1, 64, True, False, 0.3, 9001),
    (1, 32, 1, 1, 128, True, True, 0.3, 9005),
    (3, 16, 2, 1, 64, False, True, 0.0, 9009),
    (1, 8, 1, 1, 64, False, False, 0.05, 9013),
]
CASES = _cases() + ONE_ROW


def _id(c):
    B, H, Hkv, N, d, causal, bf16, scale, _ = c
    return f"B{B}H{H}kv{Hkv}N{N}d{d}{'c' if causal else 'n'}{'bf16' if bf16 else 'f32'}{'s' if scale else ''}"


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_sweep_timed_path(case):
    B, H, Hkv, N, d, causal, bf16, scale, seed = case
    q, k, v, do = make_inputs(B, H, Hkv, N, d, bf16=bf16, seeds=(seed, seed + 1, seed + 2, seed + 3))
    print(f"\n[sweep] {_id(case)} scale={scale or 'default'} seed={seed}", flush=True)
    ref = oracle_fwd_bwd(q, k, v, do, causal, scale=scale or None)
    gpu = gpu_fwd_bwd_timed(q, k, v, do, causal, bf16, scale=scale)
    errs, bad = parity(gpu, ref, TOL_BF16 if bf16 else TOL_F32, inputs=(q, k, v, do, scale or None))
    print("[sweep] " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    assert not bad, errs
