"""GPU parity of the opt-in ping-pong dK/dV kernel (bf16, d = 64), selected with
MXFA_DKV_KERNEL=pingpong, against the CPU oracle and against the default 4-wave
kernel on the same inputs. Same tolerances as the default path: 2e-2 of each
output's max magnitude."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_helpers import TOL_BF16, gpu_fwd_bwd, make_inputs, oracle_fwd_bwd, parity, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture
def pingpong(monkeypatch):
    monkeypatch.setenv("MXFA_DKV_KERNEL", "pingpong")


def _check(case, q, k, v, do, causal):
    print(f"\n[pingpong {case}] q{q.shape} k{k.shape} causal={causal}", flush=True)
    gpu = gpu_fwd_bwd(q, k, v, do, causal, True)
    ref = oracle_fwd_bwd(q, k, v, do, causal)
    errs, bad = parity(gpu, ref, TOL_BF16)
    print(f"[pingpong {case}] " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    assert not bad, f"{case}: {bad} over {TOL_BF16}: {errs}"
    return gpu


@pytest.mark.parametrize("causal", [False, True])
def test_pingpong_ragged_and_tiny(pingpong, causal):
    # N = 1, 2: one stage (the ring's prologue only); 65..300: partial last
    # stage and 2-5 stages, so every ring slot and both group loops are hit
    for n in (1, 2, 31, 63, 64, 65, 127, 128, 129, 200, 300):
        q, k, v, do = make_inputs(1, 2, 1, n, 64, bf16=True, seeds=(5, 6, 7, 8))
        _check(f"n{n}", q, k, v, do, causal)


@pytest.mark.parametrize("causal", [False, True])
def test_pingpong_gqa(pingpong, causal):
    """7 query heads per KV head: the stage sequence crosses query heads."""
    q, k, v, do = make_inputs(2, 14, 2, 512, 64, bf16=True)
    _check("qwen-gqa-n512", q, k, v, do, causal)


@pytest.mark.parametrize("causal", [False, True])
def test_pingpong_matches_default_kernel(monkeypatch, causal):
    """Same inputs through both dK/dV kernels: identical forward and dQ, and
    dK/dV within the bf16 tolerance of each other (they sum the same terms in
    a different order)."""
    q, k, v, do = make_inputs(2, 4, 2, 1024, 64, bf16=True, seeds=(21, 22, 23, 24))
    monkeypatch.delenv("MXFA_DKV_KERNEL", raising=False)
    base = gpu_fwd_bwd(q, k, v, do, causal, True)
    monkeypatch.setenv("MXFA_DKV_KERNEL", "pingpong")
    pp = gpu_fwd_bwd(q, k, v, do, causal, True)
    for i in (0, 1, 2, 3):  # O, LSE, Delta, dQ do not involve the dK/dV kernel
        assert np.array_equal(base[i], pp[i])
    for name, i in (("dK", 4), ("dV", 5)):
        e = rel_err(pp[i], base[i])
        print(f"[pingpong vs default] {name} {e:.2e}", flush=True)
        assert e <= TOL_BF16, (name, e)
