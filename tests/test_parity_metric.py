"""The parity metric's one-key case (gpu_helpers.cancel_scale), on the CPU.

With N = 1 the oracle's dQ and dK are exactly zero, so the relative bar is
applied to the magnitude of the terms that cancel. These tests pin that the
premise holds for the oracle, that rounding-sized results pass, and that a
result which drops the Delta term (dS = P dP instead of P (dP - Delta), the
mistake the cancellation hides) fails by orders of magnitude.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_helpers import TOL_F32, cancel_scale, make_inputs, oracle_fwd_bwd, parity

SHAPES = [(2, 12, 1, 64, 0.3), (1, 32, 4, 128, None), (3, 4, 4, 64, 0.05)]


def _no_delta(q, k, v, do, scale):
    """dQ, dK of one key with the Delta term dropped: dS_h = dP_h = dO_h . V_0."""
    B, Hq, _, d = q.shape
    g = Hq // k.shape[1]
    s = scale if scale else 1.0 / np.sqrt(d)
    kv = np.arange(Hq) // g
    dp = (do * v[:, kv]).sum(-1, keepdims=True)
    dq = s * dp * k[:, kv]
    dk = s * (dp * q).reshape(B, k.shape[1], g, 1, d).sum(axis=2)
    return dq.astype(np.float32), dk.astype(np.float32)


@pytest.mark.parametrize("B,Hq,Hkv,d,scale", SHAPES)
def test_one_key_metric(B, Hq, Hkv, d, scale):
    q, k, v, do = make_inputs(B, Hq, Hkv, 1, d, seeds=(71, 72, 73, 74))
    ref = oracle_fwd_bwd(q, k, v, do, True, scale=scale)
    # the premise: the oracle's own sums cancel exactly
    assert not ref[2].any() and not ref[3].any()
    lse = ref[1]
    inputs = (q, k, v, do, scale)
    dq_den, dk_den = cancel_scale(*inputs)

    # rounding of the size u |dP| (u = 2^-24), a few ulps per element: passes
    rng = np.random.RandomState(5)
    u = 2.0 ** -24
    noise_q = (rng.standard_normal(q.shape) * 8 * u * dq_den).astype(np.float32)
    noise_k = (rng.standard_normal(k.shape) * 8 * u * dk_den).astype(np.float32)
    ok = (ref[0], lse, None, noise_q, noise_k, ref[4])
    errs, bad = parity(ok, ref, TOL_F32, inputs=inputs)
    assert not bad, errs

    # Delta dropped: the error is the cancelling terms themselves
    dq_bad, dk_bad = _no_delta(q, k, v, do, scale)
    for got, name in (((ref[0], lse, None, dq_bad, noise_k, ref[4])), "dQ"), \
                     (((ref[0], lse, None, noise_q, dk_bad, ref[4])), "dK"):
        errs, bad = parity(got, ref, TOL_F32, inputs=inputs)
        assert bad == [name] and errs[name] > 1e3 * TOL_F32, errs


def test_one_key_metric_needs_one_key():
    q, k, v, do = make_inputs(1, 2, 1, 2, 64, seeds=(71, 72, 73, 74))
    with pytest.raises(AssertionError):
        cancel_scale(q, k, v, do)
