"""Shared helpers of the GPU parity tests: seeded inputs (the oracle's
generators, so CPU and GPU see identical bits), one call of the HIP path through
the C ABI, and the parity metric.

Parity metric (BASELINE / SURVEY §8c): for each output,
max|got - ref| / max|ref| <= 1e-4 for fp32 and <= 2e-2 for bf16, where the CPU
oracle consumes the bf16-rounded inputs widened to fp32.
"""
from __future__ import annotations

import os

import numpy as np

import oracle

TOL_F32 = 1e-4
TOL_BF16 = 2e-2
ORACLE_THREADS = min(16, os.cpu_count() or 1)


# Denominator floor of the parity metric. An output whose exact value is
# identically zero (N = 1 gives dQ = dK = 0, since dP - Delta cancels) has no
# magnitude to be relative to; the GPU returns fp32 cancellation noise there
# (~5e-7 for N(0,1) inputs), so without the inputs such outputs are compared
# against 1e-2 of the O(1) input scale. Given the inputs, parity() uses
# cancel_scale() instead.
ZERO_FLOOR = 1e-2


def rel_err(got, want, denom=None) -> float:
    """max|got - want| / max|want| (floored at ZERO_FLOOR), or over denom when given."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    if want.size == 0:
        return 0.0
    if denom is None:
        denom = max(float(np.abs(want).max()), ZERO_FLOOR)
    return float(np.abs(got - want).max() / denom)


def cancel_scale(q, k, v, do, scale=None):
    """The magnitudes of the terms that cancel in dQ and dK when N = 1.

    With one key every query's softmax weight is 1, O = V_0 and Delta_i =
    dO_i . O_i equals dP_i = dO_i . V_0, so dS = P (dP - Delta) and with it dQ
    and dK are exactly zero (the oracle's own sums cancel to 0). A kernel that
    forms dP and Delta in different summation orders leaves fp32 rounding of
    the size u |dP| there, summed over the group's query heads for dK. The
    relative bar applied to the magnitude of what cancels is
        dQ_i: scale |dP_i| max|K_0|,    dK_0: scale max_x sum_h |dP_h| |Q_hx|,
    so a kernel that drops or mis-weights the Delta term (error of that
    magnitude) fails it, and rounding noise (u of it) passes. Returns
    (dQ denominator, dK denominator)."""
    B, Hq, N, d = q.shape
    Hkv = k.shape[1]
    assert N == 1, "the exact cancellation holds for one key only"
    g = Hq // Hkv
    s = float(scale) if scale else 1.0 / np.sqrt(d)
    kv = np.arange(Hq) // g  # query head h reads KV head h / (Hq / Hkv), as the oracle
    q64, k64, v64, do64 = (np.asarray(x, np.float64) for x in (q, k, v, do))
    dp = np.abs((do64 * v64[:, kv]).sum(-1, keepdims=True))  # [B, Hq, 1, 1]
    dq_den = s * float((dp * np.abs(k64[:, kv])).max())
    dk_den = s * float((dp * np.abs(q64)).reshape(B, Hkv, g, 1, d).sum(axis=2).max())
    return max(dq_den, 1e-30), max(dk_den, 1e-30)


def make_inputs(B, Hq, Hkv, N, d, mult_qkv=1.0, bf16=False, seeds=(1, 2, 3, 4), uniform=False):
    """Q, K, V, dO as float32 numpy arrays ([B,H,N,d]); bf16-rounded if bf16.
    Seeds follow the reference convention Q=1, K=2, V=3, dO=4 (main.rs:584-587)."""
    qn, kn = B * Hq * N * d, B * Hkv * N * d
    if uniform:
        gen = lambda n, s, m: oracle.pseudo_rand(n, s) * np.float32(m)  # noqa: E731
    else:
        gen = lambda n, s, m: oracle.normal(n, s, m)  # noqa: E731
    q = gen(qn, seeds[0], mult_qkv).reshape(B, Hq, N, d)
    k = gen(kn, seeds[1], mult_qkv).reshape(B, Hkv, N, d)
    v = gen(kn, seeds[2], mult_qkv).reshape(B, Hkv, N, d)
    do = gen(qn, seeds[3], 1.0).reshape(B, Hq, N, d)
    if bf16:
        q, k, v, do = (oracle.bf16_round(x) for x in (q, k, v, do))
    return q, k, v, do


def to_dev(x, bf16):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x))
    return t.to(device="cuda", dtype=torch.bfloat16 if bf16 else torch.float32).contiguous()


def to_np(t):
    import torch
    return t.detach().to(torch.float32).cpu().numpy()


def gpu_fwd_bwd(q, k, v, do, causal, bf16, scale=0.0):
    """Runs forward (O, LSE), preprocess (Delta) and the tiled backward on the
    GPU through the C ABI. Returns numpy float32 (O, LSE, Delta, dQ, dK, dV)."""
    import torch
    import mx230_amd as mx
    tq, tk, tv, tdo = (to_dev(x, bf16) for x in (q, k, v, do))
    B, Hq, N, d = q.shape
    o = torch.empty_like(tq)
    lse = torch.empty((B, Hq, N), dtype=torch.float32, device="cuda")
    delta = torch.empty_like(lse)
    mx.run_flash_lse(tq, tk, tv, o, lse, causal, scale)
    mx.run_preprocess(tdo, o, delta)
    dq, dk, dv = torch.empty_like(tq), torch.empty_like(tk), torch.empty_like(tv)
    mx.run_bwd_flash(tq, tk, tv, tdo, lse, delta, dq, dk, dv, causal, scale)
    torch.cuda.synchronize()
    return tuple(to_np(t) for t in (o, lse, delta, dq, dk, dv))


def gpu_fwd_bwd_timed(q, k, v, do, causal, bf16, scale=0.0):
    """The forward, then the backward exactly as bench.py and its config table
    time it: mxfa_run_bwd_ws (one launch for bf16; the dQ work computes Delta
    itself) with the GQA split's workspace where the shape has one. Returns
    numpy float32 (O, LSE, Delta, dQ, dK, dV)."""
    import torch
    import mx230_amd as mx
    tq, tk, tv, tdo = (to_dev(x, bf16) for x in (q, k, v, do))
    B, Hq, N, d = q.shape
    o = torch.empty_like(tq)
    lse = torch.empty((B, Hq, N), dtype=torch.float32, device="cuda")
    delta = torch.empty_like(lse)
    mx.run_flash_lse(tq, tk, tv, o, lse, causal, scale)
    nws = mx.bwd_workspace_bytes(tq, tk, causal)
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda") if nws else None
    dq, dk, dv = torch.empty_like(tq), torch.empty_like(tk), torch.empty_like(tv)
    mx.run_bwd_ws(tq, tk, tv, o, tdo, lse, delta, dq, dk, dv, ws, causal, scale)
    torch.cuda.synchronize()
    return tuple(to_np(t) for t in (o, lse, delta, dq, dk, dv))


def oracle_fwd_bwd(q, k, v, do, causal, scale=None):
    B, Hq, N, d = q.shape
    Hkv = k.shape[1]
    o, lse = oracle.mha_fwd(q, k, v, B, Hq, Hkv, N, d, causal, scale=scale, nthreads=ORACLE_THREADS)
    dq, dk, dv = oracle.mha_bwd(q, k, v, do, B, Hq, Hkv, N, d, causal, scale=scale,
                                nthreads=ORACLE_THREADS)
    return o, lse, dq, dk, dv


def parity(gpu, ref, tol, inputs=None):
    """gpu = (O, LSE, Delta, dQ, dK, dV), ref = (O, LSE, dQ, dK, dV): dict of errors
    and the list of outputs over tolerance. inputs = (q, k, v, do, scale): with
    one key (N = 1) dQ and dK are measured against cancel_scale()."""
    names = ("O", "LSE", "dQ", "dK", "dV")
    got = (gpu[0], gpu[1], gpu[3], gpu[4], gpu[5])
    dens = [None] * 5
    if inputs is not None and inputs[0].shape[2] == 1:
        dens[2], dens[3] = cancel_scale(*inputs)
    errs = {n: rel_err(g, r, den) for n, g, r, den in zip(names, got, ref, dens)}
    bad = [n for n, e in errs.items() if not e <= tol]
    return errs, bad
