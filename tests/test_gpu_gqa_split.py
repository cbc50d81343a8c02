"""GPU checks of the split dK/dV pass for GQA shapes (mxfa_run_bwd_ws /
mxfa_run_bwd_dkv_ws): the query heads of a KV-head group are shared among
several work-groups per key block, which write fp32 partial sums into the
caller's workspace; they are added in a fixed order by the last work-groups
of the one-launch backward (bf16), or by a second launch.

Each case compares the split backward
- with the CPU oracle on one KV-head group (bf16 2e-2, fp32 1e-4 of each
  output's max magnitude),
- with the unsplit backward (mxfa_run_bwd) on every head: the two differ only
  in the order of the fp32 sums over a group's query heads, so dK/dV agree to
  about one bf16 rounding (3e-3 of the max; 1e-5 in fp32) and dQ is bitwise
  equal (the dQ pass is the same launch),
- with itself on a second run (bitwise: the reduction order is fixed),
- bf16: with the two-launch form (its own reduce launch; bitwise equal, the
  same planes added in the same order), with no reduce wait run out.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_helpers import TOL_BF16, TOL_F32, make_inputs, oracle_fwd_bwd, parity, rel_err, to_dev, to_np

pytestmark = pytest.mark.gpu


def _run(q, k, v, do, causal, bf16, use_ws, ws=None, one_launch=True):
    """Forward, then the backward from O (run_bwd_ws with a workspace sized
    for the shape, or run_bwd). Returns numpy (O, LSE, Delta, dQ, dK, dV) and
    the workspace tensor used."""
    import torch
    import mx230_amd as mx
    tq, tk, tv, tdo = (to_dev(x, bf16) for x in (q, k, v, do))
    B, Hq, N, d = q.shape
    o = torch.empty_like(tq)
    lse = torch.empty((B, Hq, N), dtype=torch.float32, device="cuda")
    delta = torch.empty_like(lse)
    mx.run_flash_lse(tq, tk, tv, o, lse, causal)
    dq, dk, dv = torch.empty_like(tq), torch.empty_like(tk), torch.empty_like(tv)
    old = mx.set_bwd_options(one_launch=one_launch)
    try:
        if use_ws:
            need = mx.bwd_workspace_bytes(tq, tk, causal)
            assert need > 0, "shape expected to split"
            if ws is None or ws.numel() < need:
                ws = torch.empty(need, dtype=torch.uint8, device="cuda")
            mx.run_bwd_ws(tq, tk, tv, o, tdo, lse, delta, dq, dk, dv, ws, causal)
        else:
            mx.run_bwd(tq, tk, tv, o, tdo, lse, delta, dq, dk, dv, causal)
        torch.cuda.synchronize()
    finally:
        mx.set_bwd_options(**old)
    return tuple(to_np(t) for t in (o, lse, delta, dq, dk, dv)), ws


def _check(name, q, k, v, do, causal, bf16, b=0, kvh=0):
    B, Hq, N, d = q.shape
    Hkv = k.shape[1]
    grp = Hq // Hkv
    tol = TOL_BF16 if bf16 else TOL_F32
    import mx230_amd as mx
    print(f"\n[{name}] B{B} Hq{Hq} Hkv{Hkv} N{N} d{d} causal={causal} bf16={bf16}", flush=True)
    t0 = mx.bwd_reduce_timeouts()
    split, ws = _run(q, k, v, do, causal, bf16, True)
    again, _ = _run(q, k, v, do, causal, bf16, True, ws)
    assert mx.bwd_reduce_timeouts() == t0, f"{name}: a reduce wait ran out"
    unsplit, _ = _run(q, k, v, do, causal, bf16, False)
    for a, c in zip(split, again):
        assert np.array_equal(a, c), f"{name}: split backward not deterministic"
    if bf16:
        two, _ = _run(q, k, v, do, causal, bf16, True, ws, one_launch=False)
        for i, n in ((3, "dQ"), (4, "dK"), (5, "dV")):
            assert np.array_equal(split[i], two[i]), f"{name}: {n} of one launch differs from two launches"
    assert np.array_equal(split[3], unsplit[3]), f"{name}: dQ differs from the unsplit run"
    near = 3e-3 if bf16 else 1e-5
    for i, n in ((4, "dK"), (5, "dV")):
        e = rel_err(split[i], unsplit[i])
        print(f"[{name}] split vs unsplit {n}: {e:.2e}", flush=True)
        assert e <= near, (name, n, e)
    hs = slice(kvh * grp, (kvh + 1) * grp)
    ref = oracle_fwd_bwd(q[b:b + 1, hs], k[b:b + 1, kvh:kvh + 1], v[b:b + 1, kvh:kvh + 1],
                         do[b:b + 1, hs], causal)
    sub = (split[0][b:b + 1, hs], split[1][b:b + 1, hs], split[2][b:b + 1, hs], split[3][b:b + 1, hs],
           split[4][b:b + 1, kvh:kvh + 1], split[5][b:b + 1, kvh:kvh + 1])
    errs, bad = parity(sub, ref, tol)
    print(f"[{name}] oracle, group (b={b}, kvh={kvh}): " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()),
          flush=True)
    assert not bad, (name, errs)


def test_split_cfg4_qwen_full():
    """cfg4, B2 Hq14 Hkv2 N4096 d64 causal bf16: one query head per work-group."""
    q, k, v, do = make_inputs(2, 14, 2, 4096, 64, bf16=True)
    _check("split-cfg4", q, k, v, do, True, True, b=1, kvh=1)


@pytest.mark.parametrize("d", [64, 128])
def test_split_cfg5_tinyllama_full(d):
    """cfg5, B1 Hq32 Hkv4 N2048 causal bf16, Q/K/V x0.5 (d=64: 8 shares, d=128: 4)."""
    q, k, v, do = make_inputs(1, 32, 4, 2048, d, mult_qkv=0.5, bf16=True)
    _check(f"split-cfg5-d{d}", q, k, v, do, True, True, b=0, kvh=3)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n", [1, 77, 200, 576])
def test_split_ragged(causal, n):
    """Ragged and tiny N (key blocks past N, a single row) with a 4:1 group."""
    q, k, v, do = make_inputs(1, 8, 2, n, 64, bf16=True, seeds=(31, 32, 33, 34))
    _check(f"split-n{n}", q, k, v, do, causal, True, kvh=1)


@pytest.mark.parametrize("causal", [False, True])
def test_split_d128_ragged(causal):
    """d = 128 with a ragged N (the last 16-key chunk of the in-launch reduce
    half past N) and an 8:1 group."""
    q, k, v, do = make_inputs(1, 16, 2, 1000, 128, bf16=True, seeds=(71, 72, 73, 74))
    _check(f"split-d128-n1000-{'c' if causal else 'n'}", q, k, v, do, causal, True, kvh=1)


@pytest.mark.parametrize("hq,n", [(8, 643), (10, 836)], ids=["g4-n643", "g5-n836"])
def test_split_share_starts_inside_the_diagonal(hq, n):
    """Shares are runs of a key block's (query head, stage) list: at these
    shapes some run starts at the second stage of a head, inside the two
    masked stages at its diagonal (group 5 also splits heads unevenly)."""
    q, k, v, do = make_inputs(1, hq, 2, n, 64, bf16=True, seeds=(61, 62, 63, 64))
    _check(f"split-g{hq // 2}-n{n}", q, k, v, do, True, True, kvh=1)


def test_split_fp32():
    """The fp32 parity path, 2:1 group, causal."""
    q, k, v, do = make_inputs(1, 4, 2, 300, 64, seeds=(41, 42, 43, 44))
    _check("split-f32", q, k, v, do, True, False, kvh=1)


def test_workspace_reused_for_a_smaller_shape():
    """A workspace left over from a larger call holds stale partials; a
    smaller call into it must overwrite every element it reads."""
    q, k, v, do = make_inputs(1, 8, 2, 1000, 64, bf16=True, seeds=(51, 52, 53, 54))
    _, ws = _run(q, k, v, do, True, True, True)
    q2, k2, v2, do2 = make_inputs(1, 8, 2, 333, 64, bf16=True, seeds=(55, 56, 57, 58))
    got, ws2 = _run(q2, k2, v2, do2, True, True, True, ws)
    assert ws2 is ws
    want, _ = _run(q2, k2, v2, do2, True, True, False)
    for i in (4, 5):
        assert rel_err(got[i], want[i]) <= 3e-3


def test_reduce_wait_run_out():
    """The reduce work-groups' bounded wait, forced to run out from the host
    (reduce_wait_us = 0): the kernel still ends, each work-group whose shares
    were not all done writes its 16 dK and dV rows as NaN and is counted, and
    every other row is the normal result. The next call with the default
    bound is whole again."""
    import torch
    import mx230_amd as mx
    q, k, v, do = make_inputs(1, 32, 4, 2048, 64, mult_qkv=0.5, bf16=True)
    want, ws = _run(q, k, v, do, True, True, True)
    old = mx.set_bwd_options(reduce_wait_us=0)
    try:
        t0 = mx.bwd_reduce_timeouts()
        got, _ = _run(q, k, v, do, True, True, True, ws)
        ran_out = mx.bwd_reduce_timeouts() - t0
    finally:
        mx.set_bwd_options(**old)
    nan_k = np.isnan(got[4]).any(axis=-1)
    nan_v = np.isnan(got[5]).any(axis=-1)
    print(f"\n[reduce-wait-0] waits run out {ran_out}, NaN dK rows {int(nan_k.sum())}", flush=True)
    assert ran_out > 0
    assert np.array_equal(nan_k, nan_v) and np.isnan(got[4][nan_k]).all()
    assert int(nan_k.sum()) == 16 * ran_out
    assert np.array_equal(got[4][~nan_k], want[4][~nan_k]) and np.array_equal(got[5][~nan_v], want[5][~nan_v])
    assert np.array_equal(got[3], want[3])
    again, _ = _run(q, k, v, do, True, True, True, ws)
    for a, c in zip(again, want):
        assert np.array_equal(a, c)
