"""The forward and backward that bench.py and its config table time
(mxfa_run_flash_lse_ws, mxfa_run_bwd_ws: one launch for bf16, with the GQA
split's workspace where the shape has one; for fp32 the dQ pass with Delta,
then the dK/dV pass), checked at the full BASELINE sizes: against the CPU oracle on one head or one KV-head group, and on
every head against the size-independent closed forms of the VJP
(sum_j dK_j = 0, sum_j dV_j = sum over the group's query heads of sum_i dO_i).
The long sequence (cfg3) is checked on sampled rows and keys against float64.
Also explicit softmax scales at bf16 d = 64: a power of two other than
1/sqrt(d), and a scale that is not a power of two."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_helpers import (TOL_BF16, TOL_F32, gpu_fwd_bwd, gpu_fwd_bwd_timed, make_inputs, oracle_fwd_bwd, parity,
                         rel_err)
from test_gpu_configs import _closed_forms, _keys_f64, _rows_f64

pytestmark = pytest.mark.gpu


def _one_launch(q, k, causal, bf16):
    import mx230_amd as mx
    from gpu_helpers import to_dev
    return mx.bwd_one_launch(to_dev(q[:1, :1, :1], bf16), to_dev(k[:1, :1, :1], bf16), causal)


def _group(name, q, k, v, do, causal, b, kvh, bf16=True):
    import mx230_amd as mx
    B, Hq, N, d = q.shape
    Hkv = k.shape[1]
    grp = Hq // Hkv
    n0 = mx.bwd_delta_fallbacks()
    print(f"\n[{name}] timed path B{B} Hq{Hq} Hkv{Hkv} N{N} d{d} causal={causal} bf16={bf16}", flush=True)
    gpu = gpu_fwd_bwd_timed(q, k, v, do, causal, bf16)
    print(f"[{name}] one launch {_one_launch(q, k, causal, bf16)}, Delta fallbacks {mx.bwd_delta_fallbacks() - n0}",
          flush=True)
    hs = slice(kvh * grp, (kvh + 1) * grp)
    ref = oracle_fwd_bwd(q[b:b + 1, hs], k[b:b + 1, kvh:kvh + 1], v[b:b + 1, kvh:kvh + 1],
                         do[b:b + 1, hs], causal)
    sub = (gpu[0][b:b + 1, hs], gpu[1][b:b + 1, hs], gpu[2][b:b + 1, hs], gpu[3][b:b + 1, hs],
           gpu[4][b:b + 1, kvh:kvh + 1], gpu[5][b:b + 1, kvh:kvh + 1])
    errs, bad = parity(sub, ref, TOL_BF16 if bf16 else TOL_F32)
    print(f"[{name}] group (b={b}, kvh={kvh}): " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()),
          flush=True)
    assert not bad, (name, errs)
    _closed_forms(gpu, do, Hkv)
    return gpu


def test_north_star_timed_path():
    """B4 H12 N4096 d64 causal bf16, head (b=3, h=10) against the oracle."""
    q, k, v, do = make_inputs(4, 12, 12, 4096, 64, bf16=True)
    _group("north-star", q, k, v, do, True, b=3, kvh=10)


def test_cfg4_timed_path():
    """Qwen2.5: B2 Hq14 Hkv2 N4096 causal, split over 7 shares through the workspace."""
    q, k, v, do = make_inputs(2, 14, 2, 4096, 64, bf16=True)
    _group("cfg4", q, k, v, do, True, b=0, kvh=1)


@pytest.mark.parametrize("d", [64, 128])
def test_cfg5_timed_path(d):
    """TinyLlama: B1 Hq32 Hkv4 N2048 causal, Q/K/V x0.5, split over 8 shares."""
    q, k, v, do = make_inputs(1, 32, 4, 2048, d, mult_qkv=0.5, bf16=True)
    _group(f"cfg5-d{d}", q, k, v, do, True, b=0, kvh=3)


def test_cfg1_timed_path():
    """The reference's CPU case: B1 H1 N256 d64 non-causal fp32, the whole
    tensor against the oracle."""
    q, k, v, do = make_inputs(1, 1, 1, 256, 64)
    _group("cfg1", q, k, v, do, False, b=0, kvh=0, bf16=False)


def test_cfg2_timed_path():
    """GPT-2: B4 H12 N1024 d64 causal fp32, Q/K/V x0.5, head (b=2, h=7)
    against the oracle, closed forms on every head."""
    q, k, v, do = make_inputs(4, 12, 12, 1024, 64, mult_qkv=0.5)
    _group("cfg2", q, k, v, do, True, b=2, kvh=7, bf16=False)


def test_cfg3_f32_timed_path():
    """B1 H12 N32768 d64 non-causal fp32: sampled rows and keys of head 9
    against float64 (fp32 bar, 1e-4), closed forms on every head."""
    B, H, N, d = 1, 12, 32768, 64
    q, k, v, do = make_inputs(B, H, H, N, d)
    print("\n[cfg3-f32] timed path", flush=True)
    gpu = gpu_fwd_bwd_timed(q, k, v, do, False, False)
    h = 9
    rows = np.array([0, 5, 4097, 20000, N - 1])
    o_r, lse_r, dq_r = _rows_f64(q[0, h], k[0, h], v[0, h], do[0, h], rows)
    for name, g_, r_ in (("O", gpu[0][0, h][rows], o_r), ("LSE", gpu[1][0, h][rows], lse_r),
                         ("dQ", gpu[3][0, h][rows], dq_r)):
        e = rel_err(g_, r_)
        print(f"[cfg3-f32] {name} sampled rows {e:.2e}", flush=True)
        assert e <= TOL_F32, (name, e)
    keys = np.array([2, 8191, 30000, N - 1])
    dk_r, dv_r = _keys_f64(q[0, h], k[0, h], v[0, h], do[0, h], keys)
    for name, g_, r_ in (("dK", gpu[4][0, h][keys], dk_r), ("dV", gpu[5][0, h][keys], dv_r)):
        e = rel_err(g_, r_)
        print(f"[cfg3-f32] {name} sampled keys {e:.2e}", flush=True)
        assert e <= TOL_F32, (name, e)
    _closed_forms(gpu, do, H)


def test_cfg3_bf16_timed_path():
    """B1 H12 N32768 d64 non-causal bf16: sampled rows and keys of head 4
    against float64, closed forms on every head."""
    B, H, N, d = 1, 12, 32768, 64
    q, k, v, do = make_inputs(B, H, H, N, d, bf16=True)
    print("\n[cfg3-bf16] timed path", flush=True)
    gpu = gpu_fwd_bwd_timed(q, k, v, do, False, True)
    h = 4
    rows = np.array([0, 3, 8191, 16385, 29999, N - 1])
    o_r, lse_r, dq_r = _rows_f64(q[0, h], k[0, h], v[0, h], do[0, h], rows)
    for name, g_, r_ in (("O", gpu[0][0, h][rows], o_r), ("LSE", gpu[1][0, h][rows], lse_r),
                         ("dQ", gpu[3][0, h][rows], dq_r)):
        e = rel_err(g_, r_)
        print(f"[cfg3-bf16] {name} sampled rows {e:.2e}", flush=True)
        assert e <= TOL_BF16, (name, e)
    keys = np.array([1, 4096, 25000, N - 2])
    dk_r, dv_r = _keys_f64(q[0, h], k[0, h], v[0, h], do[0, h], keys)
    for name, g_, r_ in (("dK", gpu[4][0, h][keys], dk_r), ("dV", gpu[5][0, h][keys], dv_r)):
        e = rel_err(g_, r_)
        print(f"[cfg3-bf16] {name} sampled keys {e:.2e}", flush=True)
        assert e <= TOL_BF16, (name, e)
    _closed_forms(gpu, do, H)


@pytest.mark.parametrize("scale", [0.25, 0.1], ids=["pow2", "general"])
@pytest.mark.parametrize("causal", [True, False])
def test_bf16_d64_scales(scale, causal):
    """Explicit softmax scales at bf16 d = 64, GQA with ragged N, through the
    two-launch flash backward and through the timed one launch."""
    q, k, v, do = make_inputs(2, 6, 2, 333, 64, bf16=True, seeds=(71, 72, 73, 74))
    ref = oracle_fwd_bwd(q, k, v, do, causal, scale=scale)
    for path, fn in (("flash", gpu_fwd_bwd), ("timed", gpu_fwd_bwd_timed)):
        gpu = fn(q, k, v, do, causal, True, scale=scale)
        errs, bad = parity(gpu, ref, TOL_BF16)
        print(f"\n[scale {scale} causal={causal} {path}] " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()),
              flush=True)
        assert not bad, (path, errs)
