"""The forward and backward that bench.py and its config table time
(mxfa_run_flash_lse_ws, mxfa_run_bwd_ws: one launch for bf16, with the GQA
split's workspace where the shape has one; for fp32 the dQ pass with Delta,
then the dK/dV pass), checked at the full BASELINE sizes: every element of O,
LSE, dQ, dK and dV against the CPU oracle (the whole tensor, as
run_verify_bwd compares it, 02-flash-attention/src/main.rs:477-497), and each
head or KV head against its own largest reference value as well, plus the
size-independent closed forms of the VJP (sum_j dK_j = 0, sum_j dV_j = sum over
the group's query heads of sum_i dO_i). The long sequence (cfg3) is checked on
sampled rows and keys against float64.
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


def _per_head(gpu, ref, tol):
    """The parity metric of every (batch, head) slice of each output, each
    relative to its own slice's largest reference value: the worst slice per
    output and the slices over tolerance."""
    names = ("O", "LSE", "dQ", "dK", "dV")
    got = (gpu[0], gpu[1], gpu[3], gpu[4], gpu[5])
    worst, bad = {}, []
    for n, g, r in zip(names, got, ref):
        e = [(rel_err(g[b, h], r[b, h]), b, h) for b in range(r.shape[0]) for h in range(r.shape[1])]
        worst[n] = max(e)
        bad += [(n, b, h, x) for x, b, h in e if not x <= tol]
    return worst, bad


def _whole(name, q, k, v, do, causal, bf16=True):
    """The timed launches on the whole shape against the oracle on every head."""
    import mx230_amd as mx
    B, Hq, N, d = q.shape
    Hkv = k.shape[1]
    tol = TOL_BF16 if bf16 else TOL_F32
    n0 = mx.bwd_delta_fallbacks()
    print(f"\n[{name}] timed path B{B} Hq{Hq} Hkv{Hkv} N{N} d{d} causal={causal} bf16={bf16}", flush=True)
    gpu = gpu_fwd_bwd_timed(q, k, v, do, causal, bf16)
    print(f"[{name}] one launch {_one_launch(q, k, causal, bf16)}, Delta fallbacks {mx.bwd_delta_fallbacks() - n0}",
          flush=True)
    ref = oracle_fwd_bwd(q, k, v, do, causal)
    errs, bad = parity(gpu, ref, tol)
    print(f"[{name}] whole tensors ({B * Hq} heads): " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()),
          flush=True)
    worst, bad_heads = _per_head(gpu, ref, tol)
    print(f"[{name}] worst head: " + " ".join(f"{n}={e:.2e}@(b{b},h{h})" for n, (e, b, h) in worst.items()),
          flush=True)
    assert not bad, (name, errs)
    assert not bad_heads, (name, bad_heads[:8])
    _closed_forms(gpu, do, Hkv)
    return gpu


def test_north_star_timed_path():
    """B4 H12 N4096 d64 causal bf16: all 48 heads against the oracle."""
    q, k, v, do = make_inputs(4, 12, 12, 4096, 64, bf16=True)
    _whole("north-star", q, k, v, do, True)


def test_cfg4_timed_path():
    """Qwen2.5: B2 Hq14 Hkv2 N4096 causal, split over 7 shares through the
    workspace: all 28 query heads and 4 KV heads against the oracle."""
    q, k, v, do = make_inputs(2, 14, 2, 4096, 64, bf16=True)
    _whole("cfg4", q, k, v, do, True)


@pytest.mark.parametrize("d", [64, 128])
def test_cfg5_timed_path(d):
    """TinyLlama: B1 Hq32 Hkv4 N2048 causal, Q/K/V x0.5, split over 8 shares:
    all 32 query heads and 4 KV heads against the oracle."""
    q, k, v, do = make_inputs(1, 32, 4, 2048, d, mult_qkv=0.5, bf16=True)
    _whole(f"cfg5-d{d}", q, k, v, do, True)


def test_cfg1_timed_path():
    """The reference's CPU case: B1 H1 N256 d64 non-causal fp32, the whole
    tensor against the oracle."""
    q, k, v, do = make_inputs(1, 1, 1, 256, 64)
    _whole("cfg1", q, k, v, do, False, bf16=False)


def test_cfg2_timed_path():
    """GPT-2: B4 H12 N1024 d64 causal fp32, Q/K/V x0.5: all 48 heads against
    the oracle."""
    q, k, v, do = make_inputs(4, 12, 12, 1024, 64, mult_qkv=0.5)
    _whole("cfg2", q, k, v, do, True, bf16=False)


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
