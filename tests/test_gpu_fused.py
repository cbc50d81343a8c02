"""The backward with Delta folded into the dQ pass (mxfa_run_bwd /
mxfa_run_bwd_dq_delta): dQ, dK, dV against the CPU oracle at the same
tolerances as the two-launch path (1e-4 fp32, 2e-2 bf16 of max magnitude), the
Delta it writes against the oracle's rowsum(dO * O) of the GPU's own O, and the
outputs against the reference-shaped sequence (mxfa_run_preprocess +
mxfa_run_bwd_flash), which differs only in the summation order of Delta."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_helpers import TOL_BF16, TOL_F32, make_inputs, oracle_fwd_bwd, rel_err, to_dev, to_np

pytestmark = pytest.mark.gpu


def _run(q, k, v, do, causal, bf16):
    import torch
    import mx230_amd as mx
    tq, tk, tv, tdo = (to_dev(x, bf16) for x in (q, k, v, do))
    B, Hq, N, d = q.shape
    o = torch.empty_like(tq)
    lse = torch.empty((B, Hq, N), dtype=torch.float32, device="cuda")
    mx.run_flash_lse(tq, tk, tv, o, lse, causal)
    delta_f = torch.empty_like(lse)
    dq, dk, dv = torch.empty_like(tq), torch.empty_like(tk), torch.empty_like(tv)
    mx.run_bwd(tq, tk, tv, o, tdo, lse, delta_f, dq, dk, dv, causal)
    delta_p = torch.empty_like(lse)
    mx.run_preprocess(tdo, o, delta_p)
    dq2, dk2, dv2 = torch.empty_like(tq), torch.empty_like(tk), torch.empty_like(tv)
    mx.run_bwd_flash(tq, tk, tv, tdo, lse, delta_p, dq2, dk2, dv2, causal)
    torch.cuda.synchronize()
    return [to_np(t) for t in (o, delta_f, dq, dk, dv, delta_p, dq2, dk2, dv2)]


CASES = [
    ("ref-f32-n512", dict(B=1, Hq=1, Hkv=1, N=512, d=64, bf16=False), False),
    ("ref-f32-n512-causal", dict(B=1, Hq=1, Hkv=1, N=512, d=64, bf16=False), True),
    ("gqa-bf16-ragged", dict(B=2, Hq=6, Hkv=2, N=333, d=64, bf16=True), True),
    ("bf16-d128", dict(B=1, Hq=4, Hkv=4, N=256, d=128, bf16=True), False),
    ("bf16-n1", dict(B=1, Hq=2, Hkv=1, N=1, d=64, bf16=True), True),
]


@pytest.mark.parametrize("name,shape,causal", CASES, ids=[c[0] for c in CASES])
def test_fused_backward(name, shape, causal):
    bf16 = shape.pop("bf16")
    q, k, v, do = make_inputs(shape["B"], shape["Hq"], shape["Hkv"], shape["N"], shape["d"], bf16=bf16,
                              seeds=(41, 42, 43, 44))
    print(f"\n[fused {name}] {shape} causal={causal}", flush=True)
    o, delta_f, dq, dk, dv, delta_p, dq2, dk2, dv2 = _run(q, k, v, do, causal, bf16)
    tol = TOL_BF16 if bf16 else TOL_F32
    ref = oracle_fwd_bwd(q, k, v, do, causal)
    errs = {"dQ": rel_err(dq, ref[2]), "dK": rel_err(dk, ref[3]), "dV": rel_err(dv, ref[4])}
    # Delta of the GPU's own O (attention_bwd.cu:32-44)
    delta_ref = oracle.delta(do, o, q.shape[-1]).reshape(delta_f.shape)
    errs["Delta"] = rel_err(delta_f, delta_ref)
    print(f"[fused {name}] " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    assert all(e <= tol for e in errs.values()), errs
    # against the two-launch sequence: Delta to fp32 summation-order noise, the
    # gradients to that noise propagated (bf16 outputs: one rounding step)
    assert rel_err(delta_f, delta_p) <= 1e-5
    same = 1e-5 if not bf16 else 1e-2
    for a, b in ((dq, dq2), (dk, dk2), (dv, dv2)):
        assert rel_err(a, b) <= same
