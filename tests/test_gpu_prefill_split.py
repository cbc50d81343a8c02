"""GPU parity of the prefill with its keys split over work-groups
(mxfa_run_prefill_ws, the same attn_prefill launch as mxfa_run_prefill,
03-llm-engine/kernels/llm.cu:3806-3815, for chunks whose query blocks alone
would leave most of the GPU idle).

Each split's work-group writes its unnormalised output and its rows' running
max and sum; a second launch adds them. The checks:
- the oracle, at sizes it finishes in seconds (fp32 to TOL_F32, bf16 to
  TOL_BF16), including a shape whose later splits begin at a stage that some
  of their rows precede entirely (those rows carry weight 0 into the merge);
- the unsplit prefill at the engine's shapes (Qwen2.5's 512-token chunk after
  3584 positions, a single decode-like row), to the same tolerance;
- a shape that needs no split runs the unsplit kernel: bitwise the same;
- a workspace reused by a smaller call, and one too small, refused.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_helpers import ORACLE_THREADS, TOL_BF16, TOL_F32, rel_err

pytestmark = pytest.mark.gpu


def _inputs(n_tok, pos0, nh, nkv, hd, bf16, seed):
    rng = np.random.default_rng(seed)
    nk = pos0 + n_tok
    q = rng.standard_normal((n_tok, nh * hd)).astype(np.float32)
    kc = rng.standard_normal((nk, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((nk, nkv * hd)).astype(np.float32)
    if bf16:
        q, kc, vc = (oracle.bf16_round(x) for x in (q, kc, vc))
    return q, kc, vc


def _oracle(q, kc, vc, pos0, nh, nkv, hd):
    n_tok, nk = q.shape[0], kc.shape[0]
    qf = np.zeros((1, nh, nk, hd), np.float32)
    qf[0, :, pos0:, :] = q.reshape(n_tok, nh, hd).transpose(1, 0, 2)
    kf = kc.reshape(nk, nkv, hd).transpose(1, 0, 2)[None].copy()
    vf = vc.reshape(nk, nkv, hd).transpose(1, 0, 2)[None].copy()
    o_ref, _ = oracle.mha_fwd(qf, kf, vf, 1, nh, nkv, nk, hd, True, nthreads=ORACLE_THREADS)
    return o_ref[0, :, pos0:, :].transpose(1, 0, 2).reshape(n_tok, nh * hd)


def _run(n_tok, pos0, nh, nkv, hd, bf16, seed=0, check_oracle=False, expect_split=True):
    import torch
    import mx230_amd as mx
    q, kc, vc = _inputs(n_tok, pos0, nh, nkv, hd, bf16, seed)
    dt = torch.bfloat16 if bf16 else torch.float32
    tq, tk, tv = (torch.from_numpy(x).to("cuda").to(dt) for x in (q, kc, vc))
    need = mx.prefill_workspace_bytes(n_tok, pos0, nh, nkv, hd, bf16)
    print(f"\n[prefill split] n_tok={n_tok} pos0={pos0} Hq={nh} Hkv={nkv} d={hd} bf16={bf16} ws={need}", flush=True)
    assert (need > 0) == expect_split
    out_s = torch.full((n_tok, nh * hd), 7.0, device="cuda", dtype=dt)
    out_u = torch.full_like(out_s, 7.0)
    mx.run_prefill_split(tq, tk, tv, out_s, pos0, nh, nkv, hd)
    mx.run_prefill(tq, tk, tv, out_u, pos0, nh, nkv, hd)
    torch.cuda.synchronize()
    got = out_s.float().cpu().numpy()
    assert np.isfinite(got).all()
    tol = TOL_BF16 if bf16 else TOL_F32
    if not expect_split:
        assert torch.equal(out_s, out_u)
    e = rel_err(got, out_u.float().cpu().numpy())
    print(f"[prefill split] vs unsplit {e:.2e}", flush=True)
    assert e <= tol, e
    if check_oracle:
        e = rel_err(got, _oracle(q, kc, vc, pos0, nh, nkv, hd))
        print(f"[prefill split] vs oracle {e:.2e}", flush=True)
        assert e <= tol, e


def test_split_reference_configuration():
    """fp32, head_dim 64, GQA (the reference's own types): 16 splits of 33 stages."""
    _run(n_tok=100, pos0=2000, nh=4, nkv=2, hd=64, bf16=False, check_oracle=True)


def test_split_rows_before_a_split():
    """64-query blocks straddling stage boundaries (pos0 = 100), 8 splits: the
    light blocks' last splits start at their diagonal stage, which some of their
    rows precede entirely."""
    _run(n_tok=960, pos0=100, nh=1, nkv=1, hd=64, bf16=True, seed=1, check_oracle=True)
    _run(n_tok=960, pos0=100, nh=1, nkv=1, hd=64, bf16=False, seed=2, check_oracle=True)


def test_split_d128_bf16():
    _run(n_tok=96, pos0=1000, nh=8, nkv=1, hd=128, bf16=True, seed=3, check_oracle=True)


def test_split_single_row():
    """A decode-like call: one query row after 1777 positions (14 splits), the
    GQA group's heads as the rows of one block."""
    _run(n_tok=1, pos0=1777, nh=14, nkv=2, hd=64, bf16=True, seed=4, check_oracle=True)
    _run(n_tok=1, pos0=5000, nh=4, nkv=2, hd=64, bf16=False, seed=5, check_oracle=True)


def test_single_row_group_over_two_blocks_and_mha():
    """A single row whose GQA group fills two 64-query blocks (128 query heads
    over one KV head, MQA-like: the second block's rows are heads 64-127, all at
    the row's position), bf16 and fp32, split and unsplit; and a single MHA row
    (no packing: one row per head), unsplit in bf16 and split in fp32. Each
    against the oracle (the unsplit result through its agreement with the
    split one, or directly)."""
    _run(n_tok=1, pos0=1500, nh=128, nkv=1, hd=64, bf16=True, seed=11, check_oracle=True)
    _run(n_tok=1, pos0=1500, nh=128, nkv=1, hd=64, bf16=False, seed=12, check_oracle=True)
    _run(n_tok=1, pos0=900, nh=12, nkv=12, hd=64, bf16=True, seed=13, check_oracle=True, expect_split=False)
    _run(n_tok=1, pos0=900, nh=12, nkv=12, hd=64, bf16=False, seed=14, check_oracle=True)


def test_split_engine_chunk_bf16():
    """Qwen2.5's head layout, a 512-token chunk after 3584 positions (7 splits)."""
    _run(n_tok=512, pos0=3584, nh=14, nkv=2, hd=64, bf16=True, seed=6)


def test_split_not_needed_is_unsplit():
    _run(n_tok=4096, pos0=0, nh=14, nkv=2, hd=64, bf16=True, seed=7, expect_split=False)
    _run(n_tok=1, pos0=0, nh=14, nkv=2, hd=64, bf16=True, seed=8, expect_split=False)
    _run(n_tok=512, pos0=0, nh=14, nkv=2, hd=64, bf16=True, seed=10, expect_split=False)


def test_split_workspace_reuse_and_size():
    """A workspace sized for one call serves a smaller one after it; a short one is refused."""
    import torch
    import mx230_amd as mx
    q, kc, vc = _inputs(512, 3584, 14, 2, 64, True, 9)
    tq, tk, tv = (torch.from_numpy(x).to("cuda").to(torch.bfloat16) for x in (q, kc, vc))
    out = torch.empty((512, 14 * 64), device="cuda", dtype=torch.bfloat16)
    ws = mx.run_prefill_split(tq, tk, tv, out, 3584, 14, 2, 64)
    small_q, small_out = tq[:200], torch.empty((200, 14 * 64), device="cuda", dtype=torch.bfloat16)
    # the first 200 rows at pos0 = 3584: cache rows 0..3783
    mx.run_prefill_split(small_q, tk, tv, small_out, 3584, 14, 2, 64, workspace=ws)
    ref = torch.empty_like(small_out)
    mx.run_prefill(small_q, tk, tv, ref, 3584, 14, 2, 64)
    torch.cuda.synchronize()
    assert rel_err(small_out.float().cpu().numpy(), ref.float().cpu().numpy()) <= TOL_BF16
    # causal: the first 200 rows of the large call see the same keys
    assert rel_err(small_out.float().cpu().numpy(), out[:200].float().cpu().numpy()) <= TOL_BF16
    with pytest.raises(mx.MxfaError):
        mx.run_prefill_split(tq, tk, tv, out, 3584, 14, 2, 64, workspace=ws[:ws.numel() - 16])
