"""GPU parity of the prefill over a paged KV cache (mxfa_run_prefill_paged, the
MI355X counterpart of attn_prefill_paged, 03-llm-engine/kernels/llm.cu:3827-3836).

The same for the key split (mxfa_run_prefill_paged_ws against
mxfa_run_prefill_ws). The cache's blocks sit in a pool in shuffled order, among unused blocks filled
with NaN (a read through a wrong entry would show); the block table maps each
logical block to its physical one, as the engine's does (kv_row<true>,
llm.cu:959-963). Two checks:
- the outputs are bitwise those of mxfa_run_prefill over the contiguous cache
  the pool was scattered from (the same arithmetic, only the addressing
  differs), at block sizes 1 to 256, first and later chunks, GQA, d = 128, fp32,
  and a grid large enough for the 128-query kernel;
- the oracle, on the reference's own configuration (fp32, head_dim 64, GQA,
  block size 16 = KV_BLOCK, 03-llm-engine/src/gpu.rs:209), to the tolerance of
  test_gpu_prefill.py.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_helpers import ORACLE_THREADS, TOL_BF16, TOL_F32, rel_err

pytestmark = pytest.mark.gpu


def _paged_case(n_tok, pos0, nh, nkv, hd, bs, bf16, seed=0, check_oracle=False, spare_blocks=7, split=False):
    import torch
    import mx230_amd as mx
    rng = np.random.default_rng(seed)
    width = (nh + 2 * nkv) * hd
    nk = pos0 + n_tok
    nblk = -(-nk // bs)
    qkv = rng.standard_normal((n_tok, width)).astype(np.float32)
    kc = rng.standard_normal((nblk * bs, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((nblk * bs, nkv * hd)).astype(np.float32)
    if bf16:
        qkv, kc, vc = (oracle.bf16_round(x) for x in (qkv, kc, vc))
    kc[nk:], vc[nk:] = np.nan, np.nan  # past the last position
    # the chunk's own K/V rows come from the QKV buffer, as copy_kv_batch does
    kc[pos0:nk] = qkv[:, nh * hd:(nh + nkv) * hd]
    vc[pos0:nk] = qkv[:, (nh + nkv) * hd:]

    # scatter the logical blocks over a pool with spare NaN blocks
    npool = nblk + spare_blocks
    perm = rng.permutation(npool)[:nblk].astype(np.int32)
    kp = np.full((npool * bs, nkv * hd), np.nan, np.float32)
    vp = np.full_like(kp, np.nan)
    for j, b in enumerate(perm):
        kp[b * bs:(b + 1) * bs] = kc[j * bs:(j + 1) * bs]
        vp[b * bs:(b + 1) * bs] = vc[j * bs:(j + 1) * bs]

    dt = torch.bfloat16 if bf16 else torch.float32
    tqkv = torch.from_numpy(qkv).to("cuda").to(dt)
    tk, tv, tkp, tvp = (torch.from_numpy(x).to("cuda").to(dt) for x in (kc, vc, kp, vp))
    table = torch.from_numpy(perm).to("cuda")
    out_c = torch.full((n_tok, nh * hd), 7.0, device="cuda", dtype=dt)
    out_p = torch.full((n_tok, nh * hd), 7.0, device="cuda", dtype=dt)
    print(f"\n[prefill paged] n_tok={n_tok} pos0={pos0} Hq={nh} Hkv={nkv} d={hd} bs={bs} bf16={bf16} "
          f"split={split}", flush=True)
    if split:
        assert mx.prefill_workspace_bytes(n_tok, pos0, nh, nkv, hd, bf16) > 0
        mx.run_prefill_split(tqkv[:, :nh * hd], tk, tv, out_c, pos0, nh, nkv, hd)
        mx.run_prefill_paged(tqkv[:, :nh * hd], tkp, tvp, out_p, table, bs, pos0, nh, nkv, hd, split=True)
    else:
        mx.run_prefill(tqkv[:, :nh * hd], tk, tv, out_c, pos0, nh, nkv, hd)
        mx.run_prefill_paged(tqkv[:, :nh * hd], tkp, tvp, out_p, table, bs, pos0, nh, nkv, hd)
    torch.cuda.synchronize()
    assert torch.equal(out_p, out_c), "paged prefill differs from the contiguous one"
    got = out_p.float().cpu().numpy()
    assert np.isfinite(got).all()

    if check_oracle:
        qf = np.zeros((1, nh, nk, hd), np.float32)
        qf[0, :, pos0:, :] = qkv[:, :nh * hd].reshape(n_tok, nh, hd).transpose(1, 0, 2)
        kf = kc[:nk].reshape(nk, nkv, hd).transpose(1, 0, 2)[None].copy()
        vf = vc[:nk].reshape(nk, nkv, hd).transpose(1, 0, 2)[None].copy()
        o_ref, _ = oracle.mha_fwd(qf, kf, vf, 1, nh, nkv, nk, hd, True, nthreads=ORACLE_THREADS)
        want = o_ref[0, :, pos0:, :].transpose(1, 0, 2).reshape(n_tok, nh * hd)
        e = rel_err(got, want)
        print(f"[prefill paged] O rel err {e:.2e}", flush=True)
        assert e <= (TOL_BF16 if bf16 else TOL_F32), e


def test_paged_reference_configuration():
    """fp32, head_dim 64, GQA, KV_BLOCK = 16, a chunk after history: the oracle and the contiguous prefill."""
    _paged_case(n_tok=100, pos0=37, nh=4, nkv=2, hd=64, bs=16, bf16=False, check_oracle=True)


@pytest.mark.parametrize("bs", [1, 16, 64, 256])
@pytest.mark.parametrize("n_tok,pos0", [(257, 300), (64, 64), (1, 777), (130, 5)])
def test_paged_equals_contiguous_bf16(bs, n_tok, pos0):
    """Qwen2.5 head layout, bf16, block sizes below, at and above a 64-key stage."""
    _paged_case(n_tok=n_tok, pos0=pos0, nh=14, nkv=2, hd=64, bs=bs, bf16=True, seed=bs + n_tok + pos0)


def test_paged_d128_bf16():
    _paged_case(n_tok=96, pos0=1000, nh=8, nkv=1, hd=128, bs=16, bf16=True, seed=5, check_oracle=True)


def test_paged_large_grid_bf16():
    """768 work-groups of 128 queries: the two-wave 128-query kernel."""
    _paged_case(n_tok=3072, pos0=512, nh=32, nkv=4, hd=64, bs=16, bf16=True, seed=9)


def test_paged_large_grid_d128_bf16():
    """d = 128 at a grid that the training forward would run on 128-query
    work-groups (768 of them): the prefill keeps the 64-query tiling of its
    paged form, so the two stay bitwise equal."""
    _paged_case(n_tok=3072, pos0=256, nh=32, nkv=4, hd=128, bs=16, bf16=True, seed=21)


@pytest.mark.parametrize("bs", [1, 16, 256])
@pytest.mark.parametrize("n_tok,pos0", [(512, 3584), (1, 4095), (960, 100)])
def test_paged_split_equals_contiguous_split_bf16(bs, n_tok, pos0):
    """The key split over a paged cache: bitwise the split over the gathered one."""
    nh, nkv = (1, 1) if pos0 == 100 else (14, 2)
    _paged_case(n_tok=n_tok, pos0=pos0, nh=nh, nkv=nkv, hd=64, bs=bs, bf16=True, seed=bs + n_tok, split=True)


def test_paged_single_row_mqa_oracle():
    """A single row of 128 query heads over one KV head (its group spans two
    64-query blocks) over a paged cache, unsplit and split, against the oracle."""
    _paged_case(n_tok=1, pos0=1300, nh=128, nkv=1, hd=64, bs=16, bf16=True, seed=13, check_oracle=True)
    _paged_case(n_tok=1, pos0=1300, nh=128, nkv=1, hd=64, bs=16, bf16=False, seed=14, check_oracle=True, split=True)


def test_paged_split_oracle():
    """fp32 and d = 128 bf16 splits over a paged cache against the oracle."""
    _paged_case(n_tok=100, pos0=2000, nh=4, nkv=2, hd=64, bs=16, bf16=False, seed=11, check_oracle=True, split=True)
    _paged_case(n_tok=96, pos0=1000, nh=8, nkv=1, hd=128, bs=16, bf16=True, seed=12, check_oracle=True, split=True)


def test_paged_block_size_refused():
    import torch
    import mx230_amd as mx
    q = torch.zeros((4, 64), device="cuda", dtype=torch.bfloat16)
    kv = torch.zeros((32, 64), device="cuda", dtype=torch.bfloat16)
    table = torch.zeros(4, dtype=torch.int32, device="cuda")
    with pytest.raises(mx.MxfaError):
        mx.run_prefill_paged(q, kv, kv, torch.zeros_like(q), table, 24, 0, 1, 1, 64)
