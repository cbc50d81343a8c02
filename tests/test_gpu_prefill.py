"""GPU parity of the inference-side forward (mxfa_run_prefill, the MI355X
counterpart of attn_prefill, 03-llm-engine/kernels/llm.cu:3806-3815).

Layout as in the engine: a fused token-major QKV buffer [n_tok][(Hq + 2 Hkv) d]
whose Q columns are the kernel's query rows; K and V caches [positions][Hkv d]
whose rows 0..pos0-1 hold history and rows pos0..pos0+n_tok-1 the chunk's own
K/V (copied in from the QKV buffer, as copy_kv_batch does, llm.cu:3635); output
rows [n_tok][out_stride] with padding columns.

Oracle: query row i at position pos0 + i attending to keys 0..pos0 + i is row
pos0 + i of an ordinary top-left causal attention over pos0 + n_tok positions,
so the reference is the oracle's causal forward with the chunk's queries placed
at rows pos0.. (rows before are zero and ignored). Tolerances as for the
training forward: 1e-4 (fp32) / 2e-2 (bf16) of max|O|. Cache rows past
pos0 + n_tok hold NaN, so any read past the valid rows would show up.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_helpers import ORACLE_THREADS, TOL_BF16, TOL_F32, rel_err

pytestmark = pytest.mark.gpu


def _case(n_tok, pos0, nh, nkv, hd, bf16, seed=0, pad_rows=40, out_pad=32):
    import torch
    import mx230_amd as mx
    rng = np.random.default_rng(seed)
    width = (nh + 2 * nkv) * hd
    nk = pos0 + n_tok
    qkv = rng.standard_normal((n_tok, width)).astype(np.float32)
    hist_k = rng.standard_normal((pos0, nkv * hd)).astype(np.float32)
    hist_v = rng.standard_normal((pos0, nkv * hd)).astype(np.float32)
    if bf16:
        qkv, hist_k, hist_v = (oracle.bf16_round(x) for x in (qkv, hist_k, hist_v))
    kc = np.full((nk + pad_rows, nkv * hd), np.nan, np.float32)
    vc = np.full_like(kc, np.nan)
    kc[:pos0], vc[:pos0] = hist_k, hist_v
    kc[pos0:nk] = qkv[:, nh * hd:(nh + nkv) * hd]
    vc[pos0:nk] = qkv[:, (nh + nkv) * hd:]

    dt = torch.bfloat16 if bf16 else torch.float32
    tqkv = torch.from_numpy(qkv).to("cuda").to(dt)
    tk, tv = (torch.from_numpy(x).to("cuda").to(dt) for x in (kc, vc))
    out = torch.full((n_tok, nh * hd + out_pad), 7.0, device="cuda", dtype=dt)
    print(f"\n[prefill] n_tok={n_tok} pos0={pos0} Hq={nh} Hkv={nkv} d={hd} bf16={bf16}", flush=True)
    mx.run_prefill(tqkv[:, :nh * hd], tk, tv, out[:, :nh * hd], pos0, nh, nkv, hd)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.all(got[:, nh * hd:] == 7.0), "padding columns of the output rows were written"

    # oracle: causal forward over nk positions, queries at rows pos0..
    qf = np.zeros((1, nh, nk, hd), np.float32)
    qf[0, :, pos0:, :] = qkv[:, :nh * hd].reshape(n_tok, nh, hd).transpose(1, 0, 2)
    kf = kc[:nk].reshape(nk, nkv, hd).transpose(1, 0, 2)[None].copy()
    vf = vc[:nk].reshape(nk, nkv, hd).transpose(1, 0, 2)[None].copy()
    o_ref, _ = oracle.mha_fwd(qf, kf, vf, 1, nh, nkv, nk, hd, True, nthreads=ORACLE_THREADS)
    want = o_ref[0, :, pos0:, :].transpose(1, 0, 2).reshape(n_tok, nh * hd)
    e = rel_err(got[:, :nh * hd], want)
    print(f"[prefill] O rel err {e:.2e}", flush=True)
    assert e <= (TOL_BF16 if bf16 else TOL_F32), e


def test_prefill_reference_kind0_fp32():
    """The reference's own configuration: fp32, head_dim 64, GQA, a chunk after history."""
    _case(n_tok=100, pos0=37, nh=4, nkv=2, hd=64, bf16=False)


@pytest.mark.parametrize("n_tok,pos0", [(257, 0), (257, 300), (1, 777), (64, 64), (130, 5)])
def test_prefill_qwen_heads_bf16(n_tok, pos0):
    """Qwen2.5 head layout (14 query heads over 2 KV heads), bf16: first chunk,
    later chunk, a single decode token, and chunks not aligned to the tiles."""
    _case(n_tok=n_tok, pos0=pos0, nh=14, nkv=2, hd=64, bf16=True, seed=n_tok + pos0)


def test_prefill_d128_bf16():
    _case(n_tok=96, pos0=1000, nh=8, nkv=1, hd=128, bf16=True, seed=5)


def test_prefill_fp32_long_history():
    _case(n_tok=33, pos0=2049, nh=2, nkv=1, hd=64, bf16=False, seed=6)


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
def test_prefill_at_pos0_zero_is_the_training_forward(bf16):
    """With pos0 = 0 and the chunk's K/V as the whole cache, the prefill is the
    training forward (mxfa_run_flash, causal) on the same numbers, computed by
    the same kernel with different strides: the results are bitwise equal."""
    import torch
    import mx230_amd as mx
    n, nh, nkv, hd = 200, 4, 2, 64
    dt = torch.bfloat16 if bf16 else torch.float32
    g = torch.Generator(device="cuda").manual_seed(3)
    qkv = torch.randn(n, (nh + 2 * nkv) * hd, device="cuda", generator=g).to(dt)
    kc = qkv[:, nh * hd:(nh + nkv) * hd].contiguous()
    vc = qkv[:, (nh + nkv) * hd:].contiguous()
    out = torch.empty(n, nh * hd, device="cuda", dtype=dt)
    mx.run_prefill(qkv[:, :nh * hd], kc, vc, out, 0, nh, nkv, hd)
    q4 = qkv[:, :nh * hd].reshape(n, nh, hd).transpose(0, 1).contiguous()[None]
    k4 = kc.reshape(n, nkv, hd).transpose(0, 1).contiguous()[None]
    v4 = vc.reshape(n, nkv, hd).transpose(0, 1).contiguous()[None]
    o4 = torch.empty_like(q4)
    mx.run_flash(q4, k4, v4, o4, True)
    torch.cuda.synchronize()
    assert torch.equal(out, o4[0].transpose(0, 1).reshape(n, nh * hd))


def test_prefill_rejects_short_cache():
    import torch
    import mx230_amd as mx
    q = torch.zeros(10, 128, device="cuda", dtype=torch.bfloat16)
    kc = torch.zeros(12, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="rows"):
        mx.run_prefill(q, kc, kc, torch.zeros_like(q), 5, 2, 1)
