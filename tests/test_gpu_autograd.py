"""The autograd wrapper (mx230_amd.autograd) on the GPU: values and gradients
against a float32 PyTorch restatement of attention (matmul + softmax on the GPU
in fp32; bf16 batched products are avoided on purpose), and a full attention
block's forward/backward against the same block built on that restatement.
Tolerance: 2e-2 of each tensor's max magnitude for bf16 attention outputs and
input gradients, 3e-2 for the block's weight gradients (two bf16 GEMMs more)."""
from __future__ import annotations

import math

import pytest

pytestmark = pytest.mark.gpu

TOL = 2e-2
TOL_BLOCK = 3e-2


def _rel(got, want) -> float:
    got, want = got.float(), want.float()
    return float((got - want).abs().max() / want.abs().max().clamp_min(1e-6))


def _ref_attention(q, k, v, causal, scale):
    import torch
    g = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(g, dim=1)
    v = v.repeat_interleave(g, dim=1)
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
    if causal:
        n = q.shape[2]
        s = s.masked_fill(torch.ones(n, n, dtype=torch.bool, device=q.device).triu(1), float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), v)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("hkv", [4, 2], ids=["mha", "gqa2"])
def test_flash_attention_grads(causal, hkv):
    import torch
    from mx230_amd.autograd import flash_attention
    torch.manual_seed(0)
    B, Hq, N, d = 2, 4, 320, 64
    q = torch.randn(B, Hq, N, d, device="cuda").to(torch.bfloat16).requires_grad_()
    k = torch.randn(B, hkv, N, d, device="cuda").to(torch.bfloat16).requires_grad_()
    v = torch.randn(B, hkv, N, d, device="cuda").to(torch.bfloat16).requires_grad_()
    g = torch.randn(B, Hq, N, d, device="cuda").to(torch.bfloat16)
    print(f"\n[autograd] B{B} Hq{Hq} Hkv{hkv} N{N} causal={causal}", flush=True)
    o = flash_attention(q, k, v, causal)
    (o.float() * g.float()).sum().backward()

    q32, k32, v32 = (t.detach().float().requires_grad_() for t in (q, k, v))
    o32 = _ref_attention(q32, k32, v32, causal, 1.0 / math.sqrt(d))
    (o32 * g.float()).sum().backward()
    errs = {"O": _rel(o, o32), "dQ": _rel(q.grad, q32.grad), "dK": _rel(k.grad, k32.grad),
            "dV": _rel(v.grad, v32.grad)}
    print("[autograd] " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    assert all(e <= TOL for e in errs.values()), errs


def test_attention_block_training_step():
    """A QKV-projection / flash-attention / output-projection block (8 query
    heads over 2 KV heads, causal) in bf16: outputs and every weight gradient
    against the same block in fp32 with the reference attention, then one SGD
    step changes the weights and lowers the loss of that batch."""
    import torch
    from mx230_amd.autograd import CausalSelfAttention
    torch.manual_seed(1)
    dim, B, N = 256, 2, 256
    blk = CausalSelfAttention(dim, n_heads=8, n_kv_heads=2, head_dim=64).cuda().to(torch.bfloat16)
    ref = CausalSelfAttention(dim, n_heads=8, n_kv_heads=2, head_dim=64).cuda()
    ref.load_state_dict({kk: vv.float() for kk, vv in blk.state_dict().items()})
    x = torch.randn(B, N, dim, device="cuda")
    target = torch.randn(B, N, dim, device="cuda")

    y = blk(x.to(torch.bfloat16))
    loss = ((y.float() - target) ** 2).mean()
    loss.backward()

    # the reference block runs the same projections in fp32 with the restated attention
    def ref_forward(m, xx):
        b, n, _ = xx.shape
        hq, hk, d = m.n_heads, m.n_kv_heads, m.head_dim
        q, k, v = m.qkv(xx).split([hq * d, hk * d, hk * d], dim=-1)
        q = q.view(b, n, hq, d).transpose(1, 2)
        k = k.view(b, n, hk, d).transpose(1, 2)
        v = v.view(b, n, hk, d).transpose(1, 2)
        o = _ref_attention(q, k, v, True, 1.0 / math.sqrt(d))
        return m.out(o.transpose(1, 2).reshape(b, n, hq * d))

    y32 = ref_forward(ref, x.to(torch.bfloat16).float())
    loss32 = ((y32 - target) ** 2).mean()
    loss32.backward()
    errs = {"y": _rel(y, y32), "dWqkv": _rel(blk.qkv.weight.grad, ref.qkv.weight.grad),
            "dWout": _rel(blk.out.weight.grad, ref.out.weight.grad)}
    print("\n[block] " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    assert errs["y"] <= TOL, errs
    assert errs["dWqkv"] <= TOL_BLOCK and errs["dWout"] <= TOL_BLOCK, errs

    opt = torch.optim.SGD(blk.parameters(), lr=0.5)
    w0 = blk.qkv.weight.detach().clone()
    opt.step()
    assert not torch.equal(w0, blk.qkv.weight.detach())
    with torch.no_grad():
        loss_after = ((blk(x.to(torch.bfloat16)).float() - target) ** 2).mean()
    print(f"[block] loss {float(loss):.5f} -> {float(loss_after):.5f}", flush=True)
    assert float(loss_after) < float(loss)
