"""Training-step wrapper: the flash-attention path as a ``torch.autograd.Function``.

The forward calls ``mxfa_run_flash_lse`` and saves Q, K, V, O and LSE; the
backward calls ``mxfa_run_bwd_ws`` (the dQ pass with Delta = rowsum(dO * O)
folded in, then the dK/dV pass, split over the query heads of a GQA group
through a workspace where that fills the GPU better). This is the sequence the
reference drives by hand around its kernels (02-flash-attention/src/main.rs:470-511:
flash forward with LSE, then preprocess, then ``run_bwd_flash``), packaged so a
PyTorch-ROCm training step can put it between its QKV and output projections.

Layouts as in the package: Q ``[B, Hq, N, d]``, K/V ``[B, Hkv, N, d]`` (grouped
query heads when Hkv < Hq), bf16 with d in {64, 128} or fp32 with d = 64, on a
gfx950 device. There is no fallback: CPU tensors, other dtypes or other head
sizes raise (``ValueError`` or :class:`mx230_amd.MxfaError`).
"""
from __future__ import annotations

import torch

from . import attention_bwd, attention_fwd


class FlashAttentionFunction(torch.autograd.Function):
    """O = softmax(Q K^T scale [+ causal mask]) V with the HIP forward and backward."""

    @staticmethod
    def forward(ctx, q, k, v, causal: bool, scale: float):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        o, lse = attention_fwd(q, k, v, causal, scale)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.causal, ctx.scale = causal, scale
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        do = do.to(q.dtype).contiguous()
        dq, dk, dv = attention_bwd(q, k, v, o, lse, do, ctx.causal, ctx.scale)
        return dq, dk, dv, None, None


def flash_attention(q, k, v, causal: bool = False, scale: float = 0.0):
    """Differentiable attention over the C ABI. ``scale`` 0 means 1/sqrt(d)."""
    return FlashAttentionFunction.apply(q, k, v, causal, scale)


class CausalSelfAttention(torch.nn.Module):
    """A transformer attention block around :func:`flash_attention`: fused QKV
    projection, grouped-query heads, output projection (the GEMMs on either side
    are plain torch; the attention core is the HIP path)."""

    def __init__(self, dim: int, n_heads: int, n_kv_heads: int | None = None, head_dim: int = 64,
                 causal: bool = True):
        super().__init__()
        self.n_heads = n_heads
        self.n_kv_heads = n_kv_heads or n_heads
        if self.n_heads % self.n_kv_heads:
            raise ValueError("n_heads must be a multiple of n_kv_heads")
        self.head_dim = head_dim
        self.causal = causal
        self.qkv = torch.nn.Linear(dim, (n_heads + 2 * self.n_kv_heads) * head_dim, bias=False)
        self.out = torch.nn.Linear(n_heads * head_dim, dim, bias=False)

    def forward(self, x):
        b, n, _ = x.shape
        hq, hk, d = self.n_heads, self.n_kv_heads, self.head_dim
        qkv = self.qkv(x)
        q, k, v = qkv.split([hq * d, hk * d, hk * d], dim=-1)
        q = q.view(b, n, hq, d).transpose(1, 2)
        k = k.view(b, n, hk, d).transpose(1, 2)
        v = v.view(b, n, hk, d).transpose(1, 2)
        o = flash_attention(q, k, v, self.causal)
        return self.out(o.transpose(1, 2).reshape(b, n, hq * d))
