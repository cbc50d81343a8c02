"""Writes the golden vectors in this folder (run in the build container only).

The expected outputs come from an oracle that is independent of both the
reference and ``oracle/oracle.c``: PyTorch's CPU
``torch.nn.functional.scaled_dot_product_attention`` in float64 with autograd
(torch 2.10), which is a library routine for the same mathematics
(O = softmax(QK^T * scale [+ causal top-left mask]) V and its VJP for the loss
<O, dO>, 02-flash-attention/src/main.rs:243-245,302-303). The log-sum-exp is
torch.logsumexp of the masked, scaled float64 scores.

Inputs are the reference's own generators: ``pseudo_rand`` seeds as
02-flash-attention/src/main.rs:459-462 uses them (uniform [-1, 1)), or the
seeded N(0,1) extension used by the measured configurations. They are stored
next to the outputs, so the tests do not need the generator to reproduce them.

Usage:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle  # noqa: E402  (only for the input generators)

CASES = [
    # name, B, Hq, Hkv, N, d, causal, generator, mult
    ("mha_b1h1_n64_d64_noncausal", 1, 1, 1, 64, 64, False, "uniform", 1.0),
    ("mha_b1h1_n64_d64_causal", 1, 1, 1, 64, 64, True, "uniform", 1.0),
    ("mha_b1h2_n17_d64_causal", 1, 2, 2, 17, 64, True, "normal", 1.0),
    ("mha_b1h1_n33_d64_noncausal_ragged", 1, 1, 1, 33, 64, False, "normal", 0.5),
    ("mha_b1h1_n32_d128_causal", 1, 1, 1, 32, 128, True, "normal", 0.5),
    ("gqa_b2h4kv2_n24_d64_causal", 2, 4, 2, 24, 64, True, "normal", 0.5),
    ("gqa_b1h3kv1_n20_d64_noncausal", 1, 3, 1, 20, 64, False, "normal", 1.0),
    ("mha_b1h1_n1_d64_causal", 1, 1, 1, 1, 64, True, "uniform", 1.0),
]


def gen(kind, n, seed, mult):
    if kind == "uniform":
        return oracle.pseudo_rand(n, seed) * np.float32(mult)
    return oracle.normal(n, seed, mult)


def make(name, B, Hq, Hkv, N, d, causal, kind, mult):
    qn, kn = B * Hq * N * d, B * Hkv * N * d
    q = gen(kind, qn, 1, mult).reshape(B, Hq, N, d)
    k = gen(kind, kn, 2, mult).reshape(B, Hkv, N, d)
    v = gen(kind, kn, 3, mult).reshape(B, Hkv, N, d)
    do = gen(kind, qn, 4, 1.0).reshape(B, Hq, N, d)
    scale = oracle.default_scale(d)

    tq = torch.tensor(q, dtype=torch.float64, requires_grad=True)
    tk = torch.tensor(k, dtype=torch.float64, requires_grad=True)
    tv = torch.tensor(v, dtype=torch.float64, requires_grad=True)
    out = torch.nn.functional.scaled_dot_product_attention(
        tq, tk, tv, is_causal=causal, scale=scale, enable_gqa=(Hq != Hkv))
    out.backward(torch.tensor(do, dtype=torch.float64))

    g = Hq // Hkv
    kr = torch.tensor(k, dtype=torch.float64).repeat_interleave(g, dim=1)
    s = torch.tensor(q, dtype=torch.float64) @ kr.transpose(-1, -2) * scale
    if causal:
        mask = torch.ones(N, N, dtype=torch.bool).tril()
        s = s.masked_fill(~mask, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)

    np.savez_compressed(
        os.path.join(HERE, name + ".npz"),
        meta=np.array([B, Hq, Hkv, N, d, int(causal)], np.int64),
        scale=np.array(scale, np.float32),
        q=q, k=k, v=v, do=do,
        # float64 results rounded once to float32 (6e-8 relative, far below
        # every tolerance the tests apply) to keep the fixtures small
        o=out.detach().numpy().astype(np.float32), lse=lse.numpy().astype(np.float32),
        dq=tq.grad.numpy().astype(np.float32), dk=tk.grad.numpy().astype(np.float32),
        dv=tv.grad.numpy().astype(np.float32),
    )


def main():
    for case in CASES:
        make(*case)
        print("wrote", case[0])


if __name__ == "__main__":
    main()
