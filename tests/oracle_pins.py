"""Checks that pin the CPU oracle, shared by test_oracle.py (which asserts they
all pass) and test_oracle_mutants.py (which asserts that each planted mistake
fails at least one of them).

Each pin compares the oracle with something that does not restate it: golden
vectors from float64 torch SDPA, the reference's own finite-difference gate,
closed-form invariants of the attention VJP, and special cases whose answer is
known in closed form.
"""
from __future__ import annotations

import glob
import os

import numpy as np

import oracle

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def rel_max_err(got, want) -> float:
    """max |got - want| / max |want| (the parity metric of the measured configs)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    denom = max(float(np.abs(want).max()) if want.size else 0.0, 1e-30)
    return float(np.abs(got - want).max()) / denom if want.size else 0.0


def golden_cases():
    return sorted(glob.glob(os.path.join(GOLDEN_DIR, "*.npz")))


def load_golden(path):
    with np.load(path, allow_pickle=False) as z:
        g = {k: z[k] for k in z.files}
    B, Hq, Hkv, N, d, causal = (int(x) for x in g["meta"])
    g.update(B=B, Hq=Hq, Hkv=Hkv, N=N, d=d, causal=bool(causal), scale=float(g["scale"]))
    return g


def pin_golden(lib, path, tol=2e-5):
    """Oracle forward/backward against the float64 library oracle."""
    g = load_golden(path)
    sh = (g["B"], g["Hq"], g["Hkv"], g["N"], g["d"], g["causal"])
    o, lse = oracle.mha_fwd(g["q"], g["k"], g["v"], *sh, scale=g["scale"], lib=lib)
    dq, dk, dv = oracle.mha_bwd(g["q"], g["k"], g["v"], g["do"], *sh, scale=g["scale"], lib=lib)
    errs = {
        "O": rel_max_err(o, g["o"]),
        "LSE": rel_max_err(lse, g["lse"]),
        "dQ": rel_max_err(dq, g["dq"]),
        "dK": rel_max_err(dk, g["dk"]),
        "dV": rel_max_err(dv, g["dv"]),
    }
    bad = {k: v for k, v in errs.items() if not v <= tol}
    return bad


def _rand_case(N=40, d=64, B=1, Hq=2, Hkv=1, seed=7, mult=0.7, lib=None):
    q = oracle.normal(B * Hq * N * d, seed, mult, lib=lib).reshape(B, Hq, N, d)
    k = oracle.normal(B * Hkv * N * d, seed + 1, mult, lib=lib).reshape(B, Hkv, N, d)
    v = oracle.normal(B * Hkv * N * d, seed + 2, mult, lib=lib).reshape(B, Hkv, N, d)
    do = oracle.normal(B * Hq * N * d, seed + 3, 1.0, lib=lib).reshape(B, Hq, N, d)
    return q, k, v, do


def pin_invariants(lib, causal: bool, tol=5e-5):
    """Closed forms of the softmax-attention VJP (hold for any inputs):
    sum_j dK_j = 0; sum_j dV_j = sum_i dO_i (per KV head, summed over its query
    heads); <Q,dQ> = <K,dK>; <V,dV> = <O,dO>. Returns the failing ones."""
    B, Hq, Hkv, N, d = 1, 2, 1, 40, 64
    q, k, v, do = _rand_case(N, d, B, Hq, Hkv, lib=lib)
    o, _ = oracle.mha_fwd(q, k, v, B, Hq, Hkv, N, d, causal, lib=lib)
    dq, dk, dv = oracle.mha_bwd(q, k, v, do, B, Hq, Hkv, N, d, causal, lib=lib)
    f64 = lambda a: np.asarray(a, np.float64)  # noqa: E731
    bad = {}
    s = np.abs(f64(dk)).sum()
    e = np.abs(f64(dk).sum(axis=2)).max() / max(s / N, 1e-30)
    if not e <= tol:
        bad["sum dK = 0"] = e
    want = f64(do).sum(axis=(1, 2))  # Hkv = 1: all query heads feed KV head 0
    e = np.abs(f64(dv).sum(axis=(1, 2)) - want).max() / np.abs(want).max()
    if not e <= tol:
        bad["sum dV = sum dO"] = e
    a, b = (f64(q) * f64(dq)).sum(), (f64(k) * f64(dk)).sum()
    e = abs(a - b) / max(abs(a), abs(b), 1e-30)
    if not e <= tol:
        bad["<Q,dQ> = <K,dK>"] = e
    a, b = (f64(v) * f64(dv)).sum(), (f64(o) * f64(do)).sum()
    e = abs(a - b) / max(abs(a), abs(b), 1e-30)
    if not e <= tol:
        bad["<V,dV> = <O,dO>"] = e
    return bad


def pin_fd(lib, causal: bool, gate=5e-2):
    """The reference's own gate (main.rs:504-508): fd_check(128) < 5e-2."""
    e = oracle.fd_check(128, causal, lib=lib)
    return {} if e < gate else {"fd_check": e}


def all_pins(lib):
    """Every pin; returns {pin name: failure detail} (empty when all pass)."""
    failed = {}
    for path in golden_cases():
        bad = pin_golden(lib, path)
        if bad:
            failed["golden:" + os.path.basename(path)] = bad
    for causal in (False, True):
        bad = pin_invariants(lib, causal)
        if bad:
            failed[f"invariants(causal={causal})"] = bad
        bad = pin_fd(lib, causal)
        if bad:
            failed[f"fd(causal={causal})"] = bad
    return failed
