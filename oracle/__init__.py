"""CPU oracle for the flash-attention training path (test infrastructure).

This package is the *checker*. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import it; the product library
(``mx230_amd`` / ``libmxfa.so``) never calls it and has no fallback to it.

It wraps ``liboracle.so`` (built from ``oracle.c`` by ``oracle/Makefile``), a C
restatement of the reference's Rust CPU path:

* ``pseudo_rand``            common/src/lib.rs:67-78
* ``max_rel_err``            common/src/lib.rs:46-52
* ``allclose_err``           common/src/lib.rs:58-64
* ``cpu_attention``          02-flash-attention/src/main.rs:213-241 (+ LSE, attention_flash.cu:85-87)
* ``cpu_attention_bwd``      02-flash-attention/src/main.rs:246-300
* ``attn_loss``              02-flash-attention/src/main.rs:304-333
* ``fd_check``               02-flash-attention/src/main.rs:339-390
* ``delta``                  02-flash-attention/kernels/attention_bwd.cu:32-44
* ``mha_fwd`` / ``mha_bwd``  batched [B][H][N][d] + GQA head mapping (03-llm-engine/src/cpu.rs:194,224)

Every function here is pinned by ``tests/test_oracle.py`` (golden vectors from an
independent float64 library oracle, known-answer tests, closed-form invariants,
finite differences and brute force); ``tests/test_oracle_mutants.py`` shows that
planted mistakes fail those pins.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")


def build(force: bool = False) -> str:
    """Compile ``liboracle.so`` with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        cmd = ["make", "-s", "-f", os.path.join(_HERE, "Makefile")]
        if force:
            cmd.append("-B")
        subprocess.run(cmd, check=True, cwd=_HERE)
    return _LIB_PATH


def _bind(lib):
    c = ctypes
    lib.orc_pseudo_rand.argtypes = [_f32p, c.c_size_t, c.c_uint64]
    lib.orc_normal.argtypes = [_f32p, c.c_size_t, c.c_uint64, c.c_float]
    lib.orc_bf16_round.argtypes = [_f32p, c.c_size_t]
    lib.orc_max_rel_err.argtypes = [_f32p, _f32p, c.c_size_t]
    lib.orc_max_rel_err.restype = c.c_float
    lib.orc_allclose_err.argtypes = [_f32p, _f32p, c.c_size_t, c.c_float, c.c_float]
    lib.orc_allclose_err.restype = c.c_float
    lib.orc_cpu_attention.argtypes = [_f32p, _f32p, _f32p, _f32p, c.c_void_p, c.c_int, c.c_int,
                                      c.c_int, c.c_float]
    lib.orc_cpu_attention_bwd.argtypes = [_f32p] * 7 + [c.c_int, c.c_int, c.c_int, c.c_float]
    lib.orc_attn_loss.argtypes = [_f32p] * 4 + [c.c_int, c.c_int, c.c_int]
    lib.orc_attn_loss.restype = c.c_double
    lib.orc_fd_check.argtypes = [c.c_int, c.c_int, c.c_int]
    lib.orc_fd_check.restype = c.c_float
    lib.orc_delta.argtypes = [_f32p, _f32p, _f32p, c.c_size_t, c.c_int]
    lib.orc_mha_fwd.argtypes = [c.c_int] * 6 + [c.c_float, _f32p, _f32p, _f32p, _f32p, c.c_void_p,
                                                c.c_int]
    lib.orc_mha_fwd.restype = c.c_int
    lib.orc_mha_bwd.argtypes = [c.c_int] * 6 + [c.c_float] + [_f32p] * 7 + [c.c_int]
    lib.orc_mha_bwd.restype = c.c_int
    lib.orc_mutant.restype = c.c_int
    return lib


def load(path: str | None = None):
    """Load (building if needed) the oracle library; ``path`` selects another
    build of the same source (the mutant builds of the oracle's own tests)."""
    global _lib
    if path is not None:
        return _bind(ctypes.CDLL(path))
    if _lib is None:
        build()
        _lib = _bind(ctypes.CDLL(_LIB_PATH))
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def default_scale(d: int) -> float:
    """1/sqrt(d) in f32, as main.rs:214 computes it."""
    return float(np.float32(1.0) / np.sqrt(np.float32(d)))


# ------------------------------------------------------------------ inputs --

def pseudo_rand(n: int, seed: int, lib=None) -> np.ndarray:
    out = np.empty(n, np.float32)
    (lib or load()).orc_pseudo_rand(out, n, seed)
    return out


def normal(n: int, seed: int, mult: float = 1.0, lib=None) -> np.ndarray:
    out = np.empty(n, np.float32)
    (lib or load()).orc_normal(out, n, seed, mult)
    return out


def bf16_round(x: np.ndarray, lib=None) -> np.ndarray:
    out = _f32(x).copy()
    (lib or load()).orc_bf16_round(out.reshape(-1), out.size)
    return out


# ----------------------------------------------------------------- metrics --

def max_rel_err(got, want, lib=None) -> float:
    g, w = _f32(got).reshape(-1), _f32(want).reshape(-1)
    assert g.size == w.size
    return float((lib or load()).orc_max_rel_err(g, w, g.size))


def allclose_err(got, want, rtol: float, atol: float, lib=None) -> float:
    g, w = _f32(got).reshape(-1), _f32(want).reshape(-1)
    assert g.size == w.size
    return float((lib or load()).orc_allclose_err(g, w, g.size, rtol, atol))


# ------------------------------------------------------------- single head --

def cpu_attention(q, k, v, n: int, d: int, causal: bool, scale: float | None = None, lib=None):
    """Returns (O [n][d], LSE [n])."""
    scale = default_scale(d) if scale is None else scale
    o = np.empty((n, d), np.float32)
    lse = np.empty(n, np.float32)
    (lib or load()).orc_cpu_attention(_f32(q), _f32(k), _f32(v), o, lse.ctypes.data, n, d,
                                      int(causal), scale)
    return o, lse


def cpu_attention_bwd(q, k, v, do, n: int, d: int, causal: bool, scale: float | None = None,
                      lib=None):
    """Returns (dQ, dK, dV), each [n][d]."""
    scale = default_scale(d) if scale is None else scale
    dq, dk, dv = (np.empty((n, d), np.float32) for _ in range(3))
    (lib or load()).orc_cpu_attention_bwd(_f32(q), _f32(k), _f32(v), _f32(do), dq, dk, dv, n, d,
                                          int(causal), scale)
    return dq, dk, dv


def attn_loss(q, k, v, do, n: int, d: int, causal: bool, lib=None) -> float:
    return float((lib or load()).orc_attn_loss(_f32(q), _f32(k), _f32(v), _f32(do), n, d,
                                               int(causal)))


def fd_check(n: int, causal: bool, d: int = 64, lib=None) -> float:
    return float((lib or load()).orc_fd_check(n, d, int(causal)))


def delta(do, o, d: int, lib=None) -> np.ndarray:
    dof, of = _f32(do).reshape(-1), _f32(o).reshape(-1)
    rows = dof.size // d
    out = np.empty(rows, np.float32)
    (lib or load()).orc_delta(dof, of, out, rows, d)
    return out


# ------------------------------------------------------------ multi head ---

def mha_fwd(q, k, v, B, Hq, Hkv, N, d, causal, scale=None, nthreads=1, lib=None):
    """Q [B][Hq][N][d], K/V [B][Hkv][N][d] -> (O [B][Hq][N][d], LSE [B][Hq][N])."""
    scale = default_scale(d) if scale is None else scale
    o = np.empty((B, Hq, N, d), np.float32)
    lse = np.empty((B, Hq, N), np.float32)
    rc = (lib or load()).orc_mha_fwd(B, Hq, Hkv, N, d, int(causal), scale, _f32(q), _f32(k),
                                     _f32(v), o, lse.ctypes.data, nthreads)
    if rc != 0:
        raise ValueError("invalid shape for the oracle")
    return o, lse


def mha_bwd(q, k, v, do, B, Hq, Hkv, N, d, causal, scale=None, nthreads=1, lib=None):
    """-> (dQ [B][Hq][N][d], dK [B][Hkv][N][d], dV [B][Hkv][N][d])."""
    scale = default_scale(d) if scale is None else scale
    dq = np.empty((B, Hq, N, d), np.float32)
    dk = np.empty((B, Hkv, N, d), np.float32)
    dv = np.empty((B, Hkv, N, d), np.float32)
    rc = (lib or load()).orc_mha_bwd(B, Hq, Hkv, N, d, int(causal), scale, _f32(q), _f32(k),
                                     _f32(v), _f32(do), dq, dk, dv, nthreads)
    if rc != 0:
        raise ValueError("invalid shape for the oracle")
    return dq, dk, dv
