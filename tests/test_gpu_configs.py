"""GPU checks of the full-size BASELINE.json configurations, the naive
baselines and the error/stream behaviour of the C ABI.

Full-size configs are checked against the CPU oracle on one KV-head group (the
oracle finishes that in seconds), plus size-independent properties over every
head: sum_j dK_j = 0 and sum_j dV_j = sum_i dO_i (per KV head, over its query
heads). The long-sequence config (N = 32768) is checked on sampled rows against
a float64 numpy evaluation of the same formulas, and for O(N) memory: the
library allocates nothing, so device free memory is unchanged across the calls.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from gpu_helpers import (TOL_BF16, TOL_F32, gpu_fwd_bwd, make_inputs, oracle_fwd_bwd, parity,
                         rel_err, to_dev, to_np)

pytestmark = pytest.mark.gpu


def _group_check(name, q, k, v, do, causal, b, kvh, tol):
    """Oracle parity on KV head (b, kvh) and its query heads."""
    B, Hq, N, d = q.shape
    Hkv = k.shape[1]
    grp = Hq // Hkv
    print(f"\n[{name}] B{B} Hq{Hq} Hkv{Hkv} N{N} d{d} causal={causal}", flush=True)
    gpu = gpu_fwd_bwd(q, k, v, do, causal, True)
    hs = slice(kvh * grp, (kvh + 1) * grp)
    ref = oracle_fwd_bwd(q[b:b + 1, hs], k[b:b + 1, kvh:kvh + 1], v[b:b + 1, kvh:kvh + 1],
                         do[b:b + 1, hs], causal)
    sub = (gpu[0][b:b + 1, hs], gpu[1][b:b + 1, hs], gpu[2][b:b + 1, hs], gpu[3][b:b + 1, hs],
           gpu[4][b:b + 1, kvh:kvh + 1], gpu[5][b:b + 1, kvh:kvh + 1])
    errs, bad = parity(sub, ref, tol)
    print(f"[{name}] group (b={b}, kvh={kvh}): " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()),
          flush=True)
    assert not bad, (name, errs)
    _closed_forms(gpu, do, Hkv)
    return gpu


def _closed_forms(gpu, do, Hkv):
    """sum_j dK_j = 0 and sum_j dV_j = sum over the group's query heads of sum_i dO_i."""
    dk = gpu[4].astype(np.float64)
    assert np.all(np.abs(dk.sum(axis=2)) <= 1e-2 * np.abs(dk).sum(axis=2) + 1e-6)
    B, Hq, N, d = do.shape
    sdo = do.astype(np.float64).reshape(B, Hkv, Hq // Hkv, N, d).sum(axis=(2, 3))
    assert rel_err(gpu[5].astype(np.float64).sum(axis=2), sdo) <= TOL_BF16


def test_cfg4_qwen_gqa_full():
    """Qwen2.5-0.5B: B2 Hq14 Hkv2 N4096 d64 causal bf16, 7 query heads per KV head."""
    q, k, v, do = make_inputs(2, 14, 2, 4096, 64, bf16=True)
    _group_check("cfg4", q, k, v, do, True, b=1, kvh=1, tol=TOL_BF16)


@pytest.mark.parametrize("d", [64, 128])
def test_cfg5_tinyllama_gqa_full(d):
    """TinyLlama-1.1B: B1 Hq32 Hkv4 N2048 causal bf16, d 64 and 128, Q/K/V x0.5."""
    q, k, v, do = make_inputs(1, 32, 4, 2048, d, mult_qkv=0.5, bf16=True)
    _group_check(f"cfg5-d{d}", q, k, v, do, True, b=0, kvh=2, tol=TOL_BF16)


@pytest.mark.parametrize("causal,d", [(True, 64), (False, 64), (True, 128)])
def test_forward_tilings_agree(causal, d):
    """The bf16 forward takes 64-query work-groups when fewer than 768 of 128
    queries would fill the GPU (not for non-causal d = 128). B1 H12 N4096 gives
    384 of them (so 64-query work-groups run); B2 gives 768 (128 queries). The
    same batch-0 heads in both launches agree to bf16 rounding in O (the
    tilings rescale at different stages) and to fp32 rounding in LSE, and one
    head of the B1 launch matches the oracle."""
    import torch
    import mx230_amd as mx
    q, k, v, _ = make_inputs(2, 12, 12, 4096, d, bf16=True, seeds=(61, 62, 63, 64))
    outs = []
    for B in (1, 2):
        tq, tk, tv = (to_dev(x[:B], True) for x in (q, k, v))
        o = torch.empty_like(tq)
        lse = torch.empty((B, 12, 4096), dtype=torch.float32, device="cuda")
        mx.run_flash_lse(tq, tk, tv, o, lse, causal)
        torch.cuda.synchronize()
        outs.append((to_np(o)[0], to_np(lse)[0]))
    (o1, l1), (o2, l2) = outs
    eo, el = rel_err(o1, o2), rel_err(l1, l2)
    print(f"\n[tilings causal={causal} d={d}] O {eo:.2e} LSE {el:.2e}", flush=True)
    assert eo <= 2.0 ** -7 and el <= 1e-5, (eo, el)
    h = 5
    ro, rl = oracle.mha_fwd(q[:1, h:h + 1], k[:1, h:h + 1], v[:1, h:h + 1], 1, 1, 1, 4096, d, causal,
                            nthreads=1)
    errs = (rel_err(o1[h], ro[0, 0]), rel_err(l1[h], rl[0, 0]))
    print(f"[tilings causal={causal} d={d}] oracle head {h}: O {errs[0]:.2e} LSE {errs[1]:.2e}", flush=True)
    assert max(errs) <= TOL_BF16, errs


# ---------------------------------------------------------- long sequence --

def _rows_f64(q, k, v, do, rows, cols_chunk=4096):
    """float64 reference values for the sampled query rows of one head:
    O, LSE, Delta (from the exact O) and dQ, each row computed from all keys."""
    q64, k64, v64, do64 = (x.astype(np.float64) for x in (q, k, v, do))
    d = q.shape[1]
    scale = 1.0 / np.sqrt(d)
    s = q64[rows] @ k64.T * scale
    m = s.max(axis=1, keepdims=True)
    p = np.exp(s - m)
    l = p.sum(axis=1, keepdims=True)
    p /= l
    o = p @ v64
    lse = (m + np.log(l))[:, 0]
    dp = do64[rows] @ v64.T
    delta = (do64[rows] * o).sum(axis=1)
    dq = (p * (dp - delta[:, None])) @ k64 * scale
    return o, lse, dq


def _keys_f64(q, k, v, do, keys, chunk=2048):
    """float64 dK, dV rows of the sampled keys of one head: needs LSE and Delta
    of every query, computed chunk by chunk over the query rows."""
    q64, k64, v64, do64 = (x.astype(np.float64) for x in (q, k, v, do))
    N, d = q.shape
    scale = 1.0 / np.sqrt(d)
    dk = np.zeros((len(keys), d))
    dv = np.zeros((len(keys), d))
    for i0 in range(0, N, chunk):
        s = q64[i0:i0 + chunk] @ k64.T * scale
        m = s.max(axis=1, keepdims=True)
        p = np.exp(s - m)
        p /= p.sum(axis=1, keepdims=True)
        o = p @ v64
        delta = (do64[i0:i0 + chunk] * o).sum(axis=1)
        pk = p[:, keys]
        dpk = do64[i0:i0 + chunk] @ v64[keys].T
        dv += pk.T @ do64[i0:i0 + chunk]
        dk += (pk * (dpk - delta[:, None])).T @ q64[i0:i0 + chunk] * scale
    return dk, dv


@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "f32"])
def test_cfg3_long_sequence_o_n_memory(bf16):
    """B1 H12 N32768 d64 non-causal: no N x N buffer anywhere (the library
    allocates nothing: device free memory is unchanged across forward +
    backward), and sampled rows of head 7 match float64."""
    import torch
    import mx230_amd as mx
    B, H, N, d = 1, 12, 32768, 64
    # warm-up on a tiny input: the runtime loads the code object on the first
    # launch, which is not an allocation of the library
    gpu_fwd_bwd(*make_inputs(1, 1, 1, 70, d, bf16=bf16), False, bf16)
    q, k, v, do = make_inputs(B, H, H, N, d, bf16=bf16)
    tq, tk, tv, tdo = (to_dev(x, bf16) for x in (q, k, v, do))
    o, dq = torch.empty_like(tq), torch.empty_like(tq)
    dk, dv = torch.empty_like(tk), torch.empty_like(tv)
    lse = torch.empty((B, H, N), dtype=torch.float32, device="cuda")
    delta = torch.empty_like(lse)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    alloc0 = torch.cuda.memory_allocated()
    print(f"\n[cfg3 bf16={bf16}] running", flush=True)
    mx.run_flash_lse(tq, tk, tv, o, lse, False)
    mx.run_preprocess(tdo, o, delta)
    mx.run_bwd_flash(tq, tk, tv, tdo, lse, delta, dq, dk, dv, False)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == alloc0
    assert torch.cuda.mem_get_info()[0] == free0
    tol = TOL_BF16 if bf16 else TOL_F32
    h = 7
    rows = np.array([0, 1, 4095, 16384, 30001, N - 1])
    o_r, lse_r, dq_r = _rows_f64(q[0, h], k[0, h], v[0, h], do[0, h], rows)
    got_o, got_lse, got_dq = (to_np(t)[0, h][rows] for t in (o, lse, dq))
    for name, g_, r_ in (("O", got_o, o_r), ("LSE", got_lse, lse_r), ("dQ", got_dq, dq_r)):
        e = rel_err(g_, r_)
        print(f"[cfg3] {name} sampled rows {e:.2e}", flush=True)
        assert e <= tol, (name, e)
    keys = np.array([0, 777, 20000, N - 1])
    dk_r, dv_r = _keys_f64(q[0, h], k[0, h], v[0, h], do[0, h], keys)
    for name, g_, r_ in (("dK", to_np(dk)[0, h][keys], dk_r), ("dV", to_np(dv)[0, h][keys], dv_r)):
        e = rel_err(g_, r_)
        print(f"[cfg3] {name} sampled keys {e:.2e}", flush=True)
        assert e <= tol, (name, e)
    gpu = tuple(to_np(t) for t in (o, lse, delta, dq, dk, dv))
    _closed_forms(gpu, do, H)


# --------------------------------------------------------- naive baselines --

@pytest.mark.parametrize("causal", [False, True])
def test_naive_forward_matches_oracle(causal):
    """Naive::run (main.rs:32-66): scores, softmax, S V with the N x N scratch."""
    import torch
    import mx230_amd as mx
    q, k, v, do = make_inputs(2, 4, 2, 300, 64)
    tq, tk, tv = (to_dev(x, False) for x in (q, k, v))
    s = torch.empty(mx.naive_scratch_bytes(tq, tk, causal) // 4, dtype=torch.float32, device="cuda")
    o = torch.empty_like(tq)
    mx.naive_run(tq, tk, tv, s, o, causal)
    ref_o, _ = oracle.mha_fwd(q, k, v, 2, 4, 2, 300, 64, causal)
    assert rel_err(to_np(o), ref_o) <= TOL_F32


@pytest.mark.parametrize("causal", [False, True])
def test_naive_backward_matches_oracle(causal):
    """run_bwd_naive (main.rs:147-173): atomic dK/dV into zeroed outputs."""
    import torch
    import mx230_amd as mx
    q, k, v, do = make_inputs(1, 4, 2, 257, 64, uniform=True, seeds=(11, 12, 13, 14))
    tq, tk, tv, tdo = (to_dev(x, False) for x in (q, k, v, do))
    o, lse = mx.attention_fwd(tq, tk, tv, causal)
    delta = torch.empty_like(lse)
    mx.run_preprocess(tdo, o, delta)
    dq, dk, dv = torch.zeros_like(tq), torch.zeros_like(tk), torch.zeros_like(tv)
    mx.run_bwd_naive(tq, tk, tv, tdo, lse, delta, dq, dk, dv, causal)
    ref = oracle_fwd_bwd(q, k, v, do, causal)
    for name, g_, r_ in zip(("dQ", "dK", "dV"), (dq, dk, dv), ref[2:]):
        e = rel_err(to_np(g_), r_)
        assert e <= TOL_F32, (name, e)


# ------------------------------------------------------- boundary behaviour --

def test_errors_are_returned_not_launched():
    import torch
    import mx230_amd as mx
    q = torch.zeros(1, 1, 64, 96, device="cuda", dtype=torch.bfloat16)
    o, lse = torch.empty_like(q), torch.empty(1, 1, 64, device="cuda")
    with pytest.raises(mx.MxfaError, match="UNSUPPORTED"):
        mx.run_flash_lse(q, q, q, o, lse, True)
    x = torch.zeros(1, 1, 65 * 64 + 1, device="cuda", dtype=torch.float32)
    mis = x[..., 1:].reshape(1, 1, 65, 64)  # data_ptr 4 bytes past a 16-byte boundary
    lib = mx.load_library()
    sh = mx.shape_of(mis, mis, False).c()
    rc = lib.mxfa_run_flash(ctypes.byref(sh), ctypes.c_void_p(mis.data_ptr()),
                            ctypes.c_void_p(mis.data_ptr()), ctypes.c_void_p(mis.data_ptr()),
                            ctypes.c_void_p(mis.data_ptr()), None)
    assert rc == -5
    with pytest.raises(ValueError, match="contiguous"):
        t = torch.zeros(1, 1, 64, 128, device="cuda")[..., ::2]
        mx.run_flash(t, t, t, torch.empty(1, 1, 64, 64, device="cuda"), False)
    torch.cuda.synchronize()


def test_runs_on_the_callers_stream():
    """Launches go to the stream passed in (here a side stream), in order."""
    import torch
    import mx230_amd as mx
    q, k, v, do = make_inputs(1, 2, 1, 200, 64, bf16=True)
    tq, tk, tv, tdo = (to_dev(x, True) for x in (q, k, v, do))
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        o, lse = mx.attention_fwd(tq, tk, tv, True)
        dq, dk, dv = mx.attention_bwd(tq, tk, tv, o, lse, tdo, True)
    side.synchronize()
    gpu = tuple(to_np(t) for t in (o, lse, lse, dq, dk, dv))
    ref = oracle_fwd_bwd(q, k, v, do, True)
    errs, bad = parity(gpu, ref, TOL_BF16)
    assert not bad, errs


def test_prepared_calls_match_direct_calls():
    """mx.prepare: the forward and the backward (GQA, through its workspace)
    as prepared calls, each run twice, give the direct calls' bits."""
    import torch
    import mx230_amd as mx
    q, k, v, do = make_inputs(1, 8, 2, 300, 64, bf16=True, seeds=(41, 42, 43, 44))
    tq, tk, tv, tdo = (to_dev(x, True) for x in (q, k, v, do))
    B, H, N, d = q.shape
    outs = []
    for prepared in (False, True):
        o, lse = torch.empty_like(tq), torch.empty((B, H, N), device="cuda")
        delta = torch.empty_like(lse)
        dq, dk, dv = torch.empty_like(tq), torch.empty_like(tk), torch.empty_like(tv)
        nws = mx.bwd_workspace_bytes(tq, tk, True)
        ws = torch.empty(nws, dtype=torch.uint8, device="cuda") if nws else None
        fwd_args = (tq, tk, tv, o, lse, True)
        bwd_args = (tq, tk, tv, o, tdo, lse, delta, dq, dk, dv, ws, True)
        if prepared:
            fwd, bwd = mx.prepare(mx.run_flash_lse, *fwd_args), mx.prepare(mx.run_bwd_ws, *bwd_args)
            for _ in range(2):
                fwd()
                bwd()
        else:
            mx.run_flash_lse(*fwd_args)
            mx.run_bwd_ws(*bwd_args)
        torch.cuda.synchronize()
        outs.append((o, lse, dq, dk, dv))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_code_object_load_errors_and_reload(tmp_path):
    """The kernels are a code object loaded per device: with it unloaded and
    pointed at a missing or malformed file, launches return
    MXFA_ERR_CODE_OBJECT (and nothing runs); pointed back at the built one, the
    next launch loads it again and computes as before."""
    import torch
    import mx230_amd as mx
    q, k, v, do = make_inputs(1, 2, 1, 100, 64, bf16=True)
    tq, tk, tv = (to_dev(x, True) for x in (q, k, v))
    o, lse = torch.empty_like(tq), torch.empty((1, 2, 100), dtype=torch.float32, device="cuda")
    mx.run_flash_lse(tq, tk, tv, o, lse, True)
    torch.cuda.synchronize()
    want = to_np(o)
    lib = mx.load_library()
    (tmp_path / "bad.hsaco").write_bytes(b"\x7fELF" + bytes(200))
    try:
        for path in (str(tmp_path / "missing.hsaco"), str(tmp_path / "bad.hsaco")):
            assert lib.mxfa_shutdown() == 0
            mx.set_code_object(path)
            with pytest.raises(mx.MxfaError, match="CODE_OBJECT"):
                mx.run_flash_lse(tq, tk, tv, o, lse, True)
            assert lib.mxfa_init(0) == -9
    finally:
        mx.set_code_object(None)
    assert lib.mxfa_init(0) == 0
    o.zero_()
    mx.run_flash_lse(tq, tk, tv, o, lse, True)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(o), want)
