"""mxfa_run_bwd_noalloc, the backward from O for callers that cannot allocate:
through the C ABI it gives exactly what mxfa_run_bwd_ws gives with a
caller-owned workspace (the same kernels, split and summation order, so the
outputs are bitwise equal), on consecutive calls whose second is smaller (the
static scratch keeps the first call's partial sums, which the second must not
read), for GQA shapes that split their dK/dV pass and for one that does not;
and the device's free memory does not change across a call."""
from __future__ import annotations

import ctypes

import pytest

pytestmark = pytest.mark.gpu

# (B, Hq, Hkv, N, d, causal), largest first; every call below runs both paths
CALLS = [
    [(1, 32, 4, 2048, 128, True), (1, 8, 2, 1000, 64, True)],   # 64 MiB (+8 KB) then 4.1 MB of scratch
    [(2, 14, 2, 4096, 64, True), (1, 6, 2, 577, 64, False)],     # cfg4, then non-causal ragged
    [(1, 4, 4, 300, 64, True), (1, 4, 1, 200, 128, True)],       # no split, then a d = 128 split
]


def _inputs(B, H, Hkv, N, d, seed):
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    q = torch.randn(B, H, N, d, device="cuda", generator=g).bfloat16()
    k = torch.randn(B, Hkv, N, d, device="cuda", generator=g).bfloat16()
    v = torch.randn(B, Hkv, N, d, device="cuda", generator=g).bfloat16()
    do = torch.randn(B, H, N, d, device="cuda", generator=g).bfloat16()
    return q, k, v, do


def _outs(q, k):
    import torch
    B, H, N, _ = q.shape
    return (torch.full((B, H, N), float("nan"), device="cuda"), torch.full_like(q, float("nan")),
            torch.full_like(k, float("nan")), torch.full_like(k, float("nan")))


@pytest.mark.parametrize("calls", CALLS, ids=["cfg5d128-then-small", "cfg4-then-ragged", "mha-then-d128"])
def test_noalloc_equals_workspace_path(calls):
    import torch
    import mx230_amd as mx
    lib = mx.load_library()
    assert lib.mxfa_init(0) == 0
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    for i, (B, H, Hkv, N, d, causal) in enumerate(calls):
        print(f"\n[noalloc] call {i}: B{B} Hq{H} Hkv{Hkv} N{N} d{d} causal={causal}", flush=True)
        q, k, v, do = _inputs(B, H, Hkv, N, d, seed=100 + i)
        o = torch.empty_like(q)
        lse = torch.empty((B, H, N), device="cuda")
        mx.run_flash_lse(q, k, v, o, lse, causal)
        sh = mx.shape_of(q, k, causal).c()
        nws = lib.mxfa_bwd_workspace_bytes(ctypes.byref(sh))
        assert nws <= lib.mxfa_bwd_noalloc_scratch_bytes()
        ws = torch.empty(max(nws, 16), dtype=torch.uint8, device="cuda")
        ref = _outs(q, k)
        rc = lib.mxfa_run_bwd_ws(ctypes.byref(sh), P(q), P(k), P(v), P(o), P(do), P(lse), P(ref[0]), P(ref[1]),
                                 P(ref[2]), P(ref[3]), P(ws) if nws else None, nws, None)
        assert rc == 0, rc
        got = _outs(q, k)
        stream = torch.cuda.current_stream()
        # the entry point's defining property: the device's free memory is the
        # same before and after it (no allocation by the library or a
        # runtime it calls; every buffer above was allocated before this)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        rc = lib.mxfa_run_bwd_noalloc(ctypes.byref(sh), P(q), P(k), P(v), P(o), P(do), P(lse), P(got[0]),
                                      P(got[1]), P(got[2]), P(got[3]), ctypes.c_void_p(stream.cuda_stream))
        assert rc == 0, rc
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
        assert free1 == free0, f"call {i}: device free memory changed by {free0 - free1} bytes"
        for name, a, b in zip(("Delta", "dQ", "dK", "dV"), got, ref):
            assert torch.equal(a, b), f"call {i}: {name} of mxfa_run_bwd_noalloc differs from mxfa_run_bwd_ws"
        print(f"[noalloc] call {i}: workspace {nws} bytes, outputs bitwise equal", flush=True)
