"""The one-launch backward (bwd_fused_entry, kernels mxfa_bwd_*: the default of mxfa_run_bwd for
bf16): dQ work-groups publish Delta per 128-row block behind a flag, and the
dK/dV work-groups of the same launch wait for it, or compute the rows
themselves after a wait bounded in time.

- With flags it is bitwise equal to the two-launch backward
  (set_bwd_options(one_launch=False)), over shapes and over repeated runs,
  since it stages the same Delta values. A stale or early read of Delta would
  show as a mismatch. At d = 64 the shapes whose dQ and dK/dV work-groups fit
  the three-wave kernel's slots at once (all but the north star and cfg5 here)
  run the two-wave form with batched LDS reads (kernels mxfa_bwd_b64_*_w2),
  which computes the same arithmetic in the same order.
- With every wait forced to give up (delta_wait_us < 0) the dK/dV work-groups
  compute Delta from O and dO with the dQ work-groups' own arithmetic, so the
  results are still bitwise equal, and the device's fallback counter grows by
  one per stage.
- With a GQA split through a workspace, the one launch (whose last work-groups
  add the shares' partial sums once the shares' flags are set) equals the
  two-launch split (with its reduce launch) bitwise.
- Launches in flight together on several streams, more than the flag slots,
  so later launches see other launches' Delta flags, still give each one its
  own result, bitwise. With a GQA split each launch's share flags are in its
  own workspace, with its own value: no reduce work-group waits out its bound.
"""
from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu

SHAPES = [
    ("north-star", (4, 12, 12, 4096, 64), True),
    ("cfg5-d64", (1, 32, 4, 2048, 64), True),
    ("gqa-ragged", (2, 14, 2, 777, 64), True),
    ("gqa-noncausal", (1, 6, 2, 576, 64), False),
    ("d128", (1, 8, 8, 1000, 128), True),
    ("d128-gqa-noncausal", (1, 4, 1, 2048, 128), False),
    ("n1", (1, 4, 4, 1, 64), True),
    ("n130", (2, 3, 3, 130, 64), False),
    ("w2-edge", (4, 12, 12, 1024, 64), True),    # 768 dQ + dK/dV work-groups: the two-wave form's limit
    ("w2-noncausal", (4, 12, 12, 1024, 64), False),
    ("past-w2", (4, 12, 12, 1152, 64), True),    # 864: the three-wave form
]


@pytest.fixture
def opts():
    """set(one_launch=..., delta_wait_us=...) for the test; the defaults after it."""
    import mx230_amd as mx
    old = mx.set_bwd_options(one_launch=True, delta_wait_us=200)
    yield lambda **kw: mx.set_bwd_options(**kw)
    mx.set_bwd_options(**old)


def _setup(B, H, Hkv, N, d, causal, seed=1):
    import torch
    import mx230_amd as mx
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    q = torch.randn(B, H, N, d, device="cuda", generator=g).bfloat16()
    k = torch.randn(B, Hkv, N, d, device="cuda", generator=g).bfloat16()
    v = torch.randn(B, Hkv, N, d, device="cuda", generator=g).bfloat16()
    do = torch.randn(B, H, N, d, device="cuda", generator=g).bfloat16()
    o = torch.empty_like(q)
    lse = torch.empty(B, H, N, device="cuda")
    mx.run_flash_lse(q, k, v, o, lse, causal)
    return q, k, v, do, o, lse


def _bwd(t, causal, stream=None):
    import torch
    import mx230_amd as mx
    q, k, v, do, o, lse = t
    delta = torch.full(lse.shape, float("nan"), device="cuda")
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    mx.run_bwd(q, k, v, o, do, lse, delta, dq, dk, dv, causal, stream=stream)
    return delta, dq, dk, dv


def _sync(outs):
    import torch
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("name,shape,causal", SHAPES, ids=[s[0] for s in SHAPES])
def test_one_launch_equals_two_launches(opts, name, shape, causal):
    t = _setup(*shape, causal)
    opts(one_launch=False)
    ref = _sync(_bwd(t, causal))
    opts(one_launch=True)
    import torch
    for rep in range(3):
        got = _sync(_bwd(t, causal))
        for n, a, b in zip(("Delta", "dQ", "dK", "dV"), got, ref):
            assert torch.equal(a, b), f"{name} run {rep}: {n} differs from the two-launch backward"


def test_one_launch_repeated_north_star(opts):
    import torch
    t = _setup(4, 12, 12, 4096, 64, True, seed=7)
    opts(one_launch=False)
    ref = _sync(_bwd(t, True))
    opts(one_launch=True)
    outs = [_bwd(t, True) for _ in range(20)]
    torch.cuda.synchronize()
    bad = sum(not all(torch.equal(a, b) for a, b in zip(got, ref)) for got in outs)
    assert bad == 0, f"{bad} of 20 one-launch runs differ"


@pytest.mark.parametrize("name,shape,causal", SHAPES, ids=[s[0] for s in SHAPES])
def test_one_launch_fallback(opts, name, shape, causal):
    import torch
    import mx230_amd as mx
    t = _setup(*shape, causal, seed=3)
    opts(one_launch=False)
    ref = _sync(_bwd(t, causal))
    opts(one_launch=True, delta_wait_us=-1)
    n0 = mx.bwd_delta_fallbacks()
    got = _sync(_bwd(t, causal))
    n1 = mx.bwd_delta_fallbacks()
    for n, a, b in zip(("Delta", "dQ", "dK", "dV"), got, ref):
        assert torch.equal(a, b), f"{name}: {n} of the fallback differs from the two-launch backward"
    # one fallback per stage of every dK/dV work-group (a work-group per
    # (batch, KV head, key block of 4 x 32 keys, 4 x 16 at d = 128) walks
    # every query head of its group from its diagonal in 64-query stages),
    # and none when the waits are allowed
    B, H, Hkv, N, d = shape
    bkv = 128 if d == 64 else 64
    want = B * Hkv * sum((H // Hkv) * -(-(N - (kb * bkv if causal else 0)) // 64) for kb in range(-(-N // bkv)))
    assert n1 - n0 == want, (n0, n1, want)
    opts(delta_wait_us=200)
    _sync(_bwd(t, causal))
    print(f"[{name}] fallbacks forced {n1 - n0}, then {mx.bwd_delta_fallbacks() - n1}", flush=True)


def test_one_launch_concurrent_streams(opts):
    """Six launches in flight on six streams (four flag slots)."""
    import torch
    opts(one_launch=True)
    cases = [_setup(2, 6, 2, 1000 + 64 * i, 64, True, seed=20 + i) for i in range(6)]
    opts(one_launch=False)
    refs = [_sync(_bwd(t, True)) for t in cases]
    opts(one_launch=True)
    streams = [torch.cuda.Stream() for _ in cases]
    torch.cuda.synchronize()
    outs = []
    for t, s in zip(cases, streams):
        with torch.cuda.stream(s):
            outs.append(_bwd(t, True, stream=s))
    torch.cuda.synchronize()
    for i, (got, ref) in enumerate(zip(outs, refs)):
        for n, a, b in zip(("Delta", "dQ", "dK", "dV"), got, ref):
            assert torch.equal(a, b), (i, n)


@pytest.mark.parametrize("nstreams", [6, 12])
def test_one_launch_concurrent_streams_gqa_split(opts, nstreams):
    """GQA-split launches in flight on 6 or 12 streams, each with its own
    workspace (and so its own share flags): each result is the two-launch
    one bitwise, and no reduce work-group waits out its bound."""
    import torch
    import mx230_amd as mx
    cases = [_setup(2, 6, 2, 1000 + 64 * i, 64, True, seed=40 + i) for i in range(nstreams)]
    wss = [torch.empty(mx.bwd_workspace_bytes(t[0], t[1], True), dtype=torch.uint8, device="cuda") for t in cases]
    assert all(w.numel() > 0 for w in wss)

    def bwd(t, ws, stream=None):
        q, k, v, do, o, lse = t
        delta = torch.empty_like(lse)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        mx.run_bwd_ws(q, k, v, o, do, lse, delta, dq, dk, dv, ws, True, stream=stream)
        return delta, dq, dk, dv

    opts(one_launch=False)
    refs = [_sync(bwd(t, w)) for t, w in zip(cases, wss)]
    opts(one_launch=True)
    t0 = mx.bwd_reduce_timeouts()
    streams = [torch.cuda.Stream() for _ in cases]
    torch.cuda.synchronize()
    outs = []
    for t, w, s in zip(cases, wss, streams):
        with torch.cuda.stream(s):
            outs.append(bwd(t, w, stream=s))
    torch.cuda.synchronize()
    assert mx.bwd_reduce_timeouts() == t0
    for i, (got, ref) in enumerate(zip(outs, refs)):
        for n, a, b in zip(("Delta", "dQ", "dK", "dV"), got, ref):
            assert torch.equal(a, b), (i, n)


def test_one_launch_gqa_split_queued_on_one_stream(opts):
    """Twenty GQA-split launches queued back to back on one stream (as a timed
    loop queues them) through one workspace: each finds the flags of the one
    before (another value) and waits for its own, none waits out its bound,
    and the last result is the two-launch one."""
    import torch
    import mx230_amd as mx
    t = _setup(1, 32, 4, 2048, 64, True, seed=77)
    q, k, v, do, o, lse = t
    ws = torch.empty(mx.bwd_workspace_bytes(q, k, True), dtype=torch.uint8, device="cuda")
    outs = {}
    for one in (False, True):
        opts(one_launch=one)
        delta = torch.empty_like(lse)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        call = mx.prepare(mx.run_bwd_ws, q, k, v, o, do, lse, delta, dq, dk, dv, ws, True)
        t0 = mx.bwd_reduce_timeouts()
        for _ in range(20 if one else 1):
            call()
        torch.cuda.synchronize()
        assert mx.bwd_reduce_timeouts() == t0
        outs[one] = (delta, dq, dk, dv)
    for n, a, b in zip(("Delta", "dQ", "dK", "dV"), outs[True], outs[False]):
        assert torch.equal(a, b), n


@pytest.mark.parametrize("shape", [(2, 14, 2, 4096, 64), (1, 32, 4, 2048, 64), (1, 32, 4, 2048, 128),
                                   (1, 8, 2, 300, 64), (1, 10, 2, 836, 64)],
                         ids=["cfg4", "cfg5-d64", "cfg5-d128", "ragged", "g5-mid-diagonal"])
def test_one_launch_with_gqa_split(opts, shape):
    import torch
    import mx230_amd as mx
    t = _setup(*shape, True, seed=9)
    q, k, v, do, o, lse = t
    nws = mx.bwd_workspace_bytes(q, k, True)
    assert nws > 0
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda")

    def run():
        delta = torch.full(lse.shape, float("nan"), device="cuda")
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        mx.run_bwd_ws(q, k, v, o, do, lse, delta, dq, dk, dv, ws, True)
        torch.cuda.synchronize()
        return delta, dq, dk, dv

    opts(one_launch=False)
    ref = run()
    opts(one_launch=True)
    for rep in range(3):
        got = run()
        for n, a, b in zip(("Delta", "dQ", "dK", "dV"), got, ref):
            assert torch.equal(a, b), f"run {rep}: {n} differs from the two-launch split"


def test_graph_capture_replays_correctly():
    """A captured backward (two launches: the one-launch form would replay the
    capture's flag epoch) replayed on new inputs, each replay against an eager
    run on the same inputs, with eager work in between."""
    import torch
    import mx230_amd as mx
    B, H, N, d = 2, 4, 640, 64
    q, k, v, do, o, lse = _setup(B, H, H, N, d, True, seed=30)
    delta = torch.empty_like(lse)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm-up on the capture stream
        mx.run_bwd(q, k, v, o, do, lse, delta, dq, dk, dv, True)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        mx.run_bwd(q, k, v, o, do, lse, delta, dq, dk, dv, True)
    for rep in range(3):
        t = _setup(B, H, H, N, d, True, seed=31 + rep)
        for dst, src in zip((q, k, v, do, o, lse), t):
            dst.copy_(src)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = _sync(_bwd(t, True))
        for n, a, b in zip(("Delta", "dQ", "dK", "dV"), (delta, dq, dk, dv), want):
            assert torch.equal(a, b), f"replay {rep}: {n} differs from the eager backward"
