"""Roofline probes on the MI355X: measured ceilings fall inside what the part
can physically do (AMD's published dense peaks: bf16 MFMA 2516.6 TFLOP/s, fp32
MFMA 157.3 TFLOP/s, HBM3E 8 TB/s) and above 60% of those peaks: boxes measured
so far hold 1.86-2.40 PFLOP/s bf16, 127-137 TFLOP/s fp32 and 6.3-6.4 TB/s of
streaming reads, while a broken probe (a serialised chain, a partial grid, an
accumulator round trip through memory) shows half or less."""
from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("big", [False, True], ids=["16x16x32", "32x32x16"])
def test_probe_mfma_bf16(big):
    import mx230_amd as mx
    t = mx.probe_mfma_tflops(bf16=True, big=big)
    print(f"\n[probe] bf16 MFMA {'32x32x16' if big else '16x16x32'} {t:.0f} TFLOP/s", flush=True)
    assert 0.6 * 2516.6 < t < 2600.0


def test_probe_mfma_fp32():
    import mx230_amd as mx
    t = mx.probe_mfma_tflops(bf16=False)
    print(f"\n[probe] fp32 MFMA {t:.1f} TFLOP/s", flush=True)
    assert 0.6 * 157.3 < t < 165.0


@pytest.mark.parametrize("copy", [False, True], ids=["read", "copy"])
def test_probe_hbm(copy):
    import mx230_amd as mx
    g = mx.probe_hbm_gbps(mib=1024, copy=copy)
    print(f"\n[probe] HBM {'copy' if copy else 'read'} {g:.0f} GB/s", flush=True)
    assert (0.6 if not copy else 0.45) * 8000.0 < g < 8200.0


def test_probe_dq_atomic_counts_and_rates():
    """The fused-dQ write replay: on a zeroed buffer one atomic launch leaves
    row // 128 + 1 in every element of row `row` (the key blocks at or before
    its diagonal); the store variant moves the same payload."""
    import torch
    import mx230_amd as mx
    import ctypes
    lib = mx.load_library()
    bh, n = 3, 1024
    acc = torch.zeros(bh * n * 64, dtype=torch.float32, device="cuda")
    nbytes = ctypes.c_double(0.0)
    rc = lib.mxfa_probe_dq_atomic(ctypes.c_void_p(acc.data_ptr()), bh, n, 1, ctypes.byref(nbytes), None)
    assert rc == 0
    torch.cuda.synchronize()
    want = (torch.arange(n, device="cuda") // 128 + 1).float().view(1, n, 1).expand(bh, n, 64)
    assert torch.equal(acc.view(bh, n, 64), want)
    assert nbytes.value == bh * sum(n // 64 - 2 * kb for kb in range(n // 128)) * 64 * 64 * 4
    a = mx.probe_dq_atomic(48, 4096, atomic=True)
    st = mx.probe_dq_atomic(48, 4096, atomic=False)
    print(f"\n[probe] fused-dQ writes at B*H=48 N=4096: {a['payload_bytes'] / 1e6:.0f} MB, "
          f"atomic {a['us']:.0f} us ({a['tbps']:.2f} TB/s), store {st['us']:.0f} us ({st['tbps']:.2f} TB/s)",
          flush=True)
    # the 830 MB payload lands on 50 MB of addresses: repeated stores to a line
    # merge in the write-back caches, so the store rate has no HBM bound
    assert 0.05 < a["tbps"] < 10.0 and st["tbps"] > 0.05


def test_probe_mix_ceilings_order():
    """Instruction-mix ceilings: the MFMA-only mix runs at the MFMA probe's
    rate (the same instruction, 8 independent chains); adding a kernel's VALU
    or LDS work can only lower it, and the full mix is no faster than either
    part alone."""
    import mx230_amd as mx
    mfma = mx.probe_mfma_tflops(bf16=True)
    got = {m: mx.probe_mix_tflops(m, waves_per_simd=3, iters=128) for m in mx.PROBE_MIXES}
    print("\n[probe] mix ceilings (3 waves/SIMD): " + " ".join(f"{m}={t:.0f}" for m, t in got.items())
          + f" (MFMA probe {mfma:.0f}) TFLOP/s", flush=True)
    assert 0.85 * mfma < got["mfma"] < 1.1 * mfma
    assert 0.85 * mfma < got["mfma32"] < 1.1 * mfma
    for m in ("dkv", "dkv_valu", "dkv_lds", "dq", "fwd"):
        assert 0.2 * mfma < got[m] < 1.05 * got["mfma"], m
        if m + "32" in got:
            assert 0.2 * mfma < got[m + "32"] < 1.05 * got["mfma32"], m + "32"
    assert got["dkv"] < 1.05 * min(got["dkv_valu"], got["dkv_lds"])


def test_timeline_build():
    """The timeline build of the code object stamps every work-group of a
    one-launch backward in order (start <= first stage <= end of loop <= stores
    acknowledged) and computes the same bits as the normal build; the normal
    build has no timeline (MXFA_ERR_UNSUPPORTED). The normal code object is
    loaded again at the end."""
    import numpy as np
    import torch
    import mx230_amd as mx
    B, H, N, d = 1, 4, 1024, 64
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    q, k, v, do = (torch.randn((B, H, N, d), generator=gen, device="cuda").to(torch.bfloat16) for _ in range(4))
    o = torch.empty_like(q)
    lse = torch.empty((B, H, N), device="cuda")
    delta = torch.empty_like(lse)

    def bwd():
        mx.run_flash_lse(q, k, v, o, lse, True)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        mx.run_bwd(q, k, v, o, do, lse, delta, dq, dk, dv, True)
        torch.cuda.synchronize()
        return dq, dk, dv

    ref = bwd()
    with pytest.raises(mx.MxfaError):
        mx.probe_wg_times()
    try:
        mx.shutdown()
        mx.set_code_object(mx.TIMELINE_CODE_OBJECT_PATH)
        mx.init(0)
        got = bwd()
        t = mx.probe_wg_times()
        mx.run_flash_lse(q, k, v, o, lse, True)
        torch.cuda.synchronize()
        tf = mx.probe_wg_times()
    finally:
        mx.shutdown()
        mx.set_code_object(None)
        mx.init(0)
    for a_, b_ in zip(got, ref):
        assert torch.equal(a_, b_)
    nwg = 2 * B * H * (N // 128)
    info = t[:nwg, 4:6].astype(np.int64)
    t = t[:nwg, :4].astype(np.int64)
    assert np.all(t[:, 0] > 0)
    assert np.all(np.diff(t, axis=1) >= 0)
    # dQ work-groups first (query blocks in increasing order), then dK/dV
    # (key block 0 first); causal stages: 2 (qb + 1) and N / 64 - 2 kb
    ndq = nwg // 2
    kind, block = info[:, 0] >> 32, info[:, 0] & 0xffffffff
    assert np.all(kind[:ndq] == 0) and np.all(kind[ndq:] == 1)
    assert np.array_equal(block[:ndq], np.arange(ndq) // (B * H))
    assert np.array_equal(block[ndq:], np.arange(ndq) // (B * H))
    assert np.array_equal(info[:ndq, 1], 2 * (block[:ndq] + 1))
    assert np.array_equal(info[ndq:, 1], N // 64 - 2 * block[ndq:])
    # the forward (64-query work-groups at this size, heaviest query block
    # first): kind 2, its query block, one 64-key stage per 64 queries to the
    # diagonal
    nfw = B * H * (N // 64)
    tf = tf[:nfw].astype(np.int64)
    assert np.all(np.diff(tf[:, :4], axis=1) >= 0)
    assert np.all(tf[:, 4] >> 32 == 2)
    fblock = tf[:, 4] & 0xffffffff
    assert np.array_equal(fblock, N // 64 - 1 - np.arange(nfw) // (B * H))
    assert np.array_equal(tf[:, 5], fblock + 1)
    span_us = (t[:, 3].max() - t[:, 0].min()) * 0.01
    print(f"\n[timeline] {nwg} work-groups over {span_us:.1f} us", flush=True)
    assert 1.0 < span_us < 10000.0


def test_time_median_ms():
    """mx.time_median_ms, the counterpart of common/src/lib.rs:22-43: the
    median of per-call event times after the warm-up calls; two backward
    calls per invocation take about twice as long as one."""
    import torch
    import mx230_amd as mx
    B, H, N, d = 2, 12, 2048, 64
    gen = torch.Generator(device="cuda")
    gen.manual_seed(9)
    q, k, v, do = (torch.randn((B, H, N, d), generator=gen, device="cuda").to(torch.bfloat16) for _ in range(4))
    o, dq, dk, dv = (torch.empty_like(q) for _ in range(4))
    lse = torch.empty((B, H, N), device="cuda")
    delta = torch.empty_like(lse)
    mx.run_flash_lse(q, k, v, o, lse, True)

    def bwd():
        mx.run_bwd(q, k, v, o, do, lse, delta, dq, dk, dv, True)

    calls = []
    one = mx.time_median_ms(lambda: (calls.append(1), bwd()), warmup=3, iters=9)
    assert len(calls) == 3 + 9
    two = mx.time_median_ms(lambda: (bwd(), bwd()), warmup=3, iters=9)
    print(f"\n[time_median_ms] one backward {one * 1e3:.1f} us, two {two * 1e3:.1f} us", flush=True)
    assert 0.0 < one < 10.0
    assert 1.5 < two / one < 2.3
