"""Roofline probes on the MI355X: measured ceilings fall inside what the part
can physically do (AMD's published dense peaks: bf16 MFMA 2516.6 TFLOP/s, fp32
MFMA 157.3 TFLOP/s, HBM3E 8 TB/s) and well above what a broken probe (a
serialised chain, a partial grid) would show."""
from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


def test_probe_mfma_bf16():
    import mx230_amd as mx
    t = mx.probe_mfma_tflops(bf16=True)
    print(f"\n[probe] bf16 MFMA {t:.0f} TFLOP/s", flush=True)
    assert 1000.0 < t < 2600.0


def test_probe_mfma_fp32():
    import mx230_amd as mx
    t = mx.probe_mfma_tflops(bf16=False)
    print(f"\n[probe] fp32 MFMA {t:.1f} TFLOP/s", flush=True)
    assert 60.0 < t < 165.0


@pytest.mark.parametrize("copy", [False, True], ids=["read", "copy"])
def test_probe_hbm(copy):
    import mx230_amd as mx
    g = mx.probe_hbm_gbps(mib=1024, copy=copy)
    print(f"\n[probe] HBM {'copy' if copy else 'read'} {g:.0f} GB/s", flush=True)
    assert 2000.0 < g < 8200.0
