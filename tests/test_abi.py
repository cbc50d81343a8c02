"""CPU-side checks of the C ABI (no GPU needed, no compute launched): the library
loads, exports every entry point include/mxfa.h declares, and rejects bad
arguments with the documented status codes before touching the device."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

import mx230_amd as mx

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mxfa.h")
PROBE_HEADER = os.path.join(ROOT, "include", "mxfa_probes.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(mx.LIB_PATH):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "mx230_amd", "csrc")], check=True)
    return mx.load_library()


def _declared(header=HEADER):
    text = open(header).read()
    return sorted(set(re.findall(r"\b(mxfa_[a-z0-9_]+)\s*\(", text)))


def test_header_and_python_agree():
    assert sorted(mx.EXPORTS) == _declared()
    assert sorted(mx.PROBE_EXPORTS) == _declared(PROBE_HEADER)


def test_every_declared_symbol_is_exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", mx.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (mxfa_\w+)", out))
    for name in _declared() + _declared(PROBE_HEADER):
        assert name in exported, name
        assert hasattr(lib, name)


def _shape(**kw):
    base = dict(B=1, Hq=2, Hkv=1, N=128, d=64, causal=1, dtype=mx.MXFA_BF16, scale=0.0)
    base.update(kw)
    return mx.MxfaShape(**base)


@pytest.mark.parametrize("kw,code", [
    (dict(), 0),
    (dict(dtype=7), -3),
    (dict(B=0), -2),
    (dict(N=0), -2),
    (dict(Hq=3, Hkv=2), -2),
    (dict(causal=2), -2),
    (dict(scale=-1.0), -2),
    (dict(scale=float("inf")), -2),
    (dict(d=96), -4),
    (dict(d=128, dtype=mx.MXFA_F32), -4),
    (dict(d=128), 0),
    (dict(N=64 * 65536), -2),
])
def test_check_shape(lib, kw, code):
    assert lib.mxfa_check_shape(ctypes.byref(_shape(**kw))) == code


def test_null_shape_and_pointers(lib):
    assert lib.mxfa_check_shape(None) == -1
    sh = _shape()
    p = ctypes.c_void_p(4096)
    assert lib.mxfa_run_flash_lse(ctypes.byref(sh), p, p, p, None, p, None) == -1
    assert lib.mxfa_run_flash_lse(None, p, p, p, p, p, None) == -1
    assert lib.mxfa_run_bwd_flash(ctypes.byref(sh), p, p, p, p, p, p, p, None, p, None) == -1
    assert lib.mxfa_run_preprocess(ctypes.byref(sh), None, p, p, None) == -1


def test_misaligned_pointer(lib):
    sh = _shape()
    ok, bad = ctypes.c_void_p(4096), ctypes.c_void_p(4096 + 8)
    assert lib.mxfa_run_flash(ctypes.byref(sh), ok, bad, ok, ok, None) == -5
    assert lib.mxfa_run_bwd_dkv(ctypes.byref(sh), ok, ok, ok, ok, ok, ok, ok, bad, None) == -5


def test_naive_paths_are_fp32_only(lib):
    sh = _shape(dtype=mx.MXFA_BF16)
    p = ctypes.c_void_p(4096)
    assert lib.mxfa_run_bwd_naive(ctypes.byref(sh), p, p, p, p, p, p, p, p, p, None) == -4
    assert lib.mxfa_run_naive_fwd(ctypes.byref(sh), p, p, p, p, p, None) == -4


def test_sizes_and_strings(lib):
    sh = _shape(B=2, Hq=3, Hkv=3, N=100, dtype=mx.MXFA_F32)
    assert lib.mxfa_bwd_workspace_bytes(ctypes.byref(sh)) == 0
    assert lib.mxfa_naive_scratch_bytes(ctypes.byref(sh)) == 2 * 3 * 100 * 100 * 4
    assert lib.mxfa_version() >= 100
    for code in mx.STATUS:
        assert lib.mxfa_strerror(code)
    assert lib.mxfa_strerror(12345) == b"unknown status"
    assert lib.mxfa_shutdown() == 0


# The workspace of a split: 2 x planes x B x Hkv x N x d fp32 partial sums
# (planes: the most shares any key block takes), then an 8-byte flag per
# share (all key blocks' shares) for the one-launch backward's reduce.
@pytest.mark.parametrize("kw,nbytes", [
    # no GQA: nothing to split
    (dict(B=4, Hq=12, Hkv=12, N=4096, d=64), 0),
    # cfg4 (Qwen2.5, 7:1): 2*2 (b, kv head) x 32 key blocks = 128 work-groups
    # for 2 x 768 slots; 7 is prime, so one query head per share at least;
    # about 58 stages per share gives key blocks 0-2 (7 x 64-60 stages) 8;
    # 908 shares in all
    (dict(B=2, Hq=14, Hkv=2, N=4096, d=64), 2 * 8 * 2 * 2 * 4096 * 64 * 4 + 8 * 908),
    # cfg5 d=64 (TinyLlama, 8:1): 64 work-groups; 4 shares give 256 < 1536, so
    # 8 at least; about 17 stages per share gives key block 0 (8 x 32 stages)
    # 16; 656 shares
    (dict(B=1, Hq=32, Hkv=4, N=2048, d=64), 2 * 16 * 1 * 4 * 2048 * 64 * 4 + 8 * 656),
    # cfg5 d=128: 64-key blocks, 128 work-groups for 2 x 512 slots: 8 shares
    # each, 1024
    (dict(B=1, Hq=32, Hkv=4, N=2048, d=128), 2 * 8 * 1 * 4 * 2048 * 128 * 4 + 8 * 1024),
    # 8 * 8 (b, kv head) x 32 key blocks = 2048 work-groups, twice 768 slots: no split
    (dict(B=8, Hq=16, Hkv=8, N=4096, d=64), 0),
    # 512 work-groups: 3 shares would be the first to reach 2 x 768, and 4
    # divides 8: 4 shares each, 2048
    (dict(B=4, Hq=32, Hkv=4, N=4096, d=64), 2 * 4 * 4 * 4 * 4096 * 64 * 4 + 8 * 2048),
    # fp32 parity path, tiny GQA shape: whole group split, 2 shares
    (dict(B=1, Hq=2, Hkv=1, N=128, d=64, dtype=mx.MXFA_F32), 2 * 2 * 1 * 1 * 128 * 64 * 4 + 8 * 2),
    # invalid shape
    (dict(Hq=3, Hkv=2), 0),
])
def test_bwd_workspace_bytes(lib, kw, nbytes):
    assert lib.mxfa_bwd_workspace_bytes(ctypes.byref(_shape(**kw))) == nbytes


@pytest.fixture
def default_options():
    old = mx.set_bwd_options(one_launch=True, delta_wait_us=200, reduce_wait_us=2000000)
    yield
    mx.set_bwd_options(**old)


def test_bwd_options(lib, default_options):
    o = mx.MxfaBwdOptions()
    assert lib.mxfa_get_bwd_options(ctypes.byref(o)) == 0
    assert (o.one_launch, o.delta_wait_us, o.reduce_wait_us) == (1, 200, 2000000)
    assert lib.mxfa_set_bwd_options(None) == mx_status("MXFA_ERR_NULL")
    assert lib.mxfa_get_bwd_options(None) == mx_status("MXFA_ERR_NULL")
    assert lib.mxfa_set_bwd_options(ctypes.byref(mx.MxfaBwdOptions(2, 5, 0))) == mx_status("MXFA_ERR_SHAPE")
    assert lib.mxfa_set_bwd_options(ctypes.byref(mx.MxfaBwdOptions(1, 5, -1))) == mx_status("MXFA_ERR_SHAPE")
    assert lib.mxfa_set_bwd_options(ctypes.byref(mx.MxfaBwdOptions(0, -1, 0))) == 0
    assert mx.get_bwd_options() == {"one_launch": False, "delta_wait_us": -1, "reduce_wait_us": 0}
    assert lib.mxfa_bwd_delta_fallbacks(None) == mx_status("MXFA_ERR_NULL")
    assert lib.mxfa_bwd_reduce_timeouts(None) == mx_status("MXFA_ERR_NULL")


def test_bwd_one_launch(lib, default_options):
    assert lib.mxfa_bwd_one_launch(ctypes.byref(_shape(B=4, Hq=12, Hkv=12, N=4096))) == 1
    assert lib.mxfa_bwd_one_launch(ctypes.byref(_shape(d=128))) == 1
    assert lib.mxfa_bwd_one_launch(ctypes.byref(_shape(dtype=mx.MXFA_F32))) == 0
    assert lib.mxfa_bwd_one_launch(ctypes.byref(_shape(Hq=3, Hkv=2))) == 0
    assert lib.mxfa_bwd_one_launch(None) == 0
    # more (batch, head, 128-row block) flags than one slot holds: two launches
    assert lib.mxfa_bwd_one_launch(ctypes.byref(_shape(B=64, Hq=64, Hkv=64, N=8192))) == 1  # 2^18: fits
    assert lib.mxfa_bwd_one_launch(ctypes.byref(_shape(B=64, Hq=64, Hkv=64, N=8193))) == 0
    mx.set_bwd_options(one_launch=False)
    assert lib.mxfa_bwd_one_launch(ctypes.byref(_shape(B=4, Hq=12, Hkv=12, N=4096))) == 0


def test_workspace_checks(lib):
    sh = _shape(B=2, Hq=14, Hkv=2, N=4096, d=64)
    need = lib.mxfa_bwd_workspace_bytes(ctypes.byref(sh))
    p = ctypes.c_void_p(4096)
    bad = ctypes.c_void_p(4096 + 4)
    assert lib.mxfa_run_bwd_ws(ctypes.byref(sh), p, p, p, p, p, p, p, p, p, p, p, need - 1, None) == \
        mx_status("MXFA_ERR_WORKSPACE")
    assert lib.mxfa_run_bwd_dkv_ws(ctypes.byref(sh), p, p, p, p, p, p, p, p, p, need - 16, None) == \
        mx_status("MXFA_ERR_WORKSPACE")
    assert lib.mxfa_run_bwd_dkv_ws(ctypes.byref(sh), p, p, p, p, p, p, p, p, bad, need, None) == \
        mx_status("MXFA_ERR_ALIGN")
    assert lib.mxfa_run_bwd_ws(ctypes.byref(sh), p, p, p, p, p, p, p, p, p, None, p, need, None) == \
        mx_status("MXFA_ERR_NULL")


def test_python_layer_rejects_host_tensors():
    import torch
    q = torch.zeros(1, 1, 16, 64)
    with pytest.raises(ValueError, match="device tensor"):
        mx.run_flash(q, q, q, torch.zeros_like(q), causal=False)
    with pytest.raises(ValueError):
        mx.shape_of(torch.zeros(16, 64, dtype=torch.float16), torch.zeros(16, 64, dtype=torch.float16), False)


def _prefill(**kw):
    base = dict(n_tok=100, n_head=14, n_kv_head=2, head_dim=64, pos0=37, q_stride=18 * 64, kv_stride=2 * 64,
                out_stride=14 * 64, dtype=mx.MXFA_BF16, scale=0.0)
    base.update(kw)
    return mx.MxfaPrefillShape(**base)


@pytest.mark.parametrize("kw,code", [
    (dict(), 0),
    (dict(dtype=mx.MXFA_F32), 0),
    (dict(dtype=3), -3),
    (dict(n_tok=0), -2),
    (dict(pos0=-1), -2),
    (dict(n_head=13), -2),
    (dict(q_stride=14 * 64 - 8), -2),
    (dict(kv_stride=64), -2),
    (dict(out_stride=100), -2),
    (dict(q_stride=18 * 64 + 4), -5),      # bf16 row of 2312 bytes: not a multiple of 16
    (dict(q_stride=18 * 64 + 8), 0),       # 2320 bytes: fine
    (dict(out_stride=14 * 64 + 2, dtype=mx.MXFA_F32), -5),
    (dict(head_dim=96), -4),
    (dict(head_dim=128, dtype=mx.MXFA_F32, q_stride=18 * 128, kv_stride=256, out_stride=14 * 128), -4),
    (dict(head_dim=128, q_stride=18 * 128, kv_stride=256, out_stride=14 * 128), 0),
    (dict(scale=float("nan")), -2),
    # the query blocks of the smallest prefill work-group (64 rows: fp32,
    # paged d = 128, the split kernels) must fit grid.y (65535)
    (dict(n_tok=64 * 65535, dtype=mx.MXFA_F32), 0),
    (dict(n_tok=64 * 65535 + 1, dtype=mx.MXFA_F32), -2),
    (dict(n_tok=64 * 65535 + 1, head_dim=128, q_stride=18 * 128, kv_stride=256, out_stride=14 * 128), -2),
    (dict(n_tok=128 * 65535), -2),
])
def test_check_prefill(lib, kw, code):
    assert lib.mxfa_check_prefill(ctypes.byref(_prefill(**kw))) == code


def test_prefill_null_and_alignment(lib):
    sh = _prefill()
    ok, bad = ctypes.c_void_p(4096), ctypes.c_void_p(4096 + 4)
    assert lib.mxfa_check_prefill(None) == -1
    assert lib.mxfa_run_prefill(ctypes.byref(sh), ok, None, ok, ok, None) == -1
    assert lib.mxfa_run_prefill(ctypes.byref(sh), ok, ok, bad, ok, None) == -5


@pytest.mark.parametrize("block_size,code", [(0, -4), (-16, -4), (24, -4), (1 << 25, -4)])
def test_prefill_paged_block_sizes(lib, block_size, code):
    """Block sizes are powers of two up to 2^24; others are refused before any launch."""
    ok = ctypes.c_void_p(4096)
    assert lib.mxfa_run_prefill_paged(ctypes.byref(_prefill()), ok, ok, ok, ok, ok, block_size, None) == code


def test_prefill_paged_null_and_alignment(lib):
    sh = _prefill()
    ok, bad = ctypes.c_void_p(4096), ctypes.c_void_p(4096 + 4)
    assert lib.mxfa_run_prefill_paged(ctypes.byref(sh), ok, ok, ok, ok, None, 16, None) == -1
    assert lib.mxfa_run_prefill_paged(ctypes.byref(sh), ok, ok, ok, ok, ctypes.c_void_p(4096 + 2), 16, None) == -5
    assert lib.mxfa_run_prefill_paged(ctypes.byref(sh), ok, ok, bad, ok, ok, 16, None) == -5
    assert lib.mxfa_run_prefill_paged(ctypes.byref(_prefill(head_dim=96)), ok, ok, ok, ok, ok, 16, None) == -4


@pytest.mark.parametrize("kw,splits", [
    (dict(n_tok=512, pos0=3584), 7),               # Qwen2.5 chunk after history: 112 work-groups, 64 stages
    (dict(n_tok=1, pos0=1777), 14),                # one row: 28 stages, at least 2 a split
    (dict(n_tok=1, pos0=777), 1),                  # 13 stages: too few for bf16 ...
    (dict(n_tok=1, pos0=777, dtype=mx.MXFA_F32), 6),  # ... not for fp32
    (dict(n_tok=512, pos0=0), 1),                  # 8 stages
    (dict(n_tok=1, pos0=0), 1),                    # one stage: no split
    (dict(n_tok=4096, pos0=0), 1),                 # 896 work-groups fill the GPU
    (dict(n_tok=960, pos0=100, n_head=1, n_kv_head=1, q_stride=3 * 64, kv_stride=64, out_stride=64), 8),
    (dict(n_tok=100, pos0=100000, n_head=1, n_kv_head=1, q_stride=3 * 64, kv_stride=64, out_stride=64), 32),
])
def test_prefill_split_workspace(lib, kw, splits):
    """The split prefill's workspace: splits x rows x (head_dim + 2) fp32, 0 when no split pays."""
    sh = _prefill(**kw)
    want = 0 if splits == 1 else splits * sh.n_head * sh.n_tok * (sh.head_dim + 2) * 4
    assert lib.mxfa_prefill_workspace_bytes(ctypes.byref(sh)) == want
    assert lib.mxfa_prefill_workspace_bytes(ctypes.byref(_prefill(n_tok=0))) == 0


def test_prefill_position_limit(lib):
    """Query positions stay inside int: pos0 plus the rows (a single row's GQA heads included)."""
    top = 2 ** 31 - 1 - 128
    assert lib.mxfa_check_prefill(ctypes.byref(_prefill(n_tok=1, pos0=top - 14))) == 0
    assert lib.mxfa_check_prefill(ctypes.byref(_prefill(n_tok=1, pos0=top - 13))) == -2
    assert lib.mxfa_check_prefill(ctypes.byref(_prefill(n_tok=100, pos0=top - 100))) == 0
    assert lib.mxfa_check_prefill(ctypes.byref(_prefill(n_tok=100, pos0=top - 99))) == -2


def test_prefill_split_argument_checks(lib):
    """A split shape needs an aligned workspace of the reported size; checked before any launch."""
    sh = _prefill(n_tok=512, pos0=3584)
    need = lib.mxfa_prefill_workspace_bytes(ctypes.byref(sh))
    ok = ctypes.c_void_p(4096)
    assert lib.mxfa_run_prefill_ws(ctypes.byref(sh), ok, ok, ok, ok, None, need, None) == -1
    assert lib.mxfa_run_prefill_ws(ctypes.byref(sh), ok, ok, ok, ok, ctypes.c_void_p(4104), need, None) == -5
    assert lib.mxfa_run_prefill_ws(ctypes.byref(sh), ok, ok, ok, ok, ok, need - 4, None) == -8
    assert lib.mxfa_run_prefill_ws(ctypes.byref(_prefill(head_dim=96)), ok, ok, ok, ok, ok, need, None) == -4
    # paged: the paged checks first, then the workspace's
    assert lib.mxfa_run_prefill_paged_ws(ctypes.byref(sh), ok, ok, ok, ok, None, 16, ok, need, None) == -1
    assert lib.mxfa_run_prefill_paged_ws(ctypes.byref(sh), ok, ok, ok, ok, ok, 24, ok, need, None) == -4
    assert lib.mxfa_run_prefill_paged_ws(ctypes.byref(sh), ok, ok, ok, ok, ok, 16, None, need, None) == -1
    assert lib.mxfa_run_prefill_paged_ws(ctypes.byref(sh), ok, ok, ok, ok, ok, 16, ok, need - 4, None) == -8


def test_probe_argument_checks(lib):
    """The probes validate before launching (no device needed for these)."""
    import ctypes
    flops = ctypes.c_double(0.0)
    fake = ctypes.c_void_p(4096)  # aligned, never dereferenced on the host
    assert lib.mxfa_probe_sink_len() == 2048 * 256
    assert lib.mxfa_probe_mfma(7, 16, fake, ctypes.byref(flops), None) == mx_status("MXFA_ERR_DTYPE")
    assert lib.mxfa_probe_mfma(1, 0, fake, ctypes.byref(flops), None) == mx_status("MXFA_ERR_SHAPE")
    assert lib.mxfa_probe_mfma(1, 16, None, ctypes.byref(flops), None) == mx_status("MXFA_ERR_NULL")
    assert lib.mxfa_probe_mfma(1, 16, ctypes.c_void_p(4100), ctypes.byref(flops), None) == mx_status("MXFA_ERR_ALIGN")
    assert lib.mxfa_probe_read(fake, 24, fake, None) == mx_status("MXFA_ERR_SHAPE")
    assert lib.mxfa_probe_read(None, 32, fake, None) == mx_status("MXFA_ERR_NULL")
    assert lib.mxfa_probe_copy(fake, fake, 0, None) == mx_status("MXFA_ERR_SHAPE")
    assert lib.mxfa_probe_copy(fake, ctypes.c_void_p(4104), 32, None) == mx_status("MXFA_ERR_ALIGN")
    nb = ctypes.c_double(0.0)
    assert lib.mxfa_probe_dq_atomic(None, 1, 128, 1, ctypes.byref(nb), None) == mx_status("MXFA_ERR_NULL")
    assert lib.mxfa_probe_dq_atomic(fake, 1, 192, 1, ctypes.byref(nb), None) == mx_status("MXFA_ERR_SHAPE")
    assert lib.mxfa_probe_dq_atomic(fake, 0, 128, 1, ctypes.byref(nb), None) == mx_status("MXFA_ERR_SHAPE")
    assert lib.mxfa_probe_dq_atomic(fake, 1, 128, 2, ctypes.byref(nb), None) == mx_status("MXFA_ERR_SHAPE")


def mx_status(name: str) -> int:
    return {v: k for k, v in mx.STATUS.items()}[name]


def test_autograd_wrapper_rejects_host_tensors():
    """The training-step wrapper has no CPU path either."""
    import torch
    from mx230_amd.autograd import CausalSelfAttention, flash_attention
    q = torch.zeros(1, 2, 16, 64, requires_grad=True)
    with pytest.raises(ValueError, match="device tensor"):
        flash_attention(q, q, q, causal=True)
    blk = CausalSelfAttention(128, n_heads=2, n_kv_heads=1)
    with pytest.raises(ValueError, match="device tensor"):
        blk(torch.zeros(1, 16, 128))
    with pytest.raises(ValueError, match="multiple"):
        CausalSelfAttention(128, n_heads=3, n_kv_heads=2)


def test_product_never_touches_the_oracle():
    """The checker (oracle/) is test infrastructure: the package must not
    import, load or call it."""
    pkg = os.path.join(ROOT, "mx230_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".h", "Makefile")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.lower(), os.path.join(dirpath, f)


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(ImportError, match="no fallback"):
        mx.load_library(str(tmp_path / "libmxfa.so"))


# ------------------------------------------------------------- code object --

def _patched(tmp_path, name, offset, data):
    b = bytearray(open(mx.CODE_OBJECT_PATH, "rb").read())
    b[offset:offset + len(data)] = data
    p = tmp_path / name
    p.write_bytes(bytes(b))
    return str(p)


def test_code_object_host_check(lib, tmp_path):
    """mxfa_check_code_object, the counterpart of load_ptx's empty-stub guard
    (common/src/lib.rs:11-18): the built code object passes; a missing file,
    an empty one, non-ELF bytes, another machine, another OS/ABI and another
    processor are MXFA_ERR_CODE_OBJECT, all without a device."""
    bad = mx_status("MXFA_ERR_CODE_OBJECT")
    assert mx.check_code_object() == 0
    assert mx.check_code_object(mx.CODE_OBJECT_PATH) == 0
    assert mx.check_code_object(str(tmp_path / "missing.hsaco")) == bad
    (tmp_path / "empty.hsaco").write_bytes(b"")
    assert mx.check_code_object(str(tmp_path / "empty.hsaco")) == bad
    assert mx.check_code_object(mx.LIB_PATH) == bad  # an x86-64 ELF
    assert mx.check_code_object(_patched(tmp_path, "magic.hsaco", 0, b"\x7fELG")) == bad
    assert mx.check_code_object(_patched(tmp_path, "machine.hsaco", 18, b"\x3e\x00")) == bad
    assert mx.check_code_object(_patched(tmp_path, "osabi.hsaco", 7, b"\x00")) == bad
    assert mx.check_code_object(_patched(tmp_path, "gfx942.hsaco", 48, b"\x4c")) == bad
    assert mx.check_code_object(_patched(tmp_path, "same.hsaco", 48, b"\x4f")) == 0


def test_code_object_has_every_kernel():
    """Every kernel fa_kernels.h names is a global function of the code object,
    and the counters the library reads by name are there."""
    readelf = "/opt/rocm/llvm/bin/llvm-readelf"
    if not os.path.exists(readelf):
        pytest.skip("llvm-readelf is not installed")
    text = open(os.path.join(ROOT, "mx230_amd", "csrc", "fa_kernels.h")).read()
    names = set(re.findall(r"X\((mxfa_\w+)\)", text))
    assert len(names) > 40
    out = subprocess.run([readelf, "-s", "--wide", mx.CODE_OBJECT_PATH], capture_output=True, text=True,
                         check=True).stdout
    funcs = set(re.findall(r"FUNC\s+GLOBAL\s+\w+\s+\d+\s+(mxfa_\w+)", out))
    objects = set(re.findall(r"OBJECT\s+GLOBAL\s+\w+\s+\d+\s+(mxfa_\w+)", out))
    assert names <= funcs, sorted(names - funcs)
    assert {"mxfa_delta_fallbacks", "mxfa_reduce_timeouts"} <= objects


def _vgpr_range(op: str):
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", op) or re.fullmatch(r"v(\d+)", op)
    if not m:
        return None
    lo = int(m.group(1))
    return lo, int(m.group(m.lastindex))


@pytest.mark.parametrize("which", ["CODE_OBJECT_PATH", "TIMELINE_CODE_OBJECT_PATH"])
def test_code_object_store_data_hazard(which):
    """No store of more than 64 bits has its data registers overwritten by a
    VALU instruction within the two wait states gfx950 requires. The compiler
    pads its own stores; a store it cannot see (inline asm) gets no padding,
    which is how a build with the dK/dV accumulators in AGPRs came to write
    wrong partial sums."""
    objdump = "/opt/rocm/llvm/bin/llvm-objdump"
    path = getattr(mx, which)
    if not os.path.exists(objdump) or not os.path.exists(path):
        pytest.skip("llvm-objdump or the code object is missing")
    lines = subprocess.run([objdump, "-d", "--mcpu=gfx950", path], capture_output=True, text=True,
                           check=True).stdout.splitlines()
    insts = [ln.split("//")[0].strip() for ln in lines if ln.startswith("\t")]
    store = re.compile(r"^(global|buffer|flat|scratch)_store_dwordx[34]\s")
    stores = bad = 0
    for i, ins in enumerate(insts):
        if not store.match(ins):
            continue
        ops = [o.strip() for o in ins.split(None, 1)[1].split(",")]
        data = _vgpr_range(ops[0] if ins.startswith("buffer") else ops[1])
        if data is None:  # data in AGPRs
            continue
        stores += 1
        waits = 0
        for nxt in insts[i + 1:i + 3]:
            if waits >= 2:
                break
            if nxt.startswith("s_nop"):
                waits += int(nxt.split()[1], 0) + 1
                continue
            if nxt.startswith("v_"):
                dst = _vgpr_range(nxt.split(None, 1)[1].split(",")[0].strip()) if " " in nxt else None
                if dst and dst[0] <= data[1] and data[0] <= dst[1]:
                    bad += 1
                    break
            waits += 1
    assert stores > 100
    assert bad == 0


def _sgprs(op: str):
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", op) or re.fullmatch(r"s(\d+)", op)
    return set(range(int(m.group(1)), int(m.group(m.lastindex)) + 1)) if m else set()


@pytest.mark.parametrize("which", ["CODE_OBJECT_PATH", "TIMELINE_CODE_OBJECT_PATH"])
def test_code_object_sgpr_vmem_hazard(which):
    """No vector-memory instruction reads an SGPR (its saddr or resource) that a
    VALU instruction wrote within the five wait states gfx950 requires: the
    staging loads with a scalar base are inline asm, which the compiler does
    not pad."""
    objdump = "/opt/rocm/llvm/bin/llvm-objdump"
    path = getattr(mx, which)
    if not os.path.exists(objdump) or not os.path.exists(path):
        pytest.skip("llvm-objdump or the code object is missing")
    lines = subprocess.run([objdump, "-d", "--mcpu=gfx950", path], capture_output=True, text=True,
                           check=True).stdout.splitlines()
    insts = [ln.split("//")[0].strip() for ln in lines if ln.startswith("\t")]
    vmem = re.compile(r"^(global|buffer|scratch)_(load|store)")
    checked = bad = 0
    for i, ins in enumerate(insts):
        if not vmem.match(ins) or " " not in ins:
            continue
        used = set()
        for op in ins.split(None, 1)[1].split(","):
            used |= _sgprs(op.strip())
        if not used:
            continue
        checked += 1
        waits = 0
        for prev in reversed(insts[max(0, i - 5):i]):
            if waits >= 5:
                break
            if prev.startswith("v_") and " " in prev and _sgprs(prev.split(None, 1)[1].split(",")[0].strip()) & used:
                bad += 1
                break
            waits += int(prev.split()[1], 0) + 1 if prev.startswith("s_nop") else 1
    assert checked > 500
    assert bad == 0


def test_library_has_no_kernels():
    """libmxfa.so holds no kernels (they live in the code object): its only
    device code is the scratch array of mxfa_run_bwd_noalloc."""
    out = subprocess.run(["nm", "-D", mx.LIB_PATH], capture_output=True, text=True, check=True).stdout
    assert "__hipRegisterFunction" not in out
    assert "__hipRegisterVar" in out and "hipModuleLoadData" in out


def test_noalloc_rejects_shapes_beyond_its_scratch(lib):
    """mxfa_run_bwd_noalloc: 65 MiB of scratch per device (64 MiB of planes
    and 1 MiB of share flags); a shape that needs more is MXFA_ERR_SCRATCH
    before any device work (fake pointers, no GPU)."""
    assert lib.mxfa_bwd_noalloc_scratch_bytes() == 65 << 20
    p = ctypes.c_void_p(4096)
    fits = _shape(B=1, Hq=32, Hkv=4, N=2048, d=128)  # cfg5 d = 128: 64 MiB of planes (8), 1024 flags
    assert lib.mxfa_bwd_workspace_bytes(ctypes.byref(fits)) == (64 << 20) + 8 * 1024
    big = _shape(B=1, Hq=64, Hkv=4, N=8192, d=64)  # 8 planes of 4 x 8192 rows: 128 MiB, 2048 flags
    assert lib.mxfa_bwd_workspace_bytes(ctypes.byref(big)) == 2 * 8 * 4 * 8192 * 64 * 4 + 8 * 2048
    assert lib.mxfa_run_bwd_noalloc(ctypes.byref(big), p, p, p, p, p, p, p, p, p, p, None) == \
        mx_status("MXFA_ERR_SCRATCH")
    assert lib.mxfa_run_bwd_noalloc(ctypes.byref(big), p, p, p, p, p, p, p, p, p, None, None) == \
        mx_status("MXFA_ERR_NULL")


def test_time_median_ms_needs_an_iteration():
    """mx.time_median_ms rejects iters < 1 before touching a device."""
    with pytest.raises(ValueError):
        mx.time_median_ms(lambda: None, warmup=0, iters=0)


def test_integration_rust_block_binds_every_entry_point():
    """INTEGRATION.md's Rust extern block declares every function of
    include/mxfa.h (a maintainer copying it gets the whole binding)."""
    import re
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    with open(os.path.join(root, "include", "mxfa.h")) as f:
        header = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
    names = set(re.findall(r"\b(mxfa_\w+)\s*\(", header))
    with open(os.path.join(root, "INTEGRATION.md")) as f:
        doc = f.read()
    block = doc[doc.index("// 02-flash-attention/src/mxfa.rs"):]
    block = block[:block.index("```")]
    bound = set(re.findall(r"pub fn (mxfa_\w+)\(", block))
    assert names, "no declarations parsed"
    assert names == bound, (sorted(names - bound), sorted(bound - names))


def test_prepare_checks_arguments_once_and_rejects_other_functions():
    """mx.prepare runs the wrapper's argument checks at preparation (a host
    tensor is refused there, before any launch) and covers exactly the
    launch wrappers it names."""
    import torch
    q = torch.zeros(1, 2, 16, 64, dtype=torch.bfloat16)
    lse = torch.zeros(1, 2, 16)
    with pytest.raises(ValueError, match="device tensor"):
        mx.prepare(mx.run_flash_lse, q, q, q, q, lse, True)
    with pytest.raises(ValueError, match="not a preparable"):
        mx.prepare(mx.time_median_ms, lambda: None)
    names = sorted(f.__name__ for f in mx._MARSHAL)
    assert names == sorted(["run_flash", "run_flash_lse", "run_preprocess", "run_bwd", "run_bwd_ws",
                            "run_bwd_noalloc", "run_bwd_flash", "run_bwd_dq", "run_bwd_dq_delta",
                            "run_bwd_dkv", "run_bwd_dkv_ws", "run_bwd_naive"])


def test_bench_refuses_several_gpus():
    """bench.py --gpus N > 1 exits with status 2 and says why, before touching a
    device (this build runs on one GPU; the path shards with no exchange)."""
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=root)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""
