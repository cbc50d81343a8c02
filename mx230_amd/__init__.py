"""MI355X-native flash-attention training path (forward O + LSE, FA-2 backward).

The compute lives in ``libmxfa.so`` (HIP kernels for gfx950 behind the C ABI of
``include/mxfa.h``, built from ``mx230_amd/csrc``). This module is the host-side
mirror of the reference crate's Rust wrappers
(02-flash-attention/src/main.rs:32-210): the same entry points, the same argument
meaning (caller-owned device buffers, ``n`` implied by the shapes, ``causal``
flag), the same ownership (the caller allocates O, LSE, Delta, dQ, dK, dV) and the
same "wrappers only enqueue work" contract. Where the reference panics on a
launch failure, these raise :class:`MxfaError`.

PyTorch is only plumbing here: tensors provide device memory and the current
stream. There is no CPU or PyTorch fallback: if ``libmxfa.so`` is missing or the
tensors are not on a GPU, every call raises.

Tensor layouts (contiguous): Q, O, dO, dQ ``[B, Hq, N, d]``; K, V, dK, dV
``[B, Hkv, N, d]``; LSE, Delta ``[B, Hq, N]`` float32. A 2-D ``[N, d]`` tensor is
read as B = H = 1, i.e. the reference's single-head layout.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmxfa.so")
# the kernels: one gfx950 code object the library loads per device
CODE_OBJECT_PATH = os.path.join(_HERE, "mxfa_gfx950.hsaco")
# the same kernels with per-work-group timestamps in the backward bodies
# (make -C mx230_amd/csrc timeline; read with probe_wg_times)
TIMELINE_CODE_OBJECT_PATH = os.path.join(_HERE, "mxfa_gfx950_timeline.hsaco")

MXFA_F32, MXFA_BF16 = 0, 1

STATUS = {
    0: "MXFA_OK",
    -1: "MXFA_ERR_NULL",
    -2: "MXFA_ERR_SHAPE",
    -3: "MXFA_ERR_DTYPE",
    -4: "MXFA_ERR_UNSUPPORTED",
    -5: "MXFA_ERR_ALIGN",
    -6: "MXFA_ERR_LAUNCH",
    -7: "MXFA_ERR_DEVICE",
    -8: "MXFA_ERR_WORKSPACE",
    -9: "MXFA_ERR_CODE_OBJECT",
    -10: "MXFA_ERR_SCRATCH",
}

# Every symbol include/mxfa.h declares (the tests check the library exports them).
EXPORTS = (
    "mxfa_version", "mxfa_strerror", "mxfa_init", "mxfa_shutdown", "mxfa_set_code_object",
    "mxfa_check_code_object", "mxfa_check_shape",
    "mxfa_run_flash", "mxfa_run_flash_lse", "mxfa_run_preprocess", "mxfa_run_bwd_dq",
    "mxfa_run_bwd_dkv", "mxfa_run_bwd_flash", "mxfa_run_bwd_dq_delta", "mxfa_run_bwd", "mxfa_bwd_one_launch", "mxfa_bwd_workspace_bytes",
    "mxfa_run_bwd_dkv_ws", "mxfa_run_bwd_ws", "mxfa_run_bwd_naive",
    "mxfa_naive_scratch_bytes", "mxfa_run_naive_fwd", "mxfa_check_prefill", "mxfa_run_prefill",
    "mxfa_run_prefill_paged", "mxfa_prefill_workspace_bytes", "mxfa_run_prefill_ws", "mxfa_run_prefill_paged_ws",
    "mxfa_set_bwd_options", "mxfa_get_bwd_options", "mxfa_bwd_delta_fallbacks", "mxfa_bwd_reduce_timeouts",
    "mxfa_run_bwd_noalloc", "mxfa_bwd_noalloc_scratch_bytes",
)
# Every symbol include/mxfa_probes.h declares.
PROBE_EXPORTS = (
    "mxfa_probe_sink_len", "mxfa_probe_mfma", "mxfa_probe_mfma32", "mxfa_probe_mix", "mxfa_probe_read",
    "mxfa_probe_copy", "mxfa_probe_dq_atomic", "mxfa_probe_wg_times",
)


class MxfaError(RuntimeError):
    """A non-zero status from libmxfa."""

    def __init__(self, func: str, status: int, text: str):
        super().__init__(f"{func}: {STATUS.get(status, status)} ({text})")
        self.status = status


class MxfaShape(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int), ("Hq", ctypes.c_int), ("Hkv", ctypes.c_int), ("N", ctypes.c_int),
                ("d", ctypes.c_int), ("causal", ctypes.c_int), ("dtype", ctypes.c_int),
                ("scale", ctypes.c_float)]


class MxfaBwdOptions(ctypes.Structure):
    _fields_ = [("one_launch", ctypes.c_int), ("delta_wait_us", ctypes.c_int), ("reduce_wait_us", ctypes.c_int)]


class MxfaPrefillShape(ctypes.Structure):
    _fields_ = [("n_tok", ctypes.c_int), ("n_head", ctypes.c_int), ("n_kv_head", ctypes.c_int),
                ("head_dim", ctypes.c_int), ("pos0", ctypes.c_int), ("q_stride", ctypes.c_int),
                ("kv_stride", ctypes.c_int), ("out_stride", ctypes.c_int), ("dtype", ctypes.c_int),
                ("scale", ctypes.c_float)]


_lib = None


def load_library(path: str | None = None):
    """Loads libmxfa.so (raises if it has not been built)."""
    global _lib
    if path is None and _lib is not None:
        return _lib
    p = path or LIB_PATH
    # torch first: libmxfa then binds to the HIP runtime torch already loaded, so
    # the device pointers and streams it receives from torch are valid for it
    # (loading libmxfa first would pull in a second HIP runtime)
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    if not os.path.exists(p):
        raise ImportError(f"{p} is missing: build it with `make -C mx230_amd/csrc` "
                          "(or __graft_entry__.build()); there is no fallback path")
    if path is None and not os.path.exists(CODE_OBJECT_PATH):
        raise ImportError(f"{CODE_OBJECT_PATH} (the kernels) is missing: build it with "
                          "`make -C mx230_amd/csrc`; there is no fallback path")
    lib = ctypes.CDLL(p)
    vp, sp, fp = ctypes.c_void_p, ctypes.POINTER(MxfaShape), ctypes.c_void_p
    lib.mxfa_version.restype = ctypes.c_int
    lib.mxfa_strerror.restype = ctypes.c_char_p
    lib.mxfa_strerror.argtypes = [ctypes.c_int]
    lib.mxfa_init.argtypes = [ctypes.c_int]
    lib.mxfa_set_code_object.argtypes = [ctypes.c_char_p]
    lib.mxfa_check_code_object.argtypes = [ctypes.c_char_p]
    lib.mxfa_check_shape.argtypes = [sp]
    lib.mxfa_run_flash.argtypes = [sp, vp, vp, vp, vp, vp]
    lib.mxfa_run_flash_lse.argtypes = [sp, vp, vp, vp, vp, fp, vp]
    lib.mxfa_run_preprocess.argtypes = [sp, vp, vp, fp, vp]
    lib.mxfa_run_bwd_dq.argtypes = [sp, vp, vp, vp, vp, fp, fp, vp, vp]
    lib.mxfa_run_bwd_dkv.argtypes = [sp, vp, vp, vp, vp, fp, fp, vp, vp, vp]
    lib.mxfa_run_bwd_flash.argtypes = [sp, vp, vp, vp, vp, fp, fp, vp, vp, vp, vp]
    lib.mxfa_run_bwd.argtypes = [sp, vp, vp, vp, vp, vp, fp, fp, vp, vp, vp, vp]
    lib.mxfa_run_bwd_dq_delta.argtypes = [sp, vp, vp, vp, vp, vp, fp, fp, vp, vp]
    lib.mxfa_run_bwd_naive.argtypes = [sp, vp, vp, vp, vp, fp, fp, vp, vp, vp, vp]
    lib.mxfa_bwd_one_launch.argtypes = [sp]
    lib.mxfa_bwd_workspace_bytes.argtypes = [sp]
    lib.mxfa_bwd_workspace_bytes.restype = ctypes.c_size_t
    lib.mxfa_run_bwd_dkv_ws.argtypes = [sp, vp, vp, vp, vp, fp, fp, vp, vp, vp, ctypes.c_size_t, vp]
    lib.mxfa_run_bwd_ws.argtypes = [sp, vp, vp, vp, vp, vp, fp, fp, vp, vp, vp, vp, ctypes.c_size_t, vp]
    lib.mxfa_run_bwd_noalloc.argtypes = [sp, vp, vp, vp, vp, vp, fp, fp, vp, vp, vp, vp]
    lib.mxfa_bwd_noalloc_scratch_bytes.argtypes = []
    lib.mxfa_bwd_noalloc_scratch_bytes.restype = ctypes.c_size_t
    lib.mxfa_naive_scratch_bytes.argtypes = [sp]
    lib.mxfa_naive_scratch_bytes.restype = ctypes.c_size_t
    lib.mxfa_run_naive_fwd.argtypes = [sp, vp, vp, vp, fp, vp, vp]
    pp = ctypes.POINTER(MxfaPrefillShape)
    lib.mxfa_check_prefill.argtypes = [pp]
    lib.mxfa_run_prefill.argtypes = [pp, vp, vp, vp, vp, vp]
    lib.mxfa_run_prefill_paged.argtypes = [pp, vp, vp, vp, vp, vp, ctypes.c_int, vp]
    lib.mxfa_prefill_workspace_bytes.argtypes = [pp]
    lib.mxfa_prefill_workspace_bytes.restype = ctypes.c_size_t
    lib.mxfa_run_prefill_ws.argtypes = [pp, vp, vp, vp, vp, vp, ctypes.c_size_t, vp]
    lib.mxfa_run_prefill_paged_ws.argtypes = [pp, vp, vp, vp, vp, vp, ctypes.c_int, vp, ctypes.c_size_t, vp]
    lib.mxfa_probe_sink_len.argtypes = []
    lib.mxfa_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, fp, ctypes.POINTER(ctypes.c_double), vp]
    lib.mxfa_probe_mfma32.argtypes = [ctypes.c_int, fp, ctypes.POINTER(ctypes.c_double), vp]
    lib.mxfa_probe_mix.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, fp, ctypes.POINTER(ctypes.c_double), vp]
    lib.mxfa_probe_wg_times.argtypes = [vp, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
    lib.mxfa_probe_read.argtypes = [vp, ctypes.c_size_t, fp, vp]
    lib.mxfa_probe_copy.argtypes = [vp, vp, ctypes.c_size_t, vp]
    lib.mxfa_probe_dq_atomic.argtypes = [fp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.POINTER(ctypes.c_double), vp]
    op = ctypes.POINTER(MxfaBwdOptions)
    lib.mxfa_set_bwd_options.argtypes = [op]
    lib.mxfa_get_bwd_options.argtypes = [op]
    lib.mxfa_bwd_delta_fallbacks.argtypes = [ctypes.POINTER(ctypes.c_ulonglong)]
    lib.mxfa_bwd_reduce_timeouts.argtypes = [ctypes.POINTER(ctypes.c_ulonglong)]
    for name in EXPORTS + PROBE_EXPORTS:
        if name not in ("mxfa_version", "mxfa_strerror", "mxfa_bwd_workspace_bytes",
                        "mxfa_naive_scratch_bytes", "mxfa_bwd_noalloc_scratch_bytes",
                        "mxfa_prefill_workspace_bytes"):
            getattr(lib, name).restype = ctypes.c_int
    if path is None:
        _lib = lib
    return lib


def _check(func: str, rc: int):
    if rc != 0:
        raise MxfaError(func, rc, load_library().mxfa_strerror(rc).decode())


def _invoke(func: str, args):
    _check(func, getattr(load_library(), func)(*args))


@dataclass(frozen=True)
class Shape:
    B: int
    Hq: int
    Hkv: int
    N: int
    d: int
    causal: bool
    bf16: bool
    scale: float = 0.0

    def c(self) -> MxfaShape:
        return MxfaShape(self.B, self.Hq, self.Hkv, self.N, self.d, int(self.causal),
                         MXFA_BF16 if self.bf16 else MXFA_F32, self.scale)


# --------------------------------------------------------------- torch glue --

def _torch():
    import torch
    return torch


def _dims(t, name):
    if t.dim() == 2:
        return 1, 1, t.shape[0], t.shape[1]
    if t.dim() == 4:
        return tuple(t.shape)
    raise ValueError(f"{name}: expected [N, d] or [B, H, N, d], got {tuple(t.shape)}")


def _ptr(t, name, dtype):
    torch = _torch()
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be a device tensor (got {t.device}); there is no CPU path")
    if t.dtype != dtype:
        raise ValueError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def shape_of(q, k, causal: bool, scale: float = 0.0) -> Shape:
    """Shape of an attention call from Q [B,Hq,N,d] and K [B,Hkv,N,d]."""
    torch = _torch()
    B, Hq, N, d = _dims(q, "q")
    Bk, Hkv, Nk, dk = _dims(k, "k")
    if (Bk, Nk, dk) != (B, N, d):
        raise ValueError(f"q {tuple(q.shape)} and k {tuple(k.shape)} disagree")
    if q.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"dtype {q.dtype} not supported (float32 or bfloat16)")
    return Shape(B, Hq, Hkv, N, d, bool(causal), q.dtype == torch.bfloat16, float(scale))


def _expect(t, name, shape4, dtype):
    dims = _dims(t, name)
    if tuple(dims) != tuple(shape4):
        raise ValueError(f"{name}: shape {tuple(t.shape)} does not match {tuple(shape4)}")
    return _ptr(t, name, dtype)


def _io(sh: Shape):
    torch = _torch()
    dt = torch.bfloat16 if sh.bf16 else torch.float32
    qs = (sh.B, sh.Hq, sh.N, sh.d)
    ks = (sh.B, sh.Hkv, sh.N, sh.d)
    return dt, qs, ks


def _vec_ptr(t, name, sh: Shape):
    torch = _torch()
    if t.numel() != sh.B * sh.Hq * sh.N:
        raise ValueError(f"{name}: expected {sh.B * sh.Hq * sh.N} elements, got {t.numel()}")
    return _ptr(t, name, torch.float32)


# ------------------------------------------- reference-shaped entry points --

def _call_flash(q, k, v, o, causal: bool, scale: float = 0.0, stream=None):
    sh = shape_of(q, k, causal, scale)
    dt, qs, ks = _io(sh)
    args = (_expect(q, "q", qs, dt), _expect(k, "k", ks, dt), _expect(v, "v", ks, dt),
            _expect(o, "o", qs, dt))
    return "mxfa_run_flash", (ctypes.byref(sh.c()), *args, _stream(stream))


def run_flash(q, k, v, o, causal: bool, scale: float = 0.0, stream=None):
    """Forward, O only (main.rs:68-88)."""
    _invoke(*_call_flash(q, k, v, o, causal, scale, stream))


def _call_flash_lse(q, k, v, o, lse, causal: bool, scale: float = 0.0, stream=None):
    sh = shape_of(q, k, causal, scale)
    dt, qs, ks = _io(sh)
    args = (_expect(q, "q", qs, dt), _expect(k, "k", ks, dt), _expect(v, "v", ks, dt),
            _expect(o, "o", qs, dt), _vec_ptr(lse, "lse", sh))
    return "mxfa_run_flash_lse", (ctypes.byref(sh.c()), *args, _stream(stream))


def run_flash_lse(q, k, v, o, lse, causal: bool, scale: float = 0.0, stream=None):
    """Forward with the log-sum-exp the backward needs (main.rs:102-123)."""
    _invoke(*_call_flash_lse(q, k, v, o, lse, causal, scale, stream))


def _call_preprocess(do, o, delta, stream=None):
    sh = shape_of(do, do, False)
    dt, qs, _ = _io(sh)
    args = (_expect(do, "do", qs, dt), _expect(o, "o", qs, dt), _vec_ptr(delta, "delta", sh))
    return "mxfa_run_preprocess", (ctypes.byref(sh.c()), *args, _stream(stream))


def run_preprocess(do, o, delta, stream=None):
    """Delta = rowsum(dO * O) (main.rs:126-143)."""
    _invoke(*_call_preprocess(do, o, delta, stream))


def _bwd_args(q, k, v, do, lse, delta, causal, scale):
    sh = shape_of(q, k, causal, scale)
    dt, qs, ks = _io(sh)
    args = [_expect(q, "q", qs, dt), _expect(k, "k", ks, dt), _expect(v, "v", ks, dt),
            _expect(do, "do", qs, dt), _vec_ptr(lse, "lse", sh), _vec_ptr(delta, "delta", sh)]
    return sh, dt, qs, ks, args


def _call_bwd_flash(q, k, v, do, lse, delta, dq, dk, dv, causal: bool, scale: float = 0.0,
                  stream=None):
    sh, dt, qs, ks, args = _bwd_args(q, k, v, do, lse, delta, causal, scale)
    args += [_expect(dq, "dq", qs, dt), _expect(dk, "dk", ks, dt), _expect(dv, "dv", ks, dt)]
    return "mxfa_run_bwd_flash", (ctypes.byref(sh.c()), *args, _stream(stream))


def run_bwd_flash(q, k, v, do, lse, delta, dq, dk, dv, causal: bool, scale: float = 0.0,
                  stream=None):
    """Tiled atomic-free backward: dK/dV pass then dQ pass (main.rs:179-210).
    Outputs are overwritten."""
    _invoke(*_call_bwd_flash(q, k, v, do, lse, delta, dq, dk, dv, causal, scale, stream))


def _call_bwd(q, k, v, o, do, lse, delta, dq, dk, dv, causal: bool, scale: float = 0.0, stream=None):
    sh = shape_of(q, k, causal, scale)
    dt, qs, ks = _io(sh)
    args = [_expect(q, "q", qs, dt), _expect(k, "k", ks, dt), _expect(v, "v", ks, dt), _expect(o, "o", qs, dt),
            _expect(do, "do", qs, dt), _vec_ptr(lse, "lse", sh), _vec_ptr(delta, "delta", sh),
            _expect(dq, "dq", qs, dt), _expect(dk, "dk", ks, dt), _expect(dv, "dv", ks, dt)]
    return "mxfa_run_bwd", (ctypes.byref(sh.c()), *args, _stream(stream))


def run_bwd(q, k, v, o, do, lse, delta, dq, dk, dv, causal: bool, scale: float = 0.0, stream=None):
    """The whole backward from O (mxfa_run_bwd): the dQ work computes
    Delta = rowsum(dO * O) itself and writes it to ``delta`` for the dK/dV
    work (run_preprocess + run_bwd_flash with the preprocess launch folded in);
    one launch for bf16 (bwd_one_launch), else two. Outputs are overwritten."""
    _invoke(*_call_bwd(q, k, v, o, do, lse, delta, dq, dk, dv, causal, scale, stream))


def bwd_one_launch(q, k, causal: bool) -> bool:
    """True if run_bwd runs the backward as one launch for this shape
    (mxfa_bwd_one_launch; set_bwd_options(one_launch=False) selects two
    launches)."""
    sh = shape_of(q, k, causal)
    return bool(load_library().mxfa_bwd_one_launch(ctypes.byref(sh.c())))


def get_bwd_options() -> dict:
    """The one-launch backward's process-wide settings (mxfa_get_bwd_options)."""
    o = MxfaBwdOptions()
    _check("mxfa_get_bwd_options", load_library().mxfa_get_bwd_options(ctypes.byref(o)))
    return {"one_launch": bool(o.one_launch), "delta_wait_us": o.delta_wait_us, "reduce_wait_us": o.reduce_wait_us}


def set_bwd_options(one_launch: bool | None = None, delta_wait_us: int | None = None,
                    reduce_wait_us: int | None = None) -> dict:
    """Changes the given settings (mxfa_set_bwd_options) and returns the
    previous ones. one_launch=False: always two launches; delta_wait_us < 0:
    the dK/dV work-groups never wait for Delta and compute it themselves;
    reduce_wait_us: the bound of a GQA split's reduce wait (>= 0)."""
    old = get_bwd_options()
    o = MxfaBwdOptions(int(old["one_launch"] if one_launch is None else one_launch),
                       old["delta_wait_us"] if delta_wait_us is None else int(delta_wait_us),
                       old["reduce_wait_us"] if reduce_wait_us is None else int(reduce_wait_us))
    _check("mxfa_set_bwd_options", load_library().mxfa_set_bwd_options(ctypes.byref(o)))
    return old


def bwd_delta_fallbacks() -> int:
    """Delta blocks the one-launch backward computed in its dK/dV work-groups
    on the current device since load (mxfa_bwd_delta_fallbacks; synchronise the
    launches of interest first)."""
    n = ctypes.c_ulonglong(0)
    _check("mxfa_bwd_delta_fallbacks", load_library().mxfa_bwd_delta_fallbacks(ctypes.byref(n)))
    return int(n.value)


def bwd_reduce_timeouts() -> int:
    """Work-groups of the one-launch backward that add a GQA split's partial
    sums and whose wait for them ran out (their dK/dV rows are NaN), on the
    current device since load (mxfa_bwd_reduce_timeouts; 0 in normal operation;
    synchronise the launches of interest first)."""
    n = ctypes.c_ulonglong(0)
    _check("mxfa_bwd_reduce_timeouts", load_library().mxfa_bwd_reduce_timeouts(ctypes.byref(n)))
    return int(n.value)


def bwd_workspace_bytes(q, k, causal: bool) -> int:
    """Bytes of workspace run_bwd_ws / run_bwd_dkv_ws can use for this shape
    (mxfa_bwd_workspace_bytes): nonzero only for GQA shapes whose dK/dV pass
    splits each group's query heads over several work-groups."""
    sh = shape_of(q, k, causal)
    return int(load_library().mxfa_bwd_workspace_bytes(ctypes.byref(sh.c())))


def _ws_args(workspace):
    if workspace is None:
        return [None, 0]
    torch = _torch()
    if workspace.device.type != "cuda" or not workspace.is_contiguous():
        raise ValueError("workspace: must be a contiguous device tensor")
    return [ctypes.c_void_p(workspace.data_ptr()), workspace.numel() * workspace.element_size()]


def _call_bwd_ws(q, k, v, o, do, lse, delta, dq, dk, dv, workspace, causal: bool, scale: float = 0.0,
               stream=None):
    sh = shape_of(q, k, causal, scale)
    dt, qs, ks = _io(sh)
    args = [_expect(q, "q", qs, dt), _expect(k, "k", ks, dt), _expect(v, "v", ks, dt), _expect(o, "o", qs, dt),
            _expect(do, "do", qs, dt), _vec_ptr(lse, "lse", sh), _vec_ptr(delta, "delta", sh),
            _expect(dq, "dq", qs, dt), _expect(dk, "dk", ks, dt), _expect(dv, "dv", ks, dt)]
    args += _ws_args(workspace)
    return "mxfa_run_bwd_ws", (ctypes.byref(sh.c()), *args, _stream(stream))


def run_bwd_ws(q, k, v, o, do, lse, delta, dq, dk, dv, workspace, causal: bool, scale: float = 0.0,
               stream=None):
    """run_bwd with a workspace (a device tensor of at least
    bwd_workspace_bytes(q, k, causal) bytes, or None) for the split dK/dV pass
    of GQA shapes (mxfa_run_bwd_ws)."""
    _invoke(*_call_bwd_ws(q, k, v, o, do, lse, delta, dq, dk, dv, workspace, causal, scale, stream))


def _call_bwd_noalloc(q, k, v, o, do, lse, delta, dq, dk, dv, causal: bool, scale: float = 0.0, stream=None):
    sh = shape_of(q, k, causal, scale)
    dt, qs, ks = _io(sh)
    args = [_expect(q, "q", qs, dt), _expect(k, "k", ks, dt), _expect(v, "v", ks, dt), _expect(o, "o", qs, dt),
            _expect(do, "do", qs, dt), _vec_ptr(lse, "lse", sh), _vec_ptr(delta, "delta", sh),
            _expect(dq, "dq", qs, dt), _expect(dk, "dk", ks, dt), _expect(dv, "dv", ks, dt)]
    return "mxfa_run_bwd_noalloc", (ctypes.byref(sh.c()), *args, _stream(stream))


def run_bwd_noalloc(q, k, v, o, do, lse, delta, dq, dk, dv, causal: bool, scale: float = 0.0, stream=None):
    """run_bwd_ws with the library's static scratch in place of a workspace
    (mxfa_run_bwd_noalloc): allocates nothing; calls overlapping on one device
    race on the scratch."""
    _invoke(*_call_bwd_noalloc(q, k, v, o, do, lse, delta, dq, dk, dv, causal, scale, stream))


def _call_bwd_dq_delta(q, k, v, o, do, lse, delta, dq, causal: bool, scale: float = 0.0, stream=None):
    sh = shape_of(q, k, causal, scale)
    dt, qs, ks = _io(sh)
    args = [_expect(q, "q", qs, dt), _expect(k, "k", ks, dt), _expect(v, "v", ks, dt), _expect(o, "o", qs, dt),
            _expect(do, "do", qs, dt), _vec_ptr(lse, "lse", sh), _vec_ptr(delta, "delta", sh),
            _expect(dq, "dq", qs, dt)]
    return "mxfa_run_bwd_dq_delta", (ctypes.byref(sh.c()), *args, _stream(stream))


def run_bwd_dq_delta(q, k, v, o, do, lse, delta, dq, causal: bool, scale: float = 0.0, stream=None):
    """dQ pass that computes Delta from O itself and writes it to ``delta``."""
    _invoke(*_call_bwd_dq_delta(q, k, v, o, do, lse, delta, dq, causal, scale, stream))


def _call_bwd_dq(q, k, v, do, lse, delta, dq, causal: bool, scale: float = 0.0, stream=None):
    sh, dt, qs, ks, args = _bwd_args(q, k, v, do, lse, delta, causal, scale)
    args += [_expect(dq, "dq", qs, dt)]
    return "mxfa_run_bwd_dq", (ctypes.byref(sh.c()), *args, _stream(stream))


def run_bwd_dq(q, k, v, do, lse, delta, dq, causal: bool, scale: float = 0.0, stream=None):
    """dQ pass alone (attention_bwd.cu:96-158)."""
    _invoke(*_call_bwd_dq(q, k, v, do, lse, delta, dq, causal, scale, stream))


def _call_bwd_dkv(q, k, v, do, lse, delta, dk, dv, causal: bool, scale: float = 0.0, stream=None):
    sh, dt, qs, ks, args = _bwd_args(q, k, v, do, lse, delta, causal, scale)
    args += [_expect(dk, "dk", ks, dt), _expect(dv, "dv", ks, dt)]
    return "mxfa_run_bwd_dkv", (ctypes.byref(sh.c()), *args, _stream(stream))


def run_bwd_dkv(q, k, v, do, lse, delta, dk, dv, causal: bool, scale: float = 0.0, stream=None):
    """dK/dV pass alone (attention_bwd.cu:165-243)."""
    _invoke(*_call_bwd_dkv(q, k, v, do, lse, delta, dk, dv, causal, scale, stream))


def _call_bwd_dkv_ws(q, k, v, do, lse, delta, dk, dv, workspace, causal: bool, scale: float = 0.0,
                   stream=None):
    sh, dt, qs, ks, args = _bwd_args(q, k, v, do, lse, delta, causal, scale)
    args += [_expect(dk, "dk", ks, dt), _expect(dv, "dv", ks, dt)] + _ws_args(workspace)
    return "mxfa_run_bwd_dkv_ws", (ctypes.byref(sh.c()), *args, _stream(stream))


def run_bwd_dkv_ws(q, k, v, do, lse, delta, dk, dv, workspace, causal: bool, scale: float = 0.0,
                   stream=None):
    """dK/dV pass with a workspace for the split GQA form (mxfa_run_bwd_dkv_ws)."""
    _invoke(*_call_bwd_dkv_ws(q, k, v, do, lse, delta, dk, dv, workspace, causal, scale, stream))


def _call_bwd_naive(q, k, v, do, lse, delta, dq, dk, dv, causal: bool, scale: float = 0.0,
                  stream=None):
    sh, dt, qs, ks, args = _bwd_args(q, k, v, do, lse, delta, causal, scale)
    args += [_expect(dq, "dq", qs, dt), _expect(dk, "dk", ks, dt), _expect(dv, "dv", ks, dt)]
    return "mxfa_run_bwd_naive", (ctypes.byref(sh.c()), *args, _stream(stream))


def run_bwd_naive(q, k, v, do, lse, delta, dq, dk, dv, causal: bool, scale: float = 0.0,
                  stream=None):
    """Naive atomic backward baseline, fp32; outputs must be zeroed (main.rs:147-173)."""
    _invoke(*_call_bwd_naive(q, k, v, do, lse, delta, dq, dk, dv, causal, scale, stream))


class Prepared:
    """One entry point with its arguments checked and marshalled once
    (prepare()): calling it enqueues the same launch again (the same tensors,
    shape, scale and stream) for the cost of one foreign call. It keeps the
    tensors referenced; they must keep their storage (no resize or
    reallocation) while it is in use, as their device addresses are fixed
    in it. The library validates the call again each time, as for any call."""
    __slots__ = ("func", "_fn", "_args", "_keep")

    def __init__(self, func: str, args, keep):
        self.func = func
        self._fn = getattr(load_library(), func)
        self._args = tuple(args)
        self._keep = keep

    def __call__(self):
        rc = self._fn(*self._args)
        if rc != 0:
            _check(self.func, rc)


def prepare(fn, *args, **kwargs) -> Prepared:
    """fn(*args, **kwargs) as a Prepared call, for one of run_flash,
    run_flash_lse, run_preprocess, run_bwd, run_bwd_ws, run_bwd_noalloc,
    run_bwd_flash, run_bwd_dq, run_bwd_dq_delta, run_bwd_dkv, run_bwd_dkv_ws
    and run_bwd_naive: the argument checks of fn run here, once (and raise
    here), so a loop of calls pays only the launch."""
    marshal = _MARSHAL.get(fn)
    if marshal is None:
        raise ValueError(f"prepare: {getattr(fn, '__name__', fn)!r} is not a preparable entry point")
    func, cargs = marshal(*args, **kwargs)
    return Prepared(func, cargs, (args, kwargs))


_MARSHAL = {run_flash: _call_flash, run_flash_lse: _call_flash_lse, run_preprocess: _call_preprocess,
            run_bwd: _call_bwd, run_bwd_ws: _call_bwd_ws, run_bwd_noalloc: _call_bwd_noalloc,
            run_bwd_flash: _call_bwd_flash, run_bwd_dq: _call_bwd_dq, run_bwd_dq_delta: _call_bwd_dq_delta,
            run_bwd_dkv: _call_bwd_dkv, run_bwd_dkv_ws: _call_bwd_dkv_ws, run_bwd_naive: _call_bwd_naive}


def naive_scratch_bytes(q, k, causal: bool) -> int:
    sh = shape_of(q, k, causal)
    return int(load_library().mxfa_naive_scratch_bytes(ctypes.byref(sh.c())))


def naive_run(q, k, v, s, o, causal: bool, scale: float = 0.0, stream=None):
    """Naive forward with the materialised N x N scores ``s`` (Naive::run, main.rs:32-66)."""
    torch = _torch()
    sh = shape_of(q, k, causal, scale)
    dt, qs, ks = _io(sh)
    if s.numel() * 4 < naive_scratch_bytes(q, k, causal):
        raise ValueError("s: scratch too small (needs B*Hq*N*N float32)")
    args = (_expect(q, "q", qs, dt), _expect(k, "k", ks, dt), _expect(v, "v", ks, dt),
            _ptr(s, "s", torch.float32), _expect(o, "o", qs, dt))
    _check("mxfa_run_naive_fwd",
           load_library().mxfa_run_naive_fwd(ctypes.byref(sh.c()), *args, _stream(stream)))


# ------------------------------------------------------------------ prefill --

def _rows(t, name, dtype, min_rows, min_cols):
    """A 2-D device tensor whose rows are contiguous (any row stride): returns
    (pointer, row stride in elements)."""
    torch = _torch()
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be a device tensor (got {t.device}); there is no CPU path")
    if t.dtype != dtype:
        raise ValueError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if t.dim() != 2 or (t.shape[1] > 1 and t.stride(1) != 1):
        raise ValueError(f"{name}: expected a 2-D tensor with contiguous rows, got shape {tuple(t.shape)} "
                         f"strides {t.stride()}")
    if t.shape[0] < min_rows or t.shape[1] < min_cols:
        raise ValueError(f"{name}: needs at least {min_rows} rows x {min_cols} columns, got {tuple(t.shape)}")
    return ctypes.c_void_p(t.data_ptr()), (t.stride(0) if t.shape[0] > 1 else max(t.shape[1], min_cols))


def run_prefill(q, kcache, vcache, out, pos0: int, n_head: int, n_kv_head: int, head_dim: int = 64,
                scale: float = 0.0, stream=None):
    """mxfa_run_prefill, the flash forward over a KV cache with token-major rows
    (attn_prefill, 03-llm-engine/kernels/llm.cu:3806-3815): query row i sits at
    position pos0 + i and attends to cache rows 0..pos0 + i.

    q: [n_tok, >= n_head*head_dim] (head h at columns h*head_dim..; may be a
    view into a fused QKV buffer); kcache, vcache: [>= pos0 + n_tok,
    >= n_kv_head*head_dim], same row stride, rows 0..pos0 + n_tok - 1 filled;
    out: [n_tok, >= n_head*head_dim]. All bf16, or fp32 with head_dim 64."""
    torch = _torch()
    if q.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"q: dtype {q.dtype}; bf16 or float32 expected")
    n_tok = q.shape[0] if q.dim() == 2 else -1
    qp, qs = _rows(q, "q", q.dtype, 1, n_head * head_dim)
    kp, ks = _rows(kcache, "kcache", q.dtype, pos0 + n_tok, n_kv_head * head_dim)
    vp, vs = _rows(vcache, "vcache", q.dtype, pos0 + n_tok, n_kv_head * head_dim)
    if ks != vs:
        raise ValueError(f"kcache and vcache must share a row stride ({ks} != {vs})")
    op, os_ = _rows(out, "out", q.dtype, n_tok, n_head * head_dim)
    sh = MxfaPrefillShape(n_tok, n_head, n_kv_head, head_dim, pos0, qs, ks, os_,
                          MXFA_BF16 if q.dtype == torch.bfloat16 else MXFA_F32, scale)
    _check("mxfa_run_prefill", load_library().mxfa_run_prefill(ctypes.byref(sh), qp, kp, vp, op, _stream(stream)))


def run_prefill_paged(q, kcache, vcache, out, block_table, block_size: int, pos0: int, n_head: int,
                      n_kv_head: int, head_dim: int = 64, scale: float = 0.0, stream=None, split: bool = False,
                      workspace=None):
    """mxfa_run_prefill_paged, run_prefill over a paged KV cache
    (attn_prefill_paged, 03-llm-engine/kernels/llm.cu:3827-3836): logical
    position t sits in cache row block_table[t // block_size] * block_size +
    t % block_size (kv_row<true>, llm.cu:959-963).

    kcache, vcache: [pool rows, >= n_kv_head*head_dim], same row stride, the
    pool holding every block the table names; block_table: int32 device tensor
    with at least ceil((pos0 + n_tok) / block_size) entries; block_size: a power
    of two. The rest as run_prefill; the outputs equal run_prefill's over the
    gathered cache bit for bit.

    split=True: mxfa_run_prefill_paged_ws, the keys split as run_prefill_split
    does (workspace as there, allocated here when None and returned); its
    outputs equal run_prefill_split's over the gathered cache bit for bit."""
    torch = _torch()
    if q.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"q: dtype {q.dtype}; bf16 or float32 expected")
    n_tok = q.shape[0] if q.dim() == 2 else -1
    qp, qs = _rows(q, "q", q.dtype, 1, n_head * head_dim)
    kp, ks = _rows(kcache, "kcache", q.dtype, 1, n_kv_head * head_dim)
    vp, vs = _rows(vcache, "vcache", q.dtype, 1, n_kv_head * head_dim)
    if ks != vs:
        raise ValueError(f"kcache and vcache must share a row stride ({ks} != {vs})")
    op, os_ = _rows(out, "out", q.dtype, n_tok, n_head * head_dim)
    if not isinstance(block_table, torch.Tensor) or block_table.device.type != "cuda" or \
            block_table.dtype != torch.int32 or block_table.dim() != 1 or block_table.stride(0) != 1:
        raise ValueError("block_table: expected a contiguous 1-D int32 device tensor")
    if block_size < 1:
        raise ValueError(f"block_size {block_size}: must be positive")
    need = -(-(pos0 + n_tok) // block_size)
    if block_table.numel() < need:
        raise ValueError(f"block_table: {block_table.numel()} entries, positions 0..{pos0 + n_tok - 1} need {need}")
    sh = MxfaPrefillShape(n_tok, n_head, n_kv_head, head_dim, pos0, qs, ks, os_,
                          MXFA_BF16 if q.dtype == torch.bfloat16 else MXFA_F32, scale)
    lib = load_library()
    if not split:
        _check("mxfa_run_prefill_paged",
               lib.mxfa_run_prefill_paged(ctypes.byref(sh), qp, kp, vp, op, ctypes.c_void_p(block_table.data_ptr()),
                                          int(block_size), _stream(stream)))
        return None
    workspace = _split_workspace(lib, sh, workspace, q.device)
    _check("mxfa_run_prefill_paged_ws",
           lib.mxfa_run_prefill_paged_ws(ctypes.byref(sh), qp, kp, vp, op, ctypes.c_void_p(block_table.data_ptr()),
                                         int(block_size), ctypes.c_void_p(workspace.data_ptr()),
                                         workspace.numel() * workspace.element_size(), _stream(stream)))
    return workspace


def _split_workspace(lib, sh, workspace, device):
    """The split prefill's workspace: `workspace` checked, or a new one of the size the shape needs."""
    torch = _torch()
    if workspace is None:
        need = int(lib.mxfa_prefill_workspace_bytes(ctypes.byref(sh)))
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=device)
    if not isinstance(workspace, torch.Tensor) or workspace.device.type != "cuda" or not workspace.is_contiguous():
        raise ValueError("workspace: expected a contiguous device tensor")
    return workspace


def prefill_workspace_bytes(n_tok: int, pos0: int, n_head: int, n_kv_head: int, head_dim: int = 64,
                            bf16: bool = True) -> int:
    """mxfa_prefill_workspace_bytes for contiguous rows: the fp32 partials
    run_prefill_split needs (0: the shape runs unsplit)."""
    w = n_head * head_dim
    sh = MxfaPrefillShape(n_tok, n_head, n_kv_head, head_dim, pos0, w, n_kv_head * head_dim, w,
                          MXFA_BF16 if bf16 else MXFA_F32, 0.0)
    return int(load_library().mxfa_prefill_workspace_bytes(ctypes.byref(sh)))


def run_prefill_split(q, kcache, vcache, out, pos0: int, n_head: int, n_kv_head: int, head_dim: int = 64,
                      scale: float = 0.0, workspace=None, stream=None):
    """mxfa_run_prefill_ws: run_prefill with the cache's keys split over
    work-groups when the chunk's query blocks would not fill the GPU (the same
    attn_prefill launch, 03-llm-engine/kernels/llm.cu:3806-3815). Arguments as
    run_prefill; workspace: a device tensor of at least the size
    mxfa_prefill_workspace_bytes reports (allocated here when None). Results
    equal run_prefill's to fp32 rounding, not bitwise."""
    torch = _torch()
    if q.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"q: dtype {q.dtype}; bf16 or float32 expected")
    n_tok = q.shape[0] if q.dim() == 2 else -1
    qp, qs = _rows(q, "q", q.dtype, 1, n_head * head_dim)
    kp, ks = _rows(kcache, "kcache", q.dtype, pos0 + n_tok, n_kv_head * head_dim)
    vp, vs = _rows(vcache, "vcache", q.dtype, pos0 + n_tok, n_kv_head * head_dim)
    if ks != vs:
        raise ValueError(f"kcache and vcache must share a row stride ({ks} != {vs})")
    op, os_ = _rows(out, "out", q.dtype, n_tok, n_head * head_dim)
    sh = MxfaPrefillShape(n_tok, n_head, n_kv_head, head_dim, pos0, qs, ks, os_,
                          MXFA_BF16 if q.dtype == torch.bfloat16 else MXFA_F32, scale)
    lib = load_library()
    workspace = _split_workspace(lib, sh, workspace, q.device)
    have = workspace.numel() * workspace.element_size()
    _check("mxfa_run_prefill_ws",
           lib.mxfa_run_prefill_ws(ctypes.byref(sh), qp, kp, vp, op, ctypes.c_void_p(workspace.data_ptr()),
                                   have, _stream(stream)))
    return workspace


# ------------------------------------------------------------ conveniences --

def attention_fwd(q, k, v, causal: bool, scale: float = 0.0, stream=None):
    """Allocates O and LSE and runs the forward; returns (O, LSE)."""
    torch = _torch()
    sh = shape_of(q, k, causal, scale)
    o = torch.empty_like(q)
    lse = torch.empty((sh.B, sh.Hq, sh.N), dtype=torch.float32, device=q.device)
    run_flash_lse(q, k, v, o, lse, causal, scale, stream)
    return o, lse


def attention_bwd(q, k, v, o, lse, do, causal: bool, scale: float = 0.0, stream=None):
    """Allocates Delta, dQ, dK, dV (and, for GQA shapes that use one, the dK/dV
    workspace) and runs the backward (run_bwd_ws: Delta folded into the dQ
    pass); returns (dQ, dK, dV)."""
    torch = _torch()
    sh = shape_of(q, k, causal, scale)
    delta = torch.empty((sh.B, sh.Hq, sh.N), dtype=torch.float32, device=q.device)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    nws = bwd_workspace_bytes(q, k, causal)
    ws = torch.empty(nws, dtype=torch.uint8, device=q.device) if nws else None
    run_bwd_ws(q, k, v, o, do, lse, delta, dq, dk, dv, ws, causal, scale, stream)
    return dq, dk, dv


# ----------------------------------------------------------- roofline probes --

def _time_ms(launch, reps: int) -> float:
    """Mean event time (ms) of `reps` back-to-back launches, after one warm-up."""
    torch = _torch()
    launch()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        launch()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / reps


def probe_mfma_tflops(bf16: bool = True, iters: int = 256, reps: int = 5, big: bool = False) -> float:
    """Measured MFMA throughput (TFLOP/s) of the whole device: every wave issues
    independent v_mfma_f32_16x16x32_bf16 (bf16), v_mfma_f32_32x32x16_bf16
    (bf16, big) or v_mfma_f32_16x16x4_f32 (fp32)."""
    torch = _torch()
    lib = load_library()
    sink = torch.empty(lib.mxfa_probe_sink_len(), dtype=torch.float32, device="cuda")
    flops = ctypes.c_double(0.0)
    dt = MXFA_BF16 if bf16 else MXFA_F32
    stream = _stream(None)

    def launch():
        sp = _ptr(sink, "sink", torch.float32)
        if bf16 and big:
            _check("mxfa_probe_mfma32", lib.mxfa_probe_mfma32(iters, sp, ctypes.byref(flops), stream))
        else:
            _check("mxfa_probe_mfma", lib.mxfa_probe_mfma(dt, iters, sp, ctypes.byref(flops), stream))
    ms = _time_ms(launch, reps)
    return flops.value / (ms * 1e-3) / 1e12


# The instruction mixes of mxfa_probe_mix (include/mxfa_probes.h, MXFA_PROBE_MIX_*).
PROBE_MIXES = {"mfma": 0, "dkv": 1, "dkv_valu": 2, "dkv_lds": 3, "dq": 4, "fwd": 5,
               "mfma32": 6, "dkv32": 7, "dq32": 8, "fwd32": 9}


def probe_mix_tflops(mix: str, waves_per_simd: int = 3, iters: int = 64, reps: int = 5) -> float:
    """MFMA throughput (TFLOP/s, whole device) of one of PROBE_MIXES issued with
    no dependencies between its instructions, at waves_per_simd waves per SIMD
    (mxfa_probe_mix): the instruction-issue ceiling of a kernel with that mix."""
    torch = _torch()
    lib = load_library()
    sink = torch.empty(lib.mxfa_probe_sink_len(), dtype=torch.float32, device="cuda")
    flops = ctypes.c_double(0.0)
    stream = _stream(None)
    mid = PROBE_MIXES[mix]

    def launch():
        _check("mxfa_probe_mix", lib.mxfa_probe_mix(mid, waves_per_simd, iters, _ptr(sink, "sink", torch.float32),
                                                    ctypes.byref(flops), stream))
    ms = _time_ms(launch, reps)
    return flops.value / (ms * 1e-3) / 1e12


def probe_wg_times():
    """The per-work-group timeline of the last forward or backward launch
    (mxfa_probe_wg_times; only with TIMELINE_CODE_OBJECT_PATH loaded): a uint64
    numpy array [groups, 8] by linear work-group index. Columns 0-3: 100 MHz
    real-time counter values (start, first stage staged, end of loop, stores
    acknowledged); 4: (kind << 32) | block (kind 0 = dQ and its query block,
    1 = dK/dV and its key block, 2 = forward and its query block); 5: its
    stages; 6: (XCC_ID << 32) | HW_ID, the XCD and the CU (HW_ID bits 8-11),
    shader engine (13-15) it ran on; 7: zero. Zero rows for indices the launch
    did not have (or an earlier launch's values)."""
    import numpy as np
    lib = load_library()
    avail = ctypes.c_size_t(0)
    _check("mxfa_probe_wg_times", lib.mxfa_probe_wg_times(None, 0, ctypes.byref(avail)))
    buf = np.zeros(avail.value // 8, dtype=np.uint64)
    _check("mxfa_probe_wg_times", lib.mxfa_probe_wg_times(buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes,
                                                          ctypes.byref(avail)))
    return buf.reshape(-1, 8)


def probe_dq_atomic(bh: int = 48, n: int = 4096, atomic: bool = True, reps: int = 5) -> dict:
    """Time of the global writes a dQ pass fused into the dK/dV pass would make
    at a causal (bh heads, N = n, d = 64) shape (mxfa_probe_dq_atomic): fp32
    atomic adds, or with atomic=False plain stores of the same bytes. Returns
    {"us", "payload_bytes", "tbps"} (mean of reps launches after one warm-up)."""
    torch = _torch()
    lib = load_library()
    acc = torch.zeros(bh * n * 64, dtype=torch.float32, device="cuda")
    nbytes = ctypes.c_double(0.0)
    stream = _stream(None)

    def launch():
        _check("mxfa_probe_dq_atomic", lib.mxfa_probe_dq_atomic(_ptr(acc, "acc", torch.float32), bh, n,
                                                                  int(atomic), ctypes.byref(nbytes), stream))
    ms = _time_ms(launch, reps)
    return {"us": ms * 1e3, "payload_bytes": nbytes.value, "tbps": nbytes.value / (ms * 1e-3) / 1e12}


def probe_hbm_gbps(mib: int = 1024, reps: int = 5, copy: bool = False) -> float:
    """Measured HBM streaming bandwidth (GB/s): a grid-stride read of `mib` MiB
    (or, with copy=True, a copy of that size, counting read + write bytes)."""
    torch = _torch()
    lib = load_library()
    nbytes = mib * 2**20
    x = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    stream = _stream(None)
    if copy:
        y = torch.empty_like(x)

        def launch():
            _check("mxfa_probe_copy", lib.mxfa_probe_copy(_ptr(x, "x", torch.float32), _ptr(y, "y", torch.float32),
                                                          nbytes, stream))
        moved = 2 * nbytes
    else:
        sink = torch.empty(lib.mxfa_probe_sink_len(), dtype=torch.float32, device="cuda")

        def launch():
            _check("mxfa_probe_read", lib.mxfa_probe_read(_ptr(x, "x", torch.float32), nbytes,
                                                          _ptr(sink, "sink", torch.float32), stream))
        moved = nbytes
    ms = _time_ms(launch, reps)
    return moved / (ms * 1e-3) / 1e9


def init(device: int = 0):
    """mxfa_init: checks that ``device`` is a gfx950, makes it current and
    loads the code object on it."""
    _check("mxfa_init", load_library().mxfa_init(device))


def shutdown():
    """mxfa_shutdown: unloads the code object from every device it was loaded
    on (their work must have completed); the next launch loads it again."""
    _check("mxfa_shutdown", load_library().mxfa_shutdown())


def check_code_object(path: str | None = None) -> int:
    """mxfa_check_code_object: 0 if ``path`` (default: the library's code
    object) is a gfx950 code object, else the MXFA_ERR_CODE_OBJECT status. Host
    only, no device access."""
    return int(load_library().mxfa_check_code_object(path.encode() if path else None))


def set_code_object(path: str | None):
    """mxfa_set_code_object: the code object file later loads read (None: the
    default beside libmxfa.so)."""
    _check("mxfa_set_code_object", load_library().mxfa_set_code_object(path.encode() if path else None))


# The reference's benchmark counts (02-flash-attention/src/main.rs:15-16).
WARMUP = 1
ITERS = 5


def time_median_ms(fn, warmup: int = WARMUP, iters: int = ITERS, stream=None) -> float:
    """Median time of one invocation of `fn` in milliseconds, as
    common/src/lib.rs:22-43 (time_median_ms) measures it: `warmup` calls, a
    synchronisation of the stream, then `iters` calls each bracketed by a pair
    of HIP events on the stream and waited for; the median is the sorted
    times' element iters // 2. `fn` enqueues its work on `stream` (default:
    torch's current stream)."""
    torch = _torch()
    if iters < 1:
        raise ValueError(f"iters must be at least 1 (got {iters})")
    s = stream if stream is not None else torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    s.synchronize()
    times = []
    for _ in range(iters):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(s)
        fn()
        end.record(s)
        end.synchronize()
        times.append(start.elapsed_time(end))
    times.sort()
    return times[len(times) // 2]


def fwd_flops(B, Hq, N, d, causal) -> float:
    """Algorithmic forward flops: 4 N^2 d per (batch, query head), halved if causal."""
    return 4.0 * N * N * d * B * Hq * (0.5 if causal else 1.0)


def bwd_flops(B, Hq, N, d, causal) -> float:
    """Algorithmic backward flops: 10 N^2 d per (batch, query head), halved if causal."""
    return 10.0 * N * N * d * B * Hq * (0.5 if causal else 1.0)
