"""Loaders for the in-tree libraries under ``kernels/``.

``import torch`` happens before either library is opened: PyTorch-ROCm ships
its own HIP runtime (soname ``libamdhip64.so.7``) and libharp_ra.so must bind
to that same copy so both share one device context and stream namespace.

Nothing here falls back to a CPU implementation: a missing or stale library
raises with the build command to run.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede the ctypes load, see module docstring)

ROOT = Path(__file__).resolve().parent.parent
KERNELS = ROOT / "kernels"
ABI_LIB = KERNELS / "libharp_ra.so"
OPS_LIB = KERNELS / "libring_attention_ops.so"
ASYNC_OPS_LIB = KERNELS / "libharp_async_op.so"

HARP_RA_OK = 0
HARP_RA_EINVAL = 1
HARP_RA_EUNSUPPORTED = 2
HARP_RA_ENOMEM = 3
HARP_RA_ELAUNCH = 4
HARP_RA_F32 = 0
HARP_RA_BF16 = 1
HARP_RA_MAX_CHUNKS = 16
KERNEL_KINDS = ("stats", "fwd", "delta", "dkdv", "dq")

_lock = threading.Lock()
_abi: ctypes.CDLL | None = None
_ops_loaded = False
_async_ops_loaded = False

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)
_pp = ctypes.POINTER(ctypes.c_void_p)
_sz = ctypes.c_size_t

# (restype, argtypes) of every symbol include/harp_ring_attn.h declares
ABI_PROTOTYPES = {
    "harp_ra_forward": (
        _i,
        [_p, _i64p, _pp, _pp, _i64p, _i, _i32p, _p, _i64p, _p, _i, _p,
         _i, _i, _i, _i, _i, _i, ctypes.c_float, _p, _sz, _p],
    ),
    "harp_ra_backward": (
        _i,
        [_p, _i64p, _p, _i64p, _i, _pp, _pp, _i64p, _pp, _pp, _i64p, _i,
         _i, _i32p, _p, _i64p, _p, _i, _p, _p,
         _i, _i, _i, _i, _i, _i, ctypes.c_float, _p, _sz, _p],
    ),
    "harp_ra_delta": (_i, [_p, _i64p, _p, _i64p, _p, _i, _i, _i, _i, _p]),
    "harp_ra_forward_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i, _i32p]),
    "harp_ra_backward_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i, _i32p]),
    "harp_ra_timing_enable": (_i, [_i]),
    "harp_ra_timing_read": (_i, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int), _i]),
    "harp_ra_last_error": (ctypes.c_char_p, []),
    "harp_ra_version": (ctypes.c_char_p, []),
}


HARP_QK_OK = 0
HARP_QK_F32 = 0
HARP_QK_BF16 = 1
_f = ctypes.c_float
_i64 = ctypes.c_int64


class QkvOut(ctypes.Structure):
    """harp_qkv_out_t of include/harp_qk_norm_rope.h (one projection of harp_qkv_project)."""

    _fields_ = [
        ("weight", _p),
        ("ld_weight", _i64),
        ("y", _p),
        ("ld_y", _i64),
        ("y_lin", _p),
        ("norm_weight", _p),
        ("norm_weight_dtype", _i),
        ("eps", _f),
        ("rms", _p),
    ]


# (restype, argtypes) of every symbol include/harp_qk_norm_rope.h declares
QK_PROTOTYPES = {
    "harp_qk_rmsnorm_forward": (_i, [_p, _i64p, _p, _i64p, _p, _i, _p, _f, _i, _i, _i, _i, _p]),
    "harp_qk_rmsnorm_backward": (_i, [_p, _i64p, _p, _i64p, _p, _i, _p, _p, _i64p, _p, _i, _i, _i, _i, _i,
                                      _p, _sz, _p]),
    "harp_qk_rope_forward": (_i, [_p, _i64p, _p, _i64, _i64, _p, _i64p, _i, _i, _i, _i, _p]),
    "harp_qk_rope_backward": (_i, [_p, _i64p, _p, _i64, _i64, _p, _i64p, _i, _i, _i, _i, _p]),
    "harp_qk_norm_rope_forward": (_i, [_p, _i64p, _p, _i, _f, _p, _i64, _i64, _p, _i64p, _p, _i, _i, _i, _i, _p]),
    "harp_qk_norm_rope_backward": (_i, [_p, _i64p, _p, _i64p, _p, _i, _p, _p, _i64, _i64, _p, _i64p, _p, _i,
                                        _i, _i, _i, _i, _p, _sz, _p]),
    "harp_qk_norm_rope_backward_noalloc": (_i, [_p, _i64p, _p, _i64p, _p, _i, _p, _p, _i64, _i64, _p, _i64p, _p,
                                                _i, _i, _i, _i, _i, _p]),
    "harp_qk_backward_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "harp_qkv_project": (_i, [_p, _i64, _i, _i, _i, _i, _p, _i64, _i64, ctypes.POINTER(QkvOut), _i, _p]),
    "harp_qk_last_error": (ctypes.c_char_p, []),
}


def _missing(path: Path) -> RuntimeError:
    return RuntimeError(
        f"{path} is not built; run `python -m harp_amd.build` (or __graft_entry__.build()). "
        "There is no CPU fallback."
    )


def load_abi() -> ctypes.CDLL:
    """Open libharp_ra.so (the C ABI) and attach its prototypes."""
    global _abi
    with _lock:
        if _abi is None:
            if not ABI_LIB.exists():
                raise _missing(ABI_LIB)
            lib = ctypes.CDLL(str(ABI_LIB))
            for name, (res, args) in {**ABI_PROTOTYPES, **QK_PROTOTYPES}.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _abi = lib
        return _abi


def load_ops() -> None:
    """Register torch.ops.ring_attention_ops from kernels/libring_attention_ops.so."""
    global _ops_loaded
    with _lock:
        if _ops_loaded:
            return
        if not OPS_LIB.exists():
            raise _missing(OPS_LIB)
        torch.ops.load_library(str(OPS_LIB))
        _ops_loaded = True


def load_async_ops() -> None:
    """Register torch.ops.async_op (QK RMSNorm, RoPE) from kernels/libharp_async_op.so."""
    global _async_ops_loaded
    with _lock:
        if _async_ops_loaded:
            return
        if not ASYNC_OPS_LIB.exists():
            raise _missing(ASYNC_OPS_LIB)
        torch.ops.load_library(str(ASYNC_OPS_LIB))
        _async_ops_loaded = True


def qk_check(rc: int, what: str) -> None:
    if rc != HARP_QK_OK:
        raise RuntimeError(f"{what} failed (status {rc}): {load_abi().harp_qk_last_error().decode()}")


def last_error() -> str:
    return load_abi().harp_ra_last_error().decode()


def check(rc: int, what: str) -> None:
    if rc != HARP_RA_OK:
        raise RuntimeError(f"{what} failed (status {rc}): {last_error()}")


def i64_array(vals) -> ctypes.Array:
    return (ctypes.c_int64 * len(vals))(*[int(v) for v in vals])


def ptr_array(ptrs) -> ctypes.Array:
    return (ctypes.c_void_p * len(ptrs))(*[ctypes.c_void_p(int(p)) for p in ptrs])


def i32_array(vals) -> ctypes.Array:
    return (ctypes.c_int32 * len(vals))(*[int(v) for v in vals])


def timing_enable(on: bool) -> None:
    check(load_abi().harp_ra_timing_enable(1 if on else 0), "harp_ra_timing_enable")


def timing_read() -> dict:
    """Per-kernel (ms, launches) since the last read; call after synchronising."""
    n = len(KERNEL_KINDS)
    ms = (ctypes.c_double * n)()
    cnt = (ctypes.c_int * n)()
    check(load_abi().harp_ra_timing_read(ms, cnt, n), "harp_ra_timing_read")
    return {k: (ms[i], cnt[i]) for i, k in enumerate(KERNEL_KINDS)}
