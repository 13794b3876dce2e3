"""ctypes binding of ``libsiq_kernels.so`` (the C ABI in ``include/siq_kernels.h``).

There is no fallback: if the library is missing the caller gets a RuntimeError
naming the build step, never a silent CPU or PyTorch path.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

from . import build as _build

_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None

SIQ_OK = 0
SIQ_ERR_INVALID_ARGUMENT = -1
SIQ_ERR_UNSUPPORTED = -2
SIQ_ERR_WORKSPACE = -3
SIQ_ERR_ALIGNMENT = -4
SIQ_ERR_LAUNCH = -5

_c_void_p = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_size = ctypes.c_size_t

_PROTOS = {
    "siq_abi_version": (_i32, []),
    "siq_last_error": (ctypes.c_char_p, []),
    "siq_attn_fwd_workspace_bytes": (_size, [_i32, _i64, _i64, _i32, _i32, _i32]),
    "siq_attn_bwd_workspace_bytes": (_size, [_i32, _i64, _i64, _i32, _i32, _i32, _i32]),
    "siq_attn_varlen_fwd": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i32, _i32, _i64, _i64,
         _i32, _i32, _i32, ctypes.POINTER(_i64), _f32, _i32, _c_void_p, _size, _c_void_p],
    ),
    "siq_attn_varlen_bwd": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _i32, _i32, _i32, _i64, _i64, _i32, _i32, _i32, ctypes.POINTER(_i64), _f32, _i32,
         _i32, _c_void_p, _size, _c_void_p],
    ),
    "siq_attn_varlen_fwd_noalloc": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i32, _i32, _i64, _i64,
         _i32, _i32, _i32, ctypes.POINTER(_i64), _f32, _i32, _c_void_p],
    ),
    "siq_attn_plan_bytes": (_size, [_i32, _i64, _i64]),
    "siq_attn_bwd_plan_workspace_bytes": (_size, [_i32, _i64, _i64, _i32, _i32, _i32, _i32]),
    "siq_attn_build_plan": (_i32, [_c_void_p, _c_void_p, _i32, _i64, _i64, _i32, _i32, _i32, _c_void_p, _size,
                                   _c_void_p]),
    "siq_attn_varlen_fwd_plan": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i64, _i32, _i32, _i32,
         ctypes.POINTER(_i64), _f32, _i32, _c_void_p, _size, _c_void_p],
    ),
    "siq_attn_varlen_bwd_plan": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _i32, _i64, _i64, _i32, _i32, _i32, ctypes.POINTER(_i64), _f32, _i32, _i32, _c_void_p, _size, _c_void_p,
         _size, _c_void_p],
    ),
    "siq_attn_rope_fwd_plan": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i64,
         _i32, _i32, _i32, ctypes.POINTER(_i64), _f32, _i32, _c_void_p, _size, _c_void_p],
    ),
    "siq_attn_rope_bwd_plan": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _i32, _i64, _i64, _i32, _i32, _i32, ctypes.POINTER(_i64), _f32, _i32, _c_void_p,
         _size, _c_void_p, _size, _c_void_p],
    ),
    "siq_flce_workspace_bytes": (_size, [_i64, _i64, _i64, _i64, _i32]),
    "siq_flce_fwd_bwd": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i32, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _size, _c_void_p],
    ),
    "siq_flce_loss_workspace_bytes": (_size, [_i64, _i64, _i64]),
    "siq_flce_loss": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i32, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _size, _c_void_p],
    ),
    "siq_scale_bf16": (_i32, [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p]),
    "siq_scale_bf16_inplace": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p]),
    "siq_proj_workspace_bytes": (_size, [_i64, _i64, _i64, _i32, _i64]),
    "siq_proj_fwd": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i32, _i64, _c_void_p, _size,
                            _c_void_p]),
    "siq_proj_bwd": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i32, _i64,
                            _c_void_p, _size, _c_void_p]),
    "siq_splice_workspace_bytes": (_size, [_i64]),
    "siq_splice_fwd": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _c_void_p,
                              _c_void_p, _c_void_p, _size, _c_void_p]),
    "siq_gather_rows": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p, _c_void_p]),
    "siq_embedding_bwd_workspace_bytes": (_size, [_i64, _i64]),
    "siq_embedding_bwd": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _i64, _i32, _i64, _i64, _c_void_p, _c_void_p,
                                 _size, _c_void_p]),
    "siq_probe_clock": (_i32, [_c_void_p, _i64, _c_void_p]),
    "siq_rope_fwd": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _i32, _i32,
         ctypes.POINTER(_i64), _c_void_p],
    ),
    "siq_rope_bwd": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _i32, _i32,
         ctypes.POINTER(_i64), _c_void_p],
    ),
    "siq_rope_fwd_ex": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _i32, _i32,
         ctypes.POINTER(_i64), _i32, _c_void_p],
    ),
    "siq_rope_bwd_ex": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _i32, _i32,
         ctypes.POINTER(_i64), _i32, _c_void_p],
    ),
}

EXPORTED = tuple(_PROTOS)


def lib_path() -> Path:
    return Path(os.environ.get("SIQ_KERNELS_LIB", str(_build.LIB_PATH)))


def lib() -> ctypes.CDLL:
    """Loads the library once; raises if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            path = lib_path()
            if not path.exists():
                raise RuntimeError(
                    f"{path} is missing: build the HIP kernels first "
                    "(python -c 'import __graft_entry__ as g; g.build()' or python -m siq_vl_amd.build)"
                )
            handle = ctypes.CDLL(str(path))
            for name, (res, args) in _PROTOS.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _LIB = handle
    return _LIB


def check(rc: int, what: str) -> None:
    """Maps a C status code to a Python exception."""
    if rc == SIQ_OK:
        return
    msg = lib().siq_last_error().decode(errors="replace")
    text = f"{what}: {msg} (status {rc})"
    if rc in (SIQ_ERR_INVALID_ARGUMENT, SIQ_ERR_UNSUPPORTED, SIQ_ERR_ALIGNMENT, SIQ_ERR_WORKSPACE):
        raise ValueError(text)
    raise RuntimeError(text)


def int64_array(values) -> ctypes.Array:
    arr = (_i64 * len(values))(*[int(v) for v in values])
    return arr
