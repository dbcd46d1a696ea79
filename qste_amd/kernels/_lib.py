"""ctypes binding of ``libqste_hip.so`` (declared in ``include/qste_hip.h``).

torch is imported before the library is opened: torch ships its own HIP
runtime, and the library must bind to that same runtime (the dynamic loader
matches it by soname) so that torch's device pointers and streams are the
library's too.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

LIB_PATH = Path(__file__).resolve().parent.parent / "libqste_hip.so"

_lock = threading.Lock()
_lib = None
_failure: str | None = None

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_dbl = ctypes.c_double
_flt = ctypes.c_float

# name -> (restype, argtypes); mirrors include/qste_hip.h
SIGNATURES = {
    "qste_version": (_int, []),
    "qste_error_string": (ctypes.c_char_p, [_int]),
    "qste_pack_coordinate": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "qste_unpack_rows": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _vp]),
    "qste_pack_affine_rows": (_int, [_vp, _int, _vp, _vp, _vp, _i64, _i64, _vp]),
    "qste_packed_linear_affine": (_int, [_vp, _int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "qste_packed_transpose": (_int, [_vp, _int, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "qste_evidence_from_packed_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "qste_evidence_from_packed": (_int, [_vp, _int, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    "qste_packed_row_inner": (_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "qste_linear_backward_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "qste_linear_backward_workspace_bytes_dtype": (_sz, [_i64, _i64, _i64, _int]),
    "qste_evidence_from_packed_workspace_bytes_dtype": (_sz, [_i64, _i64, _i64, _int]),
    "qste_packed_linear_affine_workspace_bytes": (_sz, [_i64, _i64, _i64, _int]),
    "qste_packed_linear_affine_ws": (_int, [_vp, _int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    "qste_packed_transpose_workspace_bytes": (_sz, [_i64, _i64, _i64, _int]),
    "qste_packed_transpose_ws": (_int, [_vp, _int, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    "qste_linear_backward": (_int, [_vp, _int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                    _i64, _i64, _i64, _vp, _sz, _vp]),
    "qste_linear_backward_offset_dot": (_int, [_vp, _int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                               _i64, _i64, _i64, _vp, _sz, _vp]),
    "qste_coordinate_update_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "qste_coordinate_update_scalars_offset": (_sz, [_i64, _i64, _i64]),
    "qste_coordinate_update_one_launch": (_int, [_i64, _i64, _i64]),
    "qste_stream_read": (_int, [_vp, _i64, _vp, _i64, _vp]),
    "qste_clock_probe": (_int, [_vp, _i64, _vp]),
    "qste_device_info": (_int, [_vp]),
    "qste_coordinate_update_static_limit": (_sz, []),
    "qste_coordinate_update_static": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _dbl, _dbl,
                                             _dbl, _dbl, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "qste_coordinate_update": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _dbl, _dbl,
                                      _dbl, _dbl, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _sz, _vp]),
    "qste_pack_bits": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "qste_unpack_bits": (_int, [_vp, _vp, _int, _i64, _i64, _vp]),
    "qste_apply_bits": (_int, [_vp, _int, _vp, _vp, _i64, _i64, _vp]),
    "qste_masked_backward": (_int, [_vp, _int, _vp, _vp, _i64, _i64, _flt, _flt, _flt, _vp]),
    "qste_masked_activation": (_int, [_vp, _int, _int, _flt, _flt, _int, _flt, _vp, _vp, _i64, _i64,
                                      _vp]),
    "qste_smooth_activation": (_int, [_vp, _int, _int, _flt, _vp, _int, _vp, _vp, _vp, _i64, _i64,
                                      _vp]),
    "qste_smooth_backward": (_int, [_vp, _int, _vp, _int, _vp, _vp, _i64, _i64, _vp]),
    "qste_swiglu_forward": (_int, [_vp, _vp, _int, _vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "qste_swiglu_backward": (_int, [_vp, _vp, _vp, _int, _vp, _vp, _i64, _vp]),
    "qste_swiglu_backward_sums_workspace_bytes": (_sz, [_i64, _i64]),
    "qste_swiglu_backward_sums": (_int, [_vp, _vp, _vp, _int, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _sz, _vp]),
    "qste_swiglu_backward_sums_into": (_int, [_vp, _vp, _vp, _int, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _sz, _vp]),
    "qste_row_scale": (_int, [_vp, _int, _vp, _vp, _i64, _flt, _flt, _vp]),
    "qste_row_scale_backward": (_int, [_vp, _vp, _int, _vp, _i64, _flt, _flt, _vp]),
    "qste_packed_embedding": (_int, [_vp, _i64, _vp, _vp, _vp, _int, _i64, _i64, _vp]),
    "qste_embedding_backward_workspace_bytes": (_sz, [_i64, _i64]),
    "qste_embedding_backward": (_int, [_vp, _i64, _vp, _int, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _sz,
                                       _vp]),
}


class KernelError(RuntimeError):
    """A HIP entry point returned a nonzero status."""


def load():
    """Open the library once; raise with the reason if it is unavailable."""

    global _lib, _failure
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            _failure = (
                f"{LIB_PATH} is not built; run `python -m qste_amd.build` "
                "(or __graft_entry__.build()) on a machine with ROCm's hipcc"
            )
            raise KernelError(_failure)
        try:
            handle = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:  # pragma: no cover - depends on the host
            _failure = f"cannot load {LIB_PATH}: {exc}"
            raise KernelError(_failure) from exc
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
        _failure = None
        return _lib


def failure() -> str | None:
    return _failure


def check(code: int, what: str) -> None:
    if code != 0:
        text = load().qste_error_string(int(code)).decode(errors="replace")
        raise KernelError(f"{what} failed ({code}): {text}")
