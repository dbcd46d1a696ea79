"""CPU oracle for QSTE's binary-linear hot path -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker (or as
the timed CPU baseline). The product package ``qste_amd`` never imports it:
its kernels run on the GPU through the HIP library or raise.

The arithmetic lives in ``qste_oracle.c`` (built by ``oracle/Makefile``);
this module is a thin numpy/ctypes wrapper. Every function follows the
reference's specification backend, ``src/qste/kernels/fallback.py``, and the
hash in ``src/qste/kernels/stream.py`` (citations per function below).

What pins each function (all checks live in ``tests/test_oracle.py``):

* hash -- golden vectors written by the reference's own ``stream`` module
  (``tests/golden/make_golden.py``) plus the uniformity / decorrelation
  properties of ``tests/test_kernels.py:250-279`` in the reference.
* pack_coordinate / unpack_rows -- brute force per bit and the round trip.
* pack_affine_rows -- golden vectors from the reference's fallback, with a
  band for elements within one ulp of the row mean; closed-form identities.
* linear / dgrad / evidence / row_inner / offset correction -- numpy dense
  products in float64 through ``unpack_rows`` (an independent route through
  matmul rather than bit loops) and golden vectors from the fallback.
* coordinate_update -- golden vectors from the fallback, compared with a
  declared rounding-margin band; invariants (packed == pack(coord), |q| and
  |coord| <= 127, reproducibility from (seed, step), first-step closed form).
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "libqste_oracle.so"
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_dbl = ctypes.c_double
_vp = ctypes.c_void_p


def build(force: bool = False) -> Path:
    """Compile the oracle with ``make`` (gcc). Idempotent unless ``force``."""

    if force or not _LIB_PATH.exists():
        args = ["make", "-s", "-C", str(_HERE)] + (["-B"] if force else [])
        subprocess.run(args, check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        handle = ctypes.CDLL(str(_LIB_PATH))
        handle.qo_scramble.restype = ctypes.c_uint32
        handle.qo_scramble.argtypes = [ctypes.c_uint32]
        handle.qo_seed_hash.restype = ctypes.c_uint32
        handle.qo_seed_hash.argtypes = [_i64]
        handle.qo_step_hash.restype = ctypes.c_uint32
        handle.qo_step_hash.argtypes = [_i64]
        handle.qo_scramble_many.argtypes = [_u32p, _i64, _u32p]
        handle.qo_uniform.argtypes = [_i64, _i64, _i64p, _i64, _f32p]
        handle.qo_pack_coordinate.argtypes = [_i8p, _i64, _i64, _u8p]
        handle.qo_unpack_rows.argtypes = [_u8p, _i64, _i64, _f32p]
        handle.qo_pack_affine_rows.argtypes = [_f32p, _i64, _i64, _u8p, _f32p, _f32p]
        handle.qo_linear_fwd.argtypes = [_f32p, _i64, _u8p, _i64, _i64, _f32p, _vp, _f64p]
        handle.qo_linear_dgrad.argtypes = [_f32p, _i64, _u8p, _i64, _i64, _vp, _f64p]
        handle.qo_evidence.argtypes = [_f32p, _i64, _i64, _u8p, _i64, _vp, _f64p]
        handle.qo_offset_correction.argtypes = [_f32p, _i64, _i64, _f32p, _f64p]
        handle.qo_row_inner.argtypes = [_f32p, _u8p, _i64, _i64, _f64p]
        handle.qo_coordinate_update.restype = _i64
        handle.qo_coordinate_update.argtypes = [
            _f32p, _i8p, _u8p, _i8p, _u16p, _u16p, _u16p, _i64, _i64,
            _dbl, _dbl, _dbl, _dbl, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
        ]
        handle.qo_step_size.restype = ctypes.c_float
        handle.qo_step_size.argtypes = [ctypes.c_float, _dbl]
        handle.qo_round_bf16.restype = ctypes.c_float
        handle.qo_round_bf16.argtypes = [ctypes.c_float]
        _lib = handle
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# -- hash (stream.py:41-83) ---------------------------------------------------


def scramble(values) -> np.ndarray:
    v = np.ascontiguousarray(np.asarray(values, dtype=np.uint64) & 0xFFFFFFFF, dtype=np.uint32)
    out = np.empty_like(v)
    lib().qo_scramble_many(v, v.size, out)
    return out


def seed_hash(seed: int) -> int:
    return int(lib().qo_seed_hash(_wrap64(seed)))


def step_hash(step: int) -> int:
    return int(lib().qo_step_hash(_wrap64(step)))


def uniform(seed: int, step: int, index) -> np.ndarray:
    idx = np.ascontiguousarray(np.asarray(index, dtype=np.int64))
    out = np.empty(idx.shape, dtype=np.float32)
    lib().qo_uniform(_wrap64(seed), _wrap64(step), idx.reshape(-1), idx.size, out.reshape(-1))
    return out


def _wrap64(value: int) -> int:
    value = int(value) & 0xFFFFFFFFFFFFFFFF
    return value - (1 << 64) if value >= (1 << 63) else value


# -- packing (fallback.py:27-92) ----------------------------------------------


def pack_coordinate(coord) -> np.ndarray:
    c = np.ascontiguousarray(coord, dtype=np.int8)
    rows, cols = c.shape
    out = np.empty((rows, (cols + 7) // 8), dtype=np.uint8)
    lib().qo_pack_coordinate(c, rows, cols, out)
    return out


def unpack_rows(packed, columns: int) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    rows = p.shape[0]
    out = np.empty((rows, columns), dtype=np.float32)
    lib().qo_unpack_rows(p, rows, columns, out)
    return out


def pack_affine_rows(x):
    """(bits, offset, scale) of fallback.py:77-88, from fp32 (or bf16-valued) rows."""

    v = _f32(x)
    rows, cols = v.shape
    bits = np.empty((rows, (cols + 7) // 8), dtype=np.uint8)
    off = np.empty(rows, dtype=np.float32)
    xs = np.empty(rows, dtype=np.float32)
    lib().qo_pack_affine_rows(v, rows, cols, bits, off, xs)
    return bits, off, xs


# -- dense products (fallback.py:95-148; functional.py:139-144) ---------------


def linear_fwd(x, packed, scale, bias, columns: int) -> np.ndarray:
    v = _f32(x).reshape(-1, columns)
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    rows = p.shape[0]
    s = _f32(scale)
    b = None if bias is None else _f32(bias)
    out = np.empty((v.shape[0], rows), dtype=np.float64)
    lib().qo_linear_fwd(v, v.shape[0], p, rows, columns, s, _ptr(b), out)
    return out


def linear_dgrad(dy, packed, columns: int, row_scale=None) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    rows = p.shape[0]
    g = _f32(dy).reshape(-1, rows)
    s = None if row_scale is None else _f32(row_scale)
    out = np.empty((g.shape[0], columns), dtype=np.float64)
    lib().qo_linear_dgrad(g, g.shape[0], p, rows, columns, _ptr(s), out)
    return out


def evidence(dy, packed_x, columns: int, row_scale=None) -> np.ndarray:
    g = _f32(dy)
    samples, rows = g.shape
    p = np.ascontiguousarray(packed_x, dtype=np.uint8)
    s = None if row_scale is None else _f32(row_scale)
    out = np.empty((rows, columns), dtype=np.float64)
    lib().qo_evidence(g, samples, rows, p, columns, _ptr(s), out)
    return out


def offset_correction(dy, offset) -> np.ndarray:
    g = _f32(dy)
    samples, rows = g.shape
    out = np.empty(rows, dtype=np.float64)
    lib().qo_offset_correction(g, samples, rows, _f32(offset), out)
    return out


def row_inner(matrix, packed, columns: int) -> np.ndarray:
    m = _f32(matrix)
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty(m.shape[0], dtype=np.float64)
    lib().qo_row_inner(m, p, m.shape[0], columns, out)
    return out


def decoded_evidence(dy, bits_x, offset, xs, columns: int) -> np.ndarray:
    """E0 = dy^T (offset + xs * sign) -- functional.py:118-145 in float64."""

    return evidence(dy, bits_x, columns, xs) + offset_correction(dy, offset)[:, None]


# -- the same products through float64 BLAS, for full-size samples ------------
# The C restatements above accumulate one product at a time and take minutes
# at config-4 sizes; these expand the signs to a float64 +-1 matrix once and
# use numpy's float64 matrix product (error ~1e-15 relative, far below any
# fp32 or bf16 bar).  tests/test_oracle.py pins them to the C versions.


def signs_f64(packed, columns: int) -> np.ndarray:
    """+-1 float64 [rows, columns] of packed signs (LSB first, pad dropped)."""

    bits = np.unpackbits(np.ascontiguousarray(packed, dtype=np.uint8), axis=1, bitorder="little")
    return bits[:, :columns].astype(np.float64) * 2.0 - 1.0


def linear_fwd_f64(x, packed, scale, bias, columns: int) -> np.ndarray:
    v = np.asarray(x, dtype=np.float32).reshape(-1, columns).astype(np.float64)
    out = v @ signs_f64(packed, columns).T
    out *= np.asarray(scale, dtype=np.float32).astype(np.float64)[None, :]
    if bias is not None:
        out += np.asarray(bias, dtype=np.float32).astype(np.float64)[None, :]
    return out


def linear_dgrad_f64(dy, packed, columns: int, row_scale=None) -> np.ndarray:
    sign = signs_f64(packed, columns)
    if row_scale is not None:
        sign *= np.asarray(row_scale, dtype=np.float32).astype(np.float64)[:, None]
    g = np.asarray(dy, dtype=np.float32).reshape(-1, sign.shape[0]).astype(np.float64)
    return g @ sign


def evidence_f64(dy, packed_x, columns: int, row_scale=None) -> np.ndarray:
    g = np.asarray(dy, dtype=np.float32).astype(np.float64)
    if row_scale is not None:
        g = g * np.asarray(row_scale, dtype=np.float32).astype(np.float64)[:, None]
    return g.T @ signs_f64(packed_x, columns)


# -- coordinate step (fallback.py:158-242) ------------------------------------


def step_size(moment_rms: float, coordinate_lr: float) -> np.float32:
    """``coordinate_lr / moment_rms`` as fallback.py:204-206 evaluates it:
    ``reciprocal(moment_rms) * fp32(coordinate_lr)``, two fp32 roundings."""

    return np.float32(lib().qo_step_size(float(np.float32(moment_rms)), float(coordinate_lr)))


def coordinate_update(grad, state: dict, *, beta1, beta2, update_clip, coordinate_lr,
                      block_size, seed, step, margins: bool = False, scalars=None,
                      scale_margin=None):
    """Run the spec step on numpy state in place; returns flips (and margins).

    ``state`` holds ``coordinate`` (int8 [R,C]), ``packed`` (uint8 [R,PB]),
    ``moment_q`` (int8 [R,C]), and ``moment_scale`` / ``row_v`` / ``col_v`` as
    float16 arrays (their bit patterns are updated through a uint16 view).
    ``scalars``, a float32 array of 4, receives sqrt(mean row statistic),
    the clip divisor, the step size and the momentum RMS.  ``scale_margin``,
    a float32 array of one value per block, receives each block's distance
    in fp16 ulps of amax / 127 from the fp16 rounding midpoint.
    """

    g = np.array(grad, dtype=np.float32, order="C", copy=True)
    rows, cols = g.shape
    for key in ("coordinate", "packed", "moment_q", "moment_scale", "row_v", "col_v"):
        if not state[key].flags["C_CONTIGUOUS"]:
            raise ValueError(f"state[{key!r}] must be C-contiguous")
    if scalars is not None and (scalars.dtype != np.float32 or scalars.size < 4
                                or not scalars.flags["C_CONTIGUOUS"]):
        raise ValueError("scalars must be a contiguous float32 array of at least 4")
    blocks = -(-rows * cols // int(block_size))
    if scale_margin is not None and (scale_margin.dtype != np.float32 or scale_margin.size < blocks
                                     or not scale_margin.flags["C_CONTIGUOUS"]):
        raise ValueError(f"scale_margin must be a contiguous float32 array of at least {blocks}")
    tm = np.empty((rows, cols), dtype=np.float32) if margins else None
    mm = np.empty((rows, cols), dtype=np.float32) if margins else None
    flips = lib().qo_coordinate_update(
        g, state["coordinate"], state["packed"], state["moment_q"],
        state["moment_scale"].view(np.uint16), state["row_v"].view(np.uint16),
        state["col_v"].view(np.uint16), rows, cols, float(beta1), float(beta2),
        float(update_clip), float(coordinate_lr), int(block_size), _wrap64(seed),
        _wrap64(step), _ptr(tm), _ptr(mm), _ptr(scalars), _ptr(scale_margin),
    )
    if margins:
        return int(flips), tm, mm
    return int(flips)


def fresh_state(coordinate, block_size: int) -> dict:
    """Optimizer state as QSTEOptimizer allocates it (optim.py:79-91)."""

    c = np.ascontiguousarray(coordinate, dtype=np.int8)
    rows, cols = c.shape
    blocks = (rows * cols + block_size - 1) // block_size
    return {
        "coordinate": c.copy(),
        "packed": pack_coordinate(c),
        "moment_q": np.zeros((rows, cols), dtype=np.int8),
        "moment_scale": np.full(blocks, 1 / 127, dtype=np.float16),
        "row_v": np.zeros(rows, dtype=np.float16),
        "col_v": np.zeros(cols, dtype=np.float16),
    }


def round_bf16(x) -> np.ndarray:
    """Round fp32 values to bfloat16 (nearest even), returned as fp32."""

    a = _f32(x)
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32)
    nan = np.isnan(a)
    out = r.view(np.float32).copy()
    out[nan] = a[nan]
    return out
