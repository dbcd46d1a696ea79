"""CPU oracle for QSTE's packed activations -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline
may import this module, and only as the checker.  It restates
``src/qste/nn.py`` and the bit helpers of ``src/qste/kernels/fallback.py``
in numpy:

* bit helpers -- ``pack_bits`` (fallback.py:32-47), ``unpack_bits``
  (fallback.py:50-54), ``apply_bits`` with the GPU backend's select
  (cuda.py:158-178: a cleared bit gives +0, not ``value * 0``);
* masked forwards and backwards -- ``_MaskedFn`` (nn.py:116-136),
  ``_PiecewiseFn`` (nn.py:139-187), ``_LeakyFn`` (nn.py:267-282),
  ``_DropoutFn`` backward (nn.py:364-368);
* smooth activations -- the derivative table (nn.py:392-481) and the row
  quantization of ``_SmoothFn`` (nn.py:487-507), ``_ReluSquareFn``
  (nn.py:315-330) and ``_AnyElementwiseFn`` (nn.py:531-555).

Arithmetic is fp32 operation by operation in the order the reference's
tensor expressions evaluate (Python scalars become fp32 operands), with a
rounding to the tensor dtype wherever the reference's expression yields a
tensor of that dtype.  Transcendental functions (exp, erf, tanh, log1p,
expm1) are evaluated in float64 and rounded once to fp32, i.e. correctly
rounded in all but rare ties; torch's and the GPU's fp32 versions are within
an ulp or two of that, so the int8 derivative payloads are compared with a
one-step band at rounding ties, not bit for bit.

What pins each function (``tests/test_oracle_activations.py``): bits against
``np.packbits(bitorder="little")`` and per-bit brute force; masked values and
gradients against torch's own ``F.relu``/``relu6``/``hardtanh``/``leaky_relu``/
``hardsigmoid`` and their autograd, bit for bit; every derivative against
float64 autograd of torch's activation (tight relative bound); the
quantization against its closed form (scale = row max / 127, |payload| <= 127,
|payload * scale - d| <= scale / 2, half-even ties) and a planted mistake.
"""

from __future__ import annotations

import math

import numpy as np

try:  # scipy's erf in float64; math.erf elementwise otherwise
    from scipy.special import erf as _erf64
except Exception:  # pragma: no cover
    _erf64 = np.vectorize(math.erf, otypes=[np.float64])

F32 = np.float32


# ---------------------------------------------------------------------------
# dtype rounding (the tensor dtypes of the reference's expressions)
# ---------------------------------------------------------------------------


def round_bf16(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 -> fp32, round to nearest even; NaN stays NaN."""

    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).copy()
    nan = np.isnan(a)
    out[nan] = a[nan]
    return out


def round_dtype(a: np.ndarray, dtype: str) -> np.ndarray:
    a = np.asarray(a, dtype=np.float32)
    if dtype == "float32":
        return a
    if dtype == "bfloat16":
        return round_bf16(a)
    if dtype == "float16":
        return a.astype(np.float16).astype(np.float32)
    raise ValueError(dtype)


def _t(fn, a: np.ndarray) -> np.ndarray:
    """A transcendental in float64, rounded once to fp32."""

    with np.errstate(all="ignore"):
        return fn(np.asarray(a, dtype=np.float64)).astype(np.float32)


def _s(v: float) -> np.float32:
    """A Python scalar as the fp32 operand torch makes of it."""

    return np.float32(v)


# ---------------------------------------------------------------------------
# bits
# ---------------------------------------------------------------------------


def pack_bits(mask: np.ndarray) -> np.ndarray:
    """One bit per element, LSB first, pad bits zero (fallback.py:32-47)."""

    mask = np.asarray(mask) != 0
    rows, cols = mask.shape
    out = np.zeros((rows, (cols + 7) // 8), dtype=np.uint8)
    for shift in range(8):
        lane = mask[:, shift::8]
        out[:, : lane.shape[1]] |= lane.astype(np.uint8) << shift
    return out


def unpack_bits(packed: np.ndarray, cols: int) -> np.ndarray:
    """0/1 per element, pad columns dropped (fallback.py:50-54)."""

    shifts = np.arange(8, dtype=np.uint8)
    bits = (packed[:, :, None] >> shifts) & 1
    return bits.reshape(packed.shape[0], -1)[:, :cols].astype(np.uint8)


def masked_backward(grad: np.ndarray, packed: np.ndarray, inside: float, outside: float,
                    dtype: str = "float32") -> np.ndarray:
    """kept = bit ? grad : +0; kept * inside, or grad * outside + kept * (inside - outside)."""

    grad = np.asarray(grad, dtype=np.float32)
    keep = unpack_bits(packed, grad.shape[1]).astype(bool)
    kept = np.where(keep, grad, np.float32(0.0))
    with np.errstate(all="ignore"):
        if outside == 0.0:
            return round_dtype(kept * _s(inside), dtype)
        first = round_dtype(grad * _s(outside), dtype)
        second = round_dtype(kept * _s(inside - outside), dtype)
        return round_dtype(first + second, dtype)


def apply_bits(values: np.ndarray, packed: np.ndarray, dtype: str = "float32") -> np.ndarray:
    return masked_backward(values, packed, 1.0, 0.0, dtype)


# ---------------------------------------------------------------------------
# masked forwards
# ---------------------------------------------------------------------------


def clamp_forward(x: np.ndarray, lower: float, upper: float | None,
                  dtype: str = "float32") -> tuple[np.ndarray, np.ndarray]:
    """clamp_max(upper) then clamp_min(lower); bit = lower < out (< upper) (nn.py:119-131)."""

    x = np.asarray(x, dtype=np.float32)
    lo = round_dtype(np.float32(lower), dtype)
    out = x.copy()
    if upper is not None:
        hi = round_dtype(np.float32(upper), dtype)
        out = np.where(out > np.float32(upper), hi, out)
    out = np.where(out < np.float32(lower), lo, out)
    keep = out > lo
    if upper is not None:
        keep &= out < hi
    return out.astype(np.float32), pack_bits(keep)


def leaky_forward(x: np.ndarray, slope: float, dtype: str = "float32") -> tuple[np.ndarray, np.ndarray]:
    """x > 0 ? x : x * slope; bit = x > 0 (nn.py:271-276)."""

    x = np.asarray(x, dtype=np.float32)
    keep = x > 0
    out = np.where(keep, x, round_dtype(x * _s(slope), dtype))
    return out.astype(np.float32), pack_bits(keep)


def interval_bits(x: np.ndarray, lower: float, upper: float | None, dtype: str = "float32") -> np.ndarray:
    """bit = lower < x (< upper) (nn.py:159-162)."""

    x = np.asarray(x, dtype=np.float32)
    keep = x > round_dtype(np.float32(lower), dtype)
    if upper is not None:
        keep &= x < round_dtype(np.float32(upper), dtype)
    return pack_bits(keep)


# ---------------------------------------------------------------------------
# smooth activations
# ---------------------------------------------------------------------------

_SQRT_2 = math.sqrt(2.0)
_SQRT_2_OVER_PI = math.sqrt(2.0 / math.pi)
_INV_SQRT_2PI = 1.0 / math.sqrt(2.0 * math.pi)
_TANH_COEFFICIENT = 0.044715
_SELU_ALPHA = 1.6732632423543772
_SELU_SCALE = 1.0507009873554805


def _sigmoid(x: np.ndarray) -> np.ndarray:
    e = _t(np.exp, -x)
    return (F32(1.0) / (F32(1.0) + e)).astype(np.float32)


def _softplus(x: np.ndarray, beta: float) -> np.ndarray:
    bx = x * _s(beta)
    return np.where(bx > F32(20.0), x, _t(np.log1p, _t(np.exp, bx)) / _s(beta)).astype(np.float32)


def value(kind: str, x: np.ndarray, param: float = 0.0) -> np.ndarray:
    """f(x) in fp32 (torch's formula for each activation, before the dtype rounding)."""

    x = np.asarray(x, dtype=np.float32)
    with np.errstate(all="ignore"):
        if kind == "gelu":
            return x * F32(0.5) * (F32(1.0) + _t(_erf64, x * _s(1.0 / _SQRT_2)))
        if kind == "gelu_tanh":
            beta = _s(_SQRT_2 * (2.0 / math.sqrt(math.pi)) * 0.5)
            cube = x * x * x
            inner = beta * (x + _s(_TANH_COEFFICIENT) * cube)
            return F32(0.5) * x * (F32(1.0) + _t(np.tanh, inner))
        if kind == "silu":
            return x / (F32(1.0) + _t(np.exp, -x))
        if kind == "tanh":
            return _t(np.tanh, x)
        if kind == "sigmoid":
            return _sigmoid(x)
        if kind == "elu":
            return np.where(x <= 0, _t(np.expm1, x) * _s(param), x).astype(np.float32)
        if kind == "celu":
            return np.where(x <= 0, _t(np.expm1, x * (F32(1.0) / _s(param))) * _s(param), x).astype(np.float32)
        if kind == "selu":
            scale = _s(_SELU_SCALE)
            return np.where(x <= 0, _t(np.expm1, x) * (_s(_SELU_ALPHA) * scale), x * scale).astype(np.float32)
        if kind == "softplus":
            return _softplus(x, param)
        if kind == "mish":
            return x * _t(np.tanh, _t(np.log1p, _t(np.exp, x)))
        if kind == "hardswish":
            return x * np.minimum(np.maximum(x + F32(3.0), F32(0.0)), F32(6.0)) / F32(6.0)
        if kind == "relu_square":
            a = np.maximum(x, F32(0.0))
            return a * a
    raise ValueError(kind)


def derivative(kind: str, x: np.ndarray, y: np.ndarray, param: float = 0.0) -> np.ndarray:
    """The retained derivative (nn.py:392-481) from x and y = f(x) as a dtype tensor."""

    x = np.asarray(x, dtype=np.float32)
    y = np.asarray(y, dtype=np.float32)
    one = F32(1.0)
    with np.errstate(all="ignore"):
        if kind == "gelu":
            cumulative = F32(0.5) * (one + _t(_erf64, x / _s(_SQRT_2)))
            e = _t(np.exp, F32(-0.5) * x * x)
            return cumulative + x * e * _s(_INV_SQRT_2PI)
        if kind == "gelu_tanh":
            s = _s(_SQRT_2_OVER_PI)
            cube = x * x * x
            inner = s * (x + _s(_TANH_COEFFICIENT) * cube)
            t = _t(np.tanh, inner)
            left = F32(0.5) * (one + t)
            right = F32(0.5) * x * (one - t * t) * s * (one + _s(3.0 * _TANH_COEFFICIENT) * x * x)
            return left + right
        if kind == "silu":
            s = _sigmoid(x)
            return s * (one + x * (one - s))
        if kind == "tanh":
            return one - y * y
        if kind == "sigmoid":
            return y * (one - y)
        if kind == "elu":
            return np.where(x > 0, one, y + _s(param)).astype(np.float32)
        if kind == "celu":
            return np.where(x > 0, one, y / _s(param) + one).astype(np.float32)
        if kind == "selu":
            return np.where(x > 0, _s(_SELU_SCALE), y + _s(_SELU_SCALE * _SELU_ALPHA)).astype(np.float32)
        if kind == "softplus":
            return _sigmoid(_s(param) * x)
        if kind == "mish":
            t = _t(np.tanh, _softplus(x, 1.0))
            return t + x * (one - t * t) * _sigmoid(x)
        if kind == "hardswish":
            inner = (F32(2.0) * x + F32(3.0)) / F32(6.0)
            return np.where(x <= -3.0, F32(0.0), np.where(x >= 3.0, one, inner)).astype(np.float32)
        if kind == "relu_square":
            return np.maximum(x, F32(0.0))
    raise ValueError(kind)


def quantize_rows(d: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """scale = max(amax |d|, 1e-8) / 127; payload = clamp(rne(d / scale), +-127) (nn.py:495-497)."""

    d = np.asarray(d, dtype=np.float32)
    amax = np.abs(d).max(axis=1) if d.shape[1] else np.zeros(d.shape[0], np.float32)
    scale = (np.maximum(amax, F32(1e-8)) / F32(127.0)).astype(np.float32)
    with np.errstate(all="ignore"):
        q = np.rint(d / scale[:, None])
    return np.clip(q, -127, 127).astype(np.int8), scale


def quantize_rows_unsigned(a: np.ndarray, dtype: str) -> tuple[np.ndarray, np.ndarray]:
    """relu(x)^2's retained byte: the same against max / 255, in the dtype (nn.py:316-318)."""

    a = np.asarray(a, dtype=np.float32)
    amax = a.max(axis=1) if a.shape[1] else np.zeros(a.shape[0], np.float32)
    scale = round_dtype(round_dtype(np.maximum(amax, F32(1e-8)), dtype) / F32(255.0), dtype)
    with np.errstate(all="ignore"):
        q = np.rint(round_dtype(a / scale[:, None], dtype))
        q = np.nan_to_num(np.clip(q, 0, 255), nan=0.0)
    return q.astype(np.uint8), scale


def smooth_forward(kind: str, x: np.ndarray, param: float = 0.0, dtype: str = "float32",
                   y: np.ndarray | None = None):
    """(y, payload, scale) of a smooth activation on rows x (fp32 values of the dtype)."""

    x = np.asarray(x, dtype=np.float32)
    if y is None:
        y = round_dtype(value(kind, x, param), dtype)
    d = derivative(kind, x, y, param)
    if kind == "relu_square":
        payload, scale = quantize_rows_unsigned(round_dtype(d, dtype), dtype)
    else:
        payload, scale = quantize_rows(d)
    return y, payload, scale


def smooth_backward(grad: np.ndarray, payload: np.ndarray, scale: np.ndarray,
                    dtype: str = "float32") -> np.ndarray:
    """grad * (payload * scale), or grad * 2 * (payload * scale) for a uint8 payload."""

    grad = np.asarray(grad, dtype=np.float32)
    s = round_dtype(np.asarray(scale, dtype=np.float32), dtype)[:, None]
    with np.errstate(all="ignore"):
        d = round_dtype(payload.astype(np.float32) * s, dtype)
        if payload.dtype == np.uint8:
            return round_dtype(round_dtype(grad * F32(2.0), dtype) * d, dtype)
        return round_dtype(grad * d, dtype)


def tie_margin(d: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Distance of d / scale from the nearest half-integer (the rounding ties)."""

    with np.errstate(all="ignore"):
        r = np.asarray(d, dtype=np.float64) / np.asarray(scale, dtype=np.float64)[:, None]
    return np.abs(np.abs(r - np.floor(r)) - 0.5)
