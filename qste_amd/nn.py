"""Packed activations: backward keeps bits or bytes of an activation, not floats.

Drop-in for the reference's ``qste.nn`` (``src/qste/nn.py``): the same
functions, modules, replacement tables and ``packed_activations()`` context,
with the forward and the retained tape produced by HIP kernels
(``csrc/activation.hip``) in one pass over the input:

    ReLU, ReLU6, Hardtanh, LeakyReLU, Hardsigmoid, Dropout   one bit per element
    GELU, SiLU, Tanh, Sigmoid, ELU, CELU, SELU, Softplus,
    Mish, Hardswish, any elementwise function                int8 derivative, fp32 scale per row
    relu(x) ** 2                                             uint8 of relu(x), scale per row

Rows are the last dimension (``_flatten``), as in the reference.  Tensors
must be on the GPU; a CPU tensor raises, as every ``qste_amd`` operator does.
"""

from __future__ import annotations

from contextlib import contextmanager

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor
from torch.autograd import Function

from . import kernels
from .functional import swiglu

# The originals, bound before ``packed_activations`` can patch them: the
# wrappers call these for values the kernels do not produce, and a patched
# name would call the wrapper back.
_TORCH_RELU = F.relu
_TORCH_RELU6 = F.relu6
_TORCH_GELU = F.gelu
_TORCH_SILU = F.silu
_TORCH_LEAKY_RELU = F.leaky_relu
_TORCH_HARDTANH = F.hardtanh
_TORCH_HARDSIGMOID = F.hardsigmoid
_TORCH_HARDSWISH = F.hardswish
_TORCH_ELU = F.elu
_TORCH_SELU = F.selu
_TORCH_CELU = F.celu
_TORCH_SOFTPLUS = F.softplus
_TORCH_MISH = F.mish
_TORCH_DROPOUT = F.dropout
_TORCH_TORCH_RELU = torch.relu

_KERNEL_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _flatten(value: Tensor) -> tuple[Tensor, tuple[int, ...], int]:
    """Rank-2 view over the last dimension (a scalar is one 1x1 row)."""

    if value.ndim == 0:
        return value.reshape(1, 1).contiguous(), value.shape, 1
    if value.ndim == 1:
        return value.reshape(1, -1).contiguous(), value.shape, value.shape[0]
    columns = value.shape[-1]
    return value.reshape(-1, columns).contiguous(), value.shape, columns


def _mark_activation_input(value: Tensor) -> Tensor:
    """Tag a converted layer's output so ``packed_activations`` packs what follows."""

    value._qste_activation_input = True
    return value


def _take_activation_input(value: Tensor) -> Tensor | None:
    return value if getattr(value, "_qste_activation_input", False) else None


def swiglu_mlp(inputs: Tensor, gate, up, down) -> Tensor:
    """``down(swiglu(gate(inputs), up(inputs)))`` for three converted layers
    (QSTELinear: gate and up d -> ffn, down ffn -> d).

    No counterpart in the reference.  Same forward values, evidence and
    scale gradients as the three layers and the gate called one by one; for
    bf16 inputs on the GPU with d and ffn multiples of 64 the whole MLP is
    one autograd node whose input gradient is one product over the gate and
    up layers, rounded once (``functional.SwiGLUMLPFn``).  Anything else is
    the layer-by-layer composition."""

    from .functional import SwiGLUMLPFn, _autocast, swiglu_mlp_fusable

    x = _autocast(inputs)
    if not swiglu_mlp_fusable(x, gate, up, down):
        return down(swiglu(gate(inputs), up(inputs)))
    surfaces = (gate.surface, up.surface, down.surface)
    for s in surfaces:
        s.note_forward()
    y = SwiGLUMLPFn.apply(x, gate.surface.packed_sign, gate.surface.log_scale, gate.bias, up.surface.packed_sign,
                          up.surface.log_scale, up.bias, down.surface.packed_sign, down.surface.log_scale, down.bias,
                          surfaces, torch.is_grad_enabled())
    return _mark_activation_input(y)


# ---------------------------------------------------------------------------
# One bit per element
# ---------------------------------------------------------------------------


def _masked_grad(grad_output: Tensor, packed: Tensor, ctx, inside: float, outside: float) -> Tensor:
    flat = grad_output.reshape(-1, ctx.columns)
    if flat.dtype in _KERNEL_DTYPES:
        out = kernels.masked_backward(flat, packed, ctx.columns, inside=inside, outside=outside)
        return out.view(ctx.shape)
    # dtypes the kernels do not take: the reference's own expression on the GPU
    kept = flat * kernels.unpack_bits(packed, ctx.columns, dtype=flat.dtype)
    if outside == 0.0:
        return (kept * inside).view(ctx.shape)
    return (flat * outside + kept * (inside - outside)).view(ctx.shape)


class _MaskedFn(Function):
    """Clamp family (ReLU, ReLU6, Hardtanh): nn.py:116-136.

    Keeps ``lower < out < upper`` -- strictly, so an element sitting on a
    clamp gets no gradient.
    """

    @staticmethod
    def forward(ctx, inputs, lower, upper):
        flat, shape, columns = _flatten(inputs)
        if flat.dtype in _KERNEL_DTYPES:
            out, packed = kernels.masked_activation(flat, kernels.MASK_CLAMP, lower=lower, upper=upper)
            output = out.view(shape)
        else:
            output = inputs if upper is None else inputs.clamp_max(upper)
            output = output.clamp_min(lower)
            kept = output.reshape(-1, columns)
            keep = kept > lower if upper is None else (kept > lower) & (kept < upper)
            packed = kernels.pack_bits(keep)
        ctx.save_for_backward(packed)
        ctx.shape, ctx.columns = shape, columns
        return output

    @staticmethod
    def backward(ctx, grad_output):
        (packed,) = ctx.saved_tensors
        return _masked_grad(grad_output, packed, ctx, 1.0, 0.0), None, None


class _PiecewiseFn(Function):
    """Piecewise-linear activations whose value is not the clamped input (nn.py:139-187).

    One bit (strictly inside the interval) plus the two slopes from a table.
    """

    @staticmethod
    def forward(ctx, inputs, kind, lower, upper):
        forward, inside_slope, outside_slope = _PIECEWISE[kind]
        output = forward(inputs)
        flat, shape, columns = _flatten(inputs)
        if flat.dtype in _KERNEL_DTYPES:
            _, packed = kernels.masked_activation(flat, kernels.MASK_INTERVAL, lower=lower, upper=upper,
                                                  want_output=False)
        else:
            inside = flat > lower
            if upper is not None:
                inside = inside & (flat < upper)
            packed = kernels.pack_bits(inside)
        ctx.save_for_backward(packed)
        ctx.shape, ctx.columns = shape, columns
        ctx.slopes = (inside_slope, outside_slope)
        return output

    @staticmethod
    def backward(ctx, grad_output):
        (packed,) = ctx.saved_tensors
        inside, outside = ctx.slopes
        return _masked_grad(grad_output, packed, ctx, inside, outside), None, None, None


_PIECEWISE: dict[str, tuple] = {
    "hardsigmoid": (lambda x: _TORCH_HARDSIGMOID(x), 1.0 / 6.0, 0.0),
}


class _LeakyFn(Function):
    """LeakyReLU: bit = x > 0; below the knee the gradient is the slope (nn.py:267-282)."""

    @staticmethod
    def forward(ctx, inputs, negative_slope):
        flat, shape, columns = _flatten(inputs)
        if flat.dtype in _KERNEL_DTYPES:
            out, packed = kernels.masked_activation(flat, kernels.MASK_LEAKY, slope=negative_slope)
            output = out.view(shape)
        else:
            packed = kernels.pack_bits(flat > 0)
            output = _TORCH_LEAKY_RELU(inputs, negative_slope, False)
        ctx.save_for_backward(packed)
        ctx.shape, ctx.columns, ctx.slope = shape, columns, negative_slope
        return output

    @staticmethod
    def backward(ctx, grad_output):
        (packed,) = ctx.saved_tensors
        return _masked_grad(grad_output, packed, ctx, 1.0, ctx.slope), None


class _DropoutFn(Function):
    """Dropout keeping its mask as bits (nn.py:352-368); the mask is torch's RNG draw."""

    @staticmethod
    def forward(ctx, inputs, probability):
        keep = torch.rand_like(inputs, dtype=torch.float32) >= probability
        flat, shape, columns = _flatten(keep)
        ctx.save_for_backward(kernels.pack_bits(flat))
        ctx.shape, ctx.columns = shape, columns
        ctx.gain = 1.0 / (1.0 - probability)
        return inputs * keep.to(inputs.dtype) * ctx.gain

    @staticmethod
    def backward(ctx, grad_output):
        (packed,) = ctx.saved_tensors
        return _masked_grad(grad_output, packed, ctx, ctx.gain, 0.0), None


def relu(inputs: Tensor) -> Tensor:
    """``F.relu`` retaining one bit per element; squaring the result fuses."""

    return _FusableReLU(_MaskedFn.apply(inputs, 0.0, None), inputs)


def relu6(inputs: Tensor) -> Tensor:
    return _MaskedFn.apply(inputs, 0.0, 6.0)


def leaky_relu(inputs: Tensor, negative_slope: float = 0.01, inplace: bool = False) -> Tensor:
    if inplace:  # an in-place op cannot retain what it overwrites
        return _TORCH_LEAKY_RELU(inputs, negative_slope, True)
    return _LeakyFn.apply(inputs, negative_slope)


def hardtanh(inputs: Tensor, min_val: float = -1.0, max_val: float = 1.0,
             inplace: bool = False) -> Tensor:
    if inplace:
        return _TORCH_HARDTANH(inputs, min_val, max_val, True)
    return _MaskedFn.apply(inputs, min_val, max_val)


def hardsigmoid(inputs: Tensor, inplace: bool = False) -> Tensor:
    if inplace:
        return _TORCH_HARDSIGMOID(inputs, True)
    return _PiecewiseFn.apply(inputs, "hardsigmoid", -3.0, 3.0)


def dropout(inputs: Tensor, p: float = 0.5, training: bool = True) -> Tensor:
    """``F.dropout`` keeping the mask as bits rather than bytes."""

    if not training or p == 0.0:
        return inputs
    if not 0.0 <= p < 1.0:
        raise ValueError("dropout probability must be in [0, 1)")
    return _DropoutFn.apply(inputs, p)


# ---------------------------------------------------------------------------
# relu(x) ** 2: one unsigned byte per element (nn.py:292-343)
# ---------------------------------------------------------------------------


class _ReluSquareFn(Function):
    """``relu(x) ** 2`` retaining ``relu(x)`` as a uint8 against its row maximum / 255."""

    @staticmethod
    def forward(ctx, inputs):
        flat, shape, columns = _flatten(inputs)
        if flat.dtype in _KERNEL_DTYPES:
            out, payload, scale = kernels.smooth_activation(flat, "relu_square")
            output = out.view(shape)
        else:
            activated = flat.clamp_min(0)
            scale = activated.amax(dim=1).clamp_min(1e-8).div_(255.0)
            payload = activated.div(scale.unsqueeze(1)).round_().clamp_(0, 255).to(torch.uint8)
            output = (activated * activated).view(shape)
        ctx.save_for_backward(payload, scale)
        ctx.shape, ctx.columns = shape, columns
        return output

    @staticmethod
    def backward(ctx, grad_output):
        payload, scale = ctx.saved_tensors
        return _dequantized_grad(grad_output, payload, scale, ctx, squared=True)


def relu_square(inputs: Tensor) -> Tensor:
    """``relu(x) ** 2`` as one op, retaining a byte per element."""

    return _ReluSquareFn.apply(inputs)


class _FusableReLU(Tensor):
    """A ReLU output that fuses with a following square (nn.py:190-247).

    Squaring it (``.square()``, ``torch.square``, ``** 2``) runs
    ``_ReluSquareFn`` on the pre-activation; every other operation sees the
    plain tensor ReLU returned, and returns plain tensors, so the subclass
    never spreads.  It pickles as an ordinary tensor.
    """

    @staticmethod
    def __new__(cls, data: Tensor, pre_activation: Tensor):
        held = data.as_subclass(cls)
        held._pre_activation = pre_activation
        return held

    def __reduce_ex__(self, protocol):
        with torch._C.DisableTorchFunctionSubclass():
            return self.as_subclass(Tensor).__reduce_ex__(protocol)

    def plain(self) -> Tensor:
        with torch._C.DisableTorchFunctionSubclass():
            return self.as_subclass(Tensor)

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = {} if kwargs is None else kwargs
        held = args[0] if args else None
        pre = getattr(held, "_pre_activation", None) if isinstance(held, cls) else None
        if pre is not None and not kwargs:
            if func in (Tensor.square, torch.square) and len(args) == 1:
                return _ReluSquareFn.apply(pre)
            if func is Tensor.__pow__ and len(args) == 2 and args[1] == 2:
                return _ReluSquareFn.apply(pre)
        with torch._C.DisableTorchFunctionSubclass():
            return func(*args, **kwargs)


# ---------------------------------------------------------------------------
# Smooth: the derivative as int8 against a per-row maximum (nn.py:385-507)
# ---------------------------------------------------------------------------

# kind -> (torch forward(x, param), kernel kind for (param)).  The forward is
# what the value must equal; the kernel computes value and derivative in one
# pass where its value is torch's bit for bit (_KERNEL_VALUE), and otherwise
# reads torch's value to derive from.
_SMOOTH: dict[str, object] = {
    "gelu": lambda x, a: _TORCH_GELU(x, approximate=a),
    "silu": lambda x, a: _TORCH_SILU(x),
    "tanh": lambda x, a: torch.tanh(x),
    "sigmoid": lambda x, a: torch.sigmoid(x),
    "elu": lambda x, a: _TORCH_ELU(x, a),
    "celu": lambda x, a: _TORCH_CELU(x, a),
    "selu": lambda x, a: _TORCH_SELU(x),
    "softplus": lambda x, a: _TORCH_SOFTPLUS(x, a),
    "mish": lambda x, a: _TORCH_MISH(x),
    "hardswish": lambda x, a: _TORCH_HARDSWISH(x),
}

# (kind, dtype) pairs whose kernel value equals torch's on the GPU (checked by
# tests/test_gpu_activations.py); the rest take torch's value and the kernel
# derives from it.  torch evaluates tanh-GELU and Hardswish in fp32 with a
# different operation order (1-ulp differences in fp32 on ~0.4% / ~27% of
# inputs), which a bf16/fp16 rounding hides only most of the time, so both
# take torch's value in every dtype.
_KERNEL_VALUE: set[tuple[str, torch.dtype]] = {
    (k, d) for k in ("gelu", "silu", "tanh", "sigmoid", "elu", "celu", "selu", "softplus", "mish")
    for d in _KERNEL_DTYPES
}


def _kernel_kind(kind: str, param) -> tuple[str, float]:
    if kind == "gelu":
        return ("gelu_tanh" if param == "tanh" else "gelu"), 0.0
    if kind in ("elu", "celu", "softplus"):
        return kind, float(param)
    return kind, 0.0


def _dequantized_grad(grad_output: Tensor, payload: Tensor, scale: Tensor, ctx, squared: bool = False):
    flat = grad_output.reshape(-1, ctx.columns)
    if flat.dtype in _KERNEL_DTYPES:
        return kernels.smooth_backward(flat, payload, scale).view(ctx.shape), None
    factor = payload.to(flat.dtype).mul_(scale.to(flat.dtype).unsqueeze(1))
    if squared:
        return (flat * 2.0 * factor).view(ctx.shape), None
    return (flat * factor).view(ctx.shape), None


class _SmoothFn(Function):
    """Smooth activation retaining its derivative as int8 with a per-row scale."""

    @staticmethod
    def forward(ctx, inputs, kind, param):
        forward = _SMOOTH.get(kind)
        if forward is None:  # pragma: no cover - guarded by the public wrappers
            raise ValueError(f"unknown smooth activation {kind!r}")
        kernel_kind, kernel_param = _kernel_kind(kind, param)
        flat, shape, columns = _flatten(inputs)
        if flat.dtype in _KERNEL_DTYPES and (kernel_kind, flat.dtype) in _KERNEL_VALUE:
            out, payload, scale = kernels.smooth_activation(flat, kernel_kind, kernel_param)
            output = out.view(shape)
        else:
            output = forward(inputs, param)
            x32 = flat if flat.dtype in _KERNEL_DTYPES else flat.float()
            y32 = output.reshape(-1, columns)
            if y32.dtype != x32.dtype:
                y32 = y32.float()
                x32 = x32.float()
            _, payload, scale = kernels.smooth_activation(x32, kernel_kind, kernel_param, output=y32)
        ctx.save_for_backward(payload, scale)
        ctx.shape, ctx.columns = shape, columns
        return output

    @staticmethod
    def backward(ctx, grad_output):
        payload, scale = ctx.saved_tensors
        grad, _ = _dequantized_grad(grad_output, payload, scale, ctx)
        return grad, None, None


class _AnyElementwiseFn(Function):
    """Any elementwise ``f``: its derivative from one autograd probe, kept as int8 (nn.py:510-555)."""

    @staticmethod
    def forward(ctx, inputs, function):
        with torch.enable_grad():
            probe = inputs.detach().requires_grad_(True)
            output = function(probe)
            if output.shape != probe.shape:
                raise ValueError(
                    "qste.nn.packed() needs an elementwise function; this one "
                    f"maps {tuple(probe.shape)} to {tuple(output.shape)}")
            (derivative,) = torch.autograd.grad(output.sum(), probe)
        flat, shape, columns = _flatten(derivative.float())
        _, payload, scale = kernels.smooth_activation(None, "provided", derivative=flat)
        ctx.save_for_backward(payload, scale)
        ctx.shape, ctx.columns = shape, columns
        return output.detach()

    @staticmethod
    def backward(ctx, grad_output):
        payload, scale = ctx.saved_tensors
        grad, _ = _dequantized_grad(grad_output, payload, scale, ctx)
        return grad, None


def elementwise(function, inputs: Tensor) -> Tensor:
    """``function(inputs)`` retaining a byte per element instead of a float."""

    return _AnyElementwiseFn.apply(inputs, function)


def packed(function):
    """``function`` wrapped so it retains a byte per element. Elementwise only."""

    def wrapper(inputs: Tensor) -> Tensor:
        return elementwise(function, inputs)

    wrapper.__name__ = getattr(function, "__name__", "packed")
    wrapper.__doc__ = f"Packed: {getattr(function, '__doc__', None) or function!r}"
    return wrapper


def gelu(inputs: Tensor, approximate: str = "none") -> Tensor:
    return _SmoothFn.apply(inputs, "gelu", approximate)


def silu(inputs: Tensor) -> Tensor:
    return _SmoothFn.apply(inputs, "silu", "none")


def tanh(inputs: Tensor) -> Tensor:
    return _SmoothFn.apply(inputs, "tanh", "none")


def sigmoid(inputs: Tensor) -> Tensor:
    return _SmoothFn.apply(inputs, "sigmoid", "none")


def elu(inputs: Tensor, alpha: float = 1.0, inplace: bool = False) -> Tensor:
    if inplace:
        return _TORCH_ELU(inputs, alpha, True)
    return _SmoothFn.apply(inputs, "elu", alpha)


def celu(inputs: Tensor, alpha: float = 1.0, inplace: bool = False) -> Tensor:
    if inplace:
        return _TORCH_CELU(inputs, alpha, True)
    return _SmoothFn.apply(inputs, "celu", alpha)


def selu(inputs: Tensor, inplace: bool = False) -> Tensor:
    if inplace:
        return _TORCH_SELU(inputs, True)
    return _SmoothFn.apply(inputs, "selu", 1.0)


def softplus(inputs: Tensor, beta: float = 1.0, threshold: float = 20.0) -> Tensor:
    # the reference's smooth softplus keeps torch's default threshold (nn.py:619-620)
    return _SmoothFn.apply(inputs, "softplus", beta)


def mish(inputs: Tensor, inplace: bool = False) -> Tensor:
    if inplace:
        return _TORCH_MISH(inputs, True)
    return _SmoothFn.apply(inputs, "mish", 1.0)


def hardswish(inputs: Tensor, inplace: bool = False) -> Tensor:
    if inplace:
        return _TORCH_HARDSWISH(inputs, True)
    return _SmoothFn.apply(inputs, "hardswish", 1.0)


# ---------------------------------------------------------------------------
# Modules, shaped like the ones they replace
# ---------------------------------------------------------------------------


class ReLU(nn.Module):
    def __init__(self, inplace: bool = False):
        super().__init__()
        self.inplace = False  # packing needs the input; in-place is not kept

    def forward(self, inputs: Tensor) -> Tensor:
        return relu(inputs)


class ReLU6(nn.Module):
    def __init__(self, inplace: bool = False):
        super().__init__()
        self.inplace = False

    def forward(self, inputs: Tensor) -> Tensor:
        return relu6(inputs)


class GELU(nn.Module):
    def __init__(self, approximate: str = "none"):
        super().__init__()
        self.approximate = approximate

    def forward(self, inputs: Tensor) -> Tensor:
        return gelu(inputs, self.approximate)

    def extra_repr(self) -> str:
        return f"approximate={self.approximate!r}"


class SiLU(nn.Module):
    def __init__(self, inplace: bool = False):
        super().__init__()
        self.inplace = False

    def forward(self, inputs: Tensor) -> Tensor:
        return silu(inputs)


class Tanh(nn.Module):
    def forward(self, inputs: Tensor) -> Tensor:
        return tanh(inputs)


class Sigmoid(nn.Module):
    def forward(self, inputs: Tensor) -> Tensor:
        return sigmoid(inputs)


class LeakyReLU(nn.Module):
    def __init__(self, negative_slope: float = 0.01):
        super().__init__()
        self.negative_slope = negative_slope

    def forward(self, inputs: Tensor) -> Tensor:
        return leaky_relu(inputs, self.negative_slope)


class Hardtanh(nn.Module):
    def __init__(self, min_val: float = -1.0, max_val: float = 1.0):
        super().__init__()
        self.min_val, self.max_val = min_val, max_val

    def forward(self, inputs: Tensor) -> Tensor:
        return hardtanh(inputs, self.min_val, self.max_val)


class Hardsigmoid(nn.Module):
    def forward(self, inputs: Tensor) -> Tensor:
        return hardsigmoid(inputs)


class ELU(nn.Module):
    def __init__(self, alpha: float = 1.0):
        super().__init__()
        self.alpha = alpha

    def forward(self, inputs: Tensor) -> Tensor:
        return elu(inputs, self.alpha)


class CELU(nn.Module):
    def __init__(self, alpha: float = 1.0):
        super().__init__()
        self.alpha = alpha

    def forward(self, inputs: Tensor) -> Tensor:
        return celu(inputs, self.alpha)


class SELU(nn.Module):
    def forward(self, inputs: Tensor) -> Tensor:
        return selu(inputs)


class Softplus(nn.Module):
    def __init__(self, beta: float = 1.0, threshold: float = 20.0):
        super().__init__()
        self.beta, self.threshold = beta, threshold

    def forward(self, inputs: Tensor) -> Tensor:
        return softplus(inputs, self.beta, self.threshold)


class Mish(nn.Module):
    def forward(self, inputs: Tensor) -> Tensor:
        return mish(inputs)


class Hardswish(nn.Module):
    def forward(self, inputs: Tensor) -> Tensor:
        return hardswish(inputs)


class Dropout(nn.Module):
    def __init__(self, p: float = 0.5, inplace: bool = False):
        super().__init__()
        self.p = p
        self.inplace = False

    def forward(self, inputs: Tensor) -> Tensor:
        return dropout(inputs, self.p, self.training)

    def extra_repr(self) -> str:
        return f"p={self.p}"


# Exact replacements change neither the value nor the gradient.
EXACT_REPLACEMENTS: dict[type, type] = {
    nn.ReLU: ReLU,
    nn.ReLU6: ReLU6,
    nn.LeakyReLU: LeakyReLU,
    nn.Hardtanh: Hardtanh,
    nn.Hardsigmoid: Hardsigmoid,
    nn.Dropout: Dropout,
}

# These quantize the retained derivative; the value is untouched.
SMOOTH_REPLACEMENTS: dict[type, type] = {
    nn.GELU: GELU,
    nn.SiLU: SiLU,
    nn.Tanh: Tanh,
    nn.Sigmoid: Sigmoid,
    nn.ELU: ELU,
    nn.CELU: CELU,
    nn.SELU: SELU,
    nn.Softplus: Softplus,
    nn.Mish: Mish,
    nn.Hardswish: Hardswish,
}

REPLACEMENTS: dict[type, type] = {**EXACT_REPLACEMENTS, **SMOOTH_REPLACEMENTS}


def replace(module: nn.Module) -> nn.Module | None:
    """A packed equivalent of ``module`` with its settings, or ``None``."""

    target = REPLACEMENTS.get(type(module))
    if target is None:
        return None
    if target is GELU:
        return GELU(getattr(module, "approximate", "none"))
    if target is Dropout:
        return Dropout(getattr(module, "p", 0.5))
    if target is LeakyReLU:
        return LeakyReLU(getattr(module, "negative_slope", 0.01))
    if target is Hardtanh:
        return Hardtanh(getattr(module, "min_val", -1.0), getattr(module, "max_val", 1.0))
    if target in (ELU, CELU):
        return target(getattr(module, "alpha", 1.0))
    if target is Softplus:
        return Softplus(getattr(module, "beta", 1.0), getattr(module, "threshold", 20.0))
    return target()


# ---------------------------------------------------------------------------
# Functional call sites (nn.py:803-932)
# ---------------------------------------------------------------------------


def _select_converted(original, replacement):
    """``replacement`` for a value a converted layer emitted; ``original`` otherwise."""

    def selected(inputs: Tensor, *args, **kwargs) -> Tensor:
        marked = _take_activation_input(inputs)
        if marked is None:
            return original(inputs, *args, **kwargs)
        return replacement(marked, *args, **kwargs)

    return selected


def _packed_relu(inputs: Tensor, inplace: bool = False) -> Tensor:
    return _TORCH_RELU(inputs, True) if inplace else relu(inputs)


def _packed_relu6(inputs: Tensor, inplace: bool = False) -> Tensor:
    return _TORCH_RELU6(inputs, True) if inplace else relu6(inputs)


def _packed_silu(inputs: Tensor, inplace: bool = False) -> Tensor:
    return _TORCH_SILU(inputs, True) if inplace else silu(inputs)


def _packed_dropout(inputs: Tensor, p: float = 0.5, training: bool = True,
                    inplace: bool = False) -> Tensor:
    return _TORCH_DROPOUT(inputs, p, training, True) if inplace else dropout(inputs, p, training)


_PATCHES = (
    (F, "relu", _select_converted(_TORCH_RELU, _packed_relu)),
    (F, "relu6", _select_converted(_TORCH_RELU6, _packed_relu6)),
    (F, "leaky_relu", _select_converted(_TORCH_LEAKY_RELU, leaky_relu)),
    (F, "hardtanh", _select_converted(_TORCH_HARDTANH, hardtanh)),
    (F, "hardsigmoid", _select_converted(_TORCH_HARDSIGMOID, hardsigmoid)),
    (torch, "relu", _select_converted(_TORCH_TORCH_RELU, relu)),
    (F, "gelu", _select_converted(_TORCH_GELU, gelu)),
    (F, "silu", _select_converted(_TORCH_SILU, _packed_silu)),
    (F, "elu", _select_converted(_TORCH_ELU, elu)),
    (F, "celu", _select_converted(_TORCH_CELU, celu)),
    (F, "selu", _select_converted(_TORCH_SELU, selu)),
    (F, "softplus", _select_converted(_TORCH_SOFTPLUS, softplus)),
    (F, "mish", _select_converted(_TORCH_MISH, mish)),
    (F, "hardswish", _select_converted(_TORCH_HARDSWISH, hardswish)),
    (F, "dropout", _select_converted(_TORCH_DROPOUT, _packed_dropout)),
)


@contextmanager
def packed_activations():
    """Pack functional activations that directly follow converted QSTE layers.

    Inside the context ``F.relu`` / ``F.gelu`` / ``F.silu`` / ... pack when
    their input was emitted by a ``QSTELinear`` and are torch's own otherwise.
    The patch is restored on exit, exceptions included.
    """

    saved = [(owner, name, getattr(owner, name)) for owner, name, _ in _PATCHES]
    for owner, name, replacement in _PATCHES:
        setattr(owner, name, replacement)
    try:
        yield
    finally:
        for owner, name, original in saved:
            setattr(owner, name, original)


__all__ = [
    "CELU", "Dropout", "ELU", "EXACT_REPLACEMENTS", "GELU", "Hardsigmoid", "Hardswish", "Hardtanh",
    "LeakyReLU", "Mish", "REPLACEMENTS", "ReLU", "ReLU6", "SELU", "SMOOTH_REPLACEMENTS", "SiLU",
    "Sigmoid", "Softplus", "Tanh", "celu", "dropout", "elementwise", "elu", "gelu", "hardsigmoid", "swiglu", "swiglu_mlp",
    "hardswish", "hardtanh", "leaky_relu", "mish", "packed", "packed_activations", "relu",
    "relu6", "relu_square", "replace", "selu", "sigmoid", "silu", "softplus", "tanh",
]
