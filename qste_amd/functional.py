"""Autograd for binary linear layers on the gfx950 kernels.

Forward (``QSTELinearFn``, reference ``src/qste/functional.py:153-171``):
``y = (x @ sign^T) * scale + bias`` and, for backward, the input kept as one
bit per element plus two floats per sample (``encode_activation``,
functional.py:98-115): ``x ~ offset + xscale * sign(x - offset)``.

Backward (functional.py:173-194) is one library call, ``linear_backward``:
the input gradient, the decoded evidence with its rank-one offset correction,
the scale gradient, the evidence times the row scale, and the bias gradient.
The evidence goes to the surface -- usually straight into the coordinate step,
inside ``loss.backward()``.
"""

from __future__ import annotations

import weakref

import torch
from torch import Tensor
from torch.autograd import Function

from . import kernels
from .surface import Surface


def _autocast(value: Tensor) -> Tensor:
    """Cast like autocast would cast a native GEMM input (functional.py:39-53)."""

    device = value.device.type
    if device not in ("cuda", "cpu") or not torch.is_autocast_enabled(device):
        return value
    return value.to(dtype=torch.get_autocast_dtype(device))


def encode_activation(flat: Tensor) -> tuple[Tensor, Tensor]:
    """``(bits, aux)`` with ``aux = stack(offset, scale)`` fp32 [2, samples]."""

    packed, offset, scale = kernels.pack_affine_rows(flat)
    return packed, kernels.stacked_pair(offset, scale)


# Layers that read the same input in one forward (a SwiGLU's gate and up
# projections) share its encoding: the last input encoded, held weakly, with
# its version counter and address.  Any backward clears it, so a reuse never
# spans a training step.
_last_encoding: tuple | None = None


def _encoding_of(inputs: Tensor, flat: Tensor, columns: int) -> tuple[Tensor, Tensor]:
    global _last_encoding
    key = (inputs._version, inputs.data_ptr(), tuple(inputs.shape), inputs.dtype, columns)
    if _last_encoding is not None:
        ref, last_key, payload, aux = _last_encoding
        if ref() is inputs and last_key == key:
            return payload, aux
    payload, aux = encode_activation(flat)
    _last_encoding = (weakref.ref(inputs), key, payload, aux)
    return payload, aux


def forget_encodings() -> None:
    global _last_encoding
    _last_encoding = None


def remember_encoding(value: Tensor, payload: Tensor, aux: Tensor) -> None:
    """Offer ``value``'s encoding (over its last dimension) to the next binary
    layer that reads ``value``, as if that layer had encoded it itself."""

    global _last_encoding
    columns = int(value.shape[-1])
    key = (value._version, value.data_ptr(), tuple(value.shape), value.dtype, columns)
    _last_encoding = (weakref.ref(value), key, payload, aux)


# A binary layer's output carries, as an attribute, the encoding aux of the
# input it was computed from: a SwiGLU gate that reads two such outputs sums
# its gradients against those inputs' offsets while it writes them
# (swiglu_backward_sums), and offers each sum to the layer whose output it
# was.  An offer names the gradient tensor it belongs to (held, with its
# version) and the aux it was summed against; a layer takes it only when
# autograd hands it exactly that gradient, unchanged, and it saved that aux.
# Offers live for one backward pass: one that no layer took (a gradient that
# autograd summed with another use of the same output) is dropped when the
# pass ends, so it holds no gradient past it.
_AUX_ATTR = "_qste_input_aux"
_offers: dict[int, tuple] = {}


def _offer_offset_dot(grad: Tensor, aux: Tensor, offset_dot: Tensor) -> None:
    _offers[grad.data_ptr()] = (grad, grad._version, aux, offset_dot)


def _take_offset_dot(grad2: Tensor, aux: Tensor) -> Tensor | None:
    offer = _offers.pop(grad2.data_ptr(), None)
    if offer is None:
        return None
    grad, version, offered_aux, offset_dot = offer
    same = (offered_aux is aux and grad._version == version and grad.numel() == grad2.numel()
            and grad.dtype == grad2.dtype and grad.is_contiguous() and grad2.is_contiguous()
            and grad.untyped_storage().data_ptr() == grad2.untyped_storage().data_ptr())
    return offset_dot if same else None


def forget_offers() -> None:
    _offers.clear()


class QSTELinearFn(Function):
    @staticmethod
    def forward(ctx, inputs, packed, scale, bias, surface: Surface):
        columns = surface.columns
        output = kernels.packed_linear_affine(inputs, packed, scale, bias, columns)
        flat = inputs.reshape(-1, columns)
        payload, aux = _encoding_of(inputs, flat, columns)
        ctx.save_for_backward(payload, aux, packed, scale)
        ctx.surface = surface
        ctx.columns = columns
        ctx.input_shape = inputs.shape
        ctx.input_dtype = inputs.dtype
        ctx.bias_dtype = None if bias is None else bias.dtype
        output = output.to(inputs.dtype)
        setattr(output, _AUX_ATTR, aux)
        return output

    @staticmethod
    def backward(ctx, grad_output):
        forget_encodings()
        payload, aux, packed, scale = ctx.saved_tensors
        grad2 = grad_output.reshape(-1, grad_output.shape[-1])
        offset_dot = _take_offset_dot(grad2, aux)
        # the input-gradient product only when autograd wants that gradient
        # (the reference always forms it, functional.py:180-183)
        grad_inputs, evidence, grad_scale, grad_bias = kernels.linear_backward(
            grad2, payload, aux[0], aux[1], packed, scale.detach(), ctx.columns,
            need_bias=ctx.bias_dtype is not None, need_input=ctx.needs_input_grad[0],
            offset_dot=offset_dot)
        ctx.surface.consume_evidence(evidence)
        if grad_inputs is not None:
            grad_inputs = grad_inputs.reshape(ctx.input_shape).to(ctx.input_dtype)
        if grad_bias is not None:
            grad_bias = grad_bias.to(ctx.bias_dtype)
        return grad_inputs, None, grad_scale.to(scale.dtype), grad_bias, None


def qste_linear(inputs: Tensor, surface: Surface, bias: Tensor | None = None) -> Tensor:
    """Functional binary linear (functional.py:197-205)."""

    surface.note_forward()
    return QSTELinearFn.apply(_autocast(inputs), surface.packed_sign, surface.scale, bias, surface)


class QSTEWeightFn(Function):
    """Differentiable dense ``sign * scale`` for code that reads ``.weight``.

    functional.py:213-245: the gradient of the dense matrix becomes the
    surface's evidence, and its row inner product with the signs the scale
    gradient.
    """

    @staticmethod
    def forward(ctx, packed, scale, surface: Surface):
        ctx.save_for_backward(packed, scale)
        ctx.surface = surface
        sign = kernels.unpack_rows(packed, surface.columns, dtype=torch.float32)
        return sign.mul_(scale.detach().float().unsqueeze(1)).to(scale.dtype)

    @staticmethod
    def backward(ctx, grad_weight):
        packed, scale = ctx.saved_tensors
        surface = ctx.surface
        grad_weight = grad_weight.float().contiguous()
        grad_scale = kernels.packed_row_inner(grad_weight, packed, surface.columns)
        evidence = grad_weight.mul_(scale.detach().float().unsqueeze(1))
        surface.consume_evidence(evidence)
        return None, grad_scale.to(scale.dtype), None


class SwiGLUFn(Function):
    """``silu(gate) * up`` in one kernel each way, rounded as torch's
    ``F.silu(gate) * up`` and its autograd round, keeping ``gate`` and ``up``
    for backward.  With ``encode`` the forward also encodes the output's rows
    for the binary layer that reads it next (a SwiGLU MLP's down
    projection), which then does not read the output again to encode it."""

    @staticmethod
    def forward(ctx, gate, up, encode: bool):
        forget_offers()
        out, encoding = kernels.swiglu_forward(gate, up, encode=encode)
        ctx.save_for_backward(gate, up)
        if encoding is not None:
            packed, offset, scale = encoding
            remember_encoding(out, packed, kernels.stacked_pair(offset, scale))
        # the encodings of the inputs of the binary layers that produced gate
        # and up (one [2, tokens] aux each), when both did
        ctx.auxes = None
        aux_g, aux_u = getattr(gate, _AUX_ATTR, None), getattr(up, _AUX_ATTR, None)
        tokens = gate.numel() // gate.shape[-1] if gate.dim() and gate.shape[-1] else 0
        if (aux_g is not None and aux_u is not None and tokens and aux_g.shape == (2, tokens)
                and aux_u.shape == (2, tokens)):
            ctx.auxes = (aux_g, aux_u)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        forget_offers()
        gate, up = ctx.saved_tensors
        if ctx.auxes is None:
            grad_gate, grad_up = kernels.swiglu_backward(grad_output.contiguous(), gate, up)
            return grad_gate, grad_up, None
        # the gradients and, for the two layers' backward, their offset sums
        aux_g, aux_u = ctx.auxes
        cols = gate.shape[-1]
        grad_gate, grad_up, sums = kernels.swiglu_backward_sums(
            grad_output.reshape(-1, cols), gate.reshape(-1, cols), up.reshape(-1, cols), aux_g[0], aux_u[0])
        grad_gate, grad_up = grad_gate.view(gate.shape), grad_up.view(up.shape)
        _offer_offset_dot(grad_gate, aux_g, sums[0])
        _offer_offset_dot(grad_up, aux_u, sums[1])
        torch.autograd.Variable._execution_engine.queue_callback(forget_offers)
        return grad_gate, grad_up, None


class SwiGLUMLPFn(Function):
    """``down(swiglu(gate(x), up(x)))`` as one autograd node, bf16.

    The values are those of the three QSTELinearFn nodes and SwiGLUFn
    composed: the same products, the same gate arithmetic, the same
    encodings (x's shared by gate and up; h's from the gate kernel), and
    the row scales of the three surfaces from their log-scales with the
    kernels of ``surface.row_scale`` (inputs are the log-scales, so their
    gradients leave this node as RowScaleFn's would).  The
    backward runs the gate and up layers as one layer of 2 ffn rows: the
    gate's backward writes their gradients side by side into one [tokens,
    2 ffn] tensor (with the two layers' offset sums, in the order the layers
    would sum them), and one ``linear_backward`` over it and the two layers'
    concatenated signs and scales gives

    * their evidence and scale gradients as the row blocks of one product
      (each element as the layer's own product forms it; a split-K plan
      chosen for the longer product may sum some tiles in another order),
    * x's gradient as one product over K = 2 ffn, rounded once, where
      autograd rounds each layer's input gradient and then their sum --
      one launch and one pass over [tokens, d] tensors fewer.

    Evidence goes to each surface after every product that reads that
    surface's signs (a delivery may step the surface, rewriting them), as in
    QSTELinearFn: down first, then gate and up."""

    @staticmethod
    def forward(ctx, inputs, packed_g, log_g, bias_g, packed_u, log_u, bias_u, packed_d, log_d, bias_d,
                surfaces, grad_on: bool):
        sg, su, sd = surfaces
        d, ffn = sg.columns, sg.rows
        flat = inputs.reshape(-1, d)
        # each layer's row scale (the kernel of surface.row_scale) right
        # before the product that needs it, so the first product is queued
        # after one small launch rather than three
        scale_g, e_g = kernels.row_scale(log_g, sg.cfg.scale_min, sg.cfg.scale_max)
        g = kernels.packed_linear_affine(flat, packed_g, scale_g, bias_g, d)
        scale_u, e_u = kernels.row_scale(log_u, su.cfg.scale_min, su.cfg.scale_max)
        u = kernels.packed_linear_affine(flat, packed_u, scale_u, bias_u, d)
        h, enc = kernels.swiglu_forward(g, u, encode=grad_on)
        scale_d, e_d = kernels.row_scale(log_d, sd.cfg.scale_min, sd.cfg.scale_max)
        y = kernels.packed_linear_affine(h, packed_d, scale_d, bias_d, ffn)
        if grad_on:
            payload_x, aux_x = _encoding_of(inputs, flat, d)
            aux_h = kernels.stacked_pair(enc[1], enc[2])
            ctx.save_for_backward(payload_x, aux_x, g, u, enc[0], aux_h, packed_g, scale_g, packed_u, scale_u,
                                  packed_d, scale_d, e_g, e_u, e_d)
        ctx.surfaces = surfaces
        ctx.input_shape = inputs.shape
        ctx.bias_dtypes = tuple(None if b is None else b.dtype for b in (bias_g, bias_u, bias_d))
        return y.reshape(*inputs.shape[:-1], d)

    @staticmethod
    def backward(ctx, grad_output):
        forget_encodings()
        (payload_x, aux_x, g, u, payload_h, aux_h, packed_g, scale_g, packed_u, scale_u, packed_d,
         scale_d, e_g, e_u, e_d) = ctx.saved_tensors
        sg, su, sd = ctx.surfaces
        d, ffn = sg.columns, sg.rows
        bg, bu, bd = ctx.bias_dtypes
        dy = grad_output.reshape(-1, d)
        # A surface's evidence may step it on delivery, rewriting its packed
        # signs in place; every product that multiplies by a layer's signs
        # runs before that layer's evidence is delivered, as in QSTELinearFn
        # (whose one call forms the input gradient before the delivery).
        dh, ev_d, gs_d, gb_d = kernels.linear_backward(
            dy, payload_h, aux_h[0], aux_h[1], packed_d, scale_d.detach(), ffn, need_bias=bd is not None)
        sd.consume_evidence(ev_d)
        del ev_d
        both, sums = kernels.swiglu_backward_sums(dh, g, u, aux_x[0], aux_x[0], side_by_side=True)
        del dh
        # gate and up as one layer of 2 ffn rows (copies of their signs and
        # scales: the deliveries below may rewrite the signs)
        packed_gu = torch.cat((packed_g, packed_u))
        scale_gu = torch.cat((scale_g.detach().float(), scale_u.detach().float()))
        need_bias = bg is not None or bu is not None
        dx, ev_gu, gs_gu, gb_gu = kernels.linear_backward(
            both, payload_x, aux_x[0], aux_x[1], packed_gu, scale_gu, d, need_bias=need_bias,
            need_input=ctx.needs_input_grad[0], offset_dot=sums.reshape(-1))
        del both
        if dx is not None:
            dx = dx.reshape(ctx.input_shape)
        sg.consume_evidence(ev_gu[:ffn])
        su.consume_evidence(ev_gu[ffn:])
        gs_g, gs_u = gs_gu[:ffn], gs_gu[ffn:]
        gb_g, gb_u = (gb_gu[:ffn], gb_gu[ffn:]) if need_bias else (None, None)

        def cast(grad, dtype):
            return None if grad is None or dtype is None else grad.to(dtype)

        def through_scale(gs, e, surface):
            # the scale's gradient carried to the log-scale, as RowScaleFn does
            return kernels.row_scale_backward(e, gs.to(e.dtype), surface.cfg.scale_min, surface.cfg.scale_max)

        return (dx, None, through_scale(gs_g, e_g, sg), cast(gb_g, bg), None, through_scale(gs_u, e_u, su),
                cast(gb_u, bu), None, through_scale(gs_d, e_d, sd), cast(gb_d, bd), None, None)


# log-scale dtypes the row-scale kernels take (surface.row_scale)
_SCALE_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def swiglu_mlp_fusable(inputs: Tensor, gate, up, down) -> bool:
    """Whether ``SwiGLUMLPFn`` takes this MLP: bf16 input on the GPU, the
    gate and up layers d -> ffn and the down layer ffn -> d, d and ffn
    multiples of 64."""

    sg, su, sd = gate.surface, up.surface, down.surface
    d, ffn = sg.columns, sg.rows
    return (inputs.is_cuda and inputs.dtype == torch.bfloat16 and inputs.dim() >= 1 and inputs.shape[-1] == d
            and su.columns == d and su.rows == ffn and sd.columns == ffn and sd.rows == d
            and d % 64 == 0 and ffn % 64 == 0 and inputs.numel() > 0
            and all(s.log_scale.is_cuda and s.log_scale.dtype in _SCALE_DTYPES for s in (sg, su, sd)))


def swiglu(gate: Tensor, up: Tensor) -> Tensor:
    """The SwiGLU gate ``F.silu(gate) * up`` (same values and gradients), fused.

    No counterpart in the reference; a SwiGLU MLP written
    ``down(swiglu(gate(x), up(x)))`` computes what
    ``down(F.silu(gate(x)) * up(x))`` computes, with two elementwise passes
    instead of five and the down projection's activation encoding produced
    with its input."""

    return SwiGLUFn.apply(gate, up, torch.is_grad_enabled())


def qste_weight(surface: Surface) -> Tensor:
    surface.note_forward()
    return QSTEWeightFn.apply(surface.packed_sign, surface.scale, surface)


class QSTEEmbeddingFn(Function):
    """Binary embedding lookup; its backward is the surface's evidence (functional.py:260-282)."""

    @staticmethod
    def forward(ctx, ids, packed, scale, surface: Surface):
        output = kernels.packed_embedding(ids, packed, scale, surface.columns)
        ctx.save_for_backward(ids, packed, scale)
        ctx.surface = surface
        return output

    @staticmethod
    def backward(ctx, grad_output):
        ids, packed, scale = ctx.saved_tensors
        evidence, grad_scale = kernels.embedding_backward(
            ids, grad_output, packed, scale.detach(), ctx.surface.columns)
        ctx.surface.consume_evidence(evidence)
        return None, None, grad_scale.to(scale.dtype), None


def qste_embedding(ids: Tensor, surface: Surface) -> Tensor:
    """Functional binary embedding (functional.py:285-287)."""

    surface.note_forward()
    return QSTEEmbeddingFn.apply(ids, surface.packed_sign, surface.scale, surface)
