"""Drop-in modules: ``QSTELinear`` / ``QSTEEmbedding`` (training) and
``PackedLinear`` / ``PackedEmbedding`` (inference).

Constructor attributes, ``weight``/``bias`` surface and call signature follow
the reference (``src/qste/modules.py:21-123``) so code that introspects an
``nn.Linear`` keeps working.
"""

from __future__ import annotations

import torch
import torch.nn as nn
from torch import Tensor

from . import kernels
from .config import QSTEConfig, coerce_config
from .functional import qste_embedding, qste_linear, qste_weight
from .nn import _mark_activation_input
from .surface import Surface


class QSTELinear(nn.Module):
    """Training-time binary linear layer over one ``Surface``.

    Its output is the input times the packed +-1 matrix (transposed), each
    output column scaled by the surface's learned row scale, plus an optional
    bias; autograd routes the coordinate evidence to the surface
    (modules.py:21-66)."""

    def __init__(self, surface: Surface, bias: Tensor | None = None):
        super().__init__()
        self.surface = surface
        self.in_features = surface.columns
        self.out_features = surface.rows
        if bias is None:
            self.register_parameter("bias", None)
        else:
            self.bias = nn.Parameter(bias.detach().float().clone())

    @classmethod
    def from_linear(cls, module: nn.Linear, cfg: QSTEConfig | None = None,
                    surface: Surface | None = None) -> "QSTELinear":
        return cls(surface or Surface(module.weight, coerce_config(cfg)), module.bias)

    @property
    def scale(self) -> Tensor:
        return self.surface.scale

    @property
    def packed_sign(self) -> Tensor:
        return self.surface.packed_sign

    @property
    def weight(self) -> Tensor:
        """Differentiable dense equivalent (materializes out x in floats)."""

        return qste_weight(self.surface)

    def forward(self, inputs: Tensor) -> Tensor:
        # tagged so packed_activations() packs an activation applied to it
        return _mark_activation_input(qste_linear(inputs, self.surface, self.bias))

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}")


class PackedLinear(nn.Module):
    """Inference-only linear over packed signs, a row scale and a bias.

    The reference casts the input to fp32, multiplies in fp32 and rounds the
    result back to the input dtype (modules.py:114-120).  Widening bf16/fp16
    to fp32 is exact, so the input goes to the kernel in its own dtype; the
    kernels multiply exact +-1 operands, accumulate in fp32 and round once to
    the input dtype.  The decode kernel (bf16, at most 16 rows) accumulates a
    biased operand and subtracts the bias, which costs a few of fp32's bits
    relative to sum |x|: well below the output's bf16 rounding.
    """

    def __init__(self, packed: Tensor, scale: Tensor, columns: int, bias: Tensor | None):
        super().__init__()
        self.register_buffer("packed_sign", packed)
        self.register_buffer("scale", scale)
        self.in_features = columns
        self.out_features = packed.shape[0]
        self.register_buffer("bias", bias)

    @torch.no_grad()
    def forward(self, inputs: Tensor) -> Tensor:
        return kernels.packed_linear_affine(
            inputs, self.packed_sign, self.scale, self.bias, self.in_features).to(inputs.dtype)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}"


class QSTEEmbedding(nn.Module):
    """Binary embedding table: a row of packed signs times the row scale (modules.py:68-97)."""

    def __init__(self, surface: Surface, padding_idx: int | None = None):
        super().__init__()
        self.surface = surface
        self.num_embeddings = surface.rows
        self.embedding_dim = surface.columns
        self.padding_idx = padding_idx

    @classmethod
    def from_embedding(cls, module: nn.Embedding, cfg: QSTEConfig | None = None,
                       surface: Surface | None = None) -> "QSTEEmbedding":
        return cls(surface or Surface(module.weight, coerce_config(cfg)), getattr(module, "padding_idx", None))

    @property
    def scale(self) -> Tensor:
        return self.surface.scale

    @property
    def packed_sign(self) -> Tensor:
        return self.surface.packed_sign

    @property
    def weight(self) -> Tensor:
        return qste_weight(self.surface)

    def forward(self, ids: Tensor) -> Tensor:
        return _mark_activation_input(qste_embedding(ids, self.surface))

    def extra_repr(self) -> str:
        return f"num_embeddings={self.num_embeddings}, embedding_dim={self.embedding_dim}"


class PackedEmbedding(nn.Module):
    """Inference-only embedding over packed signs (modules.py:126-143)."""

    def __init__(self, packed: Tensor, scale: Tensor, columns: int):
        super().__init__()
        self.register_buffer("packed_sign", packed)
        self.register_buffer("scale", scale)
        self.num_embeddings = packed.shape[0]
        self.embedding_dim = columns

    @torch.no_grad()
    def forward(self, ids: Tensor) -> Tensor:
        return kernels.packed_embedding(ids, self.packed_sign, self.scale, self.embedding_dim)

    def extra_repr(self) -> str:
        return f"num_embeddings={self.num_embeddings}, embedding_dim={self.embedding_dim}"
