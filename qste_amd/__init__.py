"""qste_amd -- QSTE's binary-linear hot path, native to MI355X (gfx950).

Drop-in for the reference's user API on this path::

    import qste_amd as qste

    qste.convert(model, include=["blocks.*.mlp.fc1", "blocks.*.mlp.fc2"])
    optimizer = torch.optim.AdamW(qste.continuous_parameters(model))
    coordinates = qste.QSTEOptimizer(model)

    loss.backward()          # the coordinate step runs inside backward
    optimizer.step(); coordinates.step()

Forward, backward and the coordinate step run as hand-written HIP kernels in
``libqste_hip.so`` (C ABI: ``include/qste_hip.h``); there is no CPU path.
"""

from .config import QSTEConfig, coerce_config
from .convert import (continuous_parameters, convert, export_packed, memory_report,
                      surfaces)
from .functional import QSTEEmbeddingFn, QSTELinearFn, qste_embedding, qste_linear, qste_weight
from .modules import PackedEmbedding, PackedLinear, QSTEEmbedding, QSTELinear
from . import nn
from .nn import packed_activations
from .optim import QSTEOptimizer
from .surface import Surface

__version__ = "0.1.0"

__all__ = [
    "PackedEmbedding",
    "PackedLinear",
    "QSTEEmbedding",
    "QSTEEmbeddingFn",
    "QSTEConfig",
    "QSTELinear",
    "QSTELinearFn",
    "QSTEOptimizer",
    "Surface",
    "coerce_config",
    "device_profile",
    "continuous_parameters",
    "convert",
    "export_packed",
    "kernel_status",
    "memory_report",
    "nn",
    "packed_activations",
    "qste_embedding",
    "qste_linear",
    "qste_weight",
    "surfaces",
    "__version__",
]


def kernel_status() -> dict:
    """Whether the HIP library is built and loads, and why not if it does not."""

    from . import kernels

    return kernels.status()


def device_profile(device=None) -> str:
    """What this build runs on a device, as one line (reference
    src/qste/__init__.py:105-120): device and architecture, compute units,
    shader clock (reported maximum and measured now), HBM and LDS sizes, the
    HIP library's version and the kernel each operator takes.  Without a GPU
    the line says that qste_amd has no CPU path."""

    from . import kernels

    return kernels.profile(device)
