"""Model surgery: replace selected ``nn.Linear`` layers with ``QSTELinear``.

Selection semantics follow ``qste.convert`` (``src/qste/convert.py:159-243``):
shell-style globs over qualified module names (``include`` then
``exclude``), ``ValueError`` when nothing is selected, tied weights sharing
one ``Surface``, the config recorded on the model as ``_qste_config``.

With ``activations`` set, activation modules are swapped for the packed
ones of ``qste_amd.nn`` (``convert.py:246-274``): ``True`` / ``"all"`` take
every replacement, ``"exact"`` only the one-bit (value- and
gradient-identical) ones.

``nn.Embedding`` layers become ``QSTEEmbedding``; ``export_packed`` turns
them into ``PackedEmbedding`` (``convert.py:327-357``).
"""

from __future__ import annotations

import copy
import fnmatch
from typing import Iterator, Sequence

import torch.nn as nn

from .config import QSTEConfig, coerce_config
from .modules import PackedEmbedding, PackedLinear, QSTEEmbedding, QSTELinear
from .surface import Surface

DEFAULT_TYPES = (nn.Linear, nn.Embedding)


def _selected(name: str, include: Sequence[str] | None, exclude: Sequence[str] | None) -> bool:
    if include is not None and not any(fnmatch.fnmatchcase(name, p) for p in include):
        return False
    return not (exclude and any(fnmatch.fnmatchcase(name, p) for p in exclude))


def _candidates(model: nn.Module, types: tuple[type, ...]) -> Iterator[tuple[str, nn.Module]]:
    converted = (QSTELinear, QSTEEmbedding)
    for name, module in model.named_modules():
        if name and isinstance(module, types + converted):
            weight = None if isinstance(module, converted) else getattr(module, "weight", None)
            if isinstance(module, converted) or (weight is not None and weight.ndim == 2):
                yield name, module


def _set_submodule(model: nn.Module, name: str, replacement: nn.Module) -> None:
    parent_name, _, leaf = name.rpartition(".")
    parent = model.get_submodule(parent_name) if parent_name else model
    setattr(parent, leaf, replacement)


def convert(
    model: nn.Module,
    include: Sequence[str] | None = None,
    exclude: Sequence[str] | None = None,
    *,
    config: QSTEConfig | None = None,
    types: tuple[type, ...] = DEFAULT_TYPES,
    activations: bool | str = True,
    verbose: bool = False,
) -> nn.Module:
    """Replace the selected layers of ``model`` in place and return it."""

    if activations not in (True, False, "exact", "all"):
        raise ValueError("activations must be True, False, 'exact', or 'all'")
    cfg = coerce_config(config)
    found = list(_candidates(model, types))
    targets = [(n, m) for n, m in found if _selected(n, include, exclude)]
    if not targets:
        raise ValueError(
            "convert() selected no layers; check `include` against "
            f"{[n for n, _ in found][:8]}")

    shared: dict[int, Surface] = {}
    converted = list(getattr(model, "_qste_converted", ()))
    for name, module in targets:
        if isinstance(module, (QSTELinear, QSTEEmbedding)):
            continue  # already binary
        surface = shared.get(id(module.weight))
        if isinstance(module, nn.Embedding):
            replacement = QSTEEmbedding.from_embedding(module, cfg, surface)
        else:
            replacement = QSTELinear.from_linear(module, cfg, surface)
        shared[id(module.weight)] = replacement.surface
        _set_submodule(model, name, replacement)
        converted.append(name)
        if verbose:
            print(f"converted {name}: {replacement.out_features} x {replacement.in_features}")

    if activations:
        converted.extend(_convert_activations(model, activations))

    model._qste_config = cfg
    model._qste_converted = tuple(converted)
    return model


def _convert_activations(model: nn.Module, mode: bool | str) -> list[str]:
    """Swap activation modules for packed ones; returns the names replaced.

    Idempotent: the packed classes are not keys of the replacement tables.
    """

    from . import nn as packed

    table = packed.EXACT_REPLACEMENTS if mode == "exact" else packed.REPLACEMENTS
    replaced: list[str] = []
    for name, module in list(model.named_modules()):
        if not name or type(module) not in table:
            continue
        substitute = packed.replace(module)
        if substitute is None:
            continue
        substitute.training = module.training
        _set_submodule(model, name, substitute)
        replaced.append(name)
    return replaced


def surfaces(model: nn.Module) -> list[Surface]:
    """Every distinct surface in the model, tied weights counted once."""

    seen: dict[int, Surface] = {}
    for module in model.modules():
        if isinstance(module, Surface):
            seen.setdefault(id(module), module)
    return list(seen.values())


def continuous_parameters(model: nn.Module):
    """Parameters the host's own optimizer owns (row scales, biases, the rest)."""

    for parameter in model.parameters():
        if parameter.requires_grad:
            yield parameter


def memory_report(model: nn.Module) -> dict[str, float]:
    """Matrix bytes before and after conversion, in megabytes."""

    flt = train = infer = 0
    for s in surfaces(model):
        m = s.memory()
        flt += m["float_equivalent"]
        train += m["packed_sign"] + m["coordinate"] + m["log_scale"]
        infer += m["packed_sign"] + m["log_scale"]
    return {
        "float_mb": flt / 1e6,
        "training_mb": train / 1e6,
        "inference_mb": infer / 1e6,
        "training_ratio": flt / train if train else 0.0,
        "inference_ratio": flt / infer if infer else 0.0,
    }


def export_packed(model: nn.Module, *, inplace: bool = False) -> nn.Module:
    """Drop the coordinates, keeping bits, scales and biases (convert.py:327-357)."""

    target = model if inplace else copy.deepcopy(model)
    for name, module in list(target.named_modules()):
        if isinstance(module, QSTELinear):
            s = module.surface
            _set_submodule(target, name, PackedLinear(
                s.packed_sign.data.clone(), s.scale.detach().clone(), s.columns,
                None if module.bias is None else module.bias.detach().clone()))
        elif isinstance(module, QSTEEmbedding):
            s = module.surface
            _set_submodule(target, name, PackedEmbedding(
                s.packed_sign.data.clone(), s.scale.detach().clone(), s.columns))
    return target
