"""The coordinate optimizer: owns the int8 coordinates and nothing else.

Behaviour of the reference's ``QSTEOptimizer`` (``src/qste/optim.py:34-232``):
per-surface state ``moment_q`` (int8), ``moment_scale`` (fp16 per block,
initialised to 1/127), ``row_v``/``col_v`` (fp16, zero); the step runs
inside backward the moment a single-use surface's evidence is complete,
with seed ``cfg.seed + 1_000_003 * position`` and the step number from
before the current ``step()`` call; ``step()`` flushes leftovers, clamps
``log_scale`` and returns the sign flips.

Flip counts stay on the device until ``step()`` returns them, so backward
never waits on the host.  Evidence all-reduce across ranks is not part of
this single-GPU build: with a multi-rank process group, pass
``gradient_reducer`` explicitly (``False`` to opt out), or construction
fails rather than letting ranks silently drift apart.
"""

from __future__ import annotations

import math
from typing import Callable, Iterable, Mapping

import torch
import torch.nn as nn
from torch import Tensor

from . import kernels
from .config import QSTEConfig, coerce_config
from .convert import surfaces as _model_surfaces
from .surface import Surface

SEED_STRIDE = 1_000_003


class QSTEOptimizer:
    def __init__(
        self,
        model: nn.Module | Iterable[Surface],
        config: QSTEConfig | None = None,
        *,
        gradient_reducer: Callable[[Tensor], Tensor] | None | bool = None,
    ):
        if isinstance(model, nn.Module):
            self.surfaces = _model_surfaces(model)
            config = config or getattr(model, "_qste_config", None)
        else:
            self.surfaces = list(model)
        if not self.surfaces:
            raise ValueError("no QSTE surfaces found; call qste_amd.convert(model, ...) first")
        self.cfg = coerce_config(config)
        self.gradient_reducer = self._resolve_reducer(gradient_reducer)
        self.step_number = 0
        self._deferred = False
        self._flips: Tensor | None = None
        self.state: dict[int, dict[str, Tensor]] = {}
        self._index: dict[int, int] = {}
        block = self.cfg.momentum_block_size
        for position, surface in enumerate(self.surfaces):
            self._index[id(surface)] = position
            device = surface.coordinate.device
            blocks = (surface.coordinate.numel() + block - 1) // block
            self.state[id(surface)] = {
                "moment_q": torch.zeros_like(surface.coordinate, dtype=torch.int8),
                "moment_scale": torch.full((blocks,), 1 / 127, dtype=torch.float16, device=device),
                "row_v": torch.zeros(surface.rows, dtype=torch.float16, device=device),
                "col_v": torch.zeros(surface.columns, dtype=torch.float16, device=device),
            }
            surface._immediate = self._apply

    @staticmethod
    def _resolve_reducer(requested):
        if requested is False:
            return None
        if requested is not None and requested is not True:
            return requested
        dist = torch.distributed
        if dist.is_available() and dist.is_initialized() and dist.get_world_size() > 1:
            raise RuntimeError(
                "a multi-rank process group is initialized: pass gradient_reducer (a callable "
                "that all-reduces fp32 evidence) or gradient_reducer=False; qste_amd does not "
                "reduce evidence across ranks on its own")
        return None

    # -- accumulation control (optim.py:120-152) --------------------------

    def defer(self, deferred: bool = True) -> None:
        self._deferred = deferred
        for surface in self.surfaces:
            surface._immediate = None if deferred else self._apply

    def prepare_accumulation(self) -> None:
        self.defer(True)
        for surface in self.surfaces:
            surface.prepare_accumulator()

    def unscale_(self, scale: float | Tensor) -> None:
        divisor = float(scale)
        for surface in self.surfaces:
            surface.scale_evidence_(divisor)

    def zero_grad(self, set_to_none: bool = True) -> None:
        del set_to_none
        for surface in self.surfaces:
            surface.flush_evidence()
            surface.reset_tracking()
        self._flips = None

    # -- the step -----------------------------------------------------------

    def seed_for(self, surface: Surface) -> int:
        return self.cfg.seed + SEED_STRIDE * self._index[id(surface)]

    @torch.no_grad()
    def _apply(self, surface: Surface, evidence: Tensor) -> None:
        state = self.state[id(surface)]
        evidence = evidence.float()
        if self.gradient_reducer is not None:
            evidence = self.gradient_reducer(evidence)
        flips = torch.empty((), dtype=torch.int64, device=evidence.device)
        kernels.coordinate_update(
            evidence, surface.coordinate.data, surface.packed_sign.data,
            state["moment_q"], state["moment_scale"], state["row_v"], state["col_v"],
            beta1=self.cfg.beta1, beta2=self.cfg.beta2, update_clip=self.cfg.update_rms_clip,
            coordinate_lr=self.cfg.coordinate_lr, block_size=self.cfg.momentum_block_size,
            seed=self.seed_for(surface), step=self.step_number, flips=flips)
        self._flips = flips if self._flips is None else self._flips + flips

    @torch.no_grad()
    def step(self) -> int:
        """Apply retained evidence, clamp scales, advance; return sign flips."""

        lo, hi = math.log(self.cfg.scale_min), math.log(self.cfg.scale_max)
        for surface in self.surfaces:
            evidence = surface.flush_evidence(keep_buffer=self._deferred)
            if evidence is not None:
                self._apply(surface, evidence)
            surface.log_scale.data.clamp_(lo, hi)
        flips = 0 if self._flips is None else int(self._flips.item())
        self._flips = None
        self.step_number += 1
        return flips

    # -- reporting and checkpointing (optim.py:205-232) -------------------------

    def state_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for s in self.state.values() for t in s.values())

    def state_dict(self) -> dict[str, object]:
        return {
            "config": self.cfg.metadata(),
            "step_number": self.step_number,
            "surfaces": [
                {k: t.detach().cpu() for k, t in self.state[id(s)].items()} for s in self.surfaces
            ],
        }

    def load_state_dict(self, state_dict: Mapping[str, object]) -> None:
        entries = state_dict["surfaces"]
        if len(entries) != len(self.surfaces):
            raise ValueError(
                f"checkpoint holds {len(entries)} surfaces, model has {len(self.surfaces)}")
        for surface, entry in zip(self.surfaces, entries):
            state = self.state[id(surface)]
            for key, tensor in entry.items():
                state[key].copy_(tensor.to(state[key].device))
        self.step_number = int(state_dict.get("step_number", 0))
