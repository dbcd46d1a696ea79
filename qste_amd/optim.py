"""The coordinate optimizer: it owns the int8 coordinates and nothing else.

Public behaviour is the reference's ``QSTEOptimizer``
(``src/qste/optim.py:34-232``); row scales and biases stay ordinary float
parameters for the host's own optimizer.  Per surface of R x C it keeps

    moment_q      int8  [R, C]            block-quantized first moment
    moment_scale  fp16  [ceil(RC/block)]  one scale per block, starts at 1/127
    row_v, col_v  fp16  [R], [C]          factored second moment, start at 0

and applies one fused HIP step (``kernels.coordinate_update``) per surface
whenever evidence for it is complete.  What "complete" means is the
surfaces' business (``surface.EvidenceLedger``): normally inside backward;
while deferred, at :meth:`QSTEOptimizer.step`.

Semantics that fix the integer trajectory and so follow the reference:

* surface ``i`` (in discovery order) draws its rounding stream from seed
  ``cfg.seed + 1_000_003 * i``;
* an application inside backward uses the step number *before* the
  ``step()`` call that follows it; ``step()`` then advances it by one;
* ``step()`` drains held evidence first, then clamps every ``log_scale``
  into ``[log scale_min, log scale_max]``, and returns the sign flips of
  all applications since the previous ``step()``.

Flip counts are written by the kernel into one preallocated device slot per
surface and read back once per ``step()``, so backward never waits on the
host and nothing is allocated per application.  That read polls an event
behind a copy into pinned host memory rather than blocking in the copy: a
blocking read returned ~70 us after the device had finished, and the
caller's next launches (the next forward) waited with it.

Evidence all-reduce across ranks is not part of this single-GPU build: with
a multi-rank process group pass ``gradient_reducer`` explicitly (``False``
to opt out), or construction fails rather than letting ranks silently drift
apart.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass, field
from typing import Callable, Iterable, Mapping

import torch
import torch.nn as nn
from torch import Tensor

from . import kernels
from .config import QSTEConfig, coerce_config
from .convert import surfaces as _model_surfaces
from .surface import Surface

SEED_STRIDE = 1_000_003
STATE_KEYS = ("moment_q", "moment_scale", "row_v", "col_v")


@dataclass
class _Slot:
    """Everything the optimizer keeps for one surface."""

    surface: Surface
    seed: int
    state: dict[str, Tensor]
    flips: Tensor                      # device int64, the last application's flips
    applied: bool = field(default=False)


def _fresh_state(surface: Surface, block: int) -> dict[str, Tensor]:
    device = surface.coordinate.device
    blocks = -(-surface.coordinate.numel() // block)
    return {
        "moment_q": torch.zeros(surface.rows, surface.columns, dtype=torch.int8, device=device),
        "moment_scale": torch.full((blocks,), 1 / 127, dtype=torch.float16, device=device),
        "row_v": torch.zeros(surface.rows, dtype=torch.float16, device=device),
        "col_v": torch.zeros(surface.columns, dtype=torch.float16, device=device),
    }


def _no_reducer_check(requested):
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


def _read_count(total: Tensor, host: Tensor | None) -> int:
    """``int(total)``.  A GPU total is copied into ``host`` (pinned int64)
    behind an event on the current stream, which is polled; the poll yields
    the interpreter lock between queries."""

    if not total.is_cuda or host is None:
        return int(total.item())
    host.copy_(total, non_blocking=True)
    done = torch.cuda.Event()
    done.record(torch.cuda.current_stream(total.device))
    while not done.query():
        time.sleep(0)
    return int(host.item())


class QSTEOptimizer:
    """Steps int8 coordinates from the evidence backward produces.

    ``model`` is a converted module or an iterable of surfaces; ``config``
    defaults to the one ``convert`` recorded on the model.
    ``gradient_reducer`` receives and returns each surface's fp32 evidence
    before it is applied.
    """

    def __init__(
        self,
        model: nn.Module | Iterable[Surface],
        config: QSTEConfig | None = None,
        *,
        gradient_reducer: Callable[[Tensor], Tensor] | None | bool = None,
    ):
        if isinstance(model, nn.Module):
            found = _model_surfaces(model)
            config = config or getattr(model, "_qste_config", None)
        else:
            found = list(model)
        if not found:
            raise ValueError("no QSTE surfaces found; call qste_amd.convert(model, ...) first")
        self.cfg = coerce_config(config)
        self.gradient_reducer = _no_reducer_check(gradient_reducer)
        self.step_number = 0
        self.deferred = False
        self._slots: dict[int, _Slot] = {}
        self._host_count: Tensor | None = None  # pinned int64 for step()'s flip total
        for position, surface in enumerate(found):
            self._slots[id(surface)] = _Slot(
                surface=surface,
                seed=self.cfg.seed + SEED_STRIDE * position,
                state=_fresh_state(surface, self.cfg.momentum_block_size),
                flips=torch.zeros((), dtype=torch.int64, device=surface.coordinate.device),
            )
            surface.route_evidence(self._apply)

    # -- the reference's public attributes ---------------------------------

    @property
    def surfaces(self) -> list[Surface]:
        return [slot.surface for slot in self._slots.values()]

    @property
    def state(self) -> dict[int, dict[str, Tensor]]:
        """Per-surface optimizer tensors, keyed by ``id(surface)``."""

        return {key: slot.state for key, slot in self._slots.items()}

    def seed_for(self, surface: Surface) -> int:
        return self._slots[id(surface)].seed

    # -- accumulation control ------------------------------------------------

    def defer(self, deferred: bool = True) -> None:
        """Hold evidence until :meth:`step` instead of applying it in backward."""

        self.deferred = bool(deferred)
        for slot in self._slots.values():
            slot.surface.route_evidence(None if self.deferred else self._apply)

    def prepare_accumulation(self) -> None:
        """Defer, into fixed zeroed evidence buffers (one per surface)."""

        self.defer(True)
        for slot in self._slots.values():
            slot.surface.prepare_accumulator()

    def unscale_(self, scale: float | Tensor) -> None:
        """Divide held evidence by an AMP loss scale."""

        divisor = float(scale)
        for slot in self._slots.values():
            slot.surface.scale_evidence_(divisor)

    def zero_grad(self, set_to_none: bool = True) -> None:
        """Drop evidence held but not applied, and flips not yet reported."""

        del set_to_none
        for slot in self._slots.values():
            slot.surface.flush_evidence()
            slot.surface.reset_tracking()
            slot.applied = False

    # -- the step ------------------------------------------------------------

    @torch.no_grad()
    def _apply(self, surface: Surface, evidence: Tensor) -> None:
        slot = self._slots[id(surface)]
        evidence = evidence.float()
        if self.gradient_reducer is not None:
            evidence = self.gradient_reducer(evidence)
        if slot.applied:
            # a second application before step() (a surface flushed after an
            # immediate apply): keep the earlier flips in the slot's total
            earlier = slot.flips.clone()
        cfg = self.cfg
        kernels.coordinate_update(
            evidence, surface.coordinate.data, surface.packed_sign.data,
            slot.state["moment_q"], slot.state["moment_scale"], slot.state["row_v"],
            slot.state["col_v"], beta1=cfg.beta1, beta2=cfg.beta2,
            update_clip=cfg.update_rms_clip, coordinate_lr=cfg.coordinate_lr,
            block_size=cfg.momentum_block_size, seed=slot.seed, step=self.step_number,
            flips=slot.flips)
        if slot.applied:
            slot.flips.add_(earlier)
        slot.applied = True

    @torch.no_grad()
    def step(self) -> int:
        """Apply held evidence, clamp row scales, advance; return the sign flips."""

        lo, hi = math.log(self.cfg.scale_min), math.log(self.cfg.scale_max)
        for slot in self._slots.values():
            pending = slot.surface.flush_evidence(keep_buffer=self.deferred)
            if pending is not None:
                self._apply(slot.surface, pending)
            slot.surface.log_scale.data.clamp_(lo, hi)
        counts = [slot.flips for slot in self._slots.values() if slot.applied]
        flips = 0
        if counts:
            total = torch.stack(counts).sum()
            if total.is_cuda and self._host_count is None:
                self._host_count = torch.empty((), dtype=torch.int64, pin_memory=True)
            flips = _read_count(total, self._host_count)
        for slot in self._slots.values():
            slot.applied = False
        self.step_number += 1
        return flips

    # -- reporting and checkpointing (layout of optim.py:205-232) -------------

    def state_bytes(self) -> int:
        return sum(t.numel() * t.element_size()
                   for slot in self._slots.values() for t in slot.state.values())

    def state_dict(self) -> dict[str, object]:
        return {
            "config": self.cfg.metadata(),
            "step_number": self.step_number,
            "surfaces": [{k: slot.state[k].detach().cpu() for k in STATE_KEYS}
                         for slot in self._slots.values()],
        }

    def load_state_dict(self, state_dict: Mapping[str, object]) -> None:
        saved = list(state_dict["surfaces"])
        if len(saved) != len(self._slots):
            raise ValueError(
                f"checkpoint holds {len(saved)} surfaces, model has {len(self._slots)}")
        for slot, entry in zip(self._slots.values(), saved):
            for key, tensor in entry.items():
                slot.state[key].copy_(tensor.to(slot.state[key].device))
        self.step_number = int(state_dict.get("step_number", 0))
