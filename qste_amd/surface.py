"""One binary matrix: its int8 coordinate, packed signs and row scale.

State layout and parameter names are the reference's ``Surface``
(``src/qste/surface.py:67-79``), so state dicts load either way:

    coordinate   int8  [rows, columns]      training state (optimizer-owned)
    packed_sign  uint8 [rows, ceil(cols/8)] forward weight, LSB-first bits
    log_scale    fp32  [rows]               learned row scale (host optimizer)

Evidence (the fp32 coordinate gradient each backward produces) does not go
through ``.grad``.  Each surface owns an :class:`EvidenceLedger` that decides
where it goes; the rules are the reference's (``surface.py:104-206``):

* a surface used once per backward hands its evidence to the optimizer inside
  that backward, without a buffer;
* a surface used several times per backward (tied weights) sums the uses, in
  the configured accumulation dtype, and hands over the sum after the last;
* while the optimizer is deferred (gradient accumulation, AMP unscaling,
  capture) evidence is held until ``QSTEOptimizer.step``, in a fixed buffer
  when one was prepared;
* the step drains whatever is held, whether or not forward and backward
  counts balanced (gradient checkpointing runs forwards that never see a
  backward).
"""

from __future__ import annotations

from typing import Callable, Optional

import torch
import torch.nn as nn
from torch import Tensor
from torch.autograd import Function

from . import kernels
from .config import QSTEConfig, coerce_config

_ACCUM_DTYPE = {"fp16": torch.float16, "fp32": torch.float32}

Sink = Callable[["Surface", Tensor], None]


def _on_gpu(fn, tensor: Tensor, *args, **kwargs) -> Tensor:
    """Run a GPU kernel on ``tensor``; a CPU tensor makes a round trip.

    Construction on a CPU model is legitimate (convert, then ``.to('cuda')``),
    but there is no CPU implementation of the kernels: the work goes to the
    current ROCm device and the result comes back.
    """

    if tensor.device.type == "cuda":
        return fn(tensor, *args, **kwargs)
    if not torch.cuda.is_available():
        raise RuntimeError(
            "qste_amd needs a ROCm GPU: its kernels have no CPU implementation "
            f"(called with a tensor on {tensor.device})"
        )
    return fn(tensor.to("cuda"), *args, **kwargs).to(tensor.device)


class RowScaleFn(Function):
    """``clamp(exp(log_scale), lo, hi)`` with torch's values and gradient, one
    HIP launch each way (surface.py:84-85) instead of torch's two forward and
    six backward kernels.  Saves exp's result, as torch's exp does."""

    @staticmethod
    def forward(ctx, log_scale, lo: float, hi: float):
        scale, e = kernels.row_scale(log_scale, lo, hi)
        ctx.save_for_backward(e)
        ctx.bounds = (lo, hi)
        return scale

    @staticmethod
    def backward(ctx, grad):
        (e,) = ctx.saved_tensors
        return kernels.row_scale_backward(e, grad, *ctx.bounds), None, None


_ROW_SCALE_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def row_scale(log_scale: Tensor, lo: float, hi: float) -> Tensor:
    """The learned row scale of surface.py:84-85; GPU log-scales (fp32, fp16,
    bf16) take the fused kernels, anything else torch's operators."""

    if log_scale.device.type == "cuda" and log_scale.dtype in _ROW_SCALE_DTYPES:
        return RowScaleFn.apply(log_scale, float(lo), float(hi))
    return log_scale.exp().clamp(lo, hi)


# Bytes of fp32 temporaries the initial quantization may hold at once; a
# vocabulary-sized weight is converted in row bands rather than copied whole.
_INIT_BUDGET = 64 << 20


def quantize_weight(weight: Tensor, cfg: QSTEConfig) -> tuple[Tensor, Tensor]:
    """Initial (row scale, int8 coordinate) from a float weight.

    The arithmetic of ``surface.py:41-62``, which fixes the starting
    coordinates: scale = max(mean |w|, 1e-5) per row; latent =
    clamp(w / scale, +-1.5) * 0.25; coordinate = round(latent / clip * 127)
    clamped to +-127, and a zero becomes +-1 after the weight's sign (a zero
    coordinate would decode to +1 whatever the weight's sign was).
    """

    rows, columns = weight.shape
    scales = torch.empty(rows, device=weight.device, dtype=torch.float32)
    coordinate = torch.empty(rows, columns, device=weight.device, dtype=torch.int8)
    band = max(1, _INIT_BUDGET // max(1, 8 * columns))
    for r0 in range(0, rows, band):
        w = weight[r0:r0 + band].float()
        s = w.abs().mean(dim=1).clamp_min_(1e-5)
        q = (w / s.unsqueeze(1)).clamp_(-1.5, 1.5).mul_(0.25)
        q = q.div_(cfg.coordinate_clip).mul_(127).round_().clamp_(-127, 127).to(torch.int8)
        away = (w >= 0).to(torch.int8).mul_(2).sub_(1)  # +1 / -1 after the sign
        coordinate[r0:r0 + band] = torch.where(q == 0, away, q)
        scales[r0:r0 + band] = s
    return scales, coordinate


class EvidenceLedger:
    """Where one surface's coordinate evidence waits between backward and the step.

    ``open_uses``  forwards run under autograd whose backward has not arrived;
    ``tied``       the running sum of the current backward's uses while more
                   are due (accumulation dtype), or None;
    ``held``       evidence kept across backwards for the step (accumulation
                   dtype), or None; a prepared buffer keeps its address;
    ``sink``       the optimizer's apply callback, or None while it defers.
    """

    __slots__ = ("open_uses", "tied", "held", "sink", "accum")

    def __init__(self, accum: torch.dtype):
        self.open_uses = 0
        self.tied: Optional[Tensor] = None
        self.held: Optional[Tensor] = None
        self.sink: Optional[Sink] = None
        self.accum = accum

    def deliver(self, surface: "Surface", evidence: Tensor) -> None:
        """One use's evidence arrives from backward."""

        self.open_uses = max(0, self.open_uses - 1)
        last = self.open_uses == 0
        if last and self.tied is None:
            if self.sink is not None and self.held is None:
                self.sink(surface, evidence.detach().float())
                return
            if self.sink is None and self.held is not None:
                self.held.add_(evidence.detach().to(self.held.dtype))
                return
        part = evidence.detach().to(self.accum)
        self.tied = part.clone() if self.tied is None else self.tied.add_(part)
        if not last:
            return
        whole, self.tied = self.tied.float(), None
        if self.sink is not None:
            if self.held is not None:
                whole.add_(self.held.float())
                self.held = None
            self.sink(surface, whole)
        elif self.held is None:
            self.held = whole.to(self.accum)
        else:
            self.held.add_(whole.to(self.accum))

    def drain(self, keep_buffer: bool) -> Optional[Tensor]:
        """Everything pending as one fp32 tensor (None if nothing is).

        With ``keep_buffer`` a held buffer stays allocated and is cleared;
        what is returned is then always a copy, never the buffer itself (an
        fp32 buffer's ``.float()`` would be the buffer, and clearing it would
        hand the step zeros).
        """

        total = None
        if self.tied is not None:
            total, self.tied = self.tied.float(), None
        if self.held is not None:
            mine = self.held.to(torch.float32, copy=keep_buffer)
            total = mine if total is None else total.add_(mine)
            if keep_buffer:
                self.held.zero_()
            else:
                self.held = None
        self.open_uses = 0
        return total

    def fix_buffer(self, shape: tuple[int, int], device: torch.device) -> None:
        """A zeroed buffer at a fixed address for accumulation or capture."""

        self.forget_uses()
        self.held = torch.zeros(shape, device=device, dtype=self.accum)

    def forget_uses(self) -> None:
        self.tied = None
        self.open_uses = 0

    def divide(self, divisor: float) -> None:
        if divisor == 0:
            raise ValueError("gradient scale must be nonzero")
        for buffer in (self.held, self.tied):
            if buffer is not None:
                buffer.div_(divisor)


class Surface(nn.Module):
    """A shareable binary matrix; tied weights share one instance."""

    def __init__(self, weight: Tensor, cfg: QSTEConfig | None = None):
        super().__init__()
        if weight.ndim != 2:
            raise ValueError("a QSTE surface must wrap a rank-2 weight")
        cfg = coerce_config(cfg)
        initial_scale, coordinate = quantize_weight(weight.detach(), cfg)
        self._install(cfg, coordinate, initial_scale.log())

    @classmethod
    def from_state(cls, coordinate: Tensor, log_scale: Tensor,
                   cfg: QSTEConfig | None = None) -> "Surface":
        """A surface holding the given int8 coordinate and fp32 log row scale.

        For restoring saved state or building seeded synthetic layers; the
        packed signs are derived from the coordinate on the GPU.
        """

        if coordinate.dtype != torch.int8 or coordinate.ndim != 2:
            raise ValueError("coordinate must be a rank-2 int8 tensor")
        if log_scale.shape != (coordinate.shape[0],):
            raise ValueError("log_scale must have one entry per row")
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self._install(coerce_config(cfg), coordinate.contiguous(), log_scale.detach().float().clone())
        return self

    def _install(self, cfg: QSTEConfig, coordinate: Tensor, log_scale: Tensor) -> None:
        self.cfg = cfg
        self.rows, self.columns = (int(s) for s in coordinate.shape)
        # parameters (not buffers) so FSDP/DDP own them; requires_grad=False
        # leaves the coordinate optimizer as their only writer
        self.coordinate = nn.Parameter(coordinate, requires_grad=False)
        self.packed_sign = nn.Parameter(_on_gpu(kernels.pack_coordinate, coordinate),
                                        requires_grad=False)
        self.log_scale = nn.Parameter(log_scale)
        self.ledger = EvidenceLedger(_ACCUM_DTYPE[cfg.evidence_accum_dtype])

    # -- forward-side state ------------------------------------------------

    @property
    def scale(self) -> Tensor:
        return row_scale(self.log_scale, self.cfg.scale_min, self.cfg.scale_max)

    @property
    def sign(self) -> Tensor:
        """Dense +-1 fp32 view of the packed matrix (allocates rows x columns)."""

        return _on_gpu(kernels.unpack_rows, self.packed_sign.data, self.columns)

    @torch.no_grad()
    def dense_weight(self) -> Tensor:
        return self.sign.mul_(self.scale.detach().unsqueeze(1).to(self.packed_sign.device))

    def extra_repr(self) -> str:
        return f"rows={self.rows}, columns={self.columns}"

    # -- evidence (the reference's Surface methods, routed by the ledger) ------

    def route_evidence(self, sink: Sink | None) -> None:
        """Where complete evidence goes: the optimizer's apply, or None to hold it."""

        self.ledger.sink = sink

    def note_forward(self) -> None:
        if torch.is_grad_enabled():
            self.ledger.open_uses += 1

    @torch.no_grad()
    def reset_tracking(self) -> None:
        self.ledger.forget_uses()

    @torch.no_grad()
    def consume_evidence(self, evidence: Tensor) -> None:
        """Accept one use's worth of coordinate evidence (fp32 [rows, columns])."""

        self.ledger.deliver(self, evidence)

    @torch.no_grad()
    def flush_evidence(self, *, keep_buffer: bool = False) -> Tensor | None:
        """Everything accumulated, whether or not the forward count balanced."""

        return self.ledger.drain(keep_buffer)

    @torch.no_grad()
    def prepare_accumulator(self) -> None:
        self.ledger.fix_buffer((self.rows, self.columns), self.coordinate.device)

    @torch.no_grad()
    def scale_evidence_(self, divisor: float) -> None:
        self.ledger.divide(divisor)

    @torch.no_grad()
    def refresh_packed(self) -> None:
        """Rebuild packed signs after an out-of-band coordinate write."""

        self.packed_sign.data.copy_(_on_gpu(kernels.pack_coordinate, self.coordinate.data))

    def memory(self) -> dict[str, int]:
        """Bytes this surface holds, by role, against an fp32 matrix."""

        return {
            "packed_sign": self.packed_sign.numel(),
            "coordinate": self.coordinate.numel(),
            "log_scale": self.log_scale.numel() * 4,
            "float_equivalent": self.rows * self.columns * 4,
        }
