"""One binary matrix: its int8 coordinate, packed signs and row scale.

State layout and parameter names match the reference's ``Surface``
(``src/qste/surface.py:30-79``) so state dicts carry over:

    coordinate   int8  [rows, columns]      training state (optimizer-owned)
    packed_sign  uint8 [rows, ceil(cols/8)] forward weight, LSB-first bits
    log_scale    fp32  [rows]               learned row scale (host optimizer)

Evidence routing (immediate apply inside backward, accumulation for tied or
deferred surfaces, the forward-count backstop) follows
``src/qste/surface.py:104-206``.
"""

from __future__ import annotations

import torch
import torch.nn as nn
from torch import Tensor

from . import kernels
from .config import QSTEConfig, coerce_config

_ACCUM_DTYPE = {"fp16": torch.float16, "fp32": torch.float32}


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


def quantize_weight(weight: Tensor, cfg: QSTEConfig) -> tuple[Tensor, Tensor]:
    """Initial (row scale, int8 coordinate) from a float weight.

    surface.py:41-62: per-row scale = mean |w| (>= 1e-5); latent =
    clamp(w / scale, +-1.5) / 4; coordinate = round(latent / clip * 127)
    clamped to +-127, with a zero pushed one step toward the weight's sign.
    """

    rows, columns = weight.shape
    row_scale = torch.empty(rows, device=weight.device, dtype=torch.float32)
    coordinate = torch.empty(rows, columns, device=weight.device, dtype=torch.int8)
    chunk = max(1, (32 << 20) // max(1, columns * 12))
    for start in range(0, rows, chunk):
        stop = min(start + chunk, rows)
        value = weight[start:stop].float()
        scale = value.abs().mean(dim=1).clamp_min(1e-5)
        latent = (value / scale[:, None]).clamp(-1.5, 1.5) * 0.25
        q = (latent / cfg.coordinate_clip * 127).round().clamp(-127, 127).to(torch.int8)
        nudge = torch.where(value >= 0, torch.ones_like(q), -torch.ones_like(q))
        coordinate[start:stop] = torch.where(q == 0, nudge, q)
        row_scale[start:stop] = scale
    return row_scale, coordinate


class Surface(nn.Module):
    """A shareable binary matrix; tied weights share one instance."""

    def __init__(self, weight: Tensor, cfg: QSTEConfig | None = None):
        super().__init__()
        if weight.ndim != 2:
            raise ValueError("a QSTE surface must wrap a rank-2 weight")
        cfg = coerce_config(cfg)
        source = weight.detach()
        row_scale, coordinate = quantize_weight(source, cfg)
        self.cfg = cfg
        self.rows, self.columns = (int(s) for s in source.shape)
        self.coordinate = nn.Parameter(coordinate, requires_grad=False)
        self.packed_sign = nn.Parameter(_on_gpu(kernels.pack_coordinate, coordinate),
                                        requires_grad=False)
        self.log_scale = nn.Parameter(row_scale.log())
        self._evidence: Tensor | None = None
        self._call_evidence: Tensor | None = None
        self._pending_calls = 0
        self._immediate = None  # set by QSTEOptimizer

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
        self.cfg = coerce_config(cfg)
        self.rows, self.columns = (int(s) for s in coordinate.shape)
        self.coordinate = nn.Parameter(coordinate.contiguous(), requires_grad=False)
        self.packed_sign = nn.Parameter(_on_gpu(kernels.pack_coordinate, self.coordinate.data),
                                        requires_grad=False)
        self.log_scale = nn.Parameter(log_scale.detach().float().clone())
        self._evidence = None
        self._call_evidence = None
        self._pending_calls = 0
        self._immediate = None
        return self

    # -- forward-side state ------------------------------------------------

    @property
    def scale(self) -> Tensor:
        return self.log_scale.exp().clamp(self.cfg.scale_min, self.cfg.scale_max)

    @property
    def sign(self) -> Tensor:
        """Dense +-1 fp32 view of the packed matrix (allocates rows x columns)."""

        return _on_gpu(kernels.unpack_rows, self.packed_sign.data, self.columns)

    @torch.no_grad()
    def dense_weight(self) -> Tensor:
        return self.sign.mul_(self.scale.detach().unsqueeze(1).to(self.packed_sign.device))

    def extra_repr(self) -> str:
        return f"rows={self.rows}, columns={self.columns}"

    # -- evidence bookkeeping (surface.py:104-206) --------------------------

    def note_forward(self) -> None:
        if torch.is_grad_enabled():
            self._pending_calls += 1

    @torch.no_grad()
    def reset_tracking(self) -> None:
        self._call_evidence = None
        self._pending_calls = 0

    @torch.no_grad()
    def consume_evidence(self, evidence: Tensor) -> None:
        """Accept one use's worth of coordinate evidence (fp32 [rows, columns]).

        The common single-use case hands it straight to the optimizer inside
        backward; a tied surface sums its uses first.
        """

        self._pending_calls = max(0, self._pending_calls - 1)
        immediate = self._immediate
        if (self._pending_calls == 0 and self._call_evidence is None
                and self._evidence is None and immediate is not None):
            immediate(self, evidence.detach().float())
            return
        if (self._pending_calls == 0 and self._call_evidence is None
                and self._evidence is not None and immediate is None):
            self._evidence.add_(evidence.detach().to(self._evidence.dtype))
            return

        accum = _ACCUM_DTYPE[self.cfg.evidence_accum_dtype]
        compact = evidence.detach().to(accum)
        if self._call_evidence is None:
            self._call_evidence = compact.clone()
        else:
            self._call_evidence.add_(compact)
        if self._pending_calls:
            return

        total = self._call_evidence.float()
        self._call_evidence = None
        if immediate is not None:
            if self._evidence is not None:
                total.add_(self._evidence.float())
                self._evidence = None
            immediate(self, total)
        elif self._evidence is None:
            self._evidence = total.to(accum)
        else:
            self._evidence.add_(total.to(accum))

    @torch.no_grad()
    def flush_evidence(self, *, keep_buffer: bool = False) -> Tensor | None:
        """Everything accumulated, whether or not the forward count balanced."""

        total = None
        if self._call_evidence is not None:
            total = self._call_evidence.float()
            self._call_evidence = None
        if self._evidence is not None:
            part = self._evidence.float()
            total = part if total is None else total.add_(part)
            if keep_buffer:
                self._evidence.zero_()
            else:
                self._evidence = None
        self._pending_calls = 0
        return total

    @torch.no_grad()
    def prepare_accumulator(self) -> None:
        self.reset_tracking()
        self._evidence = torch.zeros(
            self.rows, self.columns, device=self.coordinate.device,
            dtype=_ACCUM_DTYPE[self.cfg.evidence_accum_dtype])

    @torch.no_grad()
    def scale_evidence_(self, divisor: float) -> None:
        if divisor == 0:
            raise ValueError("gradient scale must be nonzero")
        for buffer in (self._evidence, self._call_evidence):
            if buffer is not None:
                buffer.div_(divisor)

    @torch.no_grad()
    def refresh_packed(self) -> None:
        """Rebuild packed signs after an out-of-band coordinate write."""

        self.packed_sign.data.copy_(_on_gpu(kernels.pack_coordinate, self.coordinate.data))

    def memory(self) -> dict[str, int]:
        return {
            "packed_sign": self.packed_sign.numel(),
            "coordinate": self.coordinate.numel(),
            "log_scale": self.log_scale.numel() * 4,
            "float_equivalent": self.rows * self.columns * 4,
        }
