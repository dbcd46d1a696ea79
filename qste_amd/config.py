"""Hyper-parameters of QSTE surfaces and the coordinate optimizer.

Field names, defaults and validation are the reference's
(``src/qste/config.py:8-65``) so a config object or dict moves between the two
unchanged.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass


@dataclass(frozen=True)
class QSTEConfig:
    """Immutable training recipe for binary surfaces.

    coordinate_clip      latent range the int8 coordinate spans at init
    coordinate_lr        step size, in coordinate units, per optimizer step
    beta1                first-moment decay of the coordinate optimizer
    beta2                decay of the factored row/column second moments
    update_rms_clip      global RMS ceiling of the normalized update
    momentum_block_size  elements sharing one fp16 momentum scale
    seed                 base seed of the stochastic-rounding stream
    scale_min/scale_max  clamp of the learned per-row scale
    evidence_accum_dtype dtype of deferred evidence buffers ("fp16"/"fp32")
    """

    coordinate_clip: float = 1.5
    coordinate_lr: float = 1.0
    beta1: float = 0.9
    beta2: float = 0.99
    update_rms_clip: float = 2.0
    momentum_block_size: int = 256
    seed: int = 1
    scale_min: float = 1e-6
    scale_max: float = 4.0
    evidence_accum_dtype: str = "fp16"

    def __post_init__(self) -> None:
        if self.coordinate_clip <= 0 or self.coordinate_lr <= 0:
            raise ValueError("coordinate_clip and coordinate_lr must be positive")
        if not (0 <= self.beta1 < 1 and 0 <= self.beta2 < 1):
            raise ValueError("beta1 and beta2 must be in [0, 1)")
        if self.update_rms_clip <= 0 or self.momentum_block_size <= 0:
            raise ValueError("update_rms_clip and momentum_block_size must be positive")
        if not 0 < self.scale_min < self.scale_max:
            raise ValueError("scale bounds must satisfy 0 < scale_min < scale_max")
        if self.evidence_accum_dtype not in ("fp16", "fp32"):
            raise ValueError("evidence_accum_dtype must be 'fp16' or 'fp32'")

    def metadata(self) -> dict[str, object]:
        return asdict(self)


def coerce_config(cfg) -> QSTEConfig:
    """``None`` -> defaults; a mapping -> a config; a config -> itself."""

    if cfg is None:
        return QSTEConfig()
    if isinstance(cfg, QSTEConfig):
        return cfg
    return QSTEConfig(**dict(cfg))
