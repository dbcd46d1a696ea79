"""The reference's CPU algorithm, restated for timing -- TEST INFRASTRUCTURE.

Used only by ``bench.py``'s ``cpu_baseline`` leg. It restates what the
reference's native CPU backend does (``src/qste/kernels/cpu.cpp``) with numpy:

* forward / input gradient / evidence: expand packed signs one tile of rows
  at a time through a byte -> 8 floats lookup table (cpu.cpp:59-87,
  103-125) and hand each expanded tile to an fp32 BLAS GEMM
  (cpu.cpp:342-456; numpy's matmul plays ATen's ``at::mm``), with the row
  scale folded into the expanded tile for the input gradient (cpu.cpp:402)
  and the per-sample scale folded into the gradient tile for the evidence
  (cpu.cpp:444-447);
* activation encoding and the coordinate step: the oracle's C restatement
  (``qste_oracle.c``; the reference's are ``cpu.cpp:143-203`` and
  ``cpu.cpp:578-808``).

Everything is fp32, as the reference's CPU kernels are fp32-only
(``src/qste/functional.py:56-61``; ``cpu.cpp:347-348``).
"""

from __future__ import annotations

import numpy as np

import oracle

_LUT = np.where((np.arange(256)[:, None] >> np.arange(8)[None, :]) & 1, 1.0, -1.0).astype(np.float32)
_TILE_BYTES = 1 << 20  # cpu.cpp:45, the default expansion budget


def _tile_rows(columns: int, limit: int) -> int:
    per_row = ((columns + 7) // 8) * 8 * 4
    return max(1, min(limit, max(_TILE_BYTES // per_row, 8)))


def _expand(packed: np.ndarray, columns: int) -> np.ndarray:
    return _LUT[packed].reshape(packed.shape[0], -1)[:, :columns]


def linear_forward(x: np.ndarray, packed: np.ndarray, scale: np.ndarray, columns: int) -> np.ndarray:
    rows = packed.shape[0]
    out = np.empty((x.shape[0], rows), dtype=np.float32)
    tile = _tile_rows(columns, rows)
    for r0 in range(0, rows, tile):
        w = _expand(packed[r0:r0 + tile], columns)
        out[:, r0:r0 + tile] = x @ w.T
    out *= scale[None, :]
    return out


def linear_dgrad(dy: np.ndarray, packed: np.ndarray, scale: np.ndarray, columns: int) -> np.ndarray:
    rows = packed.shape[0]
    out = np.zeros((dy.shape[0], columns), dtype=np.float32)
    tile = _tile_rows(columns, rows)
    for r0 in range(0, rows, tile):
        w = _expand(packed[r0:r0 + tile], columns) * scale[r0:r0 + tile, None]
        out += dy[:, r0:r0 + tile] @ w
    return out


def evidence(dy: np.ndarray, packed_x: np.ndarray, xs: np.ndarray, columns: int) -> np.ndarray:
    samples, rows = dy.shape
    out = np.zeros((rows, columns), dtype=np.float32)
    tile = _tile_rows(columns, samples)
    for t0 in range(0, samples, tile):
        signs = _expand(packed_x[t0:t0 + tile], columns)
        g = dy[t0:t0 + tile] * xs[t0:t0 + tile, None]
        out += g.T @ signs
    return out


def layer_backward(dy, packed_x, off, xs, packed_w, scale, columns):
    """dX, E = E0 * s and gs for one layer, as functional.py:173-194 does."""

    dx = linear_dgrad(dy, packed_w, scale, columns)
    e0 = evidence(dy, packed_x, xs, columns)
    e0 += (dy.T @ off)[:, None]
    gs = (e0 * _expand(packed_w, columns)).sum(1)
    return dx, e0 * scale[:, None], gs


def swiglu_mlp_step(x, layers, dy, block_size: int = 256, step: int = 0) -> int:
    """One fwd + bwd + coordinate step of a SwiGLU MLP on the CPU.

    ``layers`` = [(packed, scale, state) for gate, up, down]; ``state`` is an
    oracle optimizer state dict updated in place. Returns total flips.
    """

    (pg, sg, stg), (pu, su, stu), (pd, sd, std) = layers
    d = x.shape[1]
    ffn = pg.shape[0]
    bx, offx, xsx = oracle.pack_affine_rows(x)
    g = linear_forward(x, pg, sg, d)
    u = linear_forward(x, pu, su, d)
    sig = 1.0 / (1.0 + np.exp(-g))
    act = g * sig
    h = act * u
    bh, offh, xsh = oracle.pack_affine_rows(h)
    _ = linear_forward(h, pd, sd, ffn)
    flips = 0
    dh, e_down, _ = layer_backward(dy, bh, offh, xsh, pd, sd, ffn)
    flips += oracle.coordinate_update(e_down, std, beta1=0.9, beta2=0.99, update_clip=2.0,
                                      coordinate_lr=1.0, block_size=block_size, seed=1 + 2 * 1_000_003,
                                      step=step)
    du = dh * act
    dg = dh * u * (sig * (1 + g * (1 - sig)))
    _, e_up, _ = layer_backward(du, bx, offx, xsx, pu, su, d)
    flips += oracle.coordinate_update(e_up, stu, beta1=0.9, beta2=0.99, update_clip=2.0,
                                      coordinate_lr=1.0, block_size=block_size, seed=1 + 1_000_003,
                                      step=step)
    _, e_gate, _ = layer_backward(dg, bx, offx, xsx, pg, sg, d)
    flips += oracle.coordinate_update(e_gate, stg, beta1=0.9, beta2=0.99, update_clip=2.0,
                                      coordinate_lr=1.0, block_size=block_size, seed=1, step=step)
    return flips
