"""The reference's CPU algorithm, restated for timing -- TEST INFRASTRUCTURE.

Used only by ``bench.py``'s ``cpu_baseline`` leg (and its CPU test).  It runs
what the reference's native CPU backend (``src/qste/kernels/cpu.cpp``) runs,
multi-threaded on the host:

* forward / input gradient / evidence: packed signs expanded to +-1 floats
  one tile of rows at a time (``cpu_port.c`` ``cp_expand``; cpu.cpp expands
  through a byte table, cpu.cpp:59-87, 103-125) and each tile handed to torch's
  fp32 CPU GEMM (``torch.mm`` / ``addmm_`` are the reference's ``at::mm`` /
  ``addmm_``, cpu.cpp:342-456), the row scale folded into the expanded tile
  for the input gradient (cpu.cpp:402) and the per-sample scale into the
  gradient tile for the evidence (cpu.cpp:444-447);
* activation encoding, row inner product and the coordinate step's four
  dependent phases: ``cpu_port.c`` with OpenMP (cpu.cpp:143-203, 460-496,
  578-808);
* the layer's backward composition of ``functional.py:173-194``.

Everything is fp32, as the reference's CPU kernels are fp32-only
(``src/qste/functional.py:56-61``; ``cpu.cpp:347-348``).  This is not the
checker: numerics follow cpu.cpp, not the specification the oracle restates.
"""

from __future__ import annotations

import ctypes
import os
import platform
from pathlib import Path

import numpy as np
import torch

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "libqste_cpuport.so"
_lib = None

# expansion budget per tile (cpu.cpp sizes it by timing the host; 4 MiB is
# a typical per-core L2 share and keeps the BLAS calls large)
TILE_BYTES = 4 << 20


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            import oracle

            oracle.build(force=True)
        h = ctypes.CDLL(str(_LIB_PATH))
        vp, i64, dbl = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double
        h.cp_threads.restype = ctypes.c_int
        h.cp_set_threads.argtypes = [ctypes.c_int]
        h.cp_expand.argtypes = [vp, i64, i64, vp]
        h.cp_scale_rows.argtypes = [vp, i64, i64, vp]
        h.cp_pack_affine_rows.argtypes = [vp, i64, i64, vp, vp, vp]
        h.cp_row_inner.argtypes = [vp, vp, i64, i64, vp]
        h.cp_coordinate_update.restype = i64
        h.cp_coordinate_update.argtypes = [vp, vp, vp, vp, vp, vp, vp, i64, i64, dbl, dbl, dbl, dbl,
                                           i64, i64, i64]
        _lib = h
    return _lib


def set_threads(n: int) -> int:
    """Threads for the port's OpenMP loops and torch's CPU GEMMs."""

    n = max(1, int(n))
    lib().cp_set_threads(n)
    torch.set_num_threads(n)
    return n


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _p(t: torch.Tensor) -> int:
    return t.data_ptr()


def _tile_rows(stride: int, limit: int) -> int:
    return max(1, min(limit, max(TILE_BYTES // (stride * 32), 8)))


def _expanded(packed: torch.Tensor, r0: int, n: int, scratch: torch.Tensor, columns: int) -> torch.Tensor:
    stride = packed.shape[1]
    lib().cp_expand(_p(packed) + r0 * stride, n, stride, _p(scratch))
    return scratch[:n, :columns]


def pack_affine_rows(x: torch.Tensor):
    rows, cols = x.shape
    bits = torch.empty(rows, (cols + 7) // 8, dtype=torch.uint8)
    off = torch.empty(rows)
    xs = torch.empty(rows)
    lib().cp_pack_affine_rows(_p(x), rows, cols, _p(bits), _p(off), _p(xs))
    return bits, off, xs


def linear_forward(x, packed, scale, bias, columns):
    """(x @ sign^T) * scale + bias (cpu.cpp:342-371)."""

    rows, stride = packed.shape
    out = torch.empty(x.shape[0], rows)
    tile = _tile_rows(stride, rows)
    scratch = torch.empty(tile, stride * 8)
    for r0 in range(0, rows, tile):
        n = min(tile, rows - r0)
        out[:, r0:r0 + n].copy_(torch.mm(x, _expanded(packed, r0, n, scratch, columns).t()))
    out.mul_(scale.view(1, rows))
    if bias is not None:
        out.add_(bias.view(1, rows))
    return out


def linear_dgrad(dy, packed, scale, columns):
    """dy @ (scale * sign) (cpu.cpp:375-410)."""

    rows, stride = packed.shape
    out = torch.zeros(dy.shape[0], columns)
    tile = _tile_rows(stride, rows)
    scratch = torch.empty(tile, stride * 8)
    for r0 in range(0, rows, tile):
        n = min(tile, rows - r0)
        lib().cp_expand(_p(packed) + r0 * stride, n, stride, _p(scratch))
        lib().cp_scale_rows(_p(scratch), n, stride * 8, _p(scale) + 4 * r0)
        out.addmm_(dy[:, r0:r0 + n], scratch[:n, :columns])
    return out


def evidence(dy, packed_x, xs, columns):
    """dy^T @ (xs * sign(x)) (cpu.cpp:416-456)."""

    samples, rows = dy.shape
    stride = packed_x.shape[1]
    out = torch.zeros(rows, columns)
    tile = _tile_rows(stride, samples)
    scratch = torch.empty(tile, stride * 8)
    g = torch.empty(tile, rows)
    for t0 in range(0, samples, tile):
        n = min(tile, samples - t0)
        signs = _expanded(packed_x, t0, n, scratch, columns)
        torch.mul(dy[t0:t0 + n], xs[t0:t0 + n, None], out=g[:n])
        out.addmm_(g[:n].t(), signs)
    return out


def layer_backward(dy, saved, packed_w, scale, columns, need_input=True):
    """functional.py:173-194: dX, E = E0 * s, gs = row_inner(E0, sign_w), db."""

    bits, off, xs = saved
    dx = linear_dgrad(dy, packed_w, scale, columns) if need_input else None
    e0 = evidence(dy, bits, xs, columns)
    e0.add_((dy.t() @ off)[:, None])
    gs = torch.empty(e0.shape[0])
    lib().cp_row_inner(_p(e0), _p(packed_w), e0.shape[0], columns, _p(gs))
    return dx, e0.mul_(scale[:, None]), gs, dy.sum(0)


class Surface:
    """One layer's packed signs, scale and optimizer state (numpy-backed torch)."""

    def __init__(self, coord: np.ndarray, scale: np.ndarray, block: int = 256):
        rows, cols = coord.shape
        self.columns = cols
        c = torch.from_numpy(np.ascontiguousarray(coord, dtype=np.int8))
        self.coord = c.clone()
        self.packed = torch.from_numpy(np.packbits(coord >= 0, axis=1, bitorder="little"))
        self.scale = torch.from_numpy(np.ascontiguousarray(scale, dtype=np.float32))
        blocks = (rows * cols + block - 1) // block
        self.block = block
        self.moment_q = torch.zeros(rows, cols, dtype=torch.int8)
        self.moment_scale = torch.full((blocks,), 1 / 127, dtype=torch.float16)
        self.row_v = torch.zeros(rows, dtype=torch.float16)
        self.col_v = torch.zeros(cols, dtype=torch.float16)

    def step(self, evidence: torch.Tensor, seed: int, step: int, lr: float = 1.0) -> int:
        rows, cols = evidence.shape
        return int(lib().cp_coordinate_update(
            _p(evidence), _p(self.coord), _p(self.packed), _p(self.moment_q), _p(self.moment_scale),
            _p(self.row_v), _p(self.col_v), rows, cols, 0.9, 0.99, 2.0, lr, self.block, seed, step))


def cfg1_step(x, target, layer: Surface, step: int = 0) -> int:
    """Config 1: one QSTE Linear, forward, MSE against target, backward, one
    coordinate step (seed 1, the optimizer's first surface)."""

    saved = pack_affine_rows(x)
    y = linear_forward(x, layer.packed, layer.scale, None, layer.columns)
    dy = (y - target).mul_(2.0 / y.numel())
    _, ev, _, _ = layer_backward(dy, saved, layer.packed, layer.scale, layer.columns)
    return layer.step(ev, seed=1, step=step)


def swiglu_products(x, dy, layers):
    """Config 4's token-proportional work: forward of gate, up and down with
    the encodings, SwiGLU, and every layer's backward products.  Returns the
    three layers' evidence for the coordinate step."""

    gate, up, down = layers
    d = x.shape[1]
    sx = pack_affine_rows(x)
    g = linear_forward(x, gate.packed, gate.scale, None, d)
    u = linear_forward(x, up.packed, up.scale, None, d)
    sig = torch.sigmoid(g)
    act = g * sig
    h = act * u
    sh = pack_affine_rows(h)
    linear_forward(h, down.packed, down.scale, None, h.shape[1])
    dh, e_down, _, _ = layer_backward(dy, sh, down.packed, down.scale, h.shape[1])
    du = dh * act
    dg = dh * u * (sig * (1 + g * (1 - sig)))
    _, e_up, _, _ = layer_backward(du, sx, up.packed, up.scale, d)
    _, e_gate, _, _ = layer_backward(dg, sx, gate.packed, gate.scale, d)
    return e_gate, e_up, e_down


def default_threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
