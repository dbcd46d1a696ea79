"""CPU oracle for the binary embedding -- TEST INFRASTRUCTURE.

Only ``tests/`` may import it, as the checker.  It restates
``fallback.packed_embedding`` (``src/qste/kernels/fallback.py:151-155``) and
``QSTEEmbeddingFn.backward`` (``src/qste/functional.py:274-286``) in numpy:

* lookup: ``sign(packed[ids]) * scale[ids]`` (``unpack_rows`` of the selected
  rows times their scale; +-scale is exact in any dtype scale comes in);
* evidence: ``zeros(R, C)`` plus every gradient row added to its id's row in
  ascending token order in fp32 (``np.add.at`` is unbuffered and applies the
  additions in index order, as a sequential ``index_add_`` does), the scale
  gradient as the row inner product with the signs (float64, then fp32), and
  the evidence times the row scale (fp32).

Pinned in ``tests/test_oracle_embedding.py`` against torch's own
``index_add_`` on the CPU (bit for bit), dense indexing of the unpacked
matrix, and a float64 row inner product.
"""

from __future__ import annotations

import numpy as np

from . import unpack_rows


def lookup(ids: np.ndarray, packed: np.ndarray, scale: np.ndarray, cols: int) -> np.ndarray:
    flat = np.asarray(ids, dtype=np.int64).reshape(-1)
    rows = unpack_rows(packed[flat], cols).astype(np.float32)
    out = rows * np.asarray(scale, dtype=np.float32)[flat, None]
    return out.reshape(*np.shape(ids), cols)


def backward(ids: np.ndarray, grad: np.ndarray, packed: np.ndarray, scale: np.ndarray,
             cols: int) -> tuple[np.ndarray, np.ndarray]:
    """(evidence fp32 [R, C], grad_scale fp32 [R])."""

    flat = np.asarray(ids, dtype=np.int64).reshape(-1)
    g = np.asarray(grad, dtype=np.float32).reshape(-1, cols)
    rows = packed.shape[0]
    e0 = np.zeros((rows, cols), dtype=np.float32)
    np.add.at(e0, flat, g)
    sign = unpack_rows(packed, cols).astype(np.float64)
    grad_scale = (e0.astype(np.float64) * sign).sum(axis=1).astype(np.float32)
    evidence = e0 * np.asarray(scale, dtype=np.float32)[:, None]
    return evidence.astype(np.float32), grad_scale
