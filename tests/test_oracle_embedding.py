"""The embedding oracle (``oracle/embedding.py``), pinned on the CPU.

* the lookup equals dense indexing of the unpacked, scaled matrix;
* the evidence equals torch's own sequential ``index_add_`` on the CPU bit for
  bit (repeated ids included), times the row scale;
* the scale gradient equals a float64 row inner product of ``index_add_``
  with the signs, rounded once.
"""

from __future__ import annotations

import numpy as np
import torch

import oracle
from oracle import embedding as oe


def _case(rows=40, cols=21, seed=12):
    rng = np.random.default_rng(seed)
    coord = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    packed = oracle.pack_coordinate(coord)
    scale = (rng.random(rows) + 0.5).astype(np.float32)
    return coord, packed, scale


def test_lookup_is_dense_indexing():
    coord, packed, scale = _case()
    ids = np.random.default_rng(1).integers(0, 40, size=(3, 5))
    dense = np.where(coord >= 0, 1.0, -1.0).astype(np.float32) * scale[:, None]
    assert np.array_equal(oe.lookup(ids, packed, scale, 21), dense[ids])


def test_evidence_is_index_add_in_token_order():
    coord, packed, scale = _case()
    rng = np.random.default_rng(2)
    ids = rng.integers(0, 10, size=(64,))  # many repeats
    grad = rng.standard_normal((64, 21)).astype(np.float32) * 3
    ev, gs = oe.backward(ids, grad, packed, scale, 21)
    e0 = torch.zeros(40, 21).index_add_(0, torch.from_numpy(ids), torch.from_numpy(grad))
    assert np.array_equal(ev, (e0 * torch.from_numpy(scale)[:, None]).numpy())
    sign = np.where(coord >= 0, 1.0, -1.0)
    expected = (e0.numpy().astype(np.float64) * sign).sum(axis=1).astype(np.float32)
    assert np.array_equal(gs, expected)
    # rows without tokens are zero
    assert not ev[10:].any() and not gs[10:].any()
