"""The CPU baseline's port of the reference's CPU backend (oracle/cpu_baseline.py,
oracle/cpu_port.c) checked against the oracle, so the timed baseline computes
what the reference's CPU path computes and not something cheaper.

Its products must equal the float64 oracle within fp32 GEMM error, its
activation bits must equal the oracle's, and its four-phase step (cpu.cpp's
numerics: +1e-12 after the mean, fp32 sums, one division for the step size)
must keep the step's invariants and land on the specification's integers
almost everywhere.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import cpu_baseline as cb


def _rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.fixture(autouse=True)
def _threads():
    cb.set_threads(4)


def test_port_products_match_the_oracle():
    rng = np.random.default_rng(3)
    rows, cols, m = 96, 203, 40
    coord = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    scale = (np.abs(rng.standard_normal(rows)) * 0.02 + 0.01).astype(np.float32)
    layer = cb.Surface(coord, scale)
    assert np.array_equal(layer.packed.numpy(), oracle.pack_coordinate(coord))
    x = torch.from_numpy(rng.standard_normal((m, cols)).astype(np.float32))
    dy = torch.from_numpy(rng.standard_normal((m, rows)).astype(np.float32))
    bias = torch.from_numpy(rng.standard_normal(rows).astype(np.float32))
    y = cb.linear_forward(x, layer.packed, layer.scale, bias, cols)
    assert _rel(y, oracle.linear_fwd(x.numpy(), layer.packed.numpy(), scale, bias.numpy(), cols)) <= 1e-6
    dx = cb.linear_dgrad(dy, layer.packed, layer.scale, cols)
    assert _rel(dx, oracle.linear_dgrad(dy.numpy(), layer.packed.numpy(), cols, scale)) <= 1e-6
    bits, off, xs = cb.pack_affine_rows(x)
    obits, ooff, oxs = oracle.pack_affine_rows(x.numpy())
    assert np.array_equal(bits.numpy(), obits)
    assert _rel(off, ooff) <= 1e-6 and _rel(xs, oxs) <= 1e-6
    _, ev, gs, db = cb.layer_backward(dy, (bits, off, xs), layer.packed, layer.scale, cols)
    e0 = oracle.decoded_evidence(dy.numpy(), obits, ooff, oxs, cols)
    assert _rel(ev, e0 * scale.astype(np.float64)[:, None]) <= 1e-6
    assert _rel(gs, oracle.row_inner(e0.astype(np.float32), layer.packed.numpy(), cols)) <= 1e-5
    assert _rel(db, dy.numpy().astype(np.float64).sum(0)) <= 1e-6


def test_port_step_keeps_the_invariants_and_the_spec_integers():
    rng = np.random.default_rng(5)
    rows, cols = 128, 520
    coord = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    layer = cb.Surface(coord, np.ones(rows, np.float32))
    state = oracle.fresh_state(coord, 256)
    for step in range(3):
        ev = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
        before = layer.packed.numpy().copy()
        flips = layer.step(torch.from_numpy(ev.copy()), seed=7, step=step)
        oracle.coordinate_update(ev, state, beta1=0.9, beta2=0.99, update_clip=2.0, coordinate_lr=1.0,
                                 block_size=256, seed=7, step=step)
        got = layer.coord.numpy()
        assert np.array_equal(layer.packed.numpy(), oracle.pack_coordinate(got))
        assert np.abs(got.astype(int)).max() <= 127
        assert np.abs(layer.moment_q.numpy().astype(int)).max() <= 127
        diff = np.unpackbits(before ^ layer.packed.numpy(), axis=1, bitorder="little")[:, :cols]
        assert flips == int(diff.sum()) and flips > 0
        # cpu.cpp's numerics move a handful of rounding decisions by one
        assert np.mean(got != state["coordinate"]) < 0.01
        assert np.abs(got.astype(int) - state["coordinate"]).max() <= 1
