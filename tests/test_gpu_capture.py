"""Graph capture and deferred evidence, on the GPU.

* The coordinate step records into a HIP graph with a device step counter,
  a device flip count and an enable flag (the reference's capture contract,
  ``cuda.py:1724-1729``, ``tests/test_gpu.py:519-553``).  Each replay --
  with eager work and a step increment between replays -- is compared bit for
  bit with the same step run eagerly on a copy of the state (coordinates,
  packed signs, int8 momentum, fp16 scales and statistics, flips); a replay
  with the flag cleared writes nothing.
* A layer's whole backward (``linear_backward``: column sums, the split-K
  backward launch and its combine pass, at config 2's shapes) records into a
  graph; every replay, with eager work between replays, equals an eager call
  bit for bit (the products are deterministic).
* Gradient accumulation (``prepare_accumulation``, ``optim.py:120-135``):
  four microbatches leave the evidence one batch gives, to summation order,
  and coordinates within one step of it (the reference's
  ``tests/test_learning.py:174-212``); ``unscale_`` divides the held evidence.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn as nn

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _state(rows, cols, seed):
    from qste_amd import kernels

    g = torch.Generator(device=DEV).manual_seed(seed)
    coord = torch.randint(-100, 100, (rows, cols), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    return {
        "coordinate": coord,
        "packed": kernels.pack_coordinate(coord),
        "moment_q": torch.zeros_like(coord),
        "moment_scale": torch.full(((rows * cols + 255) // 256,), 1 / 127, dtype=torch.float16, device=DEV),
        "row_v": torch.zeros(rows, dtype=torch.float16, device=DEV),
        "col_v": torch.zeros(cols, dtype=torch.float16, device=DEV),
    }


def _update(st, grad, step, flips, enabled=None):
    from qste_amd import kernels

    return kernels.coordinate_update(
        grad, st["coordinate"], st["packed"], st["moment_q"], st["moment_scale"], st["row_v"], st["col_v"],
        beta1=0.9, beta2=0.99, update_clip=2.0, coordinate_lr=1.0, block_size=256, seed=1, step=step,
        flips=flips, update_enabled=enabled)


@pytest.mark.parametrize("rows,cols", [(64, 128), (256, 1024)])
def test_graph_replays_equal_eager_steps(rows, cols):
    g = torch.Generator(device=DEV).manual_seed(7)
    grad = torch.randn(rows, cols, generator=g, device=DEV)
    st = _state(rows, cols, 3)
    ref = {k: v.clone() for k, v in st.items()}
    step = torch.zeros((), dtype=torch.int64, device=DEV)
    flips = torch.zeros((), dtype=torch.int64, device=DEV)
    enabled = torch.ones((), dtype=torch.uint8, device=DEV)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm up off the capture
        warm = {k: v.clone() for k, v in st.items()}
        _update(warm, grad, step, flips, enabled)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _update(st, grad, step, flips, enabled)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        expected_flips = _update(ref, grad, i, None)
        for key in st:
            assert torch.equal(st[key], ref[key]), (i, key)
        assert int(flips) == expected_flips
        # eager work between replays, then the next step number
        _ = (grad * 2).sum().item()
        step.add_(1)
    # the enable flag cleared: a replay writes no state
    before = {k: v.clone() for k, v in st.items()}
    enabled.zero_()
    graph.replay()
    torch.cuda.synchronize()
    for key in st:
        assert torch.equal(st[key], before[key]), key
    assert int(flips) == 0


@pytest.mark.parametrize("rows,cols", [(4096, 1024), (1024, 4096)])
def test_layer_backward_graph_replays_equal_eager(rows, cols):
    from qste_amd import kernels

    T = 8192
    g = torch.Generator(device=DEV).manual_seed(rows)
    x = torch.randn(T, cols, generator=g, device=DEV).to(torch.bfloat16)
    dy = torch.randn(T, rows, generator=g, device=DEV).to(torch.bfloat16)
    coord = torch.randint(-127, 128, (rows, cols), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    packed = kernels.pack_coordinate(coord)
    scale = torch.rand(rows, generator=g, device=DEV) * 0.02 + 0.005
    xb, off, xs = kernels.pack_affine_rows(x)

    def call():
        return kernels.linear_backward(dy, xb, off, xs, packed, scale, cols, need_bias=True)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm up off the capture
        call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = call()
    for i in range(3):
        dy.mul_(-1.0 if i % 2 else 0.5)  # new gradient values, eager, between replays
        graph.replay()
        torch.cuda.synchronize()
        want = call()
        for name, got, ref in zip(("dx", "evidence", "grad_scale", "grad_bias"), outs, want):
            assert torch.equal(got, ref), (i, name)
        _ = (dy.float() * 2).sum().item()


@pytest.mark.parametrize("accum,tol", [("fp32", 1e-5), ("fp16", 2e-3)])
def test_gradient_accumulation_matches_one_large_batch(accum, tol):
    import qste_amd as qste

    def run(microbatches):
        torch.manual_seed(10)
        # the accumulation buffer takes the surface's config (convert's), as
        # in the reference (surface.py:197-206)
        cfg = {"coordinate_lr": 4.0, "evidence_accum_dtype": accum}
        model = qste.convert(nn.Sequential(nn.Linear(256, 128, bias=False)), config=cfg).to(DEV)
        coords = qste.QSTEOptimizer(model, config=cfg)
        coords.prepare_accumulation()
        data = torch.randn(512, 256, generator=torch.Generator().manual_seed(11)).to(DEV)
        for chunk in data.chunk(microbatches):
            (model(chunk).square().sum() / len(data)).backward()
        surface = qste.surfaces(model)[0]
        evidence = surface.ledger.held.float().clone()
        before = surface.coordinate.clone()
        flips = coords.step()
        # the step ran on the accumulated evidence, not on a cleared buffer
        assert flips > 0
        assert int((surface.coordinate != before).sum()) > 0
        return evidence, surface.coordinate.clone()

    one_e, one_c = run(1)
    many_e, many_c = run(4)
    scale = one_e.pow(2).mean().sqrt().clamp_min(1e-12)
    assert float((one_e - many_e).pow(2).mean().sqrt() / scale) < tol
    diff = (one_c.int() - many_c.int()).abs()
    assert int(diff.max()) <= 1
    assert float((diff > 0).float().mean()) < 0.01


def test_unscale_divides_the_held_evidence():
    import qste_amd as qste

    torch.manual_seed(2)
    cfg = {"evidence_accum_dtype": "fp32"}
    model = qste.convert(nn.Sequential(nn.Linear(64, 32, bias=False)), config=cfg).to(DEV)
    coords = qste.QSTEOptimizer(model, config=cfg)
    coords.defer()
    x = torch.randn(16, 64, device=DEV)
    (model(x).sum() * 1024.0).backward()
    surface = qste.surfaces(model)[0]
    held = surface.ledger.held.float().clone()
    coords.unscale_(1024.0)
    assert torch.allclose(surface.ledger.held.float(), held / 1024.0, rtol=1e-6, atol=0)
    before = surface.coordinate.clone()
    assert coords.step() > 0
    assert int((surface.coordinate != before).sum()) > 0
    # deferred mode keeps the buffer for the next accumulation, emptied
    assert surface.ledger.held is not None and not surface.ledger.held.any()
