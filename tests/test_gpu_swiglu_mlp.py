"""The SwiGLU MLP as one autograd node (``qste_amd.nn.swiglu_mlp``).

Its one new product, ``packed_transpose_pair`` (the gate and up layers'
input gradients as one product over K = 2 ffn), is held to the float64
oracle of the two products summed (rel-L2 <= 1e-3 against the oracle
rounded to the dtype, as every 16-bit product here), bf16 and fp16, at
ragged shapes and at config 4's shape on sampled tokens.

Then the node against the same MLP run layer by layer (``swiglu`` between
the layers): the output, every layer's evidence, scale gradient and
coordinate step bit for bit, and the input gradient within the rounding
that the single product saves.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from qste_amd import kernels

    assert kernels.native_available(), kernels.status()


def _k():
    from qste_amd import kernels

    return kernels


def _rel(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm())


def _pair_oracle(ga, pa, sa, gb, pb, sb, cols, dtype):
    rnd = oracle.round_bf16 if dtype == torch.bfloat16 else (lambda v: np.asarray(v, np.float16).astype(np.float32))
    want = oracle.linear_dgrad(ga.float().cpu().numpy(), pa.cpu().numpy(), cols, rnd(sa.cpu().numpy()))
    want = want + oracle.linear_dgrad(gb.float().cpu().numpy(), pb.cpu().numpy(), cols, rnd(sb.cpu().numpy()))
    return torch.from_numpy(np.asarray(want, np.float32)).to(dtype).double()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,rows,cols", [(512, 256, 320), (300, 192, 256), (1, 64, 64), (257, 576, 128)])
def test_packed_transpose_pair_against_the_oracle(T, rows, cols, dtype):
    k = _k()
    print(f"packed_transpose_pair {T}x{rows}x{cols} {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(T * 3 + rows + cols)
    ga = torch.randn(T, rows, generator=g, device=DEV).to(dtype)
    gb = torch.randn(T, rows, generator=g, device=DEV).to(dtype)
    ca = torch.randint(-127, 128, (rows, cols), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    cb = torch.randint(-127, 128, (rows, cols), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    pa, pb = k.pack_coordinate(ca), k.pack_coordinate(cb)
    sa = torch.rand(rows, generator=g, device=DEV) * 0.02 + 0.005
    sb = torch.rand(rows, generator=g, device=DEV) * 0.02 + 0.005
    dx = k.packed_transpose_pair(ga, pa, sa, gb, pb, sb, cols)
    torch.cuda.synchronize()
    assert dx.dtype == dtype and dx.shape == (T, cols)
    assert _rel(dx.cpu(), _pair_oracle(ga, pa, sa, gb, pb, sb, cols, dtype)) <= 1e-3
    # the two products rounded and added as autograd would: the same values
    # up to those two extra roundings
    two = (k.packed_transpose(ga, pa, cols, row_scale=sa) + k.packed_transpose(gb, pb, cols, row_scale=sb))
    assert _rel(dx, two) <= 8e-3


def test_packed_transpose_pair_config4_shape():
    """The gate and up layers' input gradient at config 4 (16384 tokens,
    ffn 14336 -> d 4096): the oracle on 64 sampled tokens."""

    k = _k()
    T, rows, cols = 16384, 14336, 4096
    g = torch.Generator(device=DEV).manual_seed(41)
    ga = torch.randn(T, rows, generator=g, device=DEV).to(torch.bfloat16)
    gb = torch.randn(T, rows, generator=g, device=DEV).to(torch.bfloat16)
    pa = k.pack_coordinate(torch.randint(-127, 128, (rows, cols), generator=g, device=DEV,
                                         dtype=torch.int32).to(torch.int8))
    pb = k.pack_coordinate(torch.randint(-127, 128, (rows, cols), generator=g, device=DEV,
                                         dtype=torch.int32).to(torch.int8))
    sa = torch.rand(rows, generator=g, device=DEV) * 0.02 + 0.005
    sb = torch.rand(rows, generator=g, device=DEV) * 0.02 + 0.005
    dx = k.packed_transpose_pair(ga, pa, sa, gb, pb, sb, cols)
    torch.cuda.synchronize()
    sel = torch.from_numpy(np.sort(np.random.default_rng(4).choice(T, 64, replace=False))).to(DEV)
    want = _pair_oracle(ga[sel], pa, sa, gb[sel], pb, sb, cols, torch.bfloat16)
    assert _rel(dx[sel].cpu(), want) <= 1e-3


def test_swiglu_mlp_node_matches_the_layer_by_layer_mlp():
    import bench
    import qste_amd as qste

    T, d, ffn = 512, 1024, 3584
    dev = torch.device(DEV)

    def run(node):
        mlp = bench.SwiGLU(d, ffn, dev)
        surfaces = [mlp.gate.surface, mlp.up.surface, mlp.down.surface]
        coords = qste.QSTEOptimizer(surfaces)
        seen = {}
        apply = coords._apply
        for name, s in zip(("gate", "up", "down"), surfaces):
            s.route_evidence(lambda srf, e, name=name: (seen.__setitem__(name, e.detach().clone()), apply(srf, e)))
        g = torch.Generator(device=dev).manual_seed(0)
        x = torch.randn(T, d, generator=g, device=dev).to(torch.bfloat16).requires_grad_(True)
        dy = torch.randn(T, d, generator=g, device=dev).to(torch.bfloat16)
        if node:
            y = qste.nn.swiglu_mlp(x, mlp.gate, mlp.up, mlp.down)
        else:
            y = mlp.down(qste.nn.swiglu(mlp.gate(x), mlp.up(x)))
        y.backward(dy)
        flips = coords.step()
        torch.cuda.synchronize()
        grads = [m.surface.log_scale.grad.clone() for m in (mlp.gate, mlp.up, mlp.down)]
        return y.detach(), x.grad, seen, grads, [s.coordinate.clone() for s in surfaces], flips

    y0, gx0, ev0, gs0, c0, f0 = run(False)
    y1, gx1, ev1, gs1, c1, f1 = run(True)
    assert torch.equal(y0, y1)
    for name in ("gate", "up", "down"):
        assert torch.equal(ev0[name], ev1[name]), name
    for a, b in zip(gs0, gs1):
        assert torch.equal(a, b)
    for a, b in zip(c0, c1):
        assert torch.equal(a, b)
    assert f0 == f1 and f1 > 0
    # one rounding of the summed product where the layer-by-layer MLP rounds
    # each layer's input gradient and then their sum
    assert _rel(gx1, gx0) <= 8e-3
