"""The SwiGLU MLP as one autograd node (``qste_amd.nn.swiglu_mlp``).

The node runs the gate and up layers' backward as one layer of 2 ffn rows:
the gate's backward writes both gradients side by side
(``swiglu_backward_sums(..., side_by_side=True)``), and one
``linear_backward`` over them and the two layers' concatenated signs and
scales gives both layers' evidence and scale gradients as its row blocks
and the input gradient as one product over K = 2 ffn.  Held here:

* the side-by-side gradients and sums bit for bit against the plain call;
* the one call against the two layers' own calls: evidence and scale
  gradients within fp32 summation order (rel <= 1e-6), the input gradient
  within the rounding the single product saves, and against the float64
  oracle of the summed products (rel-L2 <= 1e-3 against the oracle rounded
  to bf16, as every 16-bit product here), also at config 4's shape on
  sampled tokens;
* the node against the same MLP run layer by layer (``swiglu`` between the
  layers): the output bit for bit, the evidence and scale gradients within
  1e-6, the coordinate steps equal outside elements whose evidence moved,
  the input gradient within the saved rounding; also with biases on all
  three layers and a batched [2, 96, d] input (the bias gradients within
  1e-6), and with an input that takes no gradient;
* inputs the node does not take (fp16, an ffn that is not a multiple of 64)
  running the layers one by one, bit for bit.
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


def _bits(t):
    return t.contiguous().view(torch.int16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,cols", [(512, 3584), (300, 1000), (257, 520), (1, 8)])
def test_side_by_side_equals_the_plain_call(rows, cols, dtype):
    k = _k()
    g = torch.Generator(device=DEV).manual_seed(rows + cols)
    gate = (torch.randn(rows, cols, generator=g, device=DEV) * 3).to(dtype)
    up = torch.randn(rows, cols, generator=g, device=DEV).to(dtype)
    grad = torch.randn(rows, cols, generator=g, device=DEV).to(dtype)
    off = torch.randn(rows, generator=g, device=DEV)
    dg, du, sums = k.swiglu_backward_sums(grad, gate, up, off, off)
    both, sums2 = k.swiglu_backward_sums(grad, gate, up, off, off, side_by_side=True)
    torch.cuda.synchronize()
    assert both.shape == (rows, 2 * cols) and both.dtype == dtype
    assert torch.equal(_bits(both[:, :cols]), _bits(dg)) and torch.equal(_bits(both[:, cols:]), _bits(du))
    assert torch.equal(sums, sums2)


def _two_layers(T, d, ffn, seed):
    k = _k()
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(T, d, generator=g, device=DEV).to(torch.bfloat16)
    packed_x, off, xs = k.pack_affine_rows(x)
    pg = k.pack_coordinate(torch.randint(-127, 128, (ffn, d), generator=g, device=DEV,
                                         dtype=torch.int32).to(torch.int8))
    pu = k.pack_coordinate(torch.randint(-127, 128, (ffn, d), generator=g, device=DEV,
                                         dtype=torch.int32).to(torch.int8))
    sg = torch.rand(ffn, generator=g, device=DEV) * 0.02 + 0.005
    su = torch.rand(ffn, generator=g, device=DEV) * 0.02 + 0.005
    both = torch.randn(T, 2 * ffn, generator=g, device=DEV).to(torch.bfloat16)
    return packed_x, off, xs, pg, pu, sg, su, both


def _dgrad_oracle(grad, packed, cols, scale):
    want = oracle.linear_dgrad(grad.float().cpu().numpy(), packed.cpu().numpy(), cols,
                               oracle.round_bf16(scale.cpu().numpy()))
    return torch.from_numpy(np.asarray(want, np.float32)).to(torch.bfloat16)


@pytest.mark.parametrize("T,d,ffn", [(1024, 1024, 3584), (300, 256, 512)])
def test_one_call_for_two_layers_equals_their_own_calls(T, d, ffn):
    k = _k()
    print(f"two layers as one {T}x{d}x{ffn}", flush=True)
    packed_x, off, xs, pg, pu, sg, su, both = _two_layers(T, d, ffn, T + d)
    dg, du = both[:, :ffn].contiguous(), both[:, ffn:].contiguous()
    dx_g, ev_g, gs_g, _ = k.linear_backward(dg, packed_x, off, xs, pg, sg, d, need_bias=False)
    dx_u, ev_u, gs_u, _ = k.linear_backward(du, packed_x, off, xs, pu, su, d, need_bias=False)
    pgu, sgu = torch.cat((pg, pu)), torch.cat((sg, su))
    dx, ev, gs, _ = k.linear_backward(both, packed_x, off, xs, pgu, sgu, d, need_bias=False)
    torch.cuda.synchronize()
    assert _rel(ev[:ffn], ev_g) <= 1e-6 and _rel(ev[ffn:], ev_u) <= 1e-6
    assert _rel(gs[:ffn], gs_g) <= 1e-6 and _rel(gs[ffn:], gs_u) <= 1e-6
    assert _rel(dx, dx_g + dx_u) <= 8e-3
    assert _rel(dx.cpu(), _dgrad_oracle(both, pgu, d, sgu)) <= 1e-3


def test_one_call_for_two_layers_config4_shape():
    """Config 4's gate and up layers (16384 tokens, d 4096, ffn 14336) as
    one call: the input gradient against the oracle on 64 sampled tokens,
    the up layer's evidence and scale gradient against its own call."""

    k = _k()
    T, d, ffn = 16384, 4096, 14336
    packed_x, off, xs, pg, pu, sg, su, both = _two_layers(T, d, ffn, 41)
    pgu, sgu = torch.cat((pg, pu)), torch.cat((sg, su))
    dx, ev, gs, _ = k.linear_backward(both, packed_x, off, xs, pgu, sgu, d, need_bias=False)
    torch.cuda.synchronize()
    sel = torch.from_numpy(np.sort(np.random.default_rng(4).choice(T, 64, replace=False))).to(DEV)
    assert _rel(dx[sel].cpu(), _dgrad_oracle(both[sel], pgu, d, sgu)) <= 1e-3
    del dx
    _, ev_u, gs_u, _ = k.linear_backward(both[:, ffn:].contiguous(), packed_x, off, xs, pu, su, d,
                                         need_bias=False, need_input=False)
    torch.cuda.synchronize()
    assert _rel(ev[ffn:], ev_u) <= 1e-6 and _rel(gs[ffn:], gs_u) <= 1e-6


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
    assert torch.equal(ev0["down"], ev1["down"]) and torch.equal(c0[2], c1[2])
    for name in ("gate", "up"):
        assert _rel(ev1[name], ev0[name]) <= 1e-6, name
    for a, b in zip(gs0, gs1):
        assert _rel(b, a) <= 1e-6
    for a, b in zip(c0, c1):
        assert float((a != b).float().mean()) < 1e-4
    assert f1 > 0
    # one rounding of the summed product where the layer-by-layer MLP rounds
    # each layer's input gradient and then their sum
    assert _rel(gx1, gx0) <= 8e-3


def _biased_layer(rows, cols, seed, dev):
    import qste_amd as qste

    g = torch.Generator(device=dev).manual_seed(seed)
    coord = torch.randint(-127, 128, (rows, cols), generator=g, device=dev, dtype=torch.int32).to(torch.int8)
    scale = torch.randn(rows, generator=g, device=dev).abs_().mul_(0.02).clamp_min_(1e-6)
    bias = torch.randn(rows, generator=g, device=dev) * 0.1
    return qste.QSTELinear(qste.Surface.from_state(coord, scale.log()), bias)


def _node_against_layers(x_shape, needs_input):
    """The node and the layers called one by one (with the fused gate) on
    fresh copies of the same three biased layers, each with an optimizer
    stepping inside backward; returns both runs' output, input gradient,
    delivered evidence, log-scale and bias gradients and coordinates."""

    import qste_amd as qste

    d, ffn = x_shape[-1], 1024
    dev = torch.device(DEV)

    def run(node):
        gate, up, down = (_biased_layer(ffn, d, 1, dev), _biased_layer(ffn, d, 2, dev),
                          _biased_layer(d, ffn, 3, dev))
        surfaces = [gate.surface, up.surface, down.surface]
        coords = qste.QSTEOptimizer(surfaces)
        seen = {}
        apply = coords._apply
        for name, s in zip(("gate", "up", "down"), surfaces):
            s.route_evidence(lambda srf, e, name=name: (seen.__setitem__(name, e.detach().clone()), apply(srf, e)))
        g = torch.Generator(device=dev).manual_seed(9)
        x = torch.randn(*x_shape, generator=g, device=dev).to(torch.bfloat16).requires_grad_(needs_input)
        dy = torch.randn(*x_shape, generator=g, device=dev).to(torch.bfloat16)
        y = qste.nn.swiglu_mlp(x, gate, up, down) if node else down(qste.nn.swiglu(gate(x), up(x)))
        y.backward(dy)
        torch.cuda.synchronize()
        layers = (gate, up, down)
        return (y.detach(), x.grad, seen, [m.surface.log_scale.grad.clone() for m in layers],
                [m.bias.grad.clone() for m in layers], [s.coordinate.clone() for s in surfaces])

    return run(False), run(True)


def test_swiglu_mlp_node_with_biases_and_batched_input():
    """Biases on all three layers and a [2, 96, d] input: the output bit for
    bit, the bias gradients (the gate and up layers' as the two halves of
    one call's column sums) equal to the layers' own, the evidence and
    log-scale gradients within 1e-6, the input gradient within the rounding
    the single product saves, its shape the input's."""

    a, b = _node_against_layers((2, 96, 512), True)
    assert b[0].shape == (2, 96, 512) and torch.equal(a[0], b[0])
    assert b[1].shape == (2, 96, 512) and _rel(b[1], a[1]) <= 8e-3
    for name in ("gate", "up", "down"):
        assert _rel(b[2][name], a[2][name]) <= 1e-6, name
    for ga, gb in zip(a[3], b[3]):
        assert _rel(gb, ga) <= 1e-6
    for ga, gb in zip(a[4], b[4]):
        assert gb.dtype == ga.dtype == torch.float32 and _rel(gb, ga) <= 1e-6
    for ca, cb in zip(a[5], b[5]):
        assert float((ca != cb).float().mean()) < 1e-4


def test_swiglu_mlp_node_without_input_gradient():
    """An input that takes no gradient: no input-gradient product in the
    node's backward, the same evidence and scale gradients as the layers'."""

    a, b = _node_against_layers((192, 512), False)
    assert a[1] is None and b[1] is None
    assert torch.equal(a[0], b[0])
    for name in ("gate", "up", "down"):
        assert _rel(b[2][name], a[2][name]) <= 1e-6, name
    for ga, gb in zip(a[3] + a[4], b[3] + b[4]):
        assert _rel(gb, ga) <= 1e-6


@pytest.mark.parametrize("dtype,ffn", [(torch.float16, 1024), (torch.bfloat16, 1000)])
def test_swiglu_mlp_outside_the_node_is_the_layers(dtype, ffn):
    """Inputs the node does not take (fp16; an ffn that is not a multiple of
    64) run the layers one by one: output and every gradient bit for bit
    those of down(swiglu(gate(x), up(x)))."""

    import qste_amd as qste
    from qste_amd import functional

    dev = torch.device(DEV)
    d = 512

    def run(composed):
        gate, up, down = (_biased_layer(ffn, d, 1, dev), _biased_layer(ffn, d, 2, dev),
                          _biased_layer(d, ffn, 3, dev))
        g = torch.Generator(device=dev).manual_seed(4)
        x = torch.randn(128, d, generator=g, device=dev).to(dtype).requires_grad_(True)
        assert not functional.swiglu_mlp_fusable(x, gate, up, down)
        y = down(qste.nn.swiglu(gate(x), up(x))) if composed else qste.nn.swiglu_mlp(x, gate, up, down)
        y.float().square().sum().backward()
        torch.cuda.synchronize()
        layers = (gate, up, down)
        return [y.detach(), x.grad] + [m.surface.log_scale.grad for m in layers] + [m.bias.grad for m in layers]

    for a, b in zip(run(True), run(False)):
        assert a.dtype == b.dtype and torch.equal(a, b)
