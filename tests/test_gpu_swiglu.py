"""The fused SwiGLU gate against torch's own ``F.silu(g) * u``.

The reference has no SwiGLU operator: a SwiGLU MLP on it runs torch's silu
and mul between the binary layers.  That chain is therefore the oracle here,
compared bit for bit on the GPU in every dtype: the forward values, both
input gradients of its autograd (fp16's gate gradient up to one-ulp rounding
ties that torch's own fp16 kernels resolve differently by tensor size), the
one-bit encoding the fused forward
produces for the next layer (against ``pack_affine_rows`` on the same output
and against the CPU oracle), and a whole config-4-shaped MLP (smaller
tokens) whose outputs, input gradient and coordinate steps must not change
when the gate is fused.  A float64 evaluation pins the formulas themselves
(a wrong term would be far outside one rounding).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


@pytest.fixture(autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from qste_amd import kernels

    assert kernels.native_available(), kernels.status()


def _inputs(shape, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    gate = (torch.randn(shape, generator=g, device=DEV) * 3).to(dtype)
    up = torch.randn(shape, generator=g, device=DEV).to(dtype)
    grad = torch.randn(shape, generator=g, device=DEV).to(dtype)
    return gate, up, grad


def _bits(t):
    return t.contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32)


SHAPES = [(64, 4096), (33, 14336), (7, 1000), (3, 17, 24), (1, 8), (2, 5)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES)
def test_forward_and_backward_equal_torch(shape, dtype):
    import qste_amd as qste

    print(f"swiglu {shape} {dtype}", flush=True)
    gate, up, grad = _inputs(shape, dtype, sum(shape))
    g1, u1 = gate.clone().requires_grad_(True), up.clone().requires_grad_(True)
    want = F.silu(g1) * u1
    want.backward(grad)
    g2, u2 = gate.clone().requires_grad_(True), up.clone().requires_grad_(True)
    got = qste.nn.swiglu(g2, u2)
    got.backward(grad)
    torch.cuda.synchronize()
    assert got.dtype == dtype and got.shape == want.shape
    assert torch.equal(_bits(got), _bits(want.detach()))
    assert torch.equal(_bits(u2.grad), _bits(u1.grad))
    if dtype == torch.float16:
        # where dg's fp32 value lies exactly on an fp16 rounding midpoint,
        # torch's own fp16 silu_backward kernels resolve the tie differently
        # by code path (tensor size): the fused kernel rounds as the
        # vectorized one does.  Allow those one-ulp ties, nothing else.
        diff = (_bits(g2.grad).int() - _bits(g1.grad).int()).abs()
        assert int(diff.max()) <= 1
        assert int((diff > 0).sum()) <= max(1, g1.grad.numel() >> 10)
    else:
        assert torch.equal(_bits(g2.grad), _bits(g1.grad)), int((g2.grad != g1.grad).sum())
    # the formulas, in float64: h = silu(g) u, dh/du = silu(g),
    # dh/dg = u sigma (1 + g (1 - sigma)); within a few dtype roundings
    gd, ud, dd = gate.double(), up.double(), grad.double()
    sig = torch.sigmoid(gd)
    eps = {torch.bfloat16: 2e-2, torch.float16: 3e-3, torch.float32: 1e-5}[dtype]
    for got_t, ref in ((got, gd * sig * ud), (u2.grad, dd * gd * sig),
                       (g2.grad, dd * ud * sig * (1 + gd * (1 - sig)))):
        rel = float((got_t.double() - ref).norm() / ref.norm())
        assert rel <= eps, rel


@pytest.mark.parametrize("rows,cols", [(40, 14336), (64, 4096), (9, 1032), (5, 18000), (6, 100)])
def test_fused_encoding_equals_pack_affine_rows(rows, cols):
    """The encoding the forward writes equals pack_affine_rows on its output,
    byte for byte (the fused register path for bf16 rows of whole chunks up
    to 2048 chunks, the separate pass otherwise), and the CPU oracle's."""

    from qste_amd import kernels

    gate, up, _ = _inputs((rows, cols), torch.bfloat16, rows * cols)
    out, (packed, offset, scale) = kernels.swiglu_forward(gate, up, encode=True)
    p2, o2, s2 = kernels.pack_affine_rows(out)
    assert torch.equal(packed, p2)
    assert torch.equal(offset.view(torch.int32), o2.view(torch.int32))
    assert torch.equal(scale.view(torch.int32), s2.view(torch.int32))
    bits, off, xs = oracle.pack_affine_rows(out.float().cpu().numpy())
    assert np.array_equal(packed.cpu().numpy(), bits)
    assert np.array_equal(offset.cpu().numpy(), off)
    assert np.array_equal(scale.cpu().numpy(), xs)


def test_swiglu_mlp_matches_the_torch_gate():
    """A SwiGLU MLP of binary layers: swiglu(gate(x), up(x)) against
    F.silu(gate(x)) * up(x) -- identical output, input gradient, evidence
    (hence coordinates, packed signs and flips after the steps inside
    backward), and the down layer reuses the fused encoding."""

    import bench
    import qste_amd as qste
    from qste_amd import functional

    T, d, ffn = 512, 1024, 3584
    dev = torch.device(DEV)

    def run(fused):
        mlp = bench.SwiGLU(d, ffn, dev)
        coords = qste.QSTEOptimizer(list(qste.surfaces(mlp.modules)))
        g = torch.Generator(device=dev).manual_seed(0)
        x = torch.randn(T, d, generator=g, device=dev).to(torch.bfloat16).requires_grad_(True)
        dy = torch.randn(T, d, generator=g, device=dev).to(torch.bfloat16)
        gate, up = mlp.gate(x), mlp.up(x)
        h = qste.nn.swiglu(gate, up) if fused else F.silu(gate) * up
        if fused:
            # the down layer will find h's encoding waiting
            assert functional._last_encoding is not None and functional._last_encoding[0]() is h
        y = mlp.down(h)
        y.backward(dy)
        flips = coords.step()
        torch.cuda.synchronize()
        return (y.detach(), x.grad, [s.coordinate.clone() for s in qste.surfaces(mlp.modules)],
                [s.packed_sign.clone() for s in qste.surfaces(mlp.modules)], flips)

    a, b = run(False), run(True)
    assert torch.equal(a[0], b[0])
    assert torch.equal(a[1], b[1])
    for ca, cb in zip(a[2], b[2]):
        assert torch.equal(ca, cb)
    for pa, pb in zip(a[3], b[3]):
        assert torch.equal(pa, pb)
    assert a[4] == b[4] and a[4] > 0
