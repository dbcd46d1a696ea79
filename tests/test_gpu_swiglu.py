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
    from qste_amd import functional, kernels

    T, d, ffn = 512, 1024, 3584
    dev = torch.device(DEV)
    real_backward = kernels.linear_backward
    handed = []

    def spy(*args, **kw):
        handed.append(kw.get("offset_dot") is not None)
        return real_backward(*args, **kw)

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

    kernels.linear_backward = spy
    try:
        a = run(False)
        assert handed == [False, False, False]
        handed.clear()
        b = run(True)
        # down summed its own dy; gate and up took the gate kernel's sums
        assert sorted(handed) == [False, True, True]
    finally:
        kernels.linear_backward = real_backward
    assert torch.equal(a[0], b[0])
    assert torch.equal(a[1], b[1])
    for ca, cb in zip(a[2], b[2]):
        assert torch.equal(ca, cb)
    for pa, pb in zip(a[3], b[3]):
        assert torch.equal(pa, pb)
    assert a[4] == b[4] and a[4] > 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,cols", [(512, 3584), (300, 1000), (77, 14336), (1, 8), (257, 520), (9, 1001)])
def test_backward_sums_equal_the_layer_backward_sums(rows, cols, dtype):
    """swiglu_backward_sums: the same gradients as swiglu_backward, and sums
    that make linear_backward's outputs bit-identical to what it computes
    from those gradients itself (its own column sums), on both layers."""

    from qste_amd import kernels

    print(f"swiglu sums {rows}x{cols} {dtype}", flush=True)
    gate, up, grad = _inputs((rows, cols), dtype, rows + cols)
    g = torch.Generator(device=DEV).manual_seed(rows * 7 + cols)
    off_g = torch.randn(rows, generator=g, device=DEV)
    off_u = off_g if rows % 2 else torch.randn(rows, generator=g, device=DEV)
    dg0, du0 = kernels.swiglu_backward(grad, gate, up)
    dg, du, sums = kernels.swiglu_backward_sums(grad, gate, up, off_g, off_u)
    assert torch.equal(_bits(dg), _bits(dg0)) and torch.equal(_bits(du), _bits(du0))
    # within fp32 summation error of the float64 sums
    for got, dy, off in ((sums[0], dg, off_g), (sums[1], du, off_u)):
        want = dy.double().t() @ off.double()
        # a sequential fp32 sum of n terms errs by at most about n ulps of the
        # sum of magnitudes
        bound = (rows + 8) * 2.0**-24 * (dy.double().abs().t() @ off.double().abs()) + 1e-30
        assert bool(((got.double() - want).abs() <= bound).all())
    # a layer that reads dg (rows of the batch, cols = the layer's rows)
    columns = 256
    x = torch.randn(rows, columns, generator=g, device=DEV).to(dtype)
    packed_x, x_off, x_scale = kernels.pack_affine_rows(x)
    coord = torch.randint(-127, 128, (cols, columns), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    packed_w = kernels.pack_coordinate(coord)
    scale = torch.rand(cols, generator=g, device=DEV) * 0.02
    dg2, _, sums2 = kernels.swiglu_backward_sums(grad, gate, up, x_off, x_off)
    ref = kernels.linear_backward(dg2, packed_x, x_off, x_scale, packed_w, scale, columns, need_bias=False)
    got = kernels.linear_backward(dg2, packed_x, x_off, x_scale, packed_w, scale, columns, need_bias=False,
                                  offset_dot=sums2[0])
    torch.cuda.synchronize()
    assert ref[3] is None and got[3] is None
    for a, b in zip(ref[:3], got[:3]):
        assert torch.equal(a.view(torch.int16) if a.element_size() == 2 else a.view(torch.int32),
                           b.view(torch.int16) if b.element_size() == 2 else b.view(torch.int32))


def _same_or_both_nan(a, b):
    """bf16 tensors equal bit for bit, except that any NaN matches any NaN."""

    nan = torch.isnan(a.float()) & torch.isnan(b.float())
    return bool(((_bits(a) == _bits(b)) | nan).all())


@pytest.mark.parametrize("rows,cols", [(4096, 1024), (4100, 520), (4096, 14336)])
def test_tabled_forward_every_bf16_gate(rows, cols):
    """From 4096 rows on, the encoding forward takes the rounded silu of
    gates with magnitude in [2^-12, 2^8) from a table each workgroup fills
    once for several rows.  Every one of the 65536 bf16 gate values, spread
    over the rows in a seeded random order (so that waves mix tabulated gates
    with zeros, subnormals, tiny and huge magnitudes, infinities and NaNs):
    the output bit for bit against torch's F.silu(g) * u, and the encoding
    byte for byte against pack_affine_rows on that output (the even rows keep
    only gates below 2^100 in magnitude, so that their statistics are finite
    too)."""

    from qste_amd import kernels

    print(f"tabled swiglu forward {rows}x{cols}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows + cols)
    order = torch.randperm(rows * cols, generator=g, device=DEV) % 65536
    gate = (order - 32768).to(torch.int16).view(torch.bfloat16).reshape(rows, cols)
    # the even rows without their infinities, NaNs and magnitudes from 2^100
    # on (whose products can overflow), so that their statistics are finite
    # and compared exactly
    even = gate[0::2]
    even[~(even.float().abs() < 2.0**100)] = 0.5
    up = torch.randn(rows, cols, generator=g, device=DEV).bfloat16()
    want = F.silu(gate) * up
    out, (packed, offset, scale) = kernels.swiglu_forward(gate, up, encode=True)
    torch.cuda.synchronize()
    assert _same_or_both_nan(out, want)
    p2, o2, s2 = kernels.pack_affine_rows(out)
    assert torch.equal(packed, p2)
    # rows holding a NaN or an infinity have NaN statistics, whose payload
    # depends on the order the sums met them in
    for a, b in ((offset, o2), (scale, s2)):
        assert bool(((a.view(torch.int32) == b.view(torch.int32)) | (torch.isnan(a) & torch.isnan(b))).all())
    assert bool(torch.isfinite(offset[0::2]).all())


def test_backward_sums_every_bf16_gate():
    """Every one of the 65536 bf16 gate values (in and out of the range the
    kernel's sigmoid/silu tables hold: zeros, subnormals, tiny and huge
    magnitudes, infinities, NaNs), with random gradients and up values:
    dg and du bit for bit against torch's autograd chain and the plain
    kernel, and the sums against the float64 bound."""

    from qste_amd import kernels

    every = torch.arange(-32768, 32768, dtype=torch.int32, device=DEV).to(torch.int16)
    gate = every.view(torch.bfloat16).reshape(256, 256)
    g = torch.Generator(device=DEV).manual_seed(5)
    up = torch.randn(256, 256, generator=g, device=DEV).bfloat16()
    grad = torch.randn(256, 256, generator=g, device=DEV).bfloat16()
    off = torch.randn(256, generator=g, device=DEV)
    g1, u1 = gate.clone().requires_grad_(True), up.clone().requires_grad_(True)
    (F.silu(g1) * u1).backward(grad)
    dg0, du0 = kernels.swiglu_backward(grad, gate, up)
    dg, du, sums = kernels.swiglu_backward_sums(grad, gate, up, off, off)
    torch.cuda.synchronize()
    assert _same_or_both_nan(dg, g1.grad) and _same_or_both_nan(du, u1.grad)
    assert _same_or_both_nan(dg, dg0) and _same_or_both_nan(du, du0)
    finite = torch.isfinite(dg.float()).all(0) & torch.isfinite(du.float()).all(0)
    for got, dy in ((sums[0], dg), (sums[1], du)):
        want = dy.double().t() @ off.double()
        bound = 264 * 2.0**-24 * (dy.double().abs().t() @ off.double().abs()) + 1e-30
        assert bool(((got.double() - want).abs() <= bound)[finite].all())


def test_row_scale_equals_torch():
    """clamp(exp(log_scale)) and its gradient, bit for bit against torch's
    operators, over finite values across the whole exp range, the clamp
    bounds themselves, infinities and NaN."""

    import math

    from qste_amd.surface import row_scale

    lo, hi = 1e-6, 4.0
    g = torch.Generator(device=DEV).manual_seed(3)
    wide = torch.empty(1 << 20, device=DEV).uniform_(-110.0, 100.0, generator=g)
    near = torch.randn(1 << 16, device=DEV, generator=g) * 3 - 4
    special = torch.tensor([0.0, -0.0, math.log(lo), math.log(hi), float(torch.tensor(lo).log()),
                            float(torch.tensor(hi).log()), float("inf"), float("-inf"), float("nan"),
                            88.7, 88.8, -103.0, -87.3], device=DEV)
    ls = torch.cat((wide, near, special))
    grad = torch.randn(ls.numel(), device=DEV, generator=g)
    grad[-5:] = float("inf")
    a = ls.clone().requires_grad_(True)
    ref = a.exp().clamp(lo, hi)
    ref.backward(grad)
    b = ls.clone().requires_grad_(True)
    got = row_scale(b, lo, hi)
    got.backward(grad)
    torch.cuda.synchronize()
    # NaN payloads are not compared: NaN positions, then the rest bitwise
    for x, y in ((got.detach(), ref.detach()), (b.grad, a.grad)):
        assert torch.equal(torch.isnan(x), torch.isnan(y))
        keep = ~torch.isnan(y)
        assert torch.equal(x[keep].view(torch.int32), y[keep].view(torch.int32))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bounds", [(1e-6, 4.0), (1e-5, 10.0), (0.003, 0.3)])
def test_row_scale_16bit_every_value(dtype, bounds):
    """A bf16 / fp16 log-scale (a model moved to that dtype): every one of the
    65536 values of the dtype, with random gradients (and infinite ones),
    bit for bit against torch's exp().clamp() and its autograd on a tensor
    of that dtype, for bounds that are and are not representable in it."""

    from qste_amd.surface import row_scale

    lo, hi = bounds
    ls = torch.arange(-32768, 32768, dtype=torch.int32, device=DEV).to(torch.int16).view(dtype)
    g = torch.Generator(device=DEV).manual_seed(11)
    grad = torch.randn(ls.numel(), device=DEV, generator=g).to(dtype)
    grad[::4096] = float("inf")
    a = ls.clone().requires_grad_(True)
    ref = a.exp().clamp(lo, hi)
    ref.backward(grad)
    b = ls.clone().requires_grad_(True)
    got = row_scale(b, lo, hi)
    got.backward(grad)
    torch.cuda.synchronize()
    assert got.dtype == dtype and b.grad.dtype == dtype
    for x, y in ((got.detach(), ref.detach()), (b.grad, a.grad)):
        assert torch.equal(torch.isnan(x), torch.isnan(y))
        keep = ~torch.isnan(y)
        assert torch.equal(x[keep].view(torch.int16), y[keep].view(torch.int16)), int((x != y)[keep].sum())
