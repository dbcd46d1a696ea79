"""Packed activations on the GPU: the HIP kernels against the oracle and torch.

* bits and masked activations -- bit-exact against ``oracle/activations.py``
  and against torch's own activation and autograd on the same device;
* smooth activations -- the value equals torch's on the GPU bit for bit
  (the reference's forward is torch's, ``src/qste/nn.py:491``); the retained
  int8 derivative equals the oracle's except for a one-step difference at
  rounding ties (|d / scale - k - 1/2| below a stated band), the row scale
  within 4 ulp; the backward equals the oracle's on the same payload;
* the API -- the reference's own checks (``tests/test_activations.py``,
  ``tests/test_activation_coverage.py``): exact ReLU family, zero gradient at
  the kinks, dropout's gradient follows its mask, the smooth gradient within
  1% and unbiased, one bit / one byte retained per element, and
  ``packed_activations`` / ``convert(activations=...)`` routing.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import activations as oa

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
SHAPES = [(1, 1), (3, 7), (5, 33), (17, 64), (4, 1000), (2, 3000), (3, 16392)]


def _name(dtype):
    return {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16"}[dtype]


def _x(shape, seed=0, spread=3.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * spread).to(dtype)


def _np(t):
    return t.detach().float().cpu().numpy()


@pytest.fixture(scope="module")
def K():
    from qste_amd import kernels

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return kernels


# ---------------------------------------------------------------------------
# bit kernels
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("shape", SHAPES)
def test_pack_unpack_apply_bits(K, shape):
    rows, cols = shape
    print(f"bits {shape}", flush=True)
    mask = _x(shape, seed=rows + cols) > 0.2
    packed = K.pack_bits(mask.to(DEV))
    assert np.array_equal(packed.cpu().numpy(), oa.pack_bits(mask.numpy()))
    for dtype in DTYPES:
        assert torch.equal(K.unpack_bits(packed, cols, dtype=dtype).cpu(), mask.to(dtype))
        v = _x(shape, seed=1, dtype=dtype)
        out = K.apply_bits(v.to(DEV), packed, cols).cpu()
        assert np.array_equal(_np(out), oa.apply_bits(_np(v), packed.cpu().numpy(), _name(dtype)))


# ---------------------------------------------------------------------------
# masked forwards and backwards
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES)
def test_masked_activation_matches_oracle_and_torch(K, dtype, shape):
    print(f"masked {shape} {dtype}", flush=True)
    x = _x(shape, seed=2, dtype=dtype)
    x.view(-1)[:3] = torch.tensor([0.0, 6.0, -1.0])[: x.numel()].to(dtype)
    xd = x.to(DEV)
    name = _name(dtype)
    for lower, upper, fn in ((0.0, None, F.relu), (0.0, 6.0, F.relu6), (-1.0, 1.0, F.hardtanh)):
        out, packed = K.masked_activation(xd, K.MASK_CLAMP, lower=lower, upper=upper)
        ref_out, ref_packed = oa.clamp_forward(_np(x), lower, upper, name)
        assert np.array_equal(_np(out), ref_out)
        assert np.array_equal(packed.cpu().numpy(), ref_packed)
        assert torch.equal(out, fn(xd))
    out, packed = K.masked_activation(xd, K.MASK_LEAKY, slope=0.1)
    ref_out, ref_packed = oa.leaky_forward(_np(x), 0.1, name)
    assert np.array_equal(_np(out), ref_out) and np.array_equal(packed.cpu().numpy(), ref_packed)
    assert torch.equal(out, F.leaky_relu(xd, 0.1))
    none, packed = K.masked_activation(xd, K.MASK_INTERVAL, lower=-3.0, upper=3.0, want_output=False)
    assert none is None
    assert np.array_equal(packed.cpu().numpy(), oa.interval_bits(_np(x), -3.0, 3.0, name))
    # backward formulas: select, gain, slope
    g = _x(shape, seed=3, dtype=dtype)
    pk = packed.cpu().numpy()
    for inside, outside in ((1.0, 0.0), (2.0, 0.0), (1.0 / 6.0, 0.0), (1.0, 0.1), (1.0, 0.01)):
        got = K.masked_backward(g.to(DEV), packed, shape[1], inside=inside, outside=outside)
        assert np.array_equal(_np(got), oa.masked_backward(_np(g), pk, inside, outside, name)), (inside, outside)


# ---------------------------------------------------------------------------
# smooth activations
# ---------------------------------------------------------------------------

SMOOTH = [
    ("gelu", 0.0, lambda t: F.gelu(t)),
    ("gelu_tanh", 0.0, lambda t: F.gelu(t, approximate="tanh")),
    ("silu", 0.0, F.silu),
    ("tanh", 0.0, torch.tanh),
    ("sigmoid", 0.0, torch.sigmoid),
    ("elu", 0.7, lambda t: F.elu(t, 0.7)),
    ("celu", 1.3, lambda t: F.celu(t, 1.3)),
    ("selu", 0.0, F.selu),
    ("softplus", 2.0, lambda t: F.softplus(t, 2.0)),
    ("mish", 0.0, F.mish),
    ("hardswish", 0.0, F.hardswish),
]

# a payload may differ from the oracle's by one step only where d / scale is
# this close to a half-integer (fp32 transcendental ulps, relative to 127)
TIE_BAND = 2e-4


def _check_payload(payload, scale, ref_payload, ref_scale, d_ref):
    assert np.allclose(scale, ref_scale, rtol=4 * 2 ** -23, atol=0)
    diff = payload.astype(np.int32) - ref_payload.astype(np.int32)
    assert np.abs(diff).max(initial=0) <= 1
    if np.any(diff):
        margin = oa.tie_margin(d_ref, ref_scale)
        assert np.all(margin[diff != 0] < TIE_BAND), margin[diff != 0].max()
        assert np.count_nonzero(diff) <= max(2, diff.size // 1000)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("kind,param,fn", SMOOTH)
def test_smooth_activation_value_and_payload(K, dtype, kind, param, fn):
    name = _name(dtype)
    for shape in ((5, 33), (8, 2048), (3, 4104), (2, 16392)):
        print(f"smooth {kind} {dtype} {shape}", flush=True)
        x = _x(shape, seed=4, dtype=dtype)
        xd = x.to(DEV)
        y, payload, scale = K.smooth_activation(xd, kind, param)
        # the value: torch's own, computed on the same device
        ref_y_torch = fn(xd)
        ref_y, ref_payload, ref_scale = oa.smooth_forward(kind, _np(x), param, name)
        assert np.allclose(_np(y), ref_y, rtol=2e-6 if dtype == torch.float32 else 2 ** -7, atol=1e-6)
        value_exact = torch.equal(y, ref_y_torch)
        # the derivative, derived from torch's value so both sides see the same y
        d_ref = oa.derivative(kind, _np(x), _np(ref_y_torch), param)
        _, p2, s2 = K.smooth_activation(xd, kind, param, output=ref_y_torch)
        ref_p2, ref_s2 = oa.quantize_rows(d_ref)
        _check_payload(p2.cpu().numpy(), s2.cpu().numpy(), ref_p2, ref_s2, d_ref)
        if value_exact:
            assert torch.equal(payload, p2) and torch.equal(scale, s2)
        # backward on the kernel's own payload
        g = _x(shape, seed=5, dtype=dtype)
        got = K.smooth_backward(g.to(DEV), p2, s2)
        assert np.array_equal(_np(got), oa.smooth_backward(_np(g), p2.cpu().numpy(), s2.cpu().numpy(), name))


@pytest.mark.parametrize("dtype", DTYPES)
def test_kernel_value_table_is_exact_against_torch(dtype):
    """Every (kind, dtype) the API computes in the kernel equals torch's value."""

    from qste_amd import kernels as K
    from qste_amd.nn import _KERNEL_VALUE

    fns = {k: (p, f) for k, p, f in SMOOTH}
    x = _x((64, 4096), seed=6, spread=4.0, dtype=dtype).to(DEV)
    x.view(-1)[:6] = torch.tensor([0.0, -3.0, 3.0, 25.0, -25.0, 1e-3]).to(dtype)
    for kind, dt in sorted(_KERNEL_VALUE, key=str):
        if dt != dtype:
            continue
        param, fn = fns[kind]
        y, _, _ = K.smooth_activation(x, kind, param)
        ref = fn(x)
        bad = (y != ref) & ~(torch.isnan(y) & torch.isnan(ref))
        assert not bad.any(), f"{kind} {dtype}: {int(bad.sum())} values differ from torch"


@pytest.mark.parametrize("dtype", DTYPES)
def test_relu_square_and_provided_derivative(K, dtype):
    name = _name(dtype)
    x = _x((9, 300), seed=7, dtype=dtype)
    x[4] = -1.0
    y, payload, scale = K.smooth_activation(x.to(DEV), "relu_square")
    ref_y, ref_p, ref_s = oa.smooth_forward("relu_square", _np(x), 0.0, name)
    assert np.array_equal(_np(y), ref_y)
    assert np.array_equal(payload.cpu().numpy(), ref_p) and np.array_equal(scale.cpu().numpy(), ref_s)
    g = _x((9, 300), seed=8, dtype=dtype)
    got = K.smooth_backward(g.to(DEV), payload, scale)
    assert np.array_equal(_np(got), oa.smooth_backward(_np(g), ref_p, ref_s, name))
    d = _x((7, 77), seed=9)
    _, p, s = K.smooth_activation(None, "provided", derivative=d.to(DEV))
    rp, rs = oa.quantize_rows(d.numpy())
    assert np.array_equal(p.cpu().numpy(), rp) and np.array_equal(s.cpu().numpy(), rs)


def test_silu_every_bf16_input(K):
    """bf16 SiLU on every bit pattern, one element per row so the row scale is
    |d| / 127 and shows the derivative exactly: the value equals torch's, the
    payload and scale equal those derived from torch's value (the kernel's
    per-element formula), and the derivative is within a few fp32 ulps (1e-6
    absolute where 1 + x * (1 - sigmoid(x)) cancels) of
    sigmoid(x) * (1 + x * (1 - sigmoid(x))) computed by torch in fp32."""

    bits = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    x = bits.view(torch.bfloat16).reshape(-1, 1).to(DEV)
    for shape in ((65536, 1), (16, 4096), (8, 8192)):
        print(f"silu every bf16 {shape}", flush=True)
        xs = x.reshape(shape)
        y, payload, scale = K.smooth_activation(xs, "silu")
        ref = F.silu(xs)
        assert torch.equal(torch.isnan(y), torch.isnan(ref))
        assert torch.equal(y[~torch.isnan(y)], ref[~torch.isnan(ref)])
        _, p1, s1 = K.smooth_activation(xs, "silu", output=ref)
        assert torch.equal(payload, p1)
        assert torch.equal(torch.isnan(scale), torch.isnan(s1))
        assert torch.equal(scale[~torch.isnan(scale)], s1[~torch.isnan(s1)])
    xf = x.float().reshape(-1)
    sg = torch.sigmoid(xf)
    d = sg * (1 + xf * (1 - sg))
    _, payload, scale = K.smooth_activation(x, "silu")
    got = scale * payload.reshape(-1).float().sign()
    ok = torch.isfinite(d) & (d.abs() > 1e-8)
    assert torch.allclose(got[ok] * 127, d[ok], rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("dtype", DTYPES)
def test_smooth_activation_empty_rows_and_columns(K, dtype):
    for shape in ((3, 0), (0, 8), (0, 0)):
        print(f"smooth empty {shape} {dtype}", flush=True)
        x = torch.zeros(shape, dtype=dtype, device=DEV)
        y, payload, scale = K.smooth_activation(x, "silu")
        assert y.shape == shape and payload.shape == shape and scale.shape == (shape[0],)
        if shape[0]:
            assert torch.equal(scale, torch.full((shape[0],), 1e-8 / 127, device=DEV))


def test_smooth_activation_at_the_mlp_shape(K):
    """cfg4's SiLU input [16384, 14336] bf16, checked through properties."""

    g = torch.Generator(device=DEV).manual_seed(10)
    x = torch.randn(16384, 14336, generator=g, device=DEV, dtype=torch.bfloat16)
    y, payload, scale = K.smooth_activation(x, "silu")
    assert torch.equal(y, F.silu(x))
    xs = x[:64].float()
    s = torch.sigmoid(xs)
    d = s * (1 + xs * (1 - s))
    assert torch.allclose(scale[:64], d.abs().amax(1) / 127, rtol=1e-5)
    err = (payload[:64].float() * scale[:64, None] - d).abs()
    assert bool((err <= scale[:64, None] * 0.5001 + 1e-6).all())
    assert int(payload.abs().amax(1).min()) == 127


# ---------------------------------------------------------------------------
# the API (the reference's tests/test_activations.py checks, on the GPU)
# ---------------------------------------------------------------------------


def _pair(shape, seed=0, dtype=torch.float32):
    v = (_x(shape, seed=seed, spread=2.0)).to(dtype).to(DEV)
    return v.clone().requires_grad_(True), v.clone().requires_grad_(True)


def _backward(out, seed=1):
    out.backward(_x(out.shape, seed=seed, spread=1.0).to(out.dtype).to(DEV))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(8, 16), (5, 33), (3, 4, 7), (129,)])
def test_relu_family_is_bit_identical_to_torch(dtype, shape):
    from qste_amd import nn as qnn

    for ours_fn, ref_fn in ((qnn.relu, F.relu), (qnn.relu6, F.relu6), (qnn.hardtanh, F.hardtanh)):
        mine, theirs = _pair(shape, seed=3, dtype=dtype)
        ours, ref = ours_fn(mine), ref_fn(theirs)
        assert torch.equal(ours, ref)
        _backward(ours)
        _backward(ref)
        assert torch.equal(mine.grad, theirs.grad)


def test_gradients_are_zero_at_the_kinks():
    from qste_amd import nn as qnn

    x = torch.zeros(4, 8, device=DEV, requires_grad=True)
    qnn.relu(x).sum().backward()
    assert torch.equal(x.grad, torch.zeros_like(x.grad))
    x = torch.tensor([[-1.0, 0.0, 3.0, 6.0, 9.0]], device=DEV, requires_grad=True)
    qnn.relu6(x).sum().backward()
    assert torch.equal(x.grad.cpu(), torch.tensor([[0.0, 0.0, 1.0, 0.0, 0.0]]))


def test_leaky_and_hardsigmoid_follow_torch():
    from qste_amd import nn as qnn

    mine, theirs = _pair((6, 50), seed=4)
    ours, ref = qnn.leaky_relu(mine, 0.2), F.leaky_relu(theirs, 0.2)
    assert torch.equal(ours, ref)
    _backward(ours)
    _backward(ref)
    assert torch.allclose(mine.grad, theirs.grad, rtol=1e-6, atol=0)
    mine, theirs = _pair((6, 50), seed=5)
    ours, ref = qnn.hardsigmoid(mine * 2), F.hardsigmoid(theirs * 2)
    assert torch.equal(ours, ref)
    _backward(ours)
    _backward(ref)
    assert torch.allclose(mine.grad, theirs.grad, rtol=1e-6, atol=1e-7)


def test_dropout_gradient_follows_its_mask():
    from qste_amd import nn as qnn

    torch.manual_seed(0)
    x = torch.randn(64, 128, device=DEV, requires_grad=True)
    out = qnn.dropout(x, 0.5, training=True)
    out.backward(torch.ones_like(out))
    dropped = out == 0.0
    assert torch.equal(x.grad == 0.0, dropped)
    assert torch.allclose(x.grad[~dropped], torch.full_like(x.grad[~dropped], 2.0))
    assert qnn.dropout(x, 0.5, training=False) is x
    with pytest.raises(ValueError):
        qnn.dropout(x, 1.0)


API_SMOOTH = [
    ("gelu", lambda q: q.gelu, F.gelu),
    ("gelu_tanh", lambda q: (lambda t: q.gelu(t, "tanh")), lambda t: F.gelu(t, approximate="tanh")),
    ("silu", lambda q: q.silu, F.silu),
    ("tanh", lambda q: q.tanh, torch.tanh),
    ("sigmoid", lambda q: q.sigmoid, torch.sigmoid),
    ("mish", lambda q: q.mish, F.mish),
    ("softplus", lambda q: q.softplus, F.softplus),
]


@pytest.mark.parametrize("name,ours,ref", API_SMOOTH)
def test_smooth_forward_untouched_gradient_close_and_unbiased(name, ours, ref):
    from qste_amd import nn as qnn

    fn = ours(qnn)
    mine, theirs = _pair((32, 64), seed=5)
    assert torch.equal(fn(mine), ref(theirs))
    mine, theirs = _pair((64, 128), seed=7)
    _backward(fn(mine), seed=2)
    _backward(ref(theirs), seed=2)
    error = (mine.grad - theirs.grad).abs().max() / theirs.grad.abs().max()
    assert error < 0.01, f"relative gradient error {error:.4f}"
    mine, theirs = _pair((256, 256), seed=9)
    _backward(fn(mine), seed=4)
    _backward(ref(theirs), seed=4)
    bias = (mine.grad - theirs.grad).mean().abs()
    assert bias < theirs.grad.abs().mean() * 1e-3


def _retained_per_sample(function, samples=256, columns=512):
    held = []

    def pack(t):
        held.append(t.numel() * t.element_size())
        return t

    x = torch.randn(samples, columns, device=DEV, requires_grad=True)
    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
        out = function(x)
    out.sum().backward()
    return sum(held) / samples


def test_retained_bytes_per_element():
    from qste_amd import nn as qnn

    assert _retained_per_sample(qnn.relu) == pytest.approx(512 / 8, abs=1.0)
    assert _retained_per_sample(F.relu) == pytest.approx(512 * 4, abs=1.0)
    assert _retained_per_sample(lambda t: qnn.dropout(t, 0.1)) == pytest.approx(512 / 8, abs=1.0)
    assert _retained_per_sample(qnn.gelu) == pytest.approx(512 + 4, abs=1.0)
    assert _retained_per_sample(qnn.silu) == pytest.approx(512 + 4, abs=1.0)
    assert _retained_per_sample(qnn.relu_square) == pytest.approx(512 + 4, abs=1.0)


def test_relu_square_fuses_and_matches_torch():
    import qste_amd as qste
    from qste_amd import nn as qnn

    mine, theirs = _pair((16, 96), seed=11)
    ours, ref = qnn.relu_square(mine), F.relu(theirs).square()
    assert torch.equal(ours, ref)
    _backward(ours)
    _backward(ref)
    err = (mine.grad - theirs.grad).abs().max() / theirs.grad.abs().max()
    assert err < 0.01
    x = torch.randn(8, 40, device=DEV)
    with qste.packed_activations():
        r = qnn.relu(x)
        assert torch.equal(r.square(), F.relu(x).square())
        assert torch.equal(r ** 2, F.relu(x) ** 2)
        assert type(r * 3) is torch.Tensor


def test_elementwise_packs_any_function():
    from qste_amd import nn as qnn

    f = lambda t: t * torch.tanh(F.softplus(t))  # noqa: E731
    mine, theirs = _pair((32, 80), seed=12)
    ours = qnn.elementwise(f, mine)
    ref = f(theirs)
    assert torch.allclose(ours, ref)
    _backward(ours)
    _backward(ref)
    assert (mine.grad - theirs.grad).abs().max() / theirs.grad.abs().max() < 0.01
    with pytest.raises(ValueError):
        qnn.elementwise(lambda t: t.sum(-1), mine)


def test_packed_activations_route_only_converted_outputs():
    import qste_amd as qste

    class MLP(nn.Module):
        def __init__(self):
            super().__init__()
            self.gate = nn.Linear(64, 128, bias=False)
            self.up = nn.Linear(64, 128, bias=False)
            self.down = nn.Linear(128, 64, bias=False)

        def forward(self, x):
            return self.down(F.silu(self.gate(x)) * self.up(x))

    torch.manual_seed(0)
    model = qste.convert(MLP()).to(DEV)
    x = torch.randn(32, 64, device=DEV)
    kinds = []

    def pack(t):
        kinds.append(t.dtype)
        return t

    with qste.packed_activations(), torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
        out = model(x)
    assert torch.int8 in kinds  # silu kept its derivative as bytes
    out.sum().backward()
    assert F.silu is qste.nn._TORCH_SILU  # restored
    # an unconverted tensor goes to torch unchanged
    plain = torch.randn(4, 8, device=DEV)
    with qste.packed_activations():
        assert torch.equal(F.silu(plain), qste.nn._TORCH_SILU(plain))


def test_convert_replaces_activation_modules():
    import qste_amd as qste

    model = nn.Sequential(nn.Linear(32, 64), nn.GELU(), nn.Linear(64, 32), nn.ReLU(), nn.Dropout(0.1))
    qste.convert(model)
    assert isinstance(model[1], qste.nn.GELU) and isinstance(model[3], qste.nn.ReLU)
    assert isinstance(model[4], qste.nn.Dropout) and model[4].p == 0.1
    model = nn.Sequential(nn.Linear(32, 64), nn.GELU(), nn.Linear(64, 32), nn.ReLU())
    qste.convert(model, activations="exact")
    assert type(model[1]) is nn.GELU and isinstance(model[3], qste.nn.ReLU)
    model = nn.Sequential(nn.Linear(32, 64), nn.GELU())
    qste.convert(model, activations=False)
    assert type(model[1]) is nn.GELU
