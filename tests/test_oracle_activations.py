"""The packed-activation oracle (``oracle/activations.py``), pinned on the CPU.

Each restated function is checked against something independent of its own
formula:

* bits -- ``np.packbits(bitorder="little")`` and per-bit brute force;
* masked values -- torch's own ``F.relu`` / ``relu6`` / ``hardtanh`` /
  ``leaky_relu`` on the CPU, bit for bit, in fp32 and bf16 (the reference's
  forward *is* torch's, ``src/qste/nn.py:119-131, 271-276``);
* masked gradients -- torch autograd of the same functions (bit for bit for
  the clamp family, within an ulp-sized bound for the sloped ones, whose
  reference backward is a two-term expression, nn.py:278-282);
* derivatives -- float64 autograd of torch's activation, a tight relative
  bound (an fp32 restatement is ~1e-7 off; a wrong term is >1e-3 off);
* the quantization -- its closed form (scale = row max / 127 exactly,
  |payload * scale - d| <= scale / 2, ties to even) and torch evaluating the
  reference's own tensor expressions on the oracle's derivative;
* a planted mistake (a /128 scale) that the closed-form check must catch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import activations as oa

WIDTHS = [1, 7, 8, 9, 33, 64, 100]


def _x(shape, seed=0, spread=3.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * spread


# ---------------------------------------------------------------------------
# bits
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("cols", WIDTHS)
def test_pack_bits_matches_numpy_packbits_and_brute_force(cols):
    rng = np.random.default_rng(cols)
    mask = rng.random((5, cols)) < 0.4
    packed = oa.pack_bits(mask)
    assert packed.shape == (5, (cols + 7) // 8)
    assert np.array_equal(packed, np.packbits(mask, axis=1, bitorder="little"))
    for r in range(5):
        for c in range(cols):
            assert ((packed[r, c // 8] >> (c % 8)) & 1) == mask[r, c]
    assert np.array_equal(oa.unpack_bits(packed, cols).astype(bool), mask)


def test_apply_bits_is_a_select_with_positive_zero():
    values = np.array([[-1.5, 2.0, -0.0, np.inf, np.nan, 3.0, -4.0, 5.0, 6.0]], np.float32)
    keep = np.array([[0, 1, 1, 0, 0, 1, 0, 1, 1]], bool)
    out = oa.apply_bits(values, oa.pack_bits(keep))
    assert np.array_equal(out[keep], values[keep])
    dropped = out[~keep]
    assert np.all(dropped == 0) and not np.any(np.signbit(dropped))


# ---------------------------------------------------------------------------
# masked forwards / backwards against torch
# ---------------------------------------------------------------------------


CLAMPS = [("relu", 0.0, None, F.relu), ("relu6", 0.0, 6.0, F.relu6),
          ("hardtanh", -1.0, 1.0, F.hardtanh), ("hardtanh_wide", -2.5, 0.75,
                                                lambda t: F.hardtanh(t, -2.5, 0.75))]


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("name,lower,upper,fn", CLAMPS)
def test_clamp_forward_is_torch_and_its_mask(dtype, name, lower, upper, fn):
    tdt = getattr(torch, dtype)
    x = _x((6, 37), seed=3).to(tdt)
    x[0, :5] = torch.tensor([0.0, 6.0, -1.0, 1.0, 0.75])  # values on the bounds
    out, packed = oa.clamp_forward(x.float().numpy(), lower, upper, dtype)
    ref = fn(x)
    assert np.array_equal(out, ref.float().numpy())
    keep = ref > lower if upper is None else (ref > lower) & (ref < upper)
    assert np.array_equal(packed, np.packbits(keep.numpy(), axis=1, bitorder="little"))


@pytest.mark.parametrize("name,lower,upper,fn", CLAMPS)
def test_clamp_gradient_is_torch_autograd(name, lower, upper, fn):
    x = _x((4, 29), seed=4).requires_grad_(True)
    g = _x((4, 29), seed=5)
    fn(x).backward(g)
    _, packed = oa.clamp_forward(x.detach().numpy(), lower, upper)
    assert np.array_equal(oa.masked_backward(g.numpy(), packed, 1.0, 0.0), x.grad.numpy())


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_leaky_forward_is_torch_and_gradient_is_the_reference_expression(dtype):
    tdt = getattr(torch, dtype)
    slope = 0.1
    x = _x((5, 40), seed=6).to(tdt)
    out, packed = oa.leaky_forward(x.float().numpy(), slope, dtype)
    assert np.array_equal(out, F.leaky_relu(x, slope).float().numpy())
    g = _x((5, 40), seed=7).to(tdt)
    ours = oa.masked_backward(g.float().numpy(), packed, 1.0, slope, dtype)
    # nn.py:278-282 evaluated by torch on the same mask
    kept = g * (x > 0).to(tdt)
    expr = g * slope + kept * (1.0 - slope)
    assert np.array_equal(ours, expr.float().numpy())
    # and it is leaky_relu's true gradient up to the expression's roundings
    xx = x.float().clone().requires_grad_(True)
    F.leaky_relu(xx, slope).backward(g.float())
    tol = 2 ** -7 if dtype == "bfloat16" else 1e-6
    assert np.allclose(ours, xx.grad.numpy(), rtol=tol, atol=0)


def test_hardsigmoid_interval_mask_and_slope():
    x = _x((3, 50), seed=8, spread=4.0)
    x[0, :2] = torch.tensor([-3.0, 3.0])
    packed = oa.interval_bits(x.numpy(), -3.0, 3.0)
    assert np.array_equal(oa.unpack_bits(packed, 50).astype(bool), ((x > -3) & (x < 3)).numpy())
    xx = x.clone().requires_grad_(True)
    g = _x((3, 50), seed=9)
    F.hardsigmoid(xx).backward(g)
    ours = oa.masked_backward(g.numpy(), packed, 1.0 / 6.0, 0.0)
    assert np.allclose(ours, xx.grad.numpy(), rtol=1e-6, atol=0)


def test_dropout_backward_scales_kept_values_by_the_gain():
    g = _x((4, 16), seed=10)
    keep = (_x((4, 16), seed=11) > 0).numpy()
    ours = oa.masked_backward(g.numpy(), oa.pack_bits(keep), 2.0, 0.0)
    assert np.array_equal(ours, np.where(keep, g.numpy() * np.float32(2.0), 0).astype(np.float32))


# ---------------------------------------------------------------------------
# smooth derivatives against float64 autograd of torch's activation
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


@pytest.mark.parametrize("kind,param,fn", SMOOTH)
def test_derivative_formula_matches_float64_autograd(kind, param, fn):
    x64 = _x((8, 257), seed=12).double()
    x64[0, :4] = torch.tensor([0.0, -3.0, 3.0, 25.0], dtype=torch.float64)
    x64.requires_grad_(True)
    fn(x64).sum().backward()
    exact = x64.grad.numpy()
    x = x64.detach().float().numpy()
    y = oa.value(kind, x, param)
    d = oa.derivative(kind, x, y, param)
    scale = np.abs(exact).max()
    err = np.abs(d.astype(np.float64) - exact)
    if kind == "hardswish":  # the knees: torch and the reference agree off them
        err = err[np.abs(np.abs(x) - 3.0) > 1e-6]
    assert err.max() <= 2e-6 * scale, f"{kind}: {err.max() / scale:.2e}"


@pytest.mark.parametrize("kind,param,fn", SMOOTH)
def test_value_matches_torch_fp32(kind, param, fn):
    x = _x((6, 129), seed=13)
    ours = oa.value(kind, x.numpy(), param)
    ref = fn(x).numpy()
    # torch's fp32 erf/exp differ from a correctly rounded one by a few ulp,
    # which 1 + erf(x) near erf = -1 magnifies: an absolute floor of 1e-6
    assert np.allclose(ours, ref, rtol=1e-6, atol=1e-6), kind


# ---------------------------------------------------------------------------
# quantization
# ---------------------------------------------------------------------------


def test_quantize_rows_closed_form_and_ties():
    rng = np.random.default_rng(1)
    d = rng.normal(size=(16, 300)).astype(np.float32)
    d[3] = 0.0  # an all-zero row takes the 1e-8 floor
    payload, scale = oa.quantize_rows(d)
    amax = np.abs(d).max(axis=1)
    assert np.array_equal(scale, (np.maximum(amax, np.float32(1e-8)) / np.float32(127)).astype(np.float32))
    assert payload.dtype == np.int8 and np.abs(payload.astype(int)).max() <= 127
    err = np.abs(payload.astype(np.float64) * scale[:, None] - d)
    assert np.all(err <= scale[:, None] * 0.5000001)
    # the row maximum lands on +-127 exactly
    rows = np.arange(16) != 3
    assert np.all(np.abs(payload[rows]).max(axis=1) == 127)
    # ties go to even
    s = np.float32(1.0)
    ties = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5]], np.float32) * s
    p, _ = oa.quantize_rows(ties)
    assert p.tolist() == [[127, 0, 2, 2, 0, -2]]


def test_quantization_matches_the_reference_expression_in_torch():
    d = oa.derivative("silu", _x((32, 96), seed=14).numpy(), None, 0.0)
    payload, scale = oa.quantize_rows(d)
    flat = torch.from_numpy(d.copy())
    t_scale = flat.abs().amax(dim=1).clamp_min(1e-8).div_(127.0)
    t_payload = flat.div_(t_scale.unsqueeze(1)).round_().clamp_(-127, 127).to(torch.int8)
    assert np.array_equal(scale, t_scale.numpy())
    assert np.array_equal(payload, t_payload.numpy())


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_relu_square_matches_the_reference_expression_in_torch(dtype):
    tdt = getattr(torch, dtype)
    x = _x((12, 70), seed=15).to(tdt)
    x[5] = -1.0  # a row with nothing positive
    y, payload, scale = oa.smooth_forward("relu_square", x.float().numpy(), dtype=dtype)
    activated = x.clamp_min(0)
    t_scale = activated.amax(dim=1).clamp_min(1e-8).div_(255.0)
    t_payload = activated.div(t_scale.unsqueeze(1)).round_().clamp_(0, 255).to(torch.uint8)
    assert np.array_equal(y, (activated * activated).float().numpy())
    assert np.array_equal(scale, t_scale.float().numpy())
    assert np.array_equal(payload, t_payload.numpy())


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_smooth_backward_matches_the_reference_expression_in_torch(dtype):
    tdt = getattr(torch, dtype)
    x = _x((10, 48), seed=16)
    _, payload, scale = oa.smooth_forward("gelu", x.numpy())
    g = _x((10, 48), seed=17).to(tdt)
    ours = oa.smooth_backward(g.float().numpy(), payload, scale, dtype)
    t = torch.from_numpy(payload).to(tdt).mul_(torch.from_numpy(scale).to(tdt).unsqueeze(1))
    assert np.array_equal(ours, (g * t).float().numpy())
    # relu(x)^2: grad * 2.0 * activated (nn.py:325-330)
    _, up, us = oa.smooth_forward("relu_square", x.to(tdt).float().numpy(), dtype=dtype)
    ours = oa.smooth_backward(g.float().numpy(), up, us, dtype)
    act = torch.from_numpy(up).to(tdt).mul_(torch.from_numpy(us).to(tdt).unsqueeze(1))
    assert np.array_equal(ours, (g * 2.0 * act).float().numpy())


def test_a_planted_scale_mistake_is_caught():
    d = np.random.default_rng(2).normal(size=(4, 64)).astype(np.float32)
    amax = np.abs(d).max(axis=1)
    wrong_scale = np.maximum(amax, np.float32(1e-8)) / np.float32(128)
    _, scale = oa.quantize_rows(d)
    assert not np.array_equal(wrong_scale.astype(np.float32), scale)
    wrong_payload = np.clip(np.rint(d / wrong_scale[:, None]), -127, 127)
    # the 128-step payload no longer reaches the row maximum on +-127
    assert not np.all(np.abs(wrong_payload).max(axis=1) == 127) or not np.allclose(
        wrong_payload * wrong_scale[:, None], d, atol=0.5 * wrong_scale.max())
