"""Skinny-M forward (decode, M <= 16 bf16 rows) against the CPU oracle.

Two kernels serve this path: for M <= 2 an fp8 x fp4 MFMA kernel (x split
into two fp8 limbs with a per-row power-of-two scale, weight bits turned into
fp4 0 / 0.5 / 1 / 2 by masks), otherwise a bf16 MFMA kernel whose weight
operand is biased (v0(k mod 4) + 0.5 * bit, the bias removed with two per-row
sums).  Besides ordinary shapes the tests cover what those schemes could get
wrong: every M from 1 to 16 (rows of x padded to the 16 MFMA rows, limbs in
the spare rows), K that ends inside a 512-column chunk, N that ends inside a
16-row block and inside a workgroup, inputs with many exact zeros (ReLU
outputs), a row of large values next to rows of tiny ones (the row scale), an
all-zero row, and the full config-5 shape.

Bars, against the float64 oracle:
* rel-L2 <= 1e-3 against the oracle rounded to bf16 (the forward contract);
* every element within one bf16 ulp of the oracle plus 2^-12 * sum_k |x[m,k]| *
  scale[n].  The second term is the accumulation error of the M <= 2 path: its
  fp8 x fp4 MFMA sums each 128-product group keeping about 16 bits below the
  group's largest product (measured on the device: at most 3.5e-5 of the
  group's sum of magnitudes), so outputs that cancel to near zero carry an
  absolute error on the scale of sum |x|, not of |y|;
* fewer than 5% of elements differ from the rounded oracle (1-ulp rounding
  flips: 0.5% at K=1024 and 2.3% at K=8192 on the fp8 x fp4 path, about
  0.05% on the bf16 MFMA path).
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


def _bf(a: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def _check(got: torch.Tensor, want: np.ndarray, x: np.ndarray | None = None, scale: np.ndarray | None = None):
    got = got.float().cpu().numpy().astype(np.float64)
    want = np.asarray(want, dtype=np.float64)
    want_r = _bf(want).astype(np.float64)
    denom = np.linalg.norm(want_r)
    err = np.linalg.norm(got - want_r) / (denom if denom > 0 else 1.0)
    assert err <= 1e-3, err
    assert np.mean(got != want_r) < 0.05, np.mean(got != want_r)
    if x is not None:
        ulp = np.abs(want_r) * 2.0 ** -7
        mag = np.abs(x).astype(np.float64).sum(axis=1)[:, None] * np.abs(scale).astype(np.float64)[None, :]
        bound = ulp + 2.0 ** -12 * mag
        assert np.all(np.abs(got - want) <= bound), np.max(np.abs(got - want) / bound)


def _run(x: np.ndarray, packed: np.ndarray, scale: np.ndarray, bias, cols: int):
    xt = torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    pt = torch.from_numpy(packed).to(DEV)
    st = torch.from_numpy(scale).to(DEV)
    bt = None if bias is None else torch.from_numpy(bias).to(DEV)
    return _k().packed_linear_affine(xt, pt, st, bt, cols)


def _problem(rows, cols, m, seed):
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, size=(rows, cols // 8), dtype=np.uint8)
    x = _bf(rng.standard_normal((m, cols)).astype(np.float32))
    scale = (np.abs(rng.standard_normal(rows)) * 0.02 + 0.01).astype(np.float32)
    bias = (rng.standard_normal(rows) * 0.1).astype(np.float32)
    return packed, x, scale, bias


@pytest.mark.parametrize("m", list(range(1, 17)))
def test_decode_every_m(m):
    packed, x, scale, bias = _problem(300, 1024, m, 100 + m)
    _check(_run(x, packed, scale, bias, 1024), oracle.linear_fwd(x, packed, scale, bias, 1024), x, scale)


@pytest.mark.parametrize("rows,cols,m", [(16, 128, 1), (17, 384, 3), (1, 640, 2), (4097, 896, 5),
                                         (129, 4224, 16), (8192, 8192, 4), (40000, 256, 7)])
def test_decode_ragged_shapes(rows, cols, m):
    packed, x, scale, bias = _problem(rows, cols, m, rows + cols + m)
    _check(_run(x, packed, scale, bias, cols), oracle.linear_fwd(x, packed, scale, bias, cols), x, scale)
    _check(_run(x, packed, scale, None, cols), oracle.linear_fwd(x, packed, scale, None, cols), x, scale)


def test_decode_special_values():
    """Exact zeros, a large-valued row and a tiny-valued row in one batch."""

    rows, cols, m = 512, 2048, 6
    packed, x, scale, bias = _problem(rows, cols, m, 7)
    x = x.copy()
    x[0] = np.maximum(x[0], 0.0)             # ReLU-like: about half exact zeros
    x[1, ::3] = 0.0
    x[2] = _bf(x[2] * 3.0e4)                 # large magnitudes
    x[3] = _bf(x[3] * 1.0e-30)               # tiny magnitudes (still normal in bf16)
    x[4] = 0.0                               # an all-zero row gives the bias
    x[5, :] = _bf(np.float32(1.5))           # constant row
    got = _run(x, packed, scale, bias, cols)
    want = oracle.linear_fwd(x, packed, scale, bias, cols)
    for r in range(m):
        _check(got[r:r + 1], want[r:r + 1], x[r:r + 1], scale)
    assert np.array_equal(got[4].float().cpu().numpy(), _bf(bias))


@pytest.mark.parametrize("m", [1, 4, 16])
def test_decode_config5_shape(m):
    """K=8192, N=28672 (the config-5 matrix); oracle on a sample of weight rows."""

    rows, cols = 28672, 8192
    g = torch.Generator(device=DEV).manual_seed(m)
    packed = torch.randint(0, 256, (rows, cols // 8), generator=g, device=DEV, dtype=torch.int32).to(torch.uint8)
    scale = torch.randn(rows, generator=g, device=DEV).abs_().mul_(0.02)
    x = torch.randn(m, cols, generator=g, device=DEV).to(torch.bfloat16)
    y = _k().packed_linear_affine(x, packed, scale, None, cols)
    torch.cuda.synchronize()
    rng = np.random.default_rng(m)
    sel = np.sort(rng.choice(rows, 700, replace=False))
    pk = packed.cpu().numpy()[sel]
    xs = x.float().cpu().numpy()
    want = oracle.linear_fwd(xs, pk, scale.cpu().numpy()[sel], None, cols)
    _check(y[:, torch.from_numpy(sel).to(DEV)], want, xs, scale.cpu().numpy()[sel])


def test_decode_is_deterministic():
    packed, x, scale, bias = _problem(2048, 4096, 9, 3)
    a = _run(x, packed, scale, bias, 4096)
    b = _run(x, packed, scale, bias, 4096)
    assert torch.equal(a, b)
