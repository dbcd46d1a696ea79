"""Skinny-M forward (decode, M <= 16 bf16 rows) against the CPU oracle.

One kernel serves this path: a bf16 MFMA kernel whose weight operand is
biased (v0(k mod 4) + 0.5 * bit, the bias removed with two per-row sums).
Besides ordinary shapes the tests cover what that scheme could get wrong:
every M from 1 to 16 (rows of x padded to the 16 MFMA rows), K that ends
inside a 512-column chunk, N that ends inside a 16-row block and inside a
workgroup, inputs with many exact zeros (ReLU outputs), a row of large values
next to rows of tiny ones, an all-zero row, and the full config-5 shape.

Bars, against the float64 oracle (the reference's PackedLinear computes in
fp32 and rounds once to the input dtype, modules.py:114-120):
* rel-L2 <= 1e-3 against the oracle rounded to bf16 (the forward contract);
* every element within one bf16 ulp of the oracle plus 2^-16 * sum_k
  |x[m,k]| * scale[n]: the fp32 accumulation of the biased operand sums
  magnitudes up to 4.5 * sum |x| and removes the bias by a subtraction, so
  its rounding error scales with sum |x| (about 2^-20 of it), not with |y|;
* fewer than 0.5% of elements differ from the rounded oracle on random data
  (1-ulp rounding flips of outputs that sit near a bf16 rounding boundary),
  5% on single special-valued rows (sum |x| large against |y|).
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


def _check(got: torch.Tensor, want: np.ndarray, x: np.ndarray | None = None, scale: np.ndarray | None = None,
           flips: float = 0.005):
    got = got.float().cpu().numpy().astype(np.float64)
    want = np.asarray(want, dtype=np.float64)
    want_r = _bf(want).astype(np.float64)
    denom = np.linalg.norm(want_r)
    err = np.linalg.norm(got - want_r) / (denom if denom > 0 else 1.0)
    assert err <= 1e-3, err
    assert np.mean(got != want_r) < flips, np.mean(got != want_r)
    if x is not None:
        ulp = np.abs(want_r) * 2.0 ** -7
        mag = np.abs(x).astype(np.float64).sum(axis=1)[:, None] * np.abs(scale).astype(np.float64)[None, :]
        bound = ulp + 2.0 ** -16 * mag
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
    # one row at a time: a row whose outputs are small against sum |x| (the
    # large-valued row) sees more 1-ulp rounding flips than random data, so
    # the per-row flip bar is 5%; the error bound itself is unchanged
    for r in range(m):
        _check(got[r:r + 1], want[r:r + 1], x[r:r + 1], scale, flips=0.05)
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
