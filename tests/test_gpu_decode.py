"""Skinny-M forward (decode, M <= 16 bf16 or fp16 rows) against the CPU oracle.

One kernel serves this path, instantiated for bf16 and fp16 activations: an
MFMA kernel (16x16x32 in the activations' dtype) whose weight operand is
biased (v0(k mod 4) + 0.5 * bit, the bias removed with two per-row sums).
Besides ordinary shapes the tests cover what that scheme could get wrong:
every M from 1 to 16 (rows of x padded to the 16 MFMA rows), K that ends
inside a 512-column chunk, N that ends inside a 16-row block and inside a
workgroup, inputs with many exact zeros (ReLU outputs), a row of large values
next to rows of tiny ones, an all-zero row, and the full config-5 shape.

Bars, against the float64 oracle (the reference's PackedLinear computes in
fp32 and rounds once to the input dtype, modules.py:114-120):
* rel-L2 <= 1e-3 against the oracle rounded to the dtype (the forward
  contract);
* every element within one ulp of the dtype of the oracle plus 2^-16 * sum_k
  |x[m,k]| * scale[n]: the fp32 accumulation of the biased operand sums
  magnitudes up to 4.5 * sum |x| and removes the bias by a subtraction, so
  its rounding error scales with sum |x| (about 2^-20 of it), not with |y|;
* few elements differ from the rounded oracle (1-ulp rounding flips of
  outputs that sit near a rounding boundary): under 0.5% on random bf16
  data, 5% on single special-valued bf16 rows (sum |x| large against |y|).
  fp16 keeps 3 more bits, so the same accumulation error is 8x larger
  against its ulp and the flip bars are 4% and 15%; the absolute bound
  above is the same for both dtypes.
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


DTYPES = [torch.bfloat16, torch.float16]
ULP = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}


def _rd(a: np.ndarray, dtype=torch.bfloat16) -> np.ndarray:
    """Values rounded to the dtype, as float32."""

    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(dtype).float().numpy()


FLIPS = {torch.bfloat16: 0.005, torch.float16: 0.04}


def _check(got: torch.Tensor, want: np.ndarray, x: np.ndarray | None = None, scale: np.ndarray | None = None,
           flips: float | None = None):
    dtype = got.dtype
    flips = FLIPS[dtype] if flips is None else flips
    got = got.float().cpu().numpy().astype(np.float64)
    want = np.asarray(want, dtype=np.float64)
    want_r = _rd(want, dtype).astype(np.float64)
    denom = np.linalg.norm(want_r)
    err = np.linalg.norm(got - want_r) / (denom if denom > 0 else 1.0)
    assert err <= 1e-3, err
    print(f"flip rate {np.mean(got != want_r):.4f} ({dtype})", flush=True)
    assert np.mean(got != want_r) < flips, np.mean(got != want_r)
    if x is not None:
        ulp = np.abs(want_r) * ULP[dtype]
        mag = np.abs(x).astype(np.float64).sum(axis=1)[:, None] * np.abs(scale).astype(np.float64)[None, :]
        bound = ulp + 2.0 ** -16 * mag
        assert np.all(np.abs(got - want) <= bound), np.max(np.abs(got - want) / bound)


def _run(x: np.ndarray, packed: np.ndarray, scale: np.ndarray, bias, cols: int, dtype=torch.bfloat16):
    xt = torch.from_numpy(x).to(DEV).to(dtype)
    pt = torch.from_numpy(packed).to(DEV)
    st = torch.from_numpy(scale).to(DEV)
    bt = None if bias is None else torch.from_numpy(bias).to(DEV)
    y = _k().packed_linear_affine(xt, pt, st, bt, cols)
    assert y.dtype == dtype
    return y


def _problem(rows, cols, m, seed, dtype=torch.bfloat16):
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, size=(rows, cols // 8), dtype=np.uint8)
    x = _rd(rng.standard_normal((m, cols)).astype(np.float32), dtype)
    scale = (np.abs(rng.standard_normal(rows)) * 0.02 + 0.01).astype(np.float32)
    bias = (rng.standard_normal(rows) * 0.1).astype(np.float32)
    return packed, x, scale, bias


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", list(range(1, 17)))
def test_decode_every_m(m, dtype):
    packed, x, scale, bias = _problem(300, 1024, m, 100 + m, dtype)
    _check(_run(x, packed, scale, bias, 1024, dtype), oracle.linear_fwd(x, packed, scale, bias, 1024), x, scale)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,cols,m", [(16, 128, 1), (17, 384, 3), (1, 640, 2), (4097, 896, 5),
                                         (129, 4224, 16), (8192, 8192, 4), (40000, 256, 7)])
def test_decode_ragged_shapes(rows, cols, m, dtype):
    packed, x, scale, bias = _problem(rows, cols, m, rows + cols + m, dtype)
    _check(_run(x, packed, scale, bias, cols, dtype), oracle.linear_fwd(x, packed, scale, bias, cols), x, scale)
    _check(_run(x, packed, scale, None, cols, dtype), oracle.linear_fwd(x, packed, scale, None, cols), x, scale)


@pytest.mark.parametrize("dtype", DTYPES)
def test_decode_special_values(dtype):
    """Exact zeros, a large-valued row and a tiny-valued row in one batch."""

    rows, cols, m = 512, 2048, 6
    packed, x, scale, bias = _problem(rows, cols, m, 7, dtype)
    x = x.copy()
    # large and tiny magnitudes that stay finite and normal in the dtype
    big, tiny = (3.0e4, 1.0e-30) if dtype == torch.bfloat16 else (1.0e3, 1.0e-3)
    x[0] = np.maximum(x[0], 0.0)             # ReLU-like: about half exact zeros
    x[1, ::3] = 0.0
    x[2] = _rd(x[2] * big, dtype)            # large magnitudes
    x[3] = _rd(x[3] * tiny, dtype)           # tiny magnitudes
    x[4] = 0.0                               # an all-zero row gives the bias
    x[5, :] = _rd(np.float32(1.5), dtype)    # constant row
    got = _run(x, packed, scale, bias, cols, dtype)
    want = oracle.linear_fwd(x, packed, scale, bias, cols)
    # one row at a time: a row whose outputs are small against sum |x| (the
    # large-valued row) sees more 1-ulp rounding flips than random data, so
    # the per-row flip bar is 5%; the error bound itself is unchanged
    for r in range(m):
        _check(got[r:r + 1], want[r:r + 1], x[r:r + 1], scale, flips=0.05 if dtype == torch.bfloat16 else 0.15)
    assert np.array_equal(got[4].float().cpu().numpy(), _rd(bias, dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [1, 4, 16])
def test_decode_config5_shape(m, dtype):
    """K=8192, N=28672 (the config-5 matrix); oracle on a sample of weight rows."""

    rows, cols = 28672, 8192
    g = torch.Generator(device=DEV).manual_seed(m)
    packed = torch.randint(0, 256, (rows, cols // 8), generator=g, device=DEV, dtype=torch.int32).to(torch.uint8)
    scale = torch.randn(rows, generator=g, device=DEV).abs_().mul_(0.02)
    x = torch.randn(m, cols, generator=g, device=DEV).to(dtype)
    y = _k().packed_linear_affine(x, packed, scale, None, cols)
    torch.cuda.synchronize()
    assert y.dtype == dtype
    rng = np.random.default_rng(m)
    sel = np.sort(rng.choice(rows, 700, replace=False))
    pk = packed.cpu().numpy()[sel]
    xs = x.float().cpu().numpy()
    want = oracle.linear_fwd(xs, pk, scale.cpu().numpy()[sel], None, cols)
    _check(y[:, torch.from_numpy(sel).to(DEV)], want, xs, scale.cpu().numpy()[sel])


@pytest.mark.parametrize("dtype", DTYPES)
def test_decode_is_deterministic(dtype):
    packed, x, scale, bias = _problem(2048, 4096, 9, 3, dtype)
    a = _run(x, packed, scale, bias, 4096, dtype)
    b = _run(x, packed, scale, bias, 4096, dtype)
    assert torch.equal(a, b)
