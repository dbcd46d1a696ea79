"""fp32 products on the bf16 MFMA path (three bf16 limbs along K).

The forward, the input gradient and the evidence of fp32 operands run the
bf16 MFMA kernels over 3K: each fp32 value splits exactly into hi + mid + lo
bf16 limbs and each limb times +-1 is exact, so the sums carry only fp32
accumulation error.  Bars against the float64 oracle, per product: rel-L2
error <= 2e-6 (fp32 accumulation over K terms of random sign gives ~1e-7;
a dropped low limb alone gives ~2^-17 = 7.6e-6, a dropped middle limb
~2e-3), and no element off by more than 2^-20 of the sum of its terms'
magnitudes.  Also checked: the limbs path agrees with the fp32 SIMT kernels
(the plain entries) to the same bar, shapes with ragged output rows and
columns, config 1's full layer backward through ``linear_backward``, and
that the limbs path is the one that runs (it differs from the SIMT result
in the last bits somewhere).
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


def _rel(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-300))


def _bounded(got, want, mag):
    assert np.all(np.abs(np.asarray(got, np.float64) - want) <= 2.0 ** -20 * mag + 1e-30)


def _problem(m, rows, cols, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(m, cols, generator=g, device=DEV)
    coord = torch.randint(-127, 128, (rows, cols), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    from qste_amd import kernels

    packed = kernels.pack_coordinate(coord)
    scale = torch.rand(rows, generator=g, device=DEV) * 0.02 + 0.005
    bias = torch.randn(rows, generator=g, device=DEV) * 0.1
    return x, packed, scale, bias


def _plain_forward(x, packed, scale, bias, cols):
    """The plain C entry (fp32 SIMT kernel), for comparison."""

    from qste_amd import kernels

    out = torch.empty(x.shape[0], packed.shape[0], device=DEV)
    code = kernels._lib.load().qste_packed_linear_affine(
        x.data_ptr(), 0, packed.data_ptr(), scale.data_ptr(), bias.data_ptr(), out.data_ptr(), x.shape[0],
        packed.shape[0], cols, torch.cuda.current_stream().cuda_stream)
    kernels._lib.check(code, "packed_linear_affine")
    return out


@pytest.mark.parametrize("m,rows,cols", [(256, 2048, 2048), (512, 1000, 1024), (300, 640, 4096),
                                         (1024, 4096, 4096)])
def test_forward(m, rows, cols):
    from qste_amd import kernels

    print(f"fp32 forward {m}x{rows}x{cols}", flush=True)
    lib = kernels._lib.load()
    assert lib.qste_packed_linear_affine_workspace_bytes(m, rows, cols, 0) > 0
    x, packed, scale, bias = _problem(m, rows, cols, m + rows + cols)
    y = kernels.packed_linear_affine(x, packed, scale, bias, cols)
    simt = _plain_forward(x, packed, scale, bias, cols)
    torch.cuda.synchronize()
    assert y.dtype == torch.float32
    xs, pk, sc, bi = x.cpu().numpy(), packed.cpu().numpy(), scale.cpu().numpy(), bias.cpu().numpy()
    want = oracle.linear_fwd_f64(xs, pk, sc, bi, cols)
    err = _rel(y.cpu().numpy(), want)
    print(f"  rel-L2 {err:.3e} (SIMT {_rel(simt.cpu().numpy(), want):.3e})", flush=True)
    assert err <= 2e-6
    mag = np.abs(xs.astype(np.float64)).sum(1)[:, None] * sc[None, :]
    _bounded(y.cpu().numpy(), want, mag)
    assert not torch.equal(y, simt)  # a different kernel ran (fp32 roundings differ somewhere)


@pytest.mark.parametrize("m,rows,cols", [(256, 2048, 2048), (512, 4096, 1024), (384, 1024, 1000)])
def test_dgrad(m, rows, cols):
    from qste_amd import kernels

    print(f"fp32 dgrad {m}x{rows}x{cols}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows + m)
    dy = torch.randn(m, rows, generator=g, device=DEV)
    coord = torch.randint(-127, 128, (rows, cols), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    packed = kernels.pack_coordinate(coord)
    scale = torch.rand(rows, generator=g, device=DEV) * 0.02 + 0.005
    assert kernels._lib.load().qste_packed_transpose_workspace_bytes(m, rows, cols, 0) > 0
    dx = kernels.packed_transpose(dy, packed, cols, row_scale=scale)
    torch.cuda.synchronize()
    d, pk, sc = dy.cpu().numpy(), packed.cpu().numpy(), scale.cpu().numpy()
    want = oracle.linear_dgrad_f64(d, pk, cols, sc)
    err = _rel(dx.cpu().numpy(), want)
    print(f"  rel-L2 {err:.3e}", flush=True)
    assert err <= 2e-6
    mag = np.abs(d.astype(np.float64)) @ np.broadcast_to(sc[:, None].astype(np.float64), (rows, cols))
    _bounded(dx.cpu().numpy(), want, mag)


@pytest.mark.parametrize("samples,rows,cols", [(256, 2048, 2048), (1000, 1024, 512), (4096, 640, 1024)])
def test_evidence(samples, rows, cols):
    from qste_amd import kernels

    print(f"fp32 evidence {samples}x{rows}x{cols}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(samples + cols)
    dy = torch.randn(samples, rows, generator=g, device=DEV) * 0.1
    x = torch.randn(samples, cols, generator=g, device=DEV)
    packed_x, off, xs = kernels.pack_affine_rows(x)
    ev = kernels.evidence_from_packed(dy, packed_x, cols, row_scale=xs)
    torch.cuda.synchronize()
    d, px, s = dy.cpu().numpy(), packed_x.cpu().numpy(), xs.cpu().numpy()
    want = oracle.evidence_f64(d, px, cols, s)
    err = _rel(ev.cpu().numpy(), want)
    print(f"  rel-L2 {err:.3e}", flush=True)
    assert err <= 2e-6
    mag = (np.abs(d.astype(np.float64)) * s[:, None].astype(np.float64)).sum(0)[:, None] * np.ones((1, cols))
    _bounded(ev.cpu().numpy(), want, mag)


def test_config1_layer_backward():
    """Config 1's layer (2048 -> 2048 fp32, 256 tokens): every output of
    linear_backward against the float64 oracle."""

    from qste_amd import kernels

    T, R, C = 256, 2048, 2048
    g = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn(T, C, generator=g, device=DEV)
    dy = torch.randn(T, R, generator=g, device=DEV) * 1e-3
    coord = torch.randint(-127, 128, (R, C), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    packed_w = kernels.pack_coordinate(coord)
    scale = torch.rand(R, generator=g, device=DEV) * 0.02 + 0.005
    packed_x, off, xs = kernels.pack_affine_rows(x)
    lib = kernels._lib.load()
    assert lib.qste_linear_backward_workspace_bytes_dtype(T, R, C, 0) > lib.qste_linear_backward_workspace_bytes(
        T, R, C)
    dx, ev, gs, db = kernels.linear_backward(dy, packed_x, off, xs, packed_w, scale, C, need_bias=True)
    torch.cuda.synchronize()
    d, pw, sc = dy.cpu().numpy(), packed_w.cpu().numpy(), scale.cpu().numpy()
    px, o, s = packed_x.cpu().numpy(), off.cpu().numpy(), xs.cpu().numpy()
    assert _rel(dx.cpu().numpy(), oracle.linear_dgrad_f64(d, pw, C, sc)) <= 2e-6
    e0 = oracle.evidence_f64(d, px, C, s) + (d.astype(np.float64).T @ o.astype(np.float64))[:, None]
    assert _rel(ev.cpu().numpy(), e0 * sc[:, None]) <= 2e-6
    sign = oracle.signs_f64(pw, C)
    assert _rel(gs.cpu().numpy(), (e0 * sign).sum(1)) <= 2e-6
    assert _rel(db.cpu().numpy(), d.astype(np.float64).sum(0)) <= 1e-6


def _nonfinite_agree(got, want):
    """Same NaN positions, same infinities with the same signs."""

    got = np.asarray(got, np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isposinf(got), np.isposinf(want))
    assert np.array_equal(np.isneginf(got), np.isneginf(want))


def test_special_values_keep_their_ieee_results():
    """inf, NaN and values near fp32's largest through the limbs: the
    forward and the input gradient give the infinities and NaNs an fp32
    product gives (the float64 oracle on the same operands), and a finite
    value too large for bf16's rounding (above 3.3961e38) stays finite."""

    from qste_amd import kernels

    m, rows, cols = 256, 512, 1024
    x, packed, scale, bias = _problem(m, rows, cols, 11)
    big = np.float32(3.40e38)
    x[0, 5] = float("inf")                      # +-inf in every output of row 0
    x[1, 7] = float("nan")                      # NaN everywhere in row 1
    x[2, 3], x[2, 900] = float("inf"), -float("inf")  # NaN or +-inf by the two signs
    x[3, 10] = float(big)                       # finite, rounds to inf in bf16
    x[4, 20] = -float(big)
    y = kernels.packed_linear_affine(x, packed, scale, bias, cols)
    torch.cuda.synchronize()
    xs, pk, sc, bi = x.cpu().numpy(), packed.cpu().numpy(), scale.cpu().numpy(), bias.cpu().numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        want = oracle.linear_fwd_f64(xs, pk, sc, bi, cols)
    got = y.cpu().numpy()
    _nonfinite_agree(got, want)
    assert np.isfinite(got[3:]).all()
    assert np.isinf(got[0]).all() and np.isnan(got[1]).all()
    assert np.isnan(got[2]).any() and np.isinf(got[2]).any()
    fin = slice(3, m)
    assert _rel(got[fin], want[fin]) <= 2e-6
    mag = np.abs(xs[fin].astype(np.float64)).sum(1)[:, None] * sc[None, :]
    _bounded(got[fin], want[fin], mag)

    # the input gradient: the same values in dy, along K = rows
    g = torch.Generator(device=DEV).manual_seed(12)
    dy = torch.randn(m, rows, generator=g, device=DEV)
    dy[0, 5] = float("inf")
    dy[1, 7] = float("nan")
    dy[3, 10] = float(big)
    one = torch.ones(rows, device=DEV)          # row scale 1 keeps the near-max value as it is
    dx = kernels.packed_transpose(dy, packed, cols, row_scale=one)
    torch.cuda.synchronize()
    d = dy.cpu().numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        want = oracle.linear_dgrad_f64(d, pk, cols, one.cpu().numpy())
    got = dx.cpu().numpy()
    _nonfinite_agree(got, want)
    assert np.isinf(got[0]).all() and np.isnan(got[1]).all() and np.isfinite(got[2:]).all()
    assert _rel(got[2:], want[2:]) <= 2e-6


def test_products_over_row_chunks():
    """A dense operand whose limbs exceed the 512 MiB budget runs in chunks
    of output rows (8192 x 14336 fp32 -> chunks of 6144 and 2048 rows): the
    rows on both sides of the chunk boundary and the last rows against the
    float64 oracle, forward and input gradient."""

    from qste_amd import kernels

    lib = kernels._lib.load()
    m, k, n = 8192, 14336, 256
    # the workspace holds one chunk's limbs, not the whole operand's
    assert 0 < lib.qste_packed_linear_affine_workspace_bytes(m, n, k, 0) < m * k * 6
    assert 0 < lib.qste_packed_transpose_workspace_bytes(m, k, n, 0) < m * k * 6
    g = torch.Generator(device=DEV).manual_seed(13)
    x = torch.randn(m, k, generator=g, device=DEV)
    coord = torch.randint(-127, 128, (n, k), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    packed = kernels.pack_coordinate(coord)
    scale = torch.rand(n, generator=g, device=DEV) * 0.02 + 0.005
    bias = torch.randn(n, generator=g, device=DEV) * 0.1
    sel = np.r_[0:8, 6140:6150, m - 8:m]
    y = kernels.packed_linear_affine(x, packed, scale, bias, k)
    torch.cuda.synchronize()
    xs = x[torch.from_numpy(sel).to(DEV)].cpu().numpy()
    pk, sc = packed.cpu().numpy(), scale.cpu().numpy()
    want = oracle.linear_fwd_f64(xs, pk, sc, bias.cpu().numpy(), k)
    assert _rel(y[torch.from_numpy(sel).to(DEV)].cpu().numpy(), want) <= 2e-6
    del y

    # input gradient: dy [m, k] against signs [k, n] (K = k rows of signs)
    coord_t = torch.randint(-127, 128, (k, n), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    packed_t = kernels.pack_coordinate(coord_t)
    row_scale = torch.rand(k, generator=g, device=DEV) * 0.02 + 0.005
    dx = kernels.packed_transpose(x, packed_t, n, row_scale=row_scale)
    torch.cuda.synchronize()
    want = oracle.linear_dgrad_f64(xs, packed_t.cpu().numpy(), n, row_scale.cpu().numpy())
    assert _rel(dx[torch.from_numpy(sel).to(DEV)].cpu().numpy(), want) <= 2e-6
