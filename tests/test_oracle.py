"""The CPU oracle against the reference's golden vectors and the mathematics.

The oracle (``oracle/``) is the checker every HIP kernel is compared with, so
it is pinned here first: against vectors the reference's own specification
backend wrote (``tests/golden/make_golden.py``), and against closed forms and
brute force that a plausible slip (a dropped term, a swapped index, a wrong
rounding) would fail.

Integer outputs of the coordinate step depend on fp32 reductions whose order
the reference leaves to torch (``tests/test_gpu.py:440-455`` in the reference
explains why its own backends are not bit-identical). The comparison is exact
everywhere except inside a declared band: elements whose rounding decision
sits within ``TARGET_BAND`` (stochastic rounding) or ``MOMENT_BAND``
(momentum requantization) of its threshold, and the momentum of a block whose
fp32 scale sits within ``SCALE_BAND`` of an fp16 rounding tie (the stored
scale may then be its neighbour, and every q of the block moves with it).
Every mismatch must lie inside the band, and the band itself must stay a tiny
fraction of the matrix.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle

TARGET_BAND = 2.0 ** -16   # |target - floor(target) - u|
MOMENT_BAND = 2.0 ** -14  # | |m/S| - floor(|m/S|) - 1/2 |
# fp16 ulps between a block's fp32 scale amax / 127 and the fp16 rounding
# midpoint: one fp32 ulp is 2^-13 fp16 ulp, so this is three fp32 ulps
SCALE_BAND = 2.0 ** -11
STATE_KEYS = ("coordinate", "packed", "moment_q", "moment_scale", "row_v", "col_v")


# ---------------------------------------------------------------------------
# hash (stream.py:41-83)
# ---------------------------------------------------------------------------


def test_scramble_matches_reference_vectors(golden):
    g = golden("hash")
    got = oracle.scramble(g["values"])
    assert np.array_equal(got.astype(np.uint64), g["scrambled"])


def test_seed_and_step_hash_match_reference_vectors(golden):
    g = golden("hash")
    for seed, want in zip(g["seeds"], g["seed_hash"]):
        assert oracle.seed_hash(int(seed)) == int(want)
    for step, want in zip(g["steps"], g["step_hash"]):
        assert oracle.step_hash(int(step)) == int(want)


def test_uniform_draw_matches_reference_vectors(golden):
    g = golden("hash")
    for a, seed in enumerate(g["seeds"]):
        for b, step in enumerate(g["steps"]):
            got = oracle.uniform(int(seed), int(step), g["indices"].astype(np.int64))
            assert np.array_equal(got, g["uniform"][a, b]), (seed, step)


def test_scramble_is_the_published_wang_avalanche():
    """Thomas Wang's 32-bit integer hash, evaluated in Python integers.

    Catches a dropped step or a signed shift in the C spelling; the golden
    vectors above catch a wrong constant.
    """

    def wang(v):
        v &= 0xFFFFFFFF
        v = ((v ^ 61) ^ (v >> 16)) & 0xFFFFFFFF
        v = (v + (v << 3)) & 0xFFFFFFFF
        v = (v ^ (v >> 4)) & 0xFFFFFFFF
        v = (v * 0x27D4EB2D) & 0xFFFFFFFF
        return (v ^ (v >> 15)) & 0xFFFFFFFF

    values = np.random.default_rng(3).integers(0, 2**32, size=2000, dtype=np.uint64)
    assert [wang(int(v)) for v in values] == [int(x) for x in oracle.scramble(values)]


def test_stream_is_uniform_and_step_decorrelated():
    """Properties of the reference's tests/test_kernels.py:250-279."""

    draws = oracle.uniform(3, 11, np.arange(20000))
    assert 0.0 <= draws.min() and draws.max() < 1.0
    assert abs(draws.mean() - 0.5) < 0.01
    hist = np.histogram(draws, bins=10, range=(0.0, 1.0))[0] / draws.size
    assert np.all(np.abs(hist - 0.1) < 0.015)
    first = oracle.uniform(5, 100, np.arange(512))
    second = oracle.uniform(5, 101, np.arange(512))
    assert int((first == second).sum()) < 8


def test_index_enters_modulo_two_to_the_32():
    idx = np.array([5, 5 + 2**32, 5 + 2**33], dtype=np.int64)
    u = oracle.uniform(1, 2, idx)
    assert u[0] == u[1] == u[2]


# ---------------------------------------------------------------------------
# packing (fallback.py:27-92)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("cols", [1, 7, 8, 9, 63, 64, 65, 130])
def test_pack_coordinate_brute_force_and_round_trip(cols):
    rng = np.random.default_rng(cols)
    coord = rng.integers(-127, 128, size=(5, cols)).astype(np.int8)
    coord[0, 0] = 0  # zero decodes to +1
    packed = oracle.pack_coordinate(coord)
    assert packed.shape == (5, (cols + 7) // 8)
    for r in range(5):
        for c in range(cols):
            bit = (packed[r, c // 8] >> (c % 8)) & 1
            assert bit == (1 if coord[r, c] >= 0 else 0)
        # pad bits are zero
        for c in range(cols, packed.shape[1] * 8):
            assert (packed[r, c // 8] >> (c % 8)) & 1 == 0
    signs = oracle.unpack_rows(packed, cols)
    assert np.array_equal(signs, np.where(coord >= 0, 1.0, -1.0).astype(np.float32))


def test_pack_affine_matches_reference_vectors(golden):
    g = golden("pack_affine")
    names = sorted({k.split("__")[0] for k in g})
    assert names
    for name in names:
        x = g[f"{name}__x"]
        bits, off, xs = oracle.pack_affine_rows(x)
        np.testing.assert_allclose(off, g[f"{name}__offset"], rtol=1e-6, atol=1e-7)
        np.testing.assert_allclose(xs, g[f"{name}__scale"], rtol=1e-6, atol=1e-7)
        ours = oracle.unpack_rows(bits, x.shape[1])
        theirs = oracle.unpack_rows(g[f"{name}__bits"], x.shape[1])
        differ = ours != theirs
        # A bit may only differ where x sits within a few ulp of the mean.
        near = np.abs(x - off[:, None]) <= 4 * np.spacing(np.abs(off[:, None]).astype(np.float32))
        assert not np.any(differ & ~near), name
        assert int(differ.sum()) == 0, (name, int(differ.sum()))


def test_pack_affine_closed_form():
    """x ~ offset + scale * sign, offset = mean, scale = mean |x - offset|."""

    rng = np.random.default_rng(9)
    x = rng.standard_normal((7, 300)).astype(np.float32) * 3 + 1
    bits, off, xs = oracle.pack_affine_rows(x)
    np.testing.assert_allclose(off, x.astype(np.float64).mean(1), rtol=1e-6)
    np.testing.assert_allclose(xs, np.abs(x - off[:, None]).astype(np.float64).mean(1), rtol=1e-6)
    sign = oracle.unpack_rows(bits, 300)
    assert np.array_equal(sign, np.where(x - off[:, None] >= 0, 1.0, -1.0))
    # relu output: centering keeps the encoding informative (reference
    # tests/test_kernels.py:50-59)
    relu = np.maximum(rng.standard_normal((16, 64)), 0).astype(np.float32)
    frac = (oracle.unpack_rows(oracle.pack_affine_rows(relu)[0], 64) > 0).mean()
    assert 0.1 < frac < 0.9


# ---------------------------------------------------------------------------
# dense products (fallback.py:95-148) and the offset correction
# ---------------------------------------------------------------------------


def test_products_match_reference_vectors(golden):
    g = golden("products")
    names = sorted({k.split("__")[0] for k in g})
    for key in names:
        rows, cols, samples = (int(v) for v in g[f"{key}__shape"])
        packed = g[f"{key}__packed"]
        lin = oracle.linear_fwd(g[f"{key}__x"], packed, g[f"{key}__scale"], g[f"{key}__bias"], cols)
        np.testing.assert_allclose(lin, g[f"{key}__linear"], atol=1e-4, rtol=1e-5)
        tr = oracle.linear_dgrad(g[f"{key}__dy"], packed, cols, g[f"{key}__scale"])
        np.testing.assert_allclose(tr, g[f"{key}__transpose"], atol=1e-4, rtol=1e-5)
        ev = oracle.evidence(g[f"{key}__dy"], g[f"{key}__xbits"], cols, g[f"{key}__xscale"])
        np.testing.assert_allclose(ev, g[f"{key}__evidence"], atol=1e-4, rtol=1e-5)
        ri = oracle.row_inner(g[f"{key}__mat"], packed, cols)
        np.testing.assert_allclose(ri, g[f"{key}__row_inner"], atol=1e-4, rtol=1e-5)


@pytest.mark.parametrize("rows,cols,samples", [(17, 13, 5), (64, 64, 32), (33, 8, 7), (40, 96, 12)])
def test_products_equal_dense_float64_algebra(rows, cols, samples):
    rng = np.random.default_rng(rows * 1000 + cols)
    coord = rng.integers(-127, 128, size=(rows, cols)).astype(np.int8)
    packed = oracle.pack_coordinate(coord)
    sign = np.where(coord >= 0, 1.0, -1.0)  # from the coordinate, not the bits
    x = rng.standard_normal((samples, cols)).astype(np.float32)
    scale = (rng.random(rows) + 0.5).astype(np.float32)
    bias = rng.standard_normal(rows).astype(np.float32)
    dy = rng.standard_normal((samples, rows)).astype(np.float32)
    xd, dyd = x.astype(np.float64), dy.astype(np.float64)

    y = oracle.linear_fwd(x, packed, scale, bias, cols)
    np.testing.assert_allclose(y, (xd @ sign.T) * scale + bias, rtol=1e-12, atol=1e-12)
    y0 = oracle.linear_fwd(x, packed, scale, None, cols)
    np.testing.assert_allclose(y0, (xd @ sign.T) * scale, rtol=1e-12, atol=1e-12)

    dx = oracle.linear_dgrad(dy, packed, cols, scale)
    np.testing.assert_allclose(dx, (dyd * scale) @ sign, rtol=1e-12, atol=1e-12)
    dx1 = oracle.linear_dgrad(dy, packed, cols)
    np.testing.assert_allclose(dx1, dyd @ sign, rtol=1e-12, atol=1e-12)

    xbits, off, xs = oracle.pack_affine_rows(x)
    xsign = np.where(x - off[:, None] >= 0, 1.0, -1.0)
    ev = oracle.evidence(dy, xbits, cols, xs)
    np.testing.assert_allclose(ev, (dyd * xs[:, None]).T @ xsign, rtol=1e-12, atol=1e-12)
    # the decoded evidence is exactly dy^T @ x_hat with x_hat = off + xs*sign
    # (functional.py:118-145), so the offset correction is a rank-one term
    x_hat = off[:, None].astype(np.float64) + xs[:, None] * xsign
    dec = oracle.decoded_evidence(dy, xbits, off, xs, cols)
    np.testing.assert_allclose(dec, dyd.T @ x_hat, rtol=1e-10, atol=1e-10)

    mat = rng.standard_normal((rows, cols)).astype(np.float32)
    np.testing.assert_allclose(oracle.row_inner(mat, packed, cols), (mat * sign).sum(1), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# coordinate step (fallback.py:158-242)
# ---------------------------------------------------------------------------


def _golden_inputs(g, name, key):
    """A golden step's input state; a second phase stored without inputs
    starts from the first phase's (reference-written) outputs."""

    if f"{name}__in_{key}" in g:
        return g[f"{name}__in_{key}"]
    return g[f"{name[:-1]}{int(name[-1]) - 1}__out_{key}"]


def _golden_step(g, name):
    p = g[f"{name}__params"]
    state = {k: np.ascontiguousarray(_golden_inputs(g, name, k)).copy() for k in STATE_KEYS}
    kwargs = dict(beta1=p[0], beta2=p[1], update_clip=p[2], coordinate_lr=p[3],
                  block_size=int(p[4]), seed=int(p[5]), step=int(p[6]))
    return state, kwargs


def _check_golden_steps(g, names):
    """Every golden step: exact outside the declared band.  Prints, per step,
    how many elements differ from the reference (coordinates, int8 momentum,
    fp16 statistics) and how many sit inside the band at all."""

    total = banded = 0
    for name in names:
        state, kwargs = _golden_step(g, name)
        sm = np.empty(state["moment_scale"].size, np.float32)
        flips, tm, mm = oracle.coordinate_update(g[f"{name}__evidence"], state, margins=True,
                                                 scale_margin=sm, **kwargs)
        want = {k: g[f"{name}__out_{k}"] for k in STATE_KEYS}
        in_t = tm < TARGET_BAND
        # a block whose fp16 scale sits on a rounding tie may store the
        # neighbouring scale; every q of that block then moves with it
        scale_tie = sm < SCALE_BAND
        in_q = (mm < MOMENT_BAND) | np.repeat(scale_tie, kwargs["block_size"])[:mm.size].reshape(mm.shape)
        bad_c = state["coordinate"] != want["coordinate"]
        bad_q = state["moment_q"] != want["moment_q"]
        bad_s = state["moment_scale"].view(np.uint16) != want["moment_scale"].view(np.uint16)
        assert not np.any(bad_s & ~scale_tie), (name, "block scale mismatch off a rounding tie")
        fp16_bad = {key: int((state[key].view(np.uint16) != want[key].view(np.uint16)).sum())
                    for key in ("row_v", "col_v", "moment_scale")}
        print(f"golden {name}: {state['coordinate'].size} elements; differing from the reference: "
              f"coordinate {int(bad_c.sum())}, moment_q {int(bad_q.sum())}, "
              + ", ".join(f"{k} {v}" for k, v in fp16_bad.items())
              + f"; inside the band: {int(in_t.sum())} rounding, {int((mm < MOMENT_BAND).sum())} "
              f"requantization, {int(scale_tie.sum())} block scales on a tie")
        assert not np.any(bad_c & ~in_t), (name, "coordinate mismatch outside band")
        assert not np.any(bad_q & ~in_q), (name, "momentum mismatch outside band")
        assert np.abs(state["coordinate"].astype(int) - want["coordinate"]).max() <= 1
        assert np.abs(state["moment_q"].astype(int) - want["moment_q"]).max() <= 1
        if not bad_c.any():
            assert np.array_equal(state["packed"], want["packed"]), name
            assert flips == int(g[f"{name}__flips"]), name
        # fp16 statistics: equal up to one fp16 ulp (reduction order)
        for key in ("row_v", "col_v", "moment_scale"):
            diff = np.abs(state[key].view(np.uint16).astype(int) - want[key].view(np.uint16).astype(int))
            assert diff.max() <= 1, (name, key)
        total += state["coordinate"].size
        banded += int(in_t.sum() + in_q.sum())
    # the band is a sliver of the matrix, not a loophole
    assert banded < 1e-3 * total * 2, (banded, total)


def test_coordinate_update_matches_reference_vectors(golden):
    g = golden("coordinate_update")
    names = sorted({k.split("__")[0] for k in g})
    assert len(names) >= 10
    _check_golden_steps(g, names)


def test_coordinate_update_matches_reference_1024(golden):
    """A 1024 x 1024 surface (block 256), a fresh step and the next one, each
    from the reference's own state: reductions of realistic length."""

    g = golden("coordinate_update_1024")
    _check_golden_steps(g, ["u1024x1024_p0", "u1024x1024_p1"])


def _random_case(rows, cols, block, seed):
    rng = np.random.default_rng(seed)
    coord = rng.integers(-127, 128, size=(rows, cols)).astype(np.int8)
    return oracle.fresh_state(coord, block), rng.standard_normal((rows, cols)).astype(np.float32)


def test_coordinate_update_invariants():
    state, ev = _random_case(37, 45, 64, 5)
    common = dict(beta1=0.9, beta2=0.99, update_clip=2.0, coordinate_lr=4.0, block_size=64)
    before = state["packed"].copy()
    flips = oracle.coordinate_update(ev, state, seed=3, step=0, **common)
    assert np.array_equal(state["packed"], oracle.pack_coordinate(state["coordinate"]))
    assert np.abs(state["coordinate"].astype(int)).max() <= 127
    assert np.abs(state["moment_q"].astype(int)).max() <= 127
    diff = np.unpackbits(before ^ state["packed"], axis=1, bitorder="little")[:, :45]
    assert flips == int(diff.sum())
    # reproducible from (seed, step) alone
    s2, _ = _random_case(37, 45, 64, 5)
    oracle.coordinate_update(ev, s2, seed=3, step=0, **common)
    for k in STATE_KEYS:
        assert np.array_equal(state[k].view(np.uint8), s2[k].view(np.uint8))
    # a different step draws a different stream
    s3, _ = _random_case(37, 45, 64, 5)
    oracle.coordinate_update(ev, s3, seed=3, step=1, **common)
    assert not np.array_equal(state["coordinate"], s3["coordinate"])


def test_first_step_statistics_closed_form():
    """From zero state: r = (1-b2) * mean(g^2 + 1e-12), stored in fp16."""

    state, ev = _random_case(16, 24, 64, 8)
    oracle.coordinate_update(ev, state, beta1=0.9, beta2=0.99, update_clip=2.0,
                             coordinate_lr=1.0, block_size=64, seed=1, step=0)
    g64 = ev.astype(np.float64)
    row = 0.01 * (g64 ** 2 + 1e-12).mean(1)
    col = 0.01 * (g64 ** 2 + 1e-12).mean(0)
    np.testing.assert_allclose(state["row_v"].astype(np.float64), row, rtol=1e-3)
    np.testing.assert_allclose(state["col_v"].astype(np.float64), col, rtol=1e-3)
    # the new block scale is fp16(max|m| / 127) and the momentum decodes to m
    # within half a quantization step
    m_scale = state["moment_scale"].astype(np.float64)
    assert np.all(m_scale > 0)


def test_zero_learning_rate_limit_keeps_coordinates():
    """A tiny step moves a coordinate only if the draw lands below the fraction."""

    state, ev = _random_case(8, 64, 64, 11)
    before = state["coordinate"].copy()
    oracle.coordinate_update(ev, state, beta1=0.9, beta2=0.99, update_clip=2.0,
                             coordinate_lr=1e-6, block_size=64, seed=1, step=0)
    assert np.abs(state["coordinate"].astype(int) - before).max() <= 1
    assert (state["coordinate"] != before).mean() < 0.01


def test_planted_mistake_is_caught(golden):
    """A step with beta2 nudged by one fp32 ulp must fail the golden check.

    Guards the golden comparison itself against being vacuous.
    """

    g = golden("coordinate_update")
    name = "u256x512_p0"
    state, kwargs = _golden_step(g, name)
    kwargs["beta1"] = float(np.nextafter(np.float32(0.9), np.float32(1.0)))
    oracle.coordinate_update(g[f"{name}__evidence"], state, **kwargs)
    assert not np.array_equal(state["moment_q"], g[f"{name}__out_moment_q"])


def test_step_size_is_torchs_reciprocal_times_lr():
    """fallback.py:204-206 writes the step size as ``coordinate_lr / moment_rms``
    with a Python float over a 0-dim fp32 tensor.  Torch evaluates that through
    ``Tensor.__rtruediv__`` as ``reciprocal() * lr``: two roundings.  The
    oracle must equal torch's own evaluation bit for bit over learning rates
    that are and are not powers of two, and one fp32 division (the obvious
    spelling) must fail the same comparison, so the check discriminates."""

    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(2024)
    lrs = [0.3, 0.7, 0.1, 1.0, 2.0, 4.0, 0.25, 1e-3, 3.0, 0.05]
    lrs += [float(v) for v in rng.uniform(1e-4, 8.0, size=40)]
    rms = np.exp(rng.uniform(np.log(1e-8), np.log(1e3), size=30)).astype(np.float32)
    rms = np.concatenate([rms, np.float32([1e-8, 1.0, 0.5, 3.0, 127.0])])
    pairs = diff_one_division = 0
    for lr in lrs:
        for r in rms:
            want = (lr / torch.tensor(float(r), dtype=torch.float32)).item()
            got = oracle.step_size(r, lr)
            assert np.float32(want).view(np.uint32) == got.view(np.uint32), (lr, float(r))
            one = np.float32(np.float32(lr) / r)
            diff_one_division += int(one != got)
            pairs += 1
    assert pairs >= 1000
    # the single division disagrees often enough for this test to notice it
    assert diff_one_division > 0.05 * pairs, diff_one_division


def test_step_size_reaches_the_coordinate_step(golden):
    """The step reports the step size it used; it is ``step_size(rms(m), lr)``."""

    g = golden("coordinate_update")
    for name in sorted({k.split("__")[0] for k in g}):
        state, kwargs = _golden_step(g, name)
        scalars = np.zeros(4, dtype=np.float32)
        oracle.coordinate_update(g[f"{name}__evidence"], state, scalars=scalars, **kwargs)
        assert scalars[2] == oracle.step_size(scalars[3], kwargs["coordinate_lr"]), name
        assert scalars[1] >= 1.0 and scalars[3] >= np.float32(1e-8), name


def test_blas_products_equal_the_c_restatement():
    """The float64 BLAS products used for full-size samples against the C
    restatement (itself pinned to the reference-written product vectors)."""

    rng = np.random.default_rng(12)
    rows, cols, m = 70, 203, 33
    packed = rng.integers(0, 256, size=(rows, (cols + 7) // 8), dtype=np.uint8)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    dy = rng.standard_normal((m, rows)).astype(np.float32)
    scale = (rng.random(rows) + 0.5).astype(np.float32)
    bias = rng.standard_normal(rows).astype(np.float32)
    xs = (rng.random(m) + 0.1).astype(np.float32)
    xbits = rng.integers(0, 256, size=(m, (cols + 7) // 8), dtype=np.uint8)
    tol = dict(rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.linear_fwd_f64(x, packed, scale, bias, cols),
                               oracle.linear_fwd(x, packed, scale, bias, cols), **tol)
    np.testing.assert_allclose(oracle.linear_dgrad_f64(dy, packed, cols, scale),
                               oracle.linear_dgrad(dy, packed, cols, scale), **tol)
    np.testing.assert_allclose(oracle.evidence_f64(dy, xbits, cols, xs),
                               oracle.evidence(dy, xbits, cols, xs), **tol)
    np.testing.assert_array_equal(oracle.signs_f64(packed, cols), oracle.unpack_rows(packed, cols))
