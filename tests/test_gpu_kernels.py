"""HIP kernels against the CPU oracle, on the GPU, through the C ABI.

Bars (stated per test):
* integer and byte outputs -- packed signs, activation bits, coordinates,
  momentum, fp16 statistics, flip counts -- bit-exact against the oracle run
  on the same inputs;
* float outputs within a relative L2 error against the float64 oracle whose
  operands are rounded exactly as the kernel's contract says (a scale folded
  into a bf16 operand is rounded to bf16 first; a bf16 output is the oracle
  rounded to bf16).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


@pytest.fixture(autouse=True)
def _gpu():
    _need_gpu()
    from qste_amd import kernels

    assert kernels.native_available(), kernels.status()
    yield


def K():
    from qste_amd import kernels

    return kernels


def rel_l2(got, want) -> float:
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    denom = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / (denom if denom > 0 else 1.0))


def t(a, dtype=None):
    x = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return x if dtype is None else x.to(dtype)


def f32(x: torch.Tensor) -> np.ndarray:
    return x.float().cpu().numpy()


DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def as_dtype_values(a: np.ndarray, dt: str) -> np.ndarray:
    """fp32 values exactly representable in dtype ``dt`` (round once)."""

    return torch.from_numpy(a).to(DT[dt]).float().numpy()


def round_out(a: np.ndarray, dt: str) -> np.ndarray:
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(DT[dt]).float().numpy()


def round_scale(s: np.ndarray, dt: str) -> np.ndarray:
    return s if dt == "f32" else as_dtype_values(s.astype(np.float32), dt)


# ---------------------------------------------------------------------------
# packing
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 7), (3, 8), (17, 13), (64, 64), (33, 130),
                                       (128, 4096), (7, 1000)])
def test_pack_coordinate_bit_exact(rows, cols):
    rng = np.random.default_rng(rows * 7919 + cols)
    coord = rng.integers(-127, 128, size=(rows, cols)).astype(np.int8)
    coord.flat[:: max(1, coord.size // 5)] = 0
    got = K().pack_coordinate(t(coord)).cpu().numpy()
    assert np.array_equal(got, oracle.pack_coordinate(coord))


@pytest.mark.parametrize("cols", [1, 7, 8, 9, 63, 64, 65])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_unpack_rows_exact(cols, dt):
    rng = np.random.default_rng(cols)
    coord = rng.integers(-127, 128, size=(5, cols)).astype(np.int8)
    packed = oracle.pack_coordinate(coord)
    got = f32(K().unpack_rows(t(packed), cols, dtype=DT[dt]))
    assert np.array_equal(got, oracle.unpack_rows(packed, cols))


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,cols", [(9, 7), (17, 64), (16, 1024), (8, 4096), (4, 4104), (5, 1001), (3, 14336),
                                       (2, 16384), (2, 16392)])
def test_pack_affine_rows_bit_exact(dt, rows, cols):
    rng = np.random.default_rng(rows * 31 + cols)
    x = as_dtype_values((rng.standard_normal((rows, cols)) * 2 + 0.3).astype(np.float32), dt)
    bits, off, xs = K().pack_affine_rows(t(x, DT[dt]))
    ob, oo, ox = oracle.pack_affine_rows(x)
    assert np.array_equal(bits.cpu().numpy(), ob)
    assert np.array_equal(off.cpu().numpy(), oo)
    assert np.array_equal(xs.cpu().numpy(), ox)


def test_pack_affine_rows_against_reference_vectors(golden):
    g = golden("pack_affine")
    for name in sorted({k.split("__")[0] for k in g}):
        x = g[f"{name}__x"]
        bits, off, xs = K().pack_affine_rows(t(x))
        assert np.array_equal(bits.cpu().numpy(), g[f"{name}__bits"]), name
        np.testing.assert_allclose(off.cpu().numpy(), g[f"{name}__offset"], rtol=1e-6, atol=1e-7)
        np.testing.assert_allclose(xs.cpu().numpy(), g[f"{name}__scale"], rtol=1e-6, atol=1e-7)


# ---------------------------------------------------------------------------
# products
# ---------------------------------------------------------------------------

SHAPES = [(17, 13, 5), (64, 64, 32), (128, 96, 40), (33, 8, 7), (1, 1, 1), (300, 256, 129),
          (512, 1024, 256), (1024, 512, 16), (256, 4096, 4), (64, 2048, 1)]


def _problem(rows, cols, m, dt, seed):
    rng = np.random.default_rng(seed)
    coord = rng.integers(-127, 128, size=(rows, cols)).astype(np.int8)
    packed = oracle.pack_coordinate(coord)
    x = as_dtype_values(rng.standard_normal((m, cols)).astype(np.float32), dt)
    scale = (np.abs(rng.standard_normal(rows)) * 0.02 + 0.01).astype(np.float32)
    bias = rng.standard_normal(rows).astype(np.float32) * 0.1
    dy = as_dtype_values(rng.standard_normal((m, rows)).astype(np.float32), dt)
    return packed, x, scale, bias, dy


@pytest.mark.parametrize("rows,cols,m", SHAPES)
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_linear_forward(rows, cols, m, dt):
    packed, x, scale, bias, _ = _problem(rows, cols, m, dt, rows + cols + m)
    got = f32(K().packed_linear_affine(t(x, DT[dt]), t(packed), t(scale), t(bias), cols))
    want = oracle.linear_fwd(x, packed, scale, bias, cols)
    if dt == "f32":
        assert rel_l2(got, want) <= 1e-5
    else:
        want_r = round_out(want, dt)
        assert rel_l2(got, want_r) <= 1e-3
        # all but a sliver of elements equal the rounded oracle
        assert np.mean(got != want_r) < 0.01
    nob = f32(K().packed_linear_affine(t(x, DT[dt]), t(packed), t(scale), None, cols))
    want0 = oracle.linear_fwd(x, packed, scale, None, cols)
    assert rel_l2(nob, want0 if dt == "f32" else round_out(want0, dt)) <= (1e-5 if dt == "f32" else 1e-3)


@pytest.mark.parametrize("rows,cols,m", SHAPES)
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_linear_dgrad(rows, cols, m, dt):
    packed, _, scale, _, dy = _problem(rows, cols, m, dt, 3 * rows + cols + m)
    got = f32(K().packed_transpose(t(dy, DT[dt]), t(packed), cols, row_scale=t(scale)))
    want = oracle.linear_dgrad(dy, packed, cols, round_scale(scale, dt))
    if dt == "f32":
        assert rel_l2(got, want) <= 1e-5
    else:
        assert rel_l2(got, round_out(want, dt)) <= 1e-3
    plain = f32(K().packed_transpose(t(dy, DT[dt]), t(packed), cols))
    want1 = oracle.linear_dgrad(dy, packed, cols)
    assert rel_l2(plain, want1 if dt == "f32" else round_out(want1, dt)) <= (1e-5 if dt == "f32" else 1e-3)


@pytest.mark.parametrize("rows,cols,m", SHAPES)
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_evidence(rows, cols, m, dt):
    packed_w, x, scale, _, dy = _problem(rows, cols, m, dt, 5 * rows + cols + m)
    xbits, off, xs = oracle.pack_affine_rows(x)
    got = K().evidence_from_packed(t(dy, DT[dt]), t(xbits), cols, row_scale=t(xs)).cpu().numpy()
    want = oracle.evidence(dy, xbits, cols, round_scale(xs, dt))
    assert rel_l2(got, want) <= 1e-5


@pytest.mark.parametrize("rows,cols", [(17, 13), (64, 64), (300, 1000), (1024, 4096)])
def test_row_inner(rows, cols):
    rng = np.random.default_rng(rows)
    coord = rng.integers(-127, 128, size=(rows, cols)).astype(np.int8)
    packed = oracle.pack_coordinate(coord)
    mat = rng.standard_normal((rows, cols)).astype(np.float32)
    got = K().packed_row_inner(t(mat), t(packed), cols).cpu().numpy()
    assert rel_l2(got, oracle.row_inner(mat, packed, cols)) <= 1e-5


@pytest.mark.parametrize("rows,cols,m", [(17, 13, 5), (64, 64, 32), (300, 256, 129), (512, 1024, 256),
                                         (1024, 512, 64), (96, 4096, 1)])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("with_bias", [True, False])
def test_fused_linear_backward(rows, cols, m, dt, with_bias):
    packed_w, x, scale, _, dy = _problem(rows, cols, m, dt, 7 * rows + cols + m)
    xbits, off, xs = oracle.pack_affine_rows(x)
    dx, ev, gs, db = K().linear_backward(
        t(dy, DT[dt]), t(xbits), t(off), t(xs), t(packed_w), t(scale), cols, need_bias=with_bias)
    want_dx = oracle.linear_dgrad(dy, packed_w, cols, round_scale(scale, dt))
    e0 = oracle.evidence(dy, xbits, cols, round_scale(xs, dt)) + oracle.offset_correction(dy, off)[:, None]
    want_gs = oracle.row_inner(e0.astype(np.float32), packed_w, cols)
    if dt == "f32":
        assert rel_l2(f32(dx), want_dx) <= 1e-5
    else:
        assert rel_l2(f32(dx), round_out(want_dx, dt)) <= 1e-3
    assert rel_l2(ev.cpu().numpy(), e0 * scale[:, None]) <= 1e-5
    assert rel_l2(gs.cpu().numpy(), want_gs) <= 1e-4
    if with_bias:
        assert rel_l2(db.cpu().numpy(), dy.astype(np.float64).sum(0)) <= 1e-5
    else:
        assert db is None


# ---------------------------------------------------------------------------
# coordinate step
# ---------------------------------------------------------------------------

KEYS = ("coordinate", "packed", "moment_q", "moment_scale", "row_v", "col_v")


def _to_gpu_state(state):
    return {k: t(v.copy()) for k, v in state.items()}


def _gpu_step(ev, gstate, **kw):
    return K().coordinate_update(
        t(ev), gstate["coordinate"], gstate["packed"], gstate["moment_q"], gstate["moment_scale"],
        gstate["row_v"], gstate["col_v"], **kw)


def _assert_state_equal(gstate, state, tag):
    for k in KEYS:
        got = gstate[k].cpu().numpy()
        want = state[k]
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), (tag, k, int((got != want).sum()))


@pytest.mark.parametrize("file", ["coordinate_update", "coordinate_update_1024"])
def test_coordinate_update_reference_vectors(golden, file):
    """GPU vs the reference's own outputs: bit for bit against the oracle on
    the same inputs, and exact against the reference outside the rounding
    band (a stochastic-rounding decision within 2^-16 of its threshold, a
    requantization within 2^-14 of a tie, or a block whose fp32 scale lies
    within three fp32 ulps of an fp16 rounding tie).  The 1024 x 1024 file
    holds a fresh step and the next one; the second starts from the first's
    reference outputs."""

    g = golden(file)
    for name in sorted({k.split("__")[0] for k in g}):
        p = g[f"{name}__params"]
        kw = dict(beta1=p[0], beta2=p[1], update_clip=p[2], coordinate_lr=p[3],
                  block_size=int(p[4]), seed=int(p[5]), step=int(p[6]))
        src = name if f"{name}__in_coordinate" in g else f"{name[:-1]}{int(name[-1]) - 1}"
        tag = "__in_" if src == name else "__out_"
        state = {k: np.ascontiguousarray(g[f"{src}{tag}{k}"]) for k in KEYS}
        print(f"golden {file}/{name} {state['coordinate'].shape}", flush=True)
        gstate = _to_gpu_state(state)
        flips = _gpu_step(g[f"{name}__evidence"], gstate, **kw)
        # the oracle on the same inputs: GPU must equal it bit for bit
        ostate = {k: v.copy() for k, v in state.items()}
        sm = np.empty(state["moment_scale"].size, np.float32)
        oflips, tm, mm = oracle.coordinate_update(g[f"{name}__evidence"], ostate, margins=True,
                                                  scale_margin=sm, **kw)
        _assert_state_equal(gstate, ostate, name)
        assert flips == oflips, name
        # and the reference's outputs, up to the declared band
        bad = gstate["coordinate"].cpu().numpy() != g[f"{name}__out_coordinate"]
        assert not np.any(bad & (tm >= 2.0 ** -16)), name
        tie = np.repeat(sm < 2.0 ** -11, kw["block_size"])[:mm.size].reshape(mm.shape)
        bad_q = gstate["moment_q"].cpu().numpy() != g[f"{name}__out_moment_q"]
        assert not np.any(bad_q & (mm >= 2.0 ** -14) & ~tie), name


# Shapes with cols % 256 == 0 and block <= 256 take the row kernels (a wave
# per 1024-column chunk, momentum blocks as lane groups): every block size
# 8..256, a last chunk of 1, 2 or 3 slots, fewer rows than waves, and one
# chunk for a whole row (the row sums finish in the stats pass).  The rest
# take the generic kernels.
ROW_PATH = [(64, 1280, 8), (33, 2304, 16), (130, 512, 32), (3, 256, 64), (200, 3072, 128), (70, 1792, 256),
            (64, 1024, 512)]


@pytest.mark.parametrize("rows,cols,block", [(16, 32, 64), (37, 45, 64), (256, 1024, 256), (1024, 384, 256),
                                             (200, 200, 128), (3, 5000, 256), (512, 4096, 256)] + ROW_PATH)
def test_coordinate_update_matches_oracle(rows, cols, block):
    rng = np.random.default_rng(rows * cols)
    coord = rng.integers(-127, 128, size=(rows, cols)).astype(np.int8)
    state = oracle.fresh_state(coord, block)
    gstate = _to_gpu_state(state)
    for step in range(3):
        ev = (rng.standard_normal((rows, cols)) * (0.01 * (step + 1))).astype(np.float32)
        kw = dict(beta1=0.9, beta2=0.99, update_clip=2.0, coordinate_lr=1.0, block_size=block,
                  seed=1 + 1_000_003 * 2, step=step)
        flips = _gpu_step(ev, gstate, **kw)
        oflips = oracle.coordinate_update(ev, state, **kw)
        _assert_state_equal(gstate, state, (rows, cols, step))
        assert flips == oflips


# the one-launch step: strips whose rows sit in registers, in LDS and in
# memory; every power-of-two block size; strips of unequal height; fresh
# steps, speculative steps with the clip idle and with it engaged (the guess
# thrown away)
ONE_LAUNCH = [(64, 2048, 256), (512, 4096, 8), (3000, 2048, 16), (1111, 4096, 32), (700, 6144, 64),
              (9000, 4096, 128), (4096, 14336, 256)]


@pytest.mark.parametrize("rows,cols,block", ONE_LAUNCH)
def test_coordinate_update_one_launch_matches_oracle(rows, cols, block):
    from qste_amd.kernels import _lib

    assert _lib.load().qste_coordinate_update_one_launch(rows, cols, block) == 1
    print(f"one launch {rows}x{cols} block {block}", flush=True)
    rng = np.random.default_rng(rows + cols + block)
    coord = rng.integers(-127, 128, size=(rows, cols)).astype(np.int8)
    state = oracle.fresh_state(coord, block)
    gstate = _to_gpu_state(state)
    for step, clip in ((0, 2.0), (1, 2.0), (64, 1e6), (65, 0.05)):
        ev = (rng.standard_normal((rows, cols)) * 0.1).astype(np.float32)
        kw = dict(beta1=0.9, beta2=0.99, update_clip=clip, coordinate_lr=0.7, block_size=block, seed=3, step=step)
        flips = _gpu_step(ev, gstate, **kw)
        oflips = oracle.coordinate_update(ev, state, **kw)
        _assert_state_equal(gstate, state, (rows, cols, block, step))
        assert flips == oflips


@pytest.mark.parametrize("rows,cols,block", [(24, 40, 96), (50, 256, 100), (7, 33, 3), (64, 512, 384)])
def test_coordinate_update_any_block_size(rows, cols, block):
    """Momentum blocks that are not powers of two (the specification and the
    reference's config accept any positive size): the generic kernels index
    blocks by division, bit-exact against the oracle."""

    print(f"block {block} {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows * 7 + block)
    coord = rng.integers(-127, 128, size=(rows, cols)).astype(np.int8)
    state = oracle.fresh_state(coord, block)
    gstate = _to_gpu_state(state)
    for step in range(3):
        ev = (rng.standard_normal((rows, cols)) * 0.1).astype(np.float32)
        kw = dict(beta1=0.9, beta2=0.99, update_clip=2.0, coordinate_lr=0.3, block_size=block, seed=5, step=step)
        flips = _gpu_step(ev, gstate, **kw)
        oflips = oracle.coordinate_update(ev, state, **kw)
        _assert_state_equal(gstate, state, (rows, cols, block, step))
        assert flips == oflips


@pytest.mark.parametrize("clip", [0.05, 1e6])
def test_coordinate_update_clip_regimes(clip):
    """Both sides of the RMS clip on a shape where the usq pass also computes
    the momentum as if the clip divisor were 1 (host-known steps >= 64): with
    the clip engaged that guess is thrown away and the momentum pass
    recomputes; with it idle (divisor exactly 1) the guess is the result.
    Steps below 64 take the plain two-pass order.  Bit-exact either way."""

    rows, cols, block = 96, 1024, 256
    rng = np.random.default_rng(11)
    coord = rng.integers(-127, 128, size=(rows, cols)).astype(np.int8)
    state = oracle.fresh_state(coord, block)
    gstate = _to_gpu_state(state)
    for step in (0, 1, 64, 65, 200):
        ev = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        kw = dict(beta1=0.9, beta2=0.99, update_clip=clip, coordinate_lr=1.0, block_size=block,
                  seed=17, step=step)
        flips = _gpu_step(ev, gstate, **kw)
        oflips = oracle.coordinate_update(ev, state, **kw)
        _assert_state_equal(gstate, state, (clip, step))
        assert flips == oflips


def _c_step(ev, gstate, rows, cols, kw, step):
    """The C entry with a caller-held workspace; returns (flips, scalars)."""

    from qste_amd.kernels import _lib

    lib = _lib.load()
    need = lib.qste_coordinate_update_workspace_bytes(rows, cols, kw["block_size"])
    at = lib.qste_coordinate_update_scalars_offset(rows, cols, kw["block_size"])
    assert 0 <= at and at + 16 <= need
    work = torch.empty(need, dtype=torch.uint8, device=DEV)
    flips = torch.empty((), dtype=torch.int64, device=DEV)
    g = t(ev)
    rc = lib.qste_coordinate_update(
        g.data_ptr(), gstate["coordinate"].data_ptr(), gstate["packed"].data_ptr(),
        gstate["moment_q"].data_ptr(), gstate["moment_scale"].data_ptr(), gstate["row_v"].data_ptr(),
        gstate["col_v"].data_ptr(), rows, cols, kw["beta1"], kw["beta2"], kw["update_clip"],
        kw["coordinate_lr"], kw["block_size"], kw["seed"], step, None, flips.data_ptr(), None,
        work.data_ptr(), need, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    scalars = work[at:at + 16].view(torch.float32).cpu().numpy()
    return int(flips.item()), scalars


# row path (cols % 256 == 0) and the generic kernels; steps >= 64 let the
# usq pass compute the momentum speculatively
@pytest.mark.parametrize("rows,cols,block", [(64, 2048, 256), (37, 45, 64), (200, 200, 128)])
@pytest.mark.parametrize("lr", [0.3, 0.7, 0.1, 1.0])
def test_coordinate_update_step_size_matches_spec(rows, cols, block, lr):
    """The step size the kernel used -- reciprocal(rms(m)) * fp32(lr), as
    fallback.py:204-206 evaluates ``coordinate_lr / moment_rms`` -- read back
    from the workspace, equals the oracle's bit for bit, and so do the RMS
    clip divisor, the momentum RMS and the whole state."""

    print(f"step size {rows}x{cols} block {block} lr {lr}", flush=True)
    rng = np.random.default_rng(rows + cols + int(lr * 10))
    coord = rng.integers(-127, 128, size=(rows, cols)).astype(np.int8)
    state = oracle.fresh_state(coord, block)
    gstate = _to_gpu_state(state)
    kw = dict(beta1=0.9, beta2=0.99, update_clip=2.0, coordinate_lr=lr, block_size=block, seed=41)
    for step in (0, 1, 70):
        ev = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
        flips, got = _c_step(ev, gstate, rows, cols, kw, step)
        want = np.zeros(4, dtype=np.float32)
        oflips = oracle.coordinate_update(ev, state, scalars=want, step=step, **kw)
        assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist(), (step, got, want)
        assert want[2] == oracle.step_size(want[3], lr)
        _assert_state_equal(gstate, state, (rows, cols, lr, step))
        assert flips == oflips


def test_coordinate_update_device_step_flips_and_gate():
    rows, cols, block = 64, 96, 64
    rng = np.random.default_rng(5)
    coord = rng.integers(-127, 128, size=(rows, cols)).astype(np.int8)
    ev = rng.standard_normal((rows, cols)).astype(np.float32)
    kw = dict(beta1=0.9, beta2=0.99, update_clip=2.0, coordinate_lr=4.0, block_size=block, seed=9)
    # gate off: nothing changes, flips reported as zero
    state = oracle.fresh_state(coord, block)
    gstate = _to_gpu_state(state)
    flips = torch.full((), -1, dtype=torch.int64, device=DEV)
    gate = torch.zeros((), dtype=torch.uint8, device=DEV)
    out = _gpu_step(ev, gstate, step=3, flips=flips, update_enabled=gate, **kw)
    assert out is flips and int(flips.item()) == 0
    _assert_state_equal(gstate, state, "gated")
    # device step tensor == host step
    step_t = torch.tensor(3, dtype=torch.int64, device=DEV)
    gate.fill_(1)
    _gpu_step(ev, gstate, step=step_t, flips=flips, update_enabled=gate, **kw)
    oflips = oracle.coordinate_update(ev, state, step=3, **kw)
    _assert_state_equal(gstate, state, "device step")
    assert int(flips.item()) == oflips


@pytest.mark.parametrize("block", [0, -64])
def test_coordinate_update_rejects_bad_block(block):
    z = torch.zeros(4, 8, dtype=torch.int8, device=DEV)
    with pytest.raises(ValueError):
        K().coordinate_update(torch.zeros(4, 8, device=DEV), z, torch.zeros(4, 1, dtype=torch.uint8, device=DEV),
                              z.clone(), torch.zeros(1, dtype=torch.float16, device=DEV),
                              torch.zeros(4, dtype=torch.float16, device=DEV),
                              torch.zeros(8, dtype=torch.float16, device=DEV), beta1=0.9, beta2=0.99,
                              update_clip=2.0, coordinate_lr=1.0, block_size=block, seed=1, step=0)


# ---------------------------------------------------------------------------
# MFMA path: ragged tiles and the full config-4 shapes (row-sampled oracle)
# ---------------------------------------------------------------------------

MFMA_SHAPES = [(576, 320, 300), (1024, 2048, 1000), (128, 64, 17), (256, 512, 2), (4096, 1024, 257)]


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("rows,cols,m", [(4096, 4096, 64), (1000, 8192, 17), (2048, 2048, 256), (640, 4096, 100)])
def test_split_k_forward(rows, cols, m, dt):
    """16 < m with few output tiles over a long K: the forward cuts K into
    ranges (the workspace query says so), and agrees with the oracle and,
    up to rare one-ulp roundings from the other fp32 summation order, with
    the unsplit kernel the plain entry runs."""

    print(f"split-K forward {rows}x{cols} m={m} {dt}", flush=True)
    lib = K()._lib.load()
    code = {"bf16": 2, "f16": 1}[dt]
    assert lib.qste_packed_linear_affine_workspace_bytes(m, rows, cols, code) > 0
    packed, x, scale, bias, _ = _problem(rows, cols, m, dt, rows + cols + 7 * m)
    tx, tp, ts, tb = t(x, DT[dt]), t(packed), t(scale), t(bias)
    y = K().packed_linear_affine(tx, tp, ts, tb, cols)
    plain = torch.empty_like(y)
    rc = lib.qste_packed_linear_affine(tx.data_ptr(), code, tp.data_ptr(), ts.data_ptr(), tb.data_ptr(),
                                       plain.data_ptr(), m, rows, cols, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    got, ref = f32(y), f32(plain)
    want_r = round_out(oracle.linear_fwd(x, packed, scale, bias, cols), dt)
    assert rel_l2(got, want_r) <= 1e-3
    assert np.mean(got != want_r) < 0.01
    assert np.mean(got != ref) < 0.01
    ulp = np.abs(ref) * (2.0 ** -7 if dt == "bf16" else 2.0 ** -10)
    assert np.all(np.abs(got - ref) <= ulp + 1e-6)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("rows,cols,m", MFMA_SHAPES)
def test_mfma_products_ragged(rows, cols, m, dt):
    print(f"mfma {rows}x{cols} m={m} {dt}", flush=True)
    packed, x, scale, bias, dy = _problem(rows, cols, m, dt, rows * 3 + m)
    tdt = DT[dt]
    y = f32(K().packed_linear_affine(t(x, tdt), t(packed), t(scale), t(bias), cols))
    assert rel_l2(y, round_out(oracle.linear_fwd(x, packed, scale, bias, cols), dt)) <= 1e-3
    dx = f32(K().packed_transpose(t(dy, tdt), t(packed), cols, row_scale=t(scale)))
    assert rel_l2(dx, round_out(oracle.linear_dgrad(dy, packed, cols, round_scale(scale, dt)), dt)) <= 1e-3
    xbits, off, xs = oracle.pack_affine_rows(x)
    ev = K().evidence_from_packed(t(dy, tdt), t(xbits), cols, row_scale=t(xs)).cpu().numpy()
    assert rel_l2(ev, oracle.evidence(dy, xbits, cols, round_scale(xs, dt))) <= 1e-5
    dxf, evf, gs, db = K().linear_backward(t(dy, tdt), t(xbits), t(off), t(xs), t(packed), t(scale), cols,
                                           need_bias=True)
    e0 = oracle.evidence(dy, xbits, cols, round_scale(xs, dt)) + oracle.offset_correction(dy, off)[:, None]
    assert rel_l2(evf.cpu().numpy(), e0 * scale[:, None]) <= 1e-5
    assert rel_l2(gs.cpu().numpy(), oracle.row_inner(e0.astype(np.float32), packed, cols)) <= 1e-4
    assert rel_l2(f32(dxf), dx) == 0.0


# Shapes whose evidence tiles have long K (= tokens) chains against the
# launch: tiles split over K ranges, finished by a combine pass.
# (256, 256, 16384): one tile, 8 ranges; (512, 320, 3000): ragged N and a
# shorter last range (24 and 23 K steps); (1024, 4096, 8192) and
# (4096, 1024, 8192): the config-2 layers (all 64 tiles split, beside dX in
# one launch or alone); (4160, 4096, 2048): 272 tiles, ragged M, the first
# 256 whole and the last 16 split in two.
# (3072, 768, 8184) and (768, 3072, 8184): config 3's MLP layers (GPT-2 small,
# 8 x 1023 tokens), whose backward runs the pair kernel with every evidence
# tile split over a ragged K.
SPLIT_SHAPES = [(256, 256, 16384), (512, 320, 3000), (1024, 4096, 8192), (4096, 1024, 8192),
                (4160, 4096, 2048), (3072, 768, 8184), (768, 3072, 8184)]


@pytest.mark.parametrize("need_input", [True, False])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("rows,cols,m", SPLIT_SHAPES)
def test_split_evidence_backward(rows, cols, m, dt, need_input):
    """Split evidence against the oracle (at the config-2 shapes on 256
    sampled evidence rows); dX bit for bit equal to the standalone dX
    product, itself checked against the oracle above and below."""

    print(f"split {rows}x{cols} m={m} {dt} need_input={need_input}", flush=True)
    packed, x, scale, _, dy = _problem(rows, cols, m, dt, rows + 5 * cols + m)
    xbits, off, xs = oracle.pack_affine_rows(x)
    dx, ev, gs, db = K().linear_backward(t(dy, DT[dt]), t(xbits), t(off), t(xs), t(packed), t(scale), cols,
                                         need_bias=True, need_input=need_input)
    idx = np.arange(rows)
    if rows * cols * m > 1 << 31:
        idx = np.sort(np.random.default_rng(rows + cols).choice(rows, 256, replace=False))
    dys = np.ascontiguousarray(dy[:, idx])
    e0 = oracle.evidence(dys, xbits, cols, round_scale(xs, dt)) + oracle.offset_correction(dys, off)[:, None]
    assert rel_l2(ev.cpu().numpy()[idx], e0 * scale[idx, None]) <= 1e-5
    want_gs = oracle.row_inner(e0.astype(np.float32), np.ascontiguousarray(packed[idx]), cols)
    assert rel_l2(gs.cpu().numpy()[idx], want_gs) <= 1e-4
    assert rel_l2(db.cpu().numpy(), dy.astype(np.float64).sum(0)) <= 1e-5
    if need_input:
        alone = K().packed_transpose(t(dy, DT[dt]), t(packed), cols, row_scale=t(scale))
        assert torch.equal(dx, alone)
        # dX against the operand-rounded oracle (on 256 sampled tokens at the
        # larger shapes: a token's input gradient depends on its own row of dY)
        tok = np.arange(m)
        if rows * cols * m > 1 << 31:
            tok = np.sort(np.random.default_rng(m + cols).choice(m, 256, replace=False))
        want_dx = round_out(oracle.linear_dgrad(np.ascontiguousarray(dy[tok]), packed, cols,
                                                round_scale(scale, dt)), dt)
        assert rel_l2(f32(dx)[tok], want_dx) <= 1e-3
    else:
        assert dx is None


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("rows,cols,m", SPLIT_SHAPES)
def test_split_evidence_alone(rows, cols, m, dt):
    """evidence_from_packed with its split workspace, against the oracle
    (on 256 sampled rows at the larger shapes)."""

    print(f"split evidence {rows}x{cols} m={m} {dt}", flush=True)
    _, x, _, _, dy = _problem(rows, cols, m, dt, 3 * rows + cols + m)
    xbits, _, xs = oracle.pack_affine_rows(x)
    ev = K().evidence_from_packed(t(dy, DT[dt]), t(xbits), cols, row_scale=t(xs)).cpu().numpy()
    idx = np.arange(rows)
    if rows * cols * m > 1 << 31:
        idx = np.sort(np.random.default_rng(rows).choice(rows, 256, replace=False))
    want = oracle.evidence(np.ascontiguousarray(dy[:, idx]), xbits, cols, round_scale(xs, dt))
    assert rel_l2(ev[idx], want) <= 1e-5


@pytest.mark.parametrize("rows,cols,m", [(256, 256, 16384), (512, 320, 3000)])
def test_evidence_without_workspace_runs_unsplit(rows, cols, m):
    """The C entry with a NULL workspace (no split) and with the split
    workspace agree with the oracle alike."""

    from qste_amd.kernels import _lib

    _, x, _, _, dy = _problem(rows, cols, m, "bf16", rows + m)
    xbits, _, xs = oracle.pack_affine_rows(x)
    want = oracle.evidence(dy, xbits, cols, round_scale(xs, "bf16"))
    g, b, sc = t(dy, torch.bfloat16), t(xbits), t(xs)
    lib = _lib.load()
    need = lib.qste_evidence_from_packed_workspace_bytes(m, rows, cols)
    assert need > 0
    work = torch.empty(need, dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for ws, nbytes in ((None, 0), (work.data_ptr(), need)):
        out = torch.empty(rows, cols, dtype=torch.float32, device=DEV)
        rc = lib.qste_evidence_from_packed(g.data_ptr(), 2, b.data_ptr(), sc.data_ptr(), out.data_ptr(), m, rows,
                                           cols, ws, nbytes, stream)
        assert rc == 0
        outs.append(out.cpu().numpy())
    for got in outs:
        assert rel_l2(got, want) <= 1e-5


@pytest.mark.parametrize("rows,cols", [(14336, 4096), (4096, 14336)])
def test_full_size_products_sampled_rows(rows, cols):
    """Config-4 layer shapes, 16384 tokens: forward and input gradient on 256
    sampled token rows, the evidence on 256 sampled output rows, each against
    the float64 oracle (BLAS route, pinned to the C restatement), and every
    output element finite."""

    T = 16384
    print(f"full-size products {rows}x{cols}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows)
    bf = torch.bfloat16
    x = torch.randn(T, cols, generator=g, device=DEV).to(bf)
    dy = torch.randn(T, rows, generator=g, device=DEV).to(bf)
    coord = torch.randint(-127, 128, (rows, cols), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    packed = K().pack_coordinate(coord)
    scale = torch.rand(rows, generator=g, device=DEV) * 0.02 + 0.005
    y = K().packed_linear_affine(x, packed, scale, None, cols)
    dx = K().packed_transpose(dy, packed, cols, row_scale=scale)
    xbits, off, xs = K().pack_affine_rows(x)
    ev = K().evidence_from_packed(dy, xbits, cols, row_scale=xs)
    torch.cuda.synchronize()
    for out in (y, dx, ev):
        assert bool(torch.isfinite(out).all())
    pk, sc = packed.cpu().numpy(), scale.cpu().numpy()
    rng = np.random.default_rng(1)
    trows = np.sort(rng.choice(T, 256, replace=False))
    sel = torch.from_numpy(trows).to(DEV)
    want_y = round_out(oracle.linear_fwd_f64(x[sel].float().cpu().numpy(), pk, sc, None, cols), "bf16")
    assert rel_l2(f32(y[sel]), want_y) <= 1e-3
    dys = dy[sel].float().cpu().numpy()
    want_dx = round_out(oracle.linear_dgrad_f64(dys, pk, cols, round_scale(sc, "bf16")), "bf16")
    assert rel_l2(f32(dx[sel]), want_dx) <= 1e-3
    erows = np.sort(rng.choice(rows, 256, replace=False))
    esel = torch.from_numpy(erows).to(DEV)
    dy_cols = dy[:, esel].float().cpu().numpy()
    want_e = oracle.evidence_f64(dy_cols, xbits.cpu().numpy(), cols, round_scale(xs.cpu().numpy(), "bf16"))
    assert rel_l2(ev[esel].cpu().numpy(), want_e) <= 1e-5


def test_device_profile_on_the_gpu():
    """``qste_amd.device_profile()``: one line naming the gfx950 device, its
    compute-unit count and the shader clock measured by a wave."""

    import re

    import qste_amd

    line = qste_amd.device_profile()
    print(line, flush=True)
    assert "\n" not in line and "gfx950" in line
    cus = int(re.search(r"cus=(\d+)", line).group(1))
    assert cus == torch.cuda.get_device_properties(0).multi_processor_count
    mhz = float(re.search(r"/ (\d+)MHz measured", line).group(1))
    assert 500 <= mhz <= 3000
