"""The user API end to end on the GPU: QSTELinear forward/backward, the
coordinate step inside backward, PackedLinear decode, and size-independent
properties of the step at the config-4 surface shape.

Float outputs: relative L2 against the float64 oracle (bf16 outputs against
the oracle rounded to bf16, a folded scale rounded to bf16 first) -- 1e-3 for
bf16, 1e-5 for fp32. Integer state: bit-exact against the oracle's step run on
the evidence the GPU produced.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    n = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (n if n > 0 else 1.0))


def bf(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).float().numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,cols,m", [(384, 256, 200), (1024, 512, 64), (96, 130, 33)])
def test_qste_linear_forward_backward(dtype, rows, cols, m):
    import qste_amd as qste

    torch.manual_seed(rows + cols)
    lin = nn.Linear(cols, rows)
    layer = qste.QSTELinear.from_linear(lin).to(DEV)
    x = torch.randn(m, cols, device=DEV).to(dtype).requires_grad_(True)
    dy = torch.randn(m, rows, device=DEV).to(dtype)
    y = layer(x)
    y.backward(dy)
    packed = layer.surface.packed_sign.cpu().numpy()
    s = layer.scale.detach().float().cpu().numpy()
    xb = x.detach().float().cpu().numpy()
    dyb = dy.float().cpu().numpy()
    want_y = oracle.linear_fwd(xb, packed, s, layer.bias.detach().cpu().numpy(), cols)
    tol = 1e-5 if dtype == torch.float32 else 1e-3
    rnd = (lambda a: a) if dtype == torch.float32 else bf
    assert rel_l2(y.detach().float().cpu().numpy(), rnd(want_y)) <= tol
    s_op = s if dtype == torch.float32 else bf(s)
    want_dx = oracle.linear_dgrad(dyb, packed, cols, s_op)
    assert rel_l2(x.grad.float().cpu().numpy(), rnd(want_dx)) <= tol
    bits, off, xs = oracle.pack_affine_rows(xb)
    xs_op = xs if dtype == torch.float32 else bf(xs)
    e0 = oracle.evidence(dyb, bits, cols, xs_op) + oracle.offset_correction(dyb, off)[:, None]
    gs = oracle.row_inner(e0.astype(np.float32), packed, cols)
    assert rel_l2(layer.surface.log_scale.grad.cpu().numpy(), gs * s) <= 1e-4
    assert rel_l2(layer.bias.grad.cpu().numpy(), dyb.astype(np.float64).sum(0)) <= 1e-5


def test_immediate_step_equals_oracle_on_the_gpu_evidence(monkeypatch):
    """The step that runs inside backward, checked exactly."""

    import qste_amd as qste
    from qste_amd import kernels

    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(256, 512), nn.ReLU(), nn.Linear(512, 128)).to(DEV)
    qste.convert(model, include=["0", "2"], config={"seed": 3})
    coords = qste.QSTEOptimizer(model)
    real = kernels.coordinate_update
    seen = []

    def spy(gradient, coordinate, packed, moment_q, moment_scale, row_v, col_v, **kw):
        seen.append((gradient.detach().float().cpu().numpy().copy(),
                     {"coordinate": coordinate.cpu().numpy().copy(), "packed": packed.cpu().numpy().copy(),
                      "moment_q": moment_q.cpu().numpy().copy(), "moment_scale": moment_scale.cpu().numpy().copy(),
                      "row_v": row_v.cpu().numpy().copy(), "col_v": col_v.cpu().numpy().copy()},
                     dict(kw), (coordinate, packed, moment_q, moment_scale, row_v, col_v)))
        return real(gradient, coordinate, packed, moment_q, moment_scale, row_v, col_v, **kw)

    monkeypatch.setattr(kernels, "coordinate_update", spy)
    for it in range(2):
        x = torch.randn(128, 256, device=DEV, dtype=torch.bfloat16)
        model(x).float().square().mean().backward()
        coords.step()
    assert len(seen) == 4
    for ev, state, kw, after in seen:
        kw = {k: v for k, v in kw.items() if k not in ("flips", "update_enabled")}
        oracle.coordinate_update(ev, state, **kw)
    # the last step of each surface: GPU state now equals the oracle's
    for ev, state, kw, after in seen[2:]:
        names = ("coordinate", "packed", "moment_q", "moment_scale", "row_v", "col_v")
        for name, t in zip(names, after):
            assert np.array_equal(t.cpu().numpy().view(np.uint8), state[name].view(np.uint8)), name


def test_training_step_is_reproducible():
    import qste_amd as qste

    results = []
    for _ in range(2):
        torch.manual_seed(11)
        model = nn.Sequential(nn.Linear(128, 256), nn.GELU(), nn.Linear(256, 128)).to(DEV)
        qste.convert(model, include=["0", "2"])
        opt = torch.optim.AdamW(qste.continuous_parameters(model), lr=1e-3)
        coords = qste.QSTEOptimizer(model)
        g = torch.Generator(device=DEV).manual_seed(5)
        for _ in range(3):
            x = torch.randn(64, 128, device=DEV, generator=g)
            loss = model(x).square().mean()
            loss.backward()
            opt.step(); coords.step()
            opt.zero_grad(); coords.zero_grad()
        results.append([s.coordinate.detach().cpu().clone() for s in qste.surfaces(model)])
    for a, b in zip(*results):
        assert torch.equal(a, b)


@pytest.mark.parametrize("M", [1, 4, 16])
def test_packed_linear_decode(M):
    import qste_amd as qste

    K, N = 2048, 3072
    g = torch.Generator(device=DEV).manual_seed(M)
    packed = torch.randint(0, 256, (N, K // 8), generator=g, device=DEV, dtype=torch.int32).to(torch.uint8)
    scale = torch.rand(N, generator=g, device=DEV) * 0.02 + 0.001
    bias = torch.randn(N, generator=g, device=DEV) * 0.1
    layer = qste.PackedLinear(packed, scale, K, bias)
    x = torch.randn(M, K, generator=g, device=DEV).to(torch.bfloat16)
    y = layer(x)
    assert y.dtype == torch.bfloat16
    want = oracle.linear_fwd(x.float().cpu().numpy(), packed.cpu().numpy(), scale.cpu().numpy(),
                             bias.cpu().numpy(), K)
    assert rel_l2(y.float().cpu().numpy(), bf(want)) <= 1e-3


@pytest.mark.parametrize("step", [0, 70])
def test_full_size_step_matches_the_oracle(step):
    """Config-4 gate surface (14336 x 4096, the row kernels): two consecutive
    steps from fresh state, the second at ``step`` (70 lets the usq pass
    compute the momentum speculatively), bit-exact against the oracle on the
    same evidence: coordinates, packed signs, momentum, fp16 statistics and
    flip counts."""

    from qste_amd import kernels

    print(f"full-size step, second step number {step}", flush=True)
    R, C = 14336, 4096
    rng = np.random.default_rng(step + 3)
    coord0 = rng.integers(-127, 128, size=(R, C), dtype=np.int8)
    state = oracle.fresh_state(coord0, 256)
    dev = {k: torch.from_numpy(v.copy()).to(DEV) for k, v in state.items()}
    for k, number in enumerate((0, step + 1)):
        ev = (rng.standard_normal((R, C), dtype=np.float32) * np.float32(0.01 * (k + 1)))
        flips = kernels.coordinate_update(
            torch.from_numpy(ev).to(DEV), dev["coordinate"], dev["packed"], dev["moment_q"],
            dev["moment_scale"], dev["row_v"], dev["col_v"], beta1=0.9, beta2=0.99, update_clip=2.0,
            coordinate_lr=0.7, block_size=256, seed=1 + 1_000_003, step=number)
        oflips = oracle.coordinate_update(ev, state, beta1=0.9, beta2=0.99, update_clip=2.0, coordinate_lr=0.7,
                                          block_size=256, seed=1 + 1_000_003, step=number)
        for key, want in state.items():
            got = dev[key].cpu().numpy()
            assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), (number, key, int((got != want).sum()))
        assert flips == oflips and flips > 0


def test_full_size_step_properties():
    """Config-4 gate surface (14336 x 4096): integer invariants and reproducibility."""

    from qste_amd import kernels

    R, C = 14336, 4096
    g = torch.Generator(device=DEV).manual_seed(2)
    ev = torch.randn(R, C, generator=g, device=DEV) * 0.01
    coord0 = torch.randint(-127, 128, (R, C), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    outs = []
    for _ in range(2):
        coord = coord0.clone()
        packed = kernels.pack_coordinate(coord)
        before = packed.clone()
        blocks = (R * C + 255) // 256
        mq = torch.zeros_like(coord)
        ms = torch.full((blocks,), 1 / 127, dtype=torch.float16, device=DEV)
        rv = torch.zeros(R, dtype=torch.float16, device=DEV)
        cv = torch.zeros(C, dtype=torch.float16, device=DEV)
        flips = kernels.coordinate_update(ev, coord, packed, mq, ms, rv, cv, beta1=0.9, beta2=0.99,
                                          update_clip=2.0, coordinate_lr=1.0, block_size=256, seed=1, step=0)
        assert torch.equal(packed, kernels.pack_coordinate(coord))
        assert int(coord.abs().max()) <= 127 and int(mq.int().abs().max()) <= 127
        diff = torch.bitwise_xor(before, packed)
        pop = sum(int(((diff >> k) & 1).sum()) for k in range(8))
        assert flips == pop
        # a coordinate moves by about |m| / rms(m): mean |z| of a normal is 0.8
        moved = (coord.int() - coord0.int()).abs().float()
        assert 0.3 < float(moved.mean()) < 1.5
        outs.append((coord.cpu(), mq.cpu(), ms.cpu(), rv.cpu(), cv.cpu(), flips))
    for a, b in zip(outs[0][:5], outs[1][:5]):
        assert torch.equal(a.view(torch.uint8) if a.dtype == torch.float16 else a,
                           b.view(torch.uint8) if b.dtype == torch.float16 else b)
    assert outs[0][5] == outs[1][5]


def test_bf16_parameters_reach_the_kernels_intact():
    """Regression: a bf16 scale and bias (a model cast with .to(bfloat16)) are
    converted to fp32 copies for the C call; those copies must outlive the
    launch, or the allocator reuses one's block for the next (the bias) and
    the kernel reads the wrong values."""

    import qste_amd as qste

    torch.manual_seed(0)
    model = qste.convert(torch.nn.Sequential(torch.nn.Linear(256, 384)))[0].to(device="cuda", dtype=torch.bfloat16)
    x = torch.randn(64, 256, device="cuda").to(torch.bfloat16)
    sign = torch.where(model.surface.coordinate >= 0, 1.0, -1.0).double()
    ref = (x.double() @ sign.t()) * model.scale.detach().double() + model.bias.detach().double()
    with torch.no_grad():
        y = model(x)
    # against the exact product rounded to the output dtype, as the bf16
    # forward parity is stated
    ref16 = ref.to(torch.bfloat16).double()
    rel = float((y.double() - ref16).norm() / ref16.norm())
    assert rel <= 1e-3, rel
    dy = torch.randn(64, 384, device="cuda").to(torch.bfloat16)
    xr = x.clone().requires_grad_(True)
    model(xr).backward(dy)
    ref_dx = dy.double() @ (sign * model.scale.detach().double()[:, None])
    assert float((xr.grad.double() - ref_dx).norm() / ref_dx.norm()) <= 5e-3


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_weight_path_forward_evidence_and_scale_gradient(dtype):
    """``.weight`` (QSTEWeightFn, reference functional.py:213-252) for code
    that reads the dense matrix: forward is exactly sign * scale in the
    scale's dtype; backward turns dL/dW into the surface's evidence dW * s
    and the scale gradient row_inner(dW, sign) (times d scale / d log_scale),
    against the float64 oracle, and the coordinate step applied on that
    evidence inside backward equals the oracle's bit for bit."""

    import qste_amd as qste

    print(f"weight path {dtype}", flush=True)
    rows, cols, m = 384, 520, 96
    g = torch.Generator().manual_seed(31)
    coord = torch.randint(-127, 128, (rows, cols), generator=g, dtype=torch.int32).to(torch.int8)
    scale = torch.rand(rows, generator=g) * 0.02 + 0.005
    surface = qste.Surface.from_state(coord.to(DEV), scale.log().to(DEV))
    layer = qste.QSTELinear(surface, None).to(dtype=dtype)
    coords = qste.QSTEOptimizer([surface])
    seen = []
    apply = coords._apply
    surface.route_evidence(lambda s, e: (seen.append(e.detach().clone()), apply(s, e)))
    x = torch.randn(m, cols, generator=g).to(DEV)
    dy = torch.randn(m, rows, generator=g).to(DEV)

    packed_before = surface.packed_sign.detach().cpu().numpy().copy()  # the step rewrites it in backward
    w = layer.weight
    assert w.dtype == dtype
    s_eff = layer.scale.detach()
    sign = torch.where(surface.coordinate >= 0, 1.0, -1.0).to(DEV)
    assert torch.equal(w.detach().float(), (sign * s_eff.float()[:, None]).to(dtype).float())
    (x.to(dtype) @ w.t()).float().mul(dy).sum().backward()
    flips = coords.step()
    torch.cuda.synchronize()

    dw = (dy.double().t() @ x.to(dtype).double())            # dL/dW in float64
    s64 = s_eff.double()
    assert len(seen) == 1
    want_e = dw * s64[:, None]
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert float((seen[0].double() - want_e).norm() / want_e.norm()) <= tol
    gs = oracle.row_inner(dw.float().cpu().numpy(), packed_before, cols)
    want_gs = torch.from_numpy(gs).to(DEV) * s64          # d scale / d log_scale = scale
    got_gs = surface.log_scale.grad.double()
    assert float((got_gs - want_gs).norm() / want_gs.norm()) <= tol
    state = oracle.fresh_state(coord.numpy(), 256)
    oflips = oracle.coordinate_update(seen[0].cpu().numpy(), state, beta1=0.9, beta2=0.99, update_clip=2.0,
                                      coordinate_lr=1.0, block_size=256, seed=1, step=0)
    assert np.array_equal(surface.coordinate.cpu().numpy(), state["coordinate"])
    assert np.array_equal(surface.packed_sign.cpu().numpy(), state["packed"])
    assert flips == oflips and flips > 0
