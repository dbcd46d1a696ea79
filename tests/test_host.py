"""Host-side logic and the C ABI, without a GPU.

* The HIP library loads and exports every entry point `include/qste_hip.h`
  declares; argument errors come back as codes without touching a device.
* The user API (`convert`, `Surface`, `QSTELinearFn`, `QSTEOptimizer`,
  `PackedLinear`, `export_packed`) is driven on CPU through a fake operator
  layer built from the oracle -- test-only: the product's operator layer has no
  CPU path -- to check the orchestration the reference defines: layer
  selection and tying (`convert.py:159-243`), surface initialization
  (`surface.py:41-62`), the backward composition (`functional.py:173-194`),
  immediate evidence application with seed `cfg.seed + 1_000_003 * position`
  and the pre-increment step number (`optim.py:156-201`), scale clamping and
  state_dict round trips (`optim.py:212-232`).
"""

from __future__ import annotations

import ctypes
import math
import re
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from oracle import activations as oa
from oracle import embedding as oe

ROOT = Path(__file__).resolve().parents[1]


# ---------------------------------------------------------------------------
# the C ABI
# ---------------------------------------------------------------------------


def _declared():
    text = (ROOT / "include" / "qste_hip.h").read_text()
    return sorted(set(re.findall(r"\b(qste_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from qste_amd.kernels import _lib

    lib = _lib.load()
    names = _declared()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), name
    # and the binding's signature table covers them all
    assert set(names) == set(_lib.SIGNATURES)


def test_library_allocates_and_clears_no_device_memory():
    """Scratch comes from caller workspaces (or the static scratch array), and
    nothing is cleared with a memset: the built library imports no HIP
    allocation, free or memset routine."""

    import shutil
    import subprocess

    from qste_amd.kernels import _lib

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    lib = _lib.load()
    out = subprocess.run([nm, "-D", "--undefined-only", lib._name], capture_output=True, text=True, check=True)
    imported = {line.split()[-1].split("@")[0] for line in out.stdout.splitlines() if line.strip()}
    assert "hipLaunchKernel" in imported or any(n.startswith("__hip") for n in imported)
    banned = {n for n in imported if re.match(r"hip(Ext)?(Malloc|Free|Memset|HostMalloc|HostFree|MallocAsync)", n)}
    assert not banned, sorted(banned)


def test_error_codes_and_workspace_queries_need_no_gpu():
    from qste_amd.kernels import _lib

    lib = _lib.load()
    assert lib.qste_version() >= 1
    for code, word in ((-1, b"dtype"), (-2, b"shape"), (-3, b"NULL"), (-4, b"workspace"), (-5, b"block size must be positive")):
        assert word in lib.qste_error_string(code)
    assert lib.qste_coordinate_update_workspace_bytes(4096, 14336, 256) > 0
    assert lib.qste_coordinate_update_workspace_bytes(0, 8, 256) == 0
    assert lib.qste_linear_backward_workspace_bytes(16384, 14336, 4096) > 0
    # the split-K plan of the evidence (fp32 partials of 256 x 256 tiles in
    # the workspace): a one-tile evidence over 16384 tokens takes 8 K
    # ranges; config 4's 896 tiles (3.5 rounds of 256 CUs) split their last
    # 128 tiles in two; a short K splits nothing
    tile = 256 * 256 * 4
    assert lib.qste_evidence_from_packed_workspace_bytes(16384, 256, 256) == 8 * tile
    assert lib.qste_linear_backward_workspace_bytes(16384, 256, 256) > 8 * tile
    assert lib.qste_evidence_from_packed_workspace_bytes(16384, 14336, 4096) == 2 * 128 * tile
    assert lib.qste_evidence_from_packed_workspace_bytes(64, 256, 256) == 0
    assert lib.qste_linear_backward_workspace_bytes(64, 256, 256) < tile
    # argument errors are reported before any device work; a workspace
    # smaller than the split plan's is refused (NULL runs unsplit)
    need = lib.qste_evidence_from_packed_workspace_bytes(16384, 256, 256)
    assert lib.qste_evidence_from_packed(1, 2, 1, None, 1, 16384, 256, 256, 1, need - 1, None) == -4
    assert lib.qste_packed_linear_affine(None, 7, None, None, None, None, 1, 1, 8, None) == -1
    assert lib.qste_packed_transpose(None, 2, None, None, None, -1, 4, 8, None) == -2
    assert lib.qste_pack_affine_rows(None, 0, None, None, None, 4, 0, None) == -2
    # any positive momentum block size is accepted (48 is not a power of
    # two); zero or negative is refused
    assert lib.qste_coordinate_update(None, None, None, None, None, None, None, 4, 8, 0.9, 0.99, 2.0, 1.0,
                                      48, 1, 0, None, None, None, None, 0, None) == -3
    assert lib.qste_coordinate_update(None, None, None, None, None, None, None, 4, 8, 0.9, 0.99, 2.0, 1.0,
                                      0, 1, 0, None, None, None, None, 0, None) == -5
    assert lib.qste_coordinate_update(None, None, None, None, None, None, None, 4, 8, 0.9, 0.99, 2.0, 1.0,
                                      64, 1, 0, None, None, None, None, 0, None) == -3


def test_fp32_limb_workspaces_are_capped_and_shared():
    """The fp32 products' bf16 limbs (6 bytes per dense value) are held to
    512 MiB: forward and input gradient in chunks of output rows, an
    evidence whose limbs exceed it on the SIMT kernels (no limbs workspace).
    The layer backward's limbs region serves its dX and evidence products in
    turn, so it holds the larger of the two."""

    from qste_amd.kernels import _lib

    lib = _lib.load()
    f32, budget = 0, 512 << 20
    # config 4's down projection in fp32: 16384 x 14336 -> 4096
    fwd = lib.qste_packed_linear_affine_workspace_bytes(16384, 4096, 14336, f32)
    assert 0 < fwd <= budget + 4096 * 14336 * 3 // 8 + (64 << 20)
    dgr = lib.qste_packed_transpose_workspace_bytes(16384, 14336, 4096, f32)
    assert 0 < dgr <= budget + 4096 * 14336 * 3 // 8 + 4096
    assert lib.qste_evidence_from_packed_workspace_bytes_dtype(16384, 14336, 4096, f32) == 0
    assert lib.qste_evidence_from_packed_workspace_bytes_dtype(4096, 4096, 4096, f32) >= 3 * 4096 * 4096 * 2
    # small products need no chunks: the whole operand's limbs
    assert lib.qste_packed_linear_affine_workspace_bytes(256, 2048, 2048, f32) >= 256 * 2048 * 6
    for t, r, c in ((256, 2048, 2048), (4096, 4096, 4096), (16384, 14336, 4096), (16384, 4096, 14336),
                    (1024, 640, 1024), (8192, 14336, 64)):
        extra = lib.qste_linear_backward_workspace_bytes_dtype(t, r, c, f32) - lib.qste_linear_backward_workspace_bytes(
            t, r, c)
        d = lib.qste_packed_transpose_workspace_bytes(t, r, c, f32)
        e = lib.qste_evidence_from_packed_workspace_bytes_dtype(t, r, c, f32)
        assert extra >= max(d, e), (t, r, c, extra, d, e)


def test_operator_layer_refuses_cpu_tensors():
    from qste_amd import kernels

    with pytest.raises(RuntimeError, match="GPU"):
        kernels.pack_coordinate(torch.zeros(2, 8, dtype=torch.int8))
    with pytest.raises(RuntimeError, match="GPU"):
        kernels.packed_linear_affine(torch.zeros(2, 8), torch.zeros(3, 1, dtype=torch.uint8),
                                     torch.ones(3), None, 8)


def test_device_profile_without_a_gpu():
    """``qste_amd.device_profile`` on a host: one line that says the package
    has no CPU path and names the library build (reference
    src/qste/__init__.py:105-120 describes the selected kernel profile)."""

    import qste_amd

    line = qste_amd.device_profile("cpu")
    assert "\n" not in line
    assert "no QSTE kernels" in line and "gfx950" in line
    assert re.search(r"library=libqste_hip v\d+", line), line


# ---------------------------------------------------------------------------
# fake operator layer on the oracle (test-only)
# ---------------------------------------------------------------------------


class OracleKernels:
    """qste_amd.kernels' operators, computed by the oracle on CPU tensors."""

    def __init__(self):
        self.calls = []
        self.backward_calls = []

    def pack_coordinate(self, coord):
        return torch.from_numpy(oracle.pack_coordinate(coord.numpy()))

    def unpack_rows(self, packed, columns, *, dtype=None, row_scale=None):
        out = torch.from_numpy(oracle.unpack_rows(packed.numpy(), columns))
        if row_scale is not None:
            out = out * row_scale.float()[:, None]
        return out.to(dtype or torch.float32)

    def pack_affine_rows(self, values):
        b, o, s = oracle.pack_affine_rows(values.float().numpy())
        return torch.from_numpy(b), torch.from_numpy(o), torch.from_numpy(s)

    def packed_linear_affine(self, inputs, packed, scale, bias, columns):
        y = oracle.linear_fwd(inputs.float().numpy(), packed.numpy(), scale.detach().float().numpy(),
                              None if bias is None else bias.detach().float().numpy(), columns)
        return torch.from_numpy(y).float().to(inputs.dtype).view(*inputs.shape[:-1], packed.shape[0])

    def packed_row_inner(self, matrix, packed, columns):
        return torch.from_numpy(oracle.row_inner(matrix.float().numpy(), packed.numpy(), columns)).float()

    def linear_backward(self, grad, packed_x, x_offset, x_scale, packed_w, scale, columns, *, need_bias,
                        need_input=True, offset_dot=None):
        g = grad.float().numpy()
        s = scale.detach().float().numpy()
        self.backward_calls.append(need_input)
        self.offset_dots = getattr(self, "offset_dots", []) + [offset_dot is not None]
        if offset_dot is not None:
            # what was offered must be this gradient summed against this
            # layer's own saved offsets
            want = g.astype(np.float64).T @ x_offset.numpy().astype(np.float64)
            assert np.allclose(offset_dot.numpy(), want, rtol=1e-5, atol=1e-6)
        dx = oracle.linear_dgrad(g, packed_w.numpy(), columns, s)
        e0 = oracle.decoded_evidence(g, packed_x.numpy(), x_offset.numpy(), x_scale.numpy(), columns)
        gs = oracle.row_inner(e0.astype(np.float32), packed_w.numpy(), columns)
        ev = (e0 * s[:, None]).astype(np.float32)
        db = torch.from_numpy(g.astype(np.float64).sum(0)).float() if need_bias else None
        dx = torch.from_numpy(dx).float().to(grad.dtype) if need_input else None
        return dx, torch.from_numpy(ev), torch.from_numpy(gs).float(), db

    def coordinate_update(self, gradient, coordinate, packed, moment_q, moment_scale, row_v, col_v, *,
                          beta1, beta2, update_clip, coordinate_lr, block_size, seed, step, flips=None,
                          update_enabled=None):
        self.calls.append({"seed": seed, "step": int(step), "evidence": gradient.clone()})
        state = {"coordinate": coordinate.numpy(), "packed": packed.numpy(), "moment_q": moment_q.numpy(),
                 "moment_scale": moment_scale.numpy(), "row_v": row_v.numpy(), "col_v": col_v.numpy()}
        n = oracle.coordinate_update(gradient.float().numpy(), state, beta1=beta1, beta2=beta2,
                                     update_clip=update_clip, coordinate_lr=coordinate_lr,
                                     block_size=block_size, seed=seed, step=int(step))
        if flips is not None:
            flips.fill_(n)
            return flips
        return n

    # packed activations (oracle/activations.py)
    @staticmethod
    def _dt(t):
        return {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16"}[t.dtype]

    def pack_bits(self, mask):
        return torch.from_numpy(oa.pack_bits(mask.numpy()))

    def unpack_bits(self, packed, columns, *, dtype=None):
        return torch.from_numpy(oa.unpack_bits(packed.numpy(), columns)).to(dtype or torch.float32)

    def masked_backward(self, grad, packed, columns, *, inside=1.0, outside=0.0):
        out = oa.masked_backward(grad.float().numpy(), packed.numpy(), inside, outside, self._dt(grad))
        return torch.from_numpy(out).to(grad.dtype)

    def masked_activation(self, x, kind, *, lower=0.0, upper=None, slope=0.0, want_output=True):
        from qste_amd import kernels

        v, name = x.float().numpy(), self._dt(x)
        if kind == kernels.MASK_CLAMP:
            out, packed = oa.clamp_forward(v, lower, upper, name)
        elif kind == kernels.MASK_LEAKY:
            out, packed = oa.leaky_forward(v, slope, name)
        else:
            return None, torch.from_numpy(oa.interval_bits(v, lower, upper, name))
        return torch.from_numpy(out).to(x.dtype), torch.from_numpy(packed)

    def smooth_activation(self, x, kind, param=0.0, *, output=None, derivative=None):
        if kind == "provided":
            payload, scale = oa.quantize_rows(derivative.float().numpy())
            return None, torch.from_numpy(payload), torch.from_numpy(scale)
        name = self._dt(x)
        y = None if output is None else output.float().numpy()
        y, payload, scale = oa.smooth_forward(kind, x.float().numpy(), param, name, y=y)
        return torch.from_numpy(y).to(x.dtype), torch.from_numpy(payload), torch.from_numpy(scale)

    def smooth_backward(self, grad, payload, scale):
        out = oa.smooth_backward(grad.float().numpy(), payload.numpy(), scale.numpy(), self._dt(grad))
        return torch.from_numpy(out).to(grad.dtype)


    # the SwiGLU gate: torch's own chain on the CPU, encoding by the oracle
    def row_scale(self, log_scale, lo, hi):
        e = log_scale.detach().exp()
        return e.clamp(lo, hi), e

    def row_scale_backward(self, e, grad, lo, hi):
        return torch.where((e >= lo) & (e <= hi), grad.to(e.dtype), torch.zeros_like(e)) * e

    def swiglu_forward(self, gate, up, *, encode=False):
        import torch.nn.functional as F

        out = F.silu(gate) * up
        if not encode:
            return out, None
        self.swiglu_encodes = getattr(self, "swiglu_encodes", 0) + 1
        b, o, s = oracle.pack_affine_rows(out.float().reshape(-1, out.shape[-1]).numpy())
        return out, (torch.from_numpy(b), torch.from_numpy(o), torch.from_numpy(s))

    def swiglu_backward(self, grad, gate, up):
        g = gate.detach().requires_grad_(True)
        u = up.detach().requires_grad_(True)
        import torch.nn.functional as F

        with torch.enable_grad():
            (F.silu(g) * u).backward(grad)
        return g.grad, u.grad

    def swiglu_backward_sums(self, grad, gate, up, offset_gate, offset_up, *, side_by_side=False):
        dg, du = self.swiglu_backward(grad, gate, up)
        sums = torch.stack((dg.double().t() @ offset_gate.double(), du.double().t() @ offset_up.double()))
        self.swiglu_sums = getattr(self, "swiglu_sums", 0) + 1
        if side_by_side:
            return torch.cat((dg, du), dim=1), sums.float()
        return dg, du, sums.float()

    # binary embedding (oracle/embedding.py)
    def packed_embedding(self, ids, packed, scale, columns):
        out = oe.lookup(ids.numpy(), packed.numpy(), scale.detach().float().numpy(), columns)
        return torch.from_numpy(out).to(scale.dtype)

    def embedding_backward(self, ids, grad, packed, scale, columns):
        ev, gs = oe.backward(ids.numpy(), grad.float().numpy(), packed.numpy(), scale.float().numpy(), columns)
        return torch.from_numpy(ev), torch.from_numpy(gs)


ACTIVATION_OPS = ("pack_bits", "unpack_bits", "masked_backward", "masked_activation",
                  "smooth_activation", "smooth_backward", "packed_embedding", "embedding_backward",
                  "swiglu_forward", "swiglu_backward", "swiglu_backward_sums")


@pytest.fixture
def fake(monkeypatch):
    import qste_amd
    from qste_amd import kernels, surface

    ok = OracleKernels()
    for name in ("pack_coordinate", "unpack_rows", "pack_affine_rows", "packed_linear_affine",
                 "packed_row_inner", "linear_backward", "coordinate_update", "row_scale",
                 "row_scale_backward") + ACTIVATION_OPS:
        monkeypatch.setattr(kernels, name, getattr(ok, name))
    monkeypatch.setattr(surface, "_on_gpu", lambda fn, t, *a, **k: fn(t, *a, **k))
    return ok


# ---------------------------------------------------------------------------
# convert / Surface
# ---------------------------------------------------------------------------


class Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.fc1 = nn.Linear(16, 32)
        self.act = nn.ReLU()
        self.fc2 = nn.Linear(32, 16, bias=False)
        self.emb = nn.Embedding(10, 16)


def test_convert_selects_by_glob_and_records_config(fake):
    import qste_amd as qste

    torch.manual_seed(0)
    model = Block()
    qste.convert(model, include=["fc*"], exclude=["fc2"], config={"seed": 7})
    assert isinstance(model.fc1, qste.QSTELinear) and isinstance(model.fc2, nn.Linear)
    assert model._qste_config.seed == 7
    assert model.fc1.in_features == 16 and model.fc1.out_features == 32
    assert model.fc1.bias.dtype == torch.float32
    with pytest.raises(ValueError):
        qste.convert(Block(), include=["nothing*"])
    emb = qste.convert(Block(), include=["emb"]).emb
    assert isinstance(emb, qste.QSTEEmbedding) and emb.num_embeddings == 10 and emb.embedding_dim == 16
    with pytest.raises(ValueError):
        qste.convert(Block(), include=["fc1"], activations="sometimes")


def test_tied_weights_share_one_surface(fake):
    import qste_amd as qste

    a, b = nn.Linear(8, 8), nn.Linear(8, 8)
    b.weight = a.weight
    model = nn.Sequential(a, b)
    qste.convert(model)
    assert model[0].surface is model[1].surface
    assert len(qste.surfaces(model)) == 1


def test_surface_initialization_formula(fake):
    """surface.py:41-62, recomputed in float64 numpy."""

    import qste_amd as qste

    torch.manual_seed(1)
    w = torch.randn(24, 40) * 0.05
    w[3, 5] = 0.0
    s = qste.Surface(w)
    wd = w.double().numpy()
    scale = np.maximum(np.abs(wd).mean(1), 1e-5)
    latent = np.clip(wd / scale[:, None], -1.5, 1.5) * 0.25
    q = np.clip(np.round(latent / 1.5 * 127), -127, 127)
    q = np.where(q == 0, np.where(wd >= 0, 1, -1), q)
    assert np.array_equal(s.coordinate.numpy(), q.astype(np.int8))
    assert np.array_equal(s.packed_sign.numpy(), oracle.pack_coordinate(q.astype(np.int8)))
    np.testing.assert_allclose(s.log_scale.detach().numpy(), np.log(scale), rtol=1e-6)
    assert s.coordinate.requires_grad is False and s.log_scale.requires_grad is True
    torch.testing.assert_close(s.scale, s.log_scale.exp().clamp(1e-6, 4.0))


# ---------------------------------------------------------------------------
# autograd composition and the optimizer
# ---------------------------------------------------------------------------


def _mlp(seed=0):
    torch.manual_seed(seed)
    return nn.Sequential(nn.Linear(24, 40), nn.ReLU(), nn.Linear(40, 16))


def test_forward_backward_composition(fake):
    import qste_amd as qste

    model = _mlp()
    qste.convert(model, include=["0", "2"])
    layer = model[0]
    x = torch.randn(7, 24)
    y = layer(x)
    packed = layer.surface.packed_sign.numpy()
    want = oracle.linear_fwd(x.numpy(), packed, layer.scale.detach().numpy(), layer.bias.detach().numpy(), 24)
    np.testing.assert_allclose(y.detach().numpy(), want, rtol=1e-6, atol=1e-6)
    xg = x.clone().requires_grad_(True)
    dy = torch.randn(7, 40)
    layer(xg).backward(dy)
    s = layer.scale.detach().numpy()
    np.testing.assert_allclose(xg.grad.numpy(), oracle.linear_dgrad(dy.numpy(), packed, 24, s),
                               rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(layer.bias.grad.numpy(), dy.numpy().sum(0), rtol=1e-5, atol=1e-6)
    # log_scale gradient = row inner product of E0 with the signs, times
    # d scale / d log_scale = scale (clamp inactive)
    bits, off, xs = oracle.pack_affine_rows(x.numpy())
    e0 = oracle.decoded_evidence(dy.numpy(), bits, off, xs, 24)
    gs = oracle.row_inner(e0.astype(np.float32), packed, 24)
    np.testing.assert_allclose(layer.surface.log_scale.grad.numpy(), gs * s, rtol=1e-4, atol=1e-6)


def test_input_gradient_only_when_autograd_asks(fake):
    import qste_amd as qste

    model = _mlp()
    qste.convert(model, include=["0", "2"])
    x = torch.randn(5, 24)
    dy = torch.randn(5, model[2].out_features)
    # the first layer's input needs no gradient, the second's does
    model(x).backward(dy)
    assert fake.backward_calls == [True, False]
    fake.backward_calls.clear()
    xg = x.clone().requires_grad_(True)
    model(xg).backward(dy)
    assert fake.backward_calls == [True, True]
    assert xg.grad is not None and xg.grad.shape == x.shape
    # the evidence of the first layer is the same either way
    assert model[0].surface.log_scale.grad is not None


def test_optimizer_applies_inside_backward_with_reference_seeds(fake):
    import qste_amd as qste

    model = _mlp(3)
    qste.convert(model, include=["0", "2"], config={"seed": 5})
    coords = qste.QSTEOptimizer(model)
    assert coords.step_number == 0
    surfaces = qste.surfaces(model)
    before = [s.coordinate.clone() for s in surfaces]
    x = torch.randn(9, 24)
    model(x).square().mean().backward()
    # both surfaces stepped during backward, before step() is called
    assert len(fake.calls) == 2
    seeds = sorted(c["seed"] for c in fake.calls)
    assert seeds == [5, 5 + 1_000_003]
    assert all(c["step"] == 0 for c in fake.calls)
    flips = coords.step()
    assert coords.step_number == 1
    moved = sum(int((s.coordinate != b).sum()) for s, b in zip(surfaces, before))
    assert moved > 0
    assert flips == sum(int(np.unpackbits((oracle.pack_coordinate(b.numpy()) ^ s.packed_sign.numpy()),
                                          axis=1, bitorder="little")[:, :s.columns].sum())
                        for s, b in zip(surfaces, before))
    model(x).square().mean().backward()
    assert [c["step"] for c in fake.calls[2:]] == [1, 1]


def test_optimizer_flush_clamp_and_state_dict(fake):
    import qste_amd as qste

    model = _mlp(4)
    qste.convert(model, include=["0"])
    coords = qste.QSTEOptimizer(model)
    s = qste.surfaces(model)[0]
    with torch.no_grad():
        s.log_scale[0] = 10.0
        s.log_scale[1] = -50.0
    # a forward with no backward leaves a pending count; step() still clamps
    model(torch.randn(3, 24))
    coords.step()
    assert math.isclose(float(s.log_scale.detach()[0]), math.log(4.0), rel_tol=1e-6)
    assert math.isclose(float(s.log_scale.detach()[1]), math.log(1e-6), rel_tol=1e-6)
    # deferred evidence is applied by step() with the step number of that call
    coords.defer(True)
    model(torch.randn(5, 24)).sum().backward()
    assert fake.calls == []
    coords.step()
    assert [c["step"] for c in fake.calls] == [1]
    state = coords.state_dict()
    other = qste.QSTEOptimizer(model)
    other.load_state_dict(state)
    assert other.step_number == coords.step_number
    for k, v in coords.state[id(s)].items():
        assert torch.equal(other.state[id(s)][k], v)
    assert coords.state_bytes() > 0


@pytest.mark.parametrize("accum", [torch.float32, torch.float16])
def test_ledger_drain_never_returns_the_buffer_it_clears(accum):
    """A prepared buffer survives a drain with keep_buffer, emptied; what the
    drain returns is the evidence, in a tensor of its own (an fp32 buffer's
    .float() is the buffer itself, and clearing it would hand the step zeros)."""

    from qste_amd.surface import EvidenceLedger

    ledger = EvidenceLedger(accum)
    ledger.fix_buffer((3, 5), torch.device("cpu"))
    address = ledger.held.data_ptr()
    seen = []
    for _ in range(2):
        e = torch.randn(3, 5)
        seen.append(e.to(accum).float())
        ledger.open_uses += 1
        ledger.deliver(None, e)
    assert ledger.held.data_ptr() == address  # added in place
    out = ledger.drain(keep_buffer=True)
    assert out is not None and out.data_ptr() != address
    assert torch.allclose(out, (seen[0].to(accum) + seen[1].to(accum)).float())
    assert out.abs().sum() > 0
    assert ledger.held.data_ptr() == address and not ledger.held.any()
    assert ledger.drain(keep_buffer=False).abs().sum() == 0 and ledger.held is None


def test_ledger_sums_tied_uses_before_the_sink():
    from qste_amd.surface import EvidenceLedger

    got = []
    ledger = EvidenceLedger(torch.float32)
    ledger.sink = lambda owner, e: got.append((owner, e))
    parts = [torch.randn(2, 4) for _ in range(3)]
    ledger.open_uses = 3
    for i, e in enumerate(parts):
        ledger.deliver("s", e)
        assert len(got) == (1 if i == 2 else 0)
    assert got[0][0] == "s"
    assert torch.allclose(got[0][1], parts[0] + parts[1] + parts[2])
    # single use: straight through, no buffer
    ledger.open_uses = 1
    ledger.deliver("s", parts[0])
    assert torch.equal(got[1][1], parts[0]) and ledger.tied is None and ledger.held is None


def test_fp32_accumulation_steps_on_the_accumulated_evidence(fake):
    """prepare_accumulation with fp32 buffers: step() applies the sum of the
    microbatches' evidence, not a cleared buffer."""

    import qste_amd as qste

    model = _mlp(6)
    qste.convert(model, include=["0"], config={"evidence_accum_dtype": "fp32"})
    coords = qste.QSTEOptimizer(model)
    coords.prepare_accumulation()
    x = torch.randn(8, 24)
    for chunk in x.chunk(2):
        model(chunk).square().sum().backward()
    assert fake.calls == []
    coords.step()
    assert len(fake.calls) == 1
    applied = fake.calls[0]["evidence"]
    assert applied.abs().sum() > 0
    s = qste.surfaces(model)[0]
    assert s.ledger.held is not None and not s.ledger.held.any()


def test_export_packed_gives_the_same_forward(fake):
    import qste_amd as qste

    model = _mlp(6)
    qste.convert(model, include=["0", "2"])
    x = torch.randn(4, 24)
    with torch.no_grad():
        want = model(x)
    exported = qste.export_packed(model)
    assert isinstance(exported[0], qste.PackedLinear)
    with torch.no_grad():
        torch.testing.assert_close(exported(x), want)
    report = qste.memory_report(model)
    assert report["training_ratio"] > 1 and report["inference_ratio"] > report["training_ratio"]


def test_multirank_group_requires_an_explicit_reducer(monkeypatch, fake):
    import qste_amd as qste

    model = _mlp(7)
    qste.convert(model, include=["0"])
    monkeypatch.setattr(torch.distributed, "is_initialized", lambda: True)
    monkeypatch.setattr(torch.distributed, "get_world_size", lambda: 2)
    with pytest.raises(RuntimeError, match="gradient_reducer"):
        qste.QSTEOptimizer(model)
    assert qste.QSTEOptimizer(model, gradient_reducer=False).gradient_reducer is None


# ---------------------------------------------------------------------------
# packed activations: orchestration (src/qste/nn.py, convert.py:246-274)
# ---------------------------------------------------------------------------


def test_convert_swaps_activation_modules_by_mode(fake):
    import qste_amd as qste

    def model():
        return nn.Sequential(nn.Linear(8, 16), nn.GELU(approximate="tanh"), nn.Linear(16, 8),
                             nn.LeakyReLU(0.2), nn.Dropout(0.3), nn.Softplus(2.0))

    m = qste.convert(model())
    assert isinstance(m[1], qste.nn.GELU) and m[1].approximate == "tanh"
    assert isinstance(m[3], qste.nn.LeakyReLU) and m[3].negative_slope == 0.2
    assert isinstance(m[4], qste.nn.Dropout) and m[4].p == 0.3
    assert isinstance(m[5], qste.nn.Softplus) and m[5].beta == 2.0
    assert {"1", "3", "4", "5"} <= set(m._qste_converted)
    m = qste.convert(model(), activations="exact")
    assert type(m[1]) is nn.GELU and isinstance(m[3], qste.nn.LeakyReLU)
    m = qste.convert(model(), activations=False)
    assert type(m[1]) is nn.GELU and type(m[3]) is nn.LeakyReLU
    # idempotent
    m = qste.convert(model())
    again = qste.convert(m)
    assert isinstance(again[1], qste.nn.GELU)


def test_packed_activation_autograd_composition(fake):
    from qste_amd import nn as qnn

    x = torch.randn(6, 40, requires_grad=True)
    g = torch.randn(6, 40)
    qnn.relu(x).backward(g)
    assert torch.equal(x.grad, torch.where(x > 0, g, torch.zeros_like(g)))
    x.grad = None
    y = qnn.silu(x)
    assert torch.allclose(y, torch.nn.functional.silu(x), rtol=1e-6, atol=1e-6)
    y.backward(g)
    xs = x.detach()
    d = torch.sigmoid(xs) * (1 + xs * (1 - torch.sigmoid(xs)))
    scale = d.abs().amax(1, keepdim=True) / 127
    assert torch.allclose(x.grad, g * d, atol=float(scale.max() * g.abs().max()) * 0.51)
    # 0-d and 1-d inputs keep their shapes
    s = torch.tensor(0.5, requires_grad=True)
    assert qnn.gelu(s).shape == ()
    v = torch.randn(9, requires_grad=True)
    qnn.tanh(v).sum().backward()
    assert v.grad.shape == (9,)


def test_packed_activations_context_routes_marked_outputs_only(fake):
    import qste_amd as qste
    import torch.nn.functional as F

    model = qste.convert(nn.Sequential(nn.Linear(16, 24)), include=["0"])
    x = torch.randn(5, 16)
    seen = []

    def pack(t):
        seen.append(t.dtype)
        return t

    with qste.packed_activations():
        assert F.gelu is not qste.nn._TORCH_GELU
        hidden = model(x)
        with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
            F.gelu(hidden)
        assert torch.int8 in seen
        seen.clear()
        with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
            F.gelu(torch.randn(5, 24, requires_grad=True))
        assert torch.int8 not in seen
        # relu(...).square() fuses into one uint8-retaining op
        fused = qste.nn.relu(hidden).square()
        assert torch.allclose(fused, torch.relu(hidden).square())
        assert fused.grad_fn is not None and "ReluSquare" in type(fused.grad_fn).__name__
    assert F.gelu is qste.nn._TORCH_GELU and torch.relu is qste.nn._TORCH_TORCH_RELU


def test_checkpoint_layout_matches_the_reference(fake):
    """State-dict keys, dtypes and shapes of surface.py:67-74 / optim.py:212-232."""

    import qste_amd as qste

    model = qste.convert(nn.Sequential(nn.Linear(20, 12), nn.ReLU(), nn.Linear(12, 5, bias=False)))
    coords = qste.QSTEOptimizer(model)
    sd = model.state_dict()
    assert set(sd) == {"0.surface.coordinate", "0.surface.packed_sign", "0.surface.log_scale", "0.bias",
                       "2.surface.coordinate", "2.surface.packed_sign", "2.surface.log_scale"}
    assert (sd["0.surface.coordinate"].dtype, tuple(sd["0.surface.coordinate"].shape)) == (torch.int8, (12, 20))
    assert (sd["0.surface.packed_sign"].dtype, tuple(sd["0.surface.packed_sign"].shape)) == (torch.uint8, (12, 3))
    assert sd["0.surface.log_scale"].dtype == torch.float32
    osd = coords.state_dict()
    assert sorted(osd) == ["config", "step_number", "surfaces"]
    assert osd["config"] == qste.QSTEConfig().metadata()
    assert [sorted(e) for e in osd["surfaces"]] == [["col_v", "moment_q", "moment_scale", "row_v"]] * 2
    assert osd["surfaces"][1]["moment_scale"].shape == ((5 * 12 + 255) // 256,)
    restored = qste.convert(nn.Sequential(nn.Linear(20, 12), nn.ReLU(), nn.Linear(12, 5, bias=False)))
    restored.load_state_dict(sd)
    again = qste.QSTEOptimizer(restored)
    again.load_state_dict(osd)
    assert again.step_number == coords.step_number


def test_embedding_forward_and_evidence(fake):
    """functional.py:260-287 composition (the reference's test_autograd.py:231-245)."""

    import qste_amd as qste

    torch.manual_seed(12)
    surface = qste.Surface(torch.randn(40, 16))
    captured = []
    surface.route_evidence(lambda _, evidence: captured.append(evidence.clone()))
    ids = torch.randint(0, 40, (3, 5))
    grad = torch.randn(3, 5, 16)
    out = qste.qste_embedding(ids, surface)
    dense = torch.where(surface.coordinate >= 0, 1.0, -1.0) * surface.scale.detach()[:, None]
    assert torch.allclose(out, dense[ids], atol=1e-6)
    (out * grad).sum().backward()
    expected = torch.zeros(40, 16).index_add_(0, ids.reshape(-1), grad.reshape(-1, 16))
    assert len(captured) == 1
    assert torch.equal(captured[0], expected * surface.scale.detach()[:, None])
    inner = (expected.double() * torch.where(surface.coordinate >= 0, 1.0, -1.0).double()).sum(1).float()
    assert torch.allclose(surface.log_scale.grad, inner * surface.scale.detach(), rtol=1e-6, atol=1e-7)


def test_export_packed_turns_embeddings_into_packed_embeddings(fake):
    import qste_amd as qste

    torch.manual_seed(3)
    model = qste.convert(nn.Sequential(nn.Embedding(30, 8), nn.Linear(8, 4)))
    ids = torch.randint(0, 30, (2, 6))
    with torch.no_grad():
        expected = model(ids)
    exported = qste.export_packed(model)
    assert isinstance(exported[0], qste.PackedEmbedding) and isinstance(exported[1], qste.PackedLinear)
    with torch.no_grad():
        assert torch.allclose(exported(ids), expected, atol=1e-5)


def test_layers_reading_one_input_share_its_encoding(fake, monkeypatch):
    """A SwiGLU's gate and up projections read the same x: it is encoded once
    per forward, and again after a backward (no reuse across steps)."""

    import qste_amd as qste
    from qste_amd import kernels

    calls = []
    original = kernels.pack_affine_rows
    monkeypatch.setattr(kernels, "pack_affine_rows", lambda v: calls.append(v.shape) or original(v))
    model = qste.convert(nn.ModuleDict({"gate": nn.Linear(8, 16), "up": nn.Linear(8, 16),
                                        "down": nn.Linear(16, 8)}))
    x = torch.randn(5, 8)

    def forward():
        return model["down"](torch.nn.functional.silu(model["gate"](x)) * model["up"](x))

    out = forward()
    assert calls == [(5, 8), (5, 16)]
    out.sum().backward()
    calls.clear()
    forward()
    assert calls == [(5, 8), (5, 16)]
    # an in-place change of x invalidates the shared encoding
    calls.clear()
    model["gate"](x)
    x.add_(1.0)
    model["up"](x)
    assert calls == [(5, 8), (5, 8)]


def test_swiglu_hands_its_encoding_to_the_down_layer(fake, monkeypatch):
    """down(swiglu(gate(x), up(x))): x is encoded once (gate and up share
    it), h is encoded by the gate kernel and the down layer takes that
    encoding instead of encoding h again; the result and the gradients equal
    the torch gate's."""

    import qste_amd as qste
    from qste_amd import kernels

    calls = []
    real = kernels.pack_affine_rows
    monkeypatch.setattr(kernels, "pack_affine_rows", lambda v: (calls.append(tuple(v.shape)), real(v))[1])

    def layer(rows, cols, seed):
        g = torch.Generator().manual_seed(seed)
        coord = torch.randint(-127, 128, (rows, cols), generator=g, dtype=torch.int32).to(torch.int8)
        return qste.QSTELinear(qste.Surface.from_state(coord, torch.full((rows,), -3.0)), None)

    gate, up, down = layer(48, 16, 1), layer(48, 16, 2), layer(16, 48, 3)
    x = torch.randn(10, 16)

    def run(fused):
        calls.clear()
        xr = x.clone().requires_grad_(True)
        a, b = gate(xr), up(xr)
        h = qste.nn.swiglu(a, b) if fused else torch.nn.functional.silu(a) * b
        y = down(h)
        y.square().sum().backward()
        return y.detach(), xr.grad, list(calls)

    y0, g0, c0 = run(False)
    assert fake.offset_dots == [False, False, False]
    fake.offset_dots = []
    y1, g1, c1 = run(True)
    assert c0 == [(10, 16), (10, 48)]      # x once (shared), then h
    assert c1 == [(10, 16)]                 # h's encoding came from the gate kernel
    assert fake.swiglu_encodes == 1
    # the gate's backward summed dg and du for the gate and up layers, which
    # took those sums (checked against their own offsets); down summed its own
    assert fake.swiglu_sums == 1
    assert sorted(fake.offset_dots) == [False, True, True]
    assert torch.allclose(y0, y1, rtol=1e-6, atol=1e-6)
    assert torch.allclose(g0, g1, rtol=1e-5, atol=1e-6)

    # the gate layer's output also feeds the loss directly: autograd sums
    # its two gradients into a new tensor, so the offer for it is not taken;
    # the pass's end drops it (no gradient is held afterwards)
    from qste_amd import functional

    fake.offset_dots = []
    xr = x.clone().requires_grad_(True)
    a, b = gate(xr), up(xr)
    (down(qste.nn.swiglu(a, b)).square().sum() + a.sum()).backward()
    assert sorted(fake.offset_dots) == [False, False, True]
    assert functional._offers == {}


def test_swiglu_mlp_node_composes_the_layers(fake, monkeypatch):
    """qste_amd.nn.swiglu_mlp as one node (its eligibility check relaxed to
    CPU tensors so the oracle-backed operators run it): the same output as
    the layers called one by one, each surface's evidence once (the same
    evidence), the gate and up layers' backward as one call over both, and
    the steps inside backward reading each layer's signs only after every
    product that needs them."""

    import qste_amd as qste
    from qste_amd import functional

    monkeypatch.setattr(functional, "swiglu_mlp_fusable",
                        lambda x, g, u, d: x.dtype == torch.bfloat16 and x.shape[-1] % 64 == 0)

    def layer(rows, cols, seed):
        g = torch.Generator().manual_seed(seed)
        coord = torch.randint(-127, 128, (rows, cols), generator=g, dtype=torch.int32).to(torch.int8)
        return qste.QSTELinear(qste.Surface.from_state(coord, torch.full((rows,), -3.0)), None)

    def run(node):
        gate, up, down = layer(128, 64, 1), layer(128, 64, 2), layer(64, 128, 3)
        # the steps run inside backward, rewriting each surface's signs as its
        # evidence arrives: a product that read a layer's signs after that
        # layer's delivery would see the stepped ones
        coords = qste.QSTEOptimizer([gate.surface, up.surface, down.surface])
        got = {}
        for name, m in (("gate", gate), ("up", up), ("down", down)):
            m.surface.route_evidence(lambda s, e, name=name: (got.__setitem__(name, e.clone()), coords._apply(s, e)))
        x = torch.randn(10, 64, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).requires_grad_(True)
        if node:
            y = qste.nn.swiglu_mlp(x, gate, up, down)
        else:
            y = down(qste.nn.swiglu(gate(x), up(x)))
        y.float().square().sum().backward()
        return y.detach(), x.grad, got, [m.surface.log_scale.grad.clone() for m in (gate, up, down)]

    y0, g0, e0, s0 = run(False)
    fake.backward_calls = []
    fake.swiglu_sums = 0
    y1, g1, e1, s1 = run(True)
    assert fake.swiglu_sums == 1
    # the down layer, then gate and up in one call; both form input gradients
    assert fake.backward_calls == [True, True]
    assert torch.equal(y0, y1)
    assert torch.allclose(g0.float(), g1.float(), rtol=2e-2, atol=2e-2)
    for name in ("gate", "up", "down"):
        assert torch.allclose(e0[name], e1[name], rtol=1e-4, atol=1e-6), name
    for a, b in zip(s0, s1):
        assert torch.allclose(a, b, rtol=1e-4, atol=1e-6)
