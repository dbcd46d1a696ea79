"""Checkpoint interchange and resume, on the GPU.

The on-disk format is the reference's (``src/qste/surface.py:67-74``,
``src/qste/optim.py:212-232``, ``src/qste/modules.py:100-112``):

* a converted layer ``name`` holds ``name.surface.coordinate`` int8 [R, C],
  ``name.surface.packed_sign`` uint8 [R, ceil(C/8)] (LSB first, set = +1),
  ``name.surface.log_scale`` fp32 [R] and ``name.bias`` fp32 [R];
* ``QSTEOptimizer.state_dict()`` is ``{"config": QSTEConfig fields,
  "step_number": int, "surfaces": [{"moment_q": int8 [R, C], "moment_scale":
  fp16 [ceil(RC/256)], "row_v": fp16 [R], "col_v": fp16 [C]}, ...]}`` in
  surface order;
* ``export_packed`` leaves ``PackedLinear`` buffers ``packed_sign``,
  ``scale`` (fp32) and ``bias``.

Checked here as the reference's tests check it (``tests/test_convert.py:
125-160``, ``tests/test_learning.py:260-300``,
``tests/test_host_frameworks.py:112-140``): a state dict round-trips through
``torch.save`` / ``torch.load(weights_only=True)`` with the same outputs;
training resumed from a checkpoint takes the same next step bit for bit;
recomputation under gradient checkpointing leaves the same signs and flip
count; and a checkpoint written field by field in the reference's layout (no
qste_amd object involved) loads and reproduces the model.
"""

from __future__ import annotations

import io

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


class Tiny(nn.Module):
    def __init__(self, dim=64, hidden=128, out=16):
        super().__init__()
        self.fc1 = nn.Linear(dim, hidden)
        self.act = nn.ReLU()
        self.fc2 = nn.Linear(hidden, out, bias=False)

    def forward(self, x):
        return self.fc2(self.act(self.fc1(x)))


def _build(seed=13, lr=6.0):
    import qste_amd as qste

    torch.manual_seed(seed)
    model = qste.convert(Tiny()).to(DEV)
    return model, qste.QSTEOptimizer(model, config={"coordinate_lr": lr})


def _data(seed=14):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(32, 64, generator=g).to(DEV), torch.randint(0, 16, (32,), generator=g).to(DEV)


def _roundtrip(obj):
    buf = io.BytesIO()
    torch.save(obj, buf)
    buf.seek(0)
    return torch.load(buf, weights_only=True)


def test_state_dict_layout_is_the_reference_format():
    import qste_amd as qste

    model, coords = _build()
    sd = model.state_dict()
    assert set(sd) == {"fc1.surface.coordinate", "fc1.surface.packed_sign", "fc1.surface.log_scale",
                       "fc1.bias", "fc2.surface.coordinate", "fc2.surface.packed_sign",
                       "fc2.surface.log_scale"}
    assert sd["fc1.surface.coordinate"].dtype == torch.int8 and sd["fc1.surface.coordinate"].shape == (128, 64)
    assert sd["fc1.surface.packed_sign"].dtype == torch.uint8 and sd["fc1.surface.packed_sign"].shape == (128, 8)
    assert sd["fc1.surface.log_scale"].dtype == torch.float32 and sd["fc1.surface.log_scale"].shape == (128,)
    # packed_sign is the LSB-first sign of the coordinate (zero counts as +1)
    coord = sd["fc2.surface.coordinate"].cpu()
    bits = ((sd["fc2.surface.packed_sign"].cpu()[:, :, None] >> torch.arange(8)) & 1).reshape(16, -1)
    assert torch.equal(bits[:, :128].bool(), coord >= 0)
    osd = coords.state_dict()
    assert osd["config"] == qste.QSTEConfig(coordinate_lr=6.0).metadata()
    assert osd["step_number"] == 0
    first = osd["surfaces"][0]
    assert set(first) == {"moment_q", "moment_scale", "row_v", "col_v"}
    assert first["moment_q"].dtype == torch.int8 and first["moment_q"].shape == (128, 64)
    assert first["moment_scale"].dtype == torch.float16 and first["moment_scale"].shape == (32,)
    assert first["row_v"].shape == (128,) and first["col_v"].shape == (64,)


def test_state_dict_roundtrips_through_torch_save():
    model, _ = _build()
    x, _ = _data()
    expected = model(x)
    restored, _ = _build(seed=99)
    restored.load_state_dict(_roundtrip(model.state_dict()))
    assert torch.equal(restored(x), expected)


def test_training_resumes_from_a_checkpoint_bit_for_bit():
    import qste_amd as qste

    model, coords = _build()
    x, labels = _data()
    for _ in range(5):
        F.cross_entropy(model(x), labels).backward()
        coords.step()
        model.zero_grad(set_to_none=True)
    saved_model = _roundtrip(model.state_dict())
    saved_opt = _roundtrip(coords.state_dict())
    assert saved_opt["step_number"] == 5

    restored, restored_coords = _build(seed=99)
    restored.load_state_dict(saved_model)
    restored_coords.load_state_dict(saved_opt)
    for target in (model, restored):
        F.cross_entropy(target(x), labels).backward()
    coords.step()
    restored_coords.step()
    moved = 0
    for a, b in zip(qste.surfaces(model), qste.surfaces(restored)):
        assert torch.equal(a.coordinate, b.coordinate)
        assert torch.equal(a.packed_sign, b.packed_sign)
        assert torch.equal(a.log_scale.grad, b.log_scale.grad)
    for sa, sb in zip(coords.state_dict()["surfaces"], restored_coords.state_dict()["surfaces"]):
        for key in sa:
            assert torch.equal(sa[key], sb[key]), key
        moved += int(sa["moment_q"].abs().sum())
    assert moved > 0


def test_a_reference_layout_checkpoint_loads():
    """Field-by-field in the reference's format, built from plain tensors."""

    import qste_amd as qste

    g = torch.Generator().manual_seed(3)
    coord1 = torch.randint(-127, 128, (128, 64), generator=g, dtype=torch.int32).to(torch.int8)
    coord2 = torch.randint(-127, 128, (16, 128), generator=g, dtype=torch.int32).to(torch.int8)

    def pack(c):
        bits = (c >= 0).to(torch.uint8).reshape(c.shape[0], -1, 8)
        return (bits << torch.arange(8, dtype=torch.uint8)).sum(-1, dtype=torch.uint8)

    sd = {
        "fc1.surface.coordinate": coord1, "fc1.surface.packed_sign": pack(coord1),
        "fc1.surface.log_scale": torch.full((128,), -3.0), "fc1.bias": torch.linspace(-1, 1, 128),
        "fc2.surface.coordinate": coord2, "fc2.surface.packed_sign": pack(coord2),
        "fc2.surface.log_scale": torch.full((16,), -2.0),
    }
    model, _ = _build()
    model.load_state_dict(_roundtrip(sd))
    assert torch.equal(model.fc1.surface.packed_sign.cpu(),
                       qste.kernels.pack_coordinate(coord1.to(DEV)).cpu())
    x, _ = _data()
    with torch.no_grad():
        h = torch.relu(x @ (torch.where(coord1 >= 0, 1.0, -1.0).to(DEV) * torch.exp(torch.tensor(-3.0))).t()
                       + torch.linspace(-1, 1, 128, device=DEV))
        ref = h @ (torch.where(coord2 >= 0, 1.0, -1.0).to(DEV) * torch.exp(torch.tensor(-2.0))).t()
        out = model(x)
    assert torch.allclose(out, ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("reentrant", [False, True])
def test_gradient_checkpointing_gives_the_same_signs(reentrant):
    """Recomputation runs forward twice; the signs and flips must not depend on it.

    As the reference checks it (tests/test_host_frameworks.py:112-140): the
    packed signs and the flip count.  Under non-reentrant checkpointing the
    first forward also counts, so the evidence waits in the surface's
    accumulation buffer (fp16 by the config, surface.py:140-168) until
    QSTEOptimizer.step() flushes it: a coordinate may then sit one step from
    where the immediate path puts it, but no sign differs.  Under reentrant
    checkpointing the first forward runs without grad and the path is the
    immediate one, so the coordinates agree as well.
    """

    import qste_amd as qste

    def run(checkpointed):
        torch.manual_seed(4)
        block = qste.convert(nn.Sequential(nn.Linear(32, 32), nn.ReLU(), nn.Linear(32, 32))).to(DEV)
        coords = qste.QSTEOptimizer(block, config={"coordinate_lr": 8.0})
        x = torch.randn(8, 32, generator=torch.Generator().manual_seed(5)).to(DEV).requires_grad_(True)
        out = torch.utils.checkpoint.checkpoint(block, x, use_reentrant=reentrant) if checkpointed else block(x)
        out.square().mean().backward()
        flips = coords.step()
        surfaces = qste.surfaces(block)
        return [s.packed_sign.clone() for s in surfaces], [s.coordinate.clone() for s in surfaces], flips

    plain_signs, plain_coords, plain_flips = run(False)
    signs, coords, flips = run(True)
    assert plain_flips > 0
    assert flips == plain_flips
    for a, b in zip(plain_signs, signs):
        assert torch.equal(a, b)
    if reentrant:
        for a, b in zip(plain_coords, coords):
            assert torch.equal(a, b)
    else:
        for a, b in zip(plain_coords, coords):
            assert int((a.int() - b.int()).abs().max()) <= 1


def test_more_forwards_than_backwards_still_applies_evidence():
    """A discarded forward leaves the count unbalanced; step() flushes anyway."""

    import qste_amd as qste

    torch.manual_seed(6)
    model = qste.convert(nn.Sequential(nn.Linear(16, 16))).to(DEV)
    coords = qste.QSTEOptimizer(model, config={"coordinate_lr": 8.0})
    surface = qste.surfaces(model)[0]
    model(torch.randn(4, 16, device=DEV))  # never backwarded
    model(torch.randn(4, 16, device=DEV)).sum().backward()
    before = surface.packed_sign.clone()
    assert coords.step() > 0
    assert not torch.equal(before, surface.packed_sign)


def test_export_packed_keeps_outputs_and_drops_training_state():
    import qste_amd as qste

    model, _ = _build()
    model.eval()
    x, _ = _data()
    with torch.no_grad():
        expected = model(x)
    exported = qste.export_packed(model)
    with torch.no_grad():
        assert torch.allclose(exported(x), expected, rtol=1e-5, atol=1e-5)
    assert not any(isinstance(m, qste.Surface) for m in exported.modules())
    assert isinstance(exported.fc1, qste.PackedLinear)
    sd = _roundtrip(exported.state_dict())
    assert set(sd) == {"fc1.packed_sign", "fc1.scale", "fc1.bias", "fc2.packed_sign", "fc2.scale"}
    assert sd["fc1.scale"].dtype == torch.float32
