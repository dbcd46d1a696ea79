"""The BASELINE configurations 1, 2 and 3 end to end, at their real shapes.

* config 1 -- one QSTE Linear 2048 -> 2048 in fp32 (256 tokens, MSE against a
  target, backward, one coordinate step): forward, input gradient, evidence
  and bias gradient against the float64 oracle (rel-L2 <= 1e-5), the step on
  the GPU's own evidence bit-exact against the oracle;

* config 2 -- the converted ReLU MLP (1024 -> 4096 -> 1024, bf16, 8192
  tokens): each layer's forward against a float64 product over the same signs
  and scales rounded to bf16 (rel-L2 <= 1e-3), the input gradient of the whole
  block against float32 autograd through the dense weights, and one
  fwd+bwd+coordinate step that moves the coordinates with packed == pack(coord);
* config 3 -- GPT-2 small (12 layers, d=768, vocab 50257, batch 8 x 1024),
  MLPs converted: one AdamW + QSTEOptimizer training step with a finite loss,
  every MLP surface moved and its packed signs consistent, attention weights
  updated, and the first MLP layer's forward at the real shape against float64.

The workloads are bench.py's own (``relu_mlp``, ``GPT2Small``).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _rel(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm())


def _dense(layer):
    sign = torch.where(layer.surface.coordinate >= 0, 1.0, -1.0).double()
    return sign * layer.scale.detach().double()[:, None]


def _reference_linear(layer, x):
    y = x.double() @ _dense(layer).t()
    if layer.bias is not None:
        y = y + layer.bias.detach().double()
    return y


def _packed_of(coord):
    from qste_amd import kernels

    return kernels.pack_coordinate(coord)


@pytest.mark.parametrize("base", [0, 100])
def test_config1_single_linear_fp32(base):
    """Config 1's workload (2048 -> 2048, 256 tokens, fp32, MSE against a
    target, backward, one coordinate step from fresh state), with the
    recipe's seeds 0..3 (offset by ``base``): y, the input gradient and the
    evidence within rel-L2 1e-5 of the float64 oracle, and the step on the
    GPU's own evidence bit-exact against the oracle's."""

    import numpy as np

    import oracle
    import qste_amd as qste
    from bench import cfg1_workload

    print(f"config 1 base {base}", flush=True)
    layer, x, target = cfg1_workload(DEV, base)
    surface = layer.surface
    coords = qste.QSTEOptimizer([surface])
    seen = []
    apply = coords._apply
    surface.route_evidence(lambda s, e: (seen.append(e.detach().clone()), apply(s, e)))
    packed = surface.packed_sign.detach().cpu().numpy()
    coord0 = surface.coordinate.detach().cpu().numpy().copy()
    scale = layer.scale.detach().cpu().numpy()
    xr = x.clone().requires_grad_(True)
    y = layer(xr)
    loss = F.mse_loss(y, target)
    loss.backward()
    flips = coords.step()
    torch.cuda.synchronize()

    xs = x.cpu().numpy()
    want_y = oracle.linear_fwd(xs, packed, scale, np.zeros(2048, np.float32), 2048)
    assert _rel(y.detach().cpu(), torch.from_numpy(want_y)) <= 1e-5
    dy = (2.0 / y.numel()) * (y.detach() - target)
    dy_np = dy.cpu().numpy()
    want_dx = oracle.linear_dgrad(dy_np, packed, 2048, scale)
    assert _rel(xr.grad.cpu(), torch.from_numpy(want_dx)) <= 1e-5
    bits, off, xsc = oracle.pack_affine_rows(xs)
    want_e = oracle.decoded_evidence(dy_np, bits, off, xsc, 2048) * scale.astype(np.float64)[:, None]
    assert len(seen) == 1
    assert _rel(seen[0].cpu(), torch.from_numpy(want_e)) <= 1e-5
    assert _rel(layer.bias.grad.cpu(), torch.from_numpy(dy_np.astype(np.float64).sum(0))) <= 1e-5

    state = oracle.fresh_state(coord0, 256)
    oflips = oracle.coordinate_update(seen[0].cpu().numpy(), state, beta1=0.9, beta2=0.99, update_clip=2.0,
                                      coordinate_lr=1.0, block_size=256, seed=1, step=0)
    assert np.array_equal(surface.coordinate.cpu().numpy(), state["coordinate"])
    assert np.array_equal(surface.packed_sign.cpu().numpy(), state["packed"])
    got = coords.state[id(surface)]
    for k in ("moment_q", "moment_scale", "row_v", "col_v"):
        assert np.array_equal(got[k].cpu().numpy().view(np.uint8), state[k].view(np.uint8)), k
    assert flips == oflips and flips > 0


def test_config2_relu_mlp():
    import qste_amd as qste
    from bench import relu_mlp

    model = relu_mlp(device=DEV)
    g = torch.Generator(device=DEV).manual_seed(0)
    x = torch.randn(8192, 1024, generator=g, device=DEV).to(torch.bfloat16)
    dy = torch.randn(8192, 1024, generator=g, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        h = model[0](x)
        ref_h = _reference_linear(model[0], x)
        assert _rel(h, ref_h.to(torch.bfloat16)) <= 1e-3
        y = model[2](torch.relu(h))
        assert _rel(y, _reference_linear(model[2], torch.relu(h)).to(torch.bfloat16)) <= 1e-3

    # input gradient of the block against float32 autograd through dense weights
    xr = x.float().requires_grad_(True)
    w1, w2 = _dense(model[0]).float(), _dense(model[2]).float()
    b1, b2 = model[0].bias.detach().float(), model[2].bias.detach().float()
    (F.linear(torch.relu(F.linear(xr, w1, b1)), w2, b2) * dy.float()).sum().backward()

    coords = qste.QSTEOptimizer(model)
    surfaces = qste.surfaces(model)
    before = [s.coordinate.clone() for s in surfaces]
    # the signs the backward multiplies by (the optimizer moves the
    # coordinates, and so the packed signs, inside the backward)
    signs = {id(layer): layer.surface.packed_sign.cpu().numpy().copy() for layer in (model[0], model[2])}
    xq = x.clone().requires_grad_(True)
    h = model[0](xq)
    r = model[1](h)
    r.retain_grad()
    model[2](r).backward(dy)
    assert _rel(xq.grad, xr.grad) <= 1.5e-2  # against fp32 autograd through dense weights
    # each layer's input gradient against the operand-rounded float64 oracle
    # (the row scale rounded to bf16 inside the contraction, as the MFMA
    # operand holds it; the product rounded to bf16), on 512 sampled tokens:
    # the second layer's on the upstream gradient, the first layer's on the
    # ReLU's output gradient the block formed
    tok = np.sort(np.random.default_rng(2).choice(8192, 512, replace=False))

    def dgrad_oracle(layer, grad, columns):
        scale = oracle.round_bf16(layer.scale.detach().float().cpu().numpy())
        want = oracle.linear_dgrad(grad, signs[id(layer)], columns, scale)
        return torch.from_numpy(want.astype(np.float32)).to(torch.bfloat16).double()

    dy_s = np.ascontiguousarray(dy.float().cpu().numpy()[tok])
    assert _rel(r.grad[tok].cpu(), dgrad_oracle(model[2], dy_s, 4096)) <= 1e-3
    dh = torch.where(h > 0, r.grad, torch.zeros_like(r.grad))
    dh_s = np.ascontiguousarray(dh.float().cpu().numpy()[tok])
    assert _rel(xq.grad[tok].cpu(), dgrad_oracle(model[0], dh_s, 1024)) <= 1e-3
    flips = coords.step()
    assert flips > 0
    for s, b in zip(surfaces, before):
        assert not torch.equal(s.coordinate, b)
        assert torch.equal(s.packed_sign, _packed_of(s.coordinate))
        assert int(s.coordinate.abs().max()) <= 127


def test_config3_gpt2_small_training_step():
    import qste_amd as qste
    from bench import GPT2Small

    model = GPT2Small(device=DEV)
    mlp_layers = [m for m in model.modules() if isinstance(m, qste.QSTELinear)]
    assert len(mlp_layers) == 24
    assert all(isinstance(b.mlp[1], qste.nn.GELU) for b in model.blocks)
    adam = torch.optim.AdamW(list(qste.continuous_parameters(model)), lr=1e-3)
    coords = qste.QSTEOptimizer(model)
    g = torch.Generator(device=DEV).manual_seed(1)
    ids = torch.randint(0, 50257, (8, 1024), generator=g, device=DEV)

    # the first MLP layer at its real shape (8192 x 768 -> 3072)
    with torch.no_grad():
        x = torch.randn(8192, 768, generator=g, device=DEV).to(torch.bfloat16)
        fc = model.blocks[0].mlp[0]
        assert _rel(fc(x), _reference_linear(fc, x).to(torch.bfloat16)) <= 1e-3

    before = [s.coordinate.clone() for s in qste.surfaces(model)]
    qkv_before = model.blocks[0].qkv.weight.detach().clone()
    logits = model(ids[:, :-1])
    loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]).float(), ids[:, 1:].reshape(-1))
    assert torch.isfinite(loss)
    assert abs(float(loss) - 10.8) < 1.5  # ~log(50257) at random init
    loss.backward()
    adam.step()
    flips = coords.step()
    assert flips > 0
    for s, b in zip(qste.surfaces(model), before):
        assert not torch.equal(s.coordinate, b)
        assert torch.equal(s.packed_sign, _packed_of(s.coordinate))
    assert not torch.equal(model.blocks[0].qkv.weight, qkv_before)
