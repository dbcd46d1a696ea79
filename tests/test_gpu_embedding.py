"""Binary embedding on the GPU: lookup and evidence against the oracle.

* lookup -- bit-exact against ``oracle/embedding.py`` (+-scale per element);
* backward -- the evidence bit-exact against the oracle's token-order fp32
  sums (a sequential ``index_add_``), including repeated ids and rows no token
  touches; the scale gradient within 1e-6 relative (a float64 row sum here,
  torch's fp32 reduction in the reference);
* at a GPT-2-sized table (50257 x 768, 8192 tokens) against torch's own CPU
  ``index_add_``, bit for bit;
* out-of-range ids raise, and a converted ``nn.Embedding`` trains and exports.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from oracle import embedding as oe

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def K():
    from qste_amd import kernels

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return kernels


def _table(rows, cols, seed):
    rng = np.random.default_rng(seed)
    coord = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    packed = oracle.pack_coordinate(coord)
    scale = (rng.random(rows) + 0.1).astype(np.float32)
    return packed, scale


@pytest.mark.parametrize("rows,cols", [(40, 16), (4096, 129), (7, 1), (300, 64), (1000, 771)])
def test_lookup_matches_oracle(K, rows, cols):
    print(f"lookup {rows}x{cols}", flush=True)
    packed, scale = _table(rows, cols, rows + cols)
    ids = np.random.default_rng(1).integers(0, rows, size=(7, 11))
    got = K.packed_embedding(torch.from_numpy(ids).to(DEV), torch.from_numpy(packed).to(DEV),
                             torch.from_numpy(scale).to(DEV), cols)
    assert got.shape == (7, 11, cols) and got.dtype == torch.float32
    assert np.array_equal(got.cpu().numpy(), oe.lookup(ids, packed, scale, cols))
    got16 = K.packed_embedding(torch.from_numpy(ids).to(DEV), torch.from_numpy(packed).to(DEV),
                               torch.from_numpy(scale).to(DEV).bfloat16(), cols)
    assert got16.dtype == torch.bfloat16
    ref16 = oe.lookup(ids, packed, torch.from_numpy(scale).bfloat16().float().numpy(), cols)
    assert np.array_equal(got16.float().cpu().numpy(), ref16)


@pytest.mark.parametrize("rows,cols,count,vocab_used", [(40, 16, 15, 40), (300, 64, 500, 20),
                                                        (1000, 771, 64, 1000), (5, 8, 0, 5),
                                                        # three 8-bit sort passes, a ragged last block,
                                                        # many tokens per id (order within an id matters)
                                                        (70000, 64, 20001, 300), (70000, 32, 5000, 70000)])
def test_backward_matches_oracle(K, rows, cols, count, vocab_used):
    print(f"backward {rows}x{cols} count={count}", flush=True)
    packed, scale = _table(rows, cols, 7)
    rng = np.random.default_rng(count)
    ids = rng.integers(0, vocab_used, size=(count,))
    grad = (rng.standard_normal((count, cols)) * 2).astype(np.float32)
    ev, gs = K.embedding_backward(torch.from_numpy(ids).to(DEV), torch.from_numpy(grad).to(DEV),
                                  torch.from_numpy(packed).to(DEV), torch.from_numpy(scale).to(DEV), cols)
    rev, rgs = oe.backward(ids, grad, packed, scale, cols)
    assert np.array_equal(ev.cpu().numpy(), rev)
    assert np.allclose(gs.cpu().numpy(), rgs, rtol=1e-6, atol=1e-6)


def test_backward_at_gpt2_vocabulary_matches_torch_cpu_index_add(K):
    rows, cols, count = 50257, 768, 8192
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, rows, (count,), generator=g)
    ids[:512] = 50256  # a heavily repeated id (an end-of-text token)
    grad = torch.randn(count, cols, generator=g).bfloat16()
    coord = torch.randint(-127, 128, (rows, cols), generator=g, dtype=torch.int32).to(torch.int8)
    packed = K.pack_coordinate(coord.to(DEV))
    scale = (torch.rand(rows, generator=g) + 0.1)
    ev, gs = K.embedding_backward(ids.to(DEV), grad.to(DEV), packed, scale.to(DEV), cols)
    e0 = torch.zeros(rows, cols).index_add_(0, ids, grad.float())
    assert torch.equal(ev.cpu(), e0 * scale[:, None])
    sign = torch.where(coord >= 0, 1.0, -1.0).double()
    ref = (e0.double() * sign).sum(1).float()
    assert torch.allclose(gs.cpu(), ref, rtol=1e-6, atol=1e-5)


def test_out_of_range_ids_raise(K):
    packed, scale = _table(10, 8, 2)
    p, s = torch.from_numpy(packed).to(DEV), torch.from_numpy(scale).to(DEV)
    for bad in (10, -1):
        with pytest.raises(IndexError):
            K.packed_embedding(torch.tensor([0, bad], device=DEV), p, s, 8)


def test_converted_embedding_trains_and_exports():
    import qste_amd as qste

    torch.manual_seed(0)
    model = qste.convert(nn.Sequential(nn.Embedding(64, 32), nn.Linear(32, 64))).to(DEV)
    assert isinstance(model[0], qste.QSTEEmbedding)
    coords = qste.QSTEOptimizer(model, config={"coordinate_lr": 8.0})
    before = model[0].surface.coordinate.clone()
    ids = torch.randint(0, 64, (16, 8), device=DEV)
    torch.nn.functional.cross_entropy(model(ids).reshape(-1, 64), ids.reshape(-1)).backward()
    assert model[0].surface.log_scale.grad is not None
    flips = coords.step()
    assert flips >= 0 and not torch.equal(before, model[0].surface.coordinate)
    model.eval()
    with torch.no_grad():
        expected = model(ids)
        exported = qste.export_packed(model)
        assert isinstance(exported[0], qste.PackedEmbedding)
        assert torch.allclose(exported(ids), expected, rtol=1e-5, atol=1e-5)
