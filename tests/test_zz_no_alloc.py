"""The coordinate step's no-allocation entry point against the workspace one.

``qste_coordinate_update_static`` runs the same kernels as
``qste_coordinate_update`` on a static device array instead of a caller
workspace.  Through the C ABI, on identical copies of the state, both must
give the same coordinates, packed signs, momentum, fp16 statistics and flip
count, bit for bit: first on a config-4 surface (14336 x 4096, row kernels),
then, reusing the array, on a smaller ragged one (generic kernels) -- so a
stale byte left by the first call would show in the second.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
KEYS = ("coordinate", "packed", "moment_q", "moment_scale", "row_v", "col_v")


@pytest.fixture(autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from qste_amd import kernels

    assert kernels.native_available(), kernels.status()


def _state(rows, cols, block, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    coord = torch.randint(-127, 128, (rows, cols), generator=g, device=DEV, dtype=torch.int32).to(torch.int8)
    from qste_amd import kernels

    blocks = (rows * cols + block - 1) // block
    return {
        "coordinate": coord,
        "packed": kernels.pack_coordinate(coord),
        "moment_q": torch.randint(-127, 128, (rows, cols), generator=g, device=DEV,
                                  dtype=torch.int32).to(torch.int8),
        "moment_scale": (torch.rand(blocks, generator=g, device=DEV) * 0.01 + 1e-3).to(torch.float16),
        "row_v": (torch.rand(rows, generator=g, device=DEV) * 1e-3).to(torch.float16),
        "col_v": (torch.rand(cols, generator=g, device=DEV) * 1e-3).to(torch.float16),
    }


def _call(lib, static, ev, st, rows, cols, block, step, flips, stream):
    args = [ev.data_ptr(), st["coordinate"].data_ptr(), st["packed"].data_ptr(), st["moment_q"].data_ptr(),
            st["moment_scale"].data_ptr(), st["row_v"].data_ptr(), st["col_v"].data_ptr(), rows, cols,
            0.9, 0.99, 2.0, 0.3, block, 77, step, None, flips.data_ptr(), None]
    if static:
        return lib.qste_coordinate_update_static(*args, stream)
    need = lib.qste_coordinate_update_workspace_bytes(rows, cols, block)
    work = torch.empty(need, dtype=torch.uint8, device=DEV)
    rc = lib.qste_coordinate_update(*args, work.data_ptr(), need, stream)
    torch.cuda.synchronize()
    return rc


def test_static_entry_matches_the_workspace_entry_twice():
    from qste_amd.kernels import _lib

    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    limit = lib.qste_coordinate_update_static_limit()
    assert limit == 16 << 20
    # a surface whose workspace exceeds the static array is refused, nothing written
    big_rows, big_cols = 28672, 8192
    assert lib.qste_coordinate_update_workspace_bytes(big_rows, big_cols, 256) > limit
    one = torch.zeros(1, device=DEV)
    assert lib.qste_coordinate_update_static(
        one.data_ptr(), one.data_ptr(), one.data_ptr(), one.data_ptr(), one.data_ptr(), one.data_ptr(),
        one.data_ptr(), big_rows, big_cols, 0.9, 0.99, 2.0, 1.0, 256, 1, 0, None, None, None, stream) == -7
    for rows, cols, block, step in ((14336, 4096, 256, 3), (300, 520, 96, 70)):
        print(f"no-alloc step {rows}x{cols} block {block} step {step}", flush=True)
        assert lib.qste_coordinate_update_workspace_bytes(rows, cols, block) <= limit
        ev = torch.randn(rows, cols, generator=torch.Generator(device=DEV).manual_seed(rows), device=DEV) * 0.05
        ref = _state(rows, cols, block, rows + cols)
        mine = {k: v.clone() for k, v in ref.items()}
        f_ref = torch.full((), -1, dtype=torch.int64, device=DEV)
        f_mine = torch.full((), -1, dtype=torch.int64, device=DEV)
        assert _call(lib, False, ev, ref, rows, cols, block, step, f_ref, stream) == 0
        assert _call(lib, True, ev, mine, rows, cols, block, step, f_mine, stream) == 0
        torch.cuda.synchronize()
        for k in KEYS:
            assert torch.equal(mine[k].view(torch.uint8), ref[k].view(torch.uint8)), (rows, cols, k)
        assert int(f_mine.item()) == int(f_ref.item()) and int(f_ref.item()) > 0
