"""Write the golden input/output vectors under tests/golden/.

Run once, in the build container, where the reference checkout is mounted:

    python tests/golden/make_golden.py /root/reference

It imports the reference's *specification* backend
(``src/qste/kernels/fallback.py``) and its hash module
(``src/qste/kernels/stream.py``) to compute outputs for seeded inputs, and
stores inputs and outputs as compressed ``.npz`` data. Only the functions
whose outputs nothing else pins exactly are generated this way:

* the hash (``stream.scramble``/``seed_hash``/``step_hash``/``uniform``): the
  reference's tests hold no literal known-answer values;
* ``fallback.pack_affine_rows``: bits of elements within rounding of the row
  mean depend on torch's reduction order;
* ``fallback.coordinate_update``: integer outputs depend on torch's fp32
  reduction order and fused multiply-adds;
* small ``packed_linear_affine`` / ``packed_transpose`` /
  ``evidence_from_packed`` / ``packed_row_inner`` cases, as an extra anchor
  for the float products (which float64 dense algebra also pins).

Nothing here is loaded by the GPU tests at run time except the ``.npz``
files; the reference itself never leaves this container.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def _load_reference(root: Path):
    sys.path.insert(0, str(root / "src"))
    from qste.kernels import fallback, stream  # noqa: E402

    return fallback, stream


def _hash_vectors(stream) -> dict:
    values = [0, 1, 2, 61, 255, 4095, 2**16, 2**24, 2**31, 2**31 + 7, 2**32 - 1,
              12345678, 987654321]
    rng = np.random.default_rng(20240501)
    values += [int(v) for v in rng.integers(0, 2**32, size=243, dtype=np.uint64)]
    scrambled = [stream.scramble(v) for v in values]
    seeds = [0, 1, 7, 17, 99, 1000004, 2**31 + 5, 2**31 + 11, 3_000_010]
    steps = [0, 1, 3, 5, 7, 99, 1234, 2**32 + 3]
    indices = [0, 1, 2, 63, 4095, 2**20 + 17, 2**33 + 5, 58_720_255, 2**32 - 1]
    uni = np.zeros((len(seeds), len(steps), len(indices)), dtype=np.float32)
    for a, seed in enumerate(seeds):
        for b, step in enumerate(steps):
            for c, index in enumerate(indices):
                uni[a, b, c] = stream.uniform(seed, step, index)
    return {
        "values": np.array(values, dtype=np.uint64),
        "scrambled": np.array(scrambled, dtype=np.uint64),
        "seeds": np.array(seeds, dtype=np.uint64),
        "seed_hash": np.array([stream.seed_hash(s) for s in seeds], dtype=np.uint64),
        "steps": np.array(steps, dtype=np.uint64),
        "step_hash": np.array([stream.step_hash(s) for s in steps], dtype=np.uint64),
        "indices": np.array(indices, dtype=np.uint64),
        "uniform": uni,
    }


def _affine_cases(fallback) -> dict:
    out = {}
    cases = [
        ("f32_c7", 9, 7, "normal", 0),
        ("f32_c64", 17, 64, "normal", 1),
        ("f32_c1024", 16, 1024, "normal", 2),
        ("f32_c4096", 8, 4096, "normal", 3),
        ("bf16_c1024", 16, 1024, "bf16", 4),
        ("bf16_c4096", 8, 4096, "bf16", 5),
        ("relu_c96", 12, 96, "relu", 6),
        ("const_c33", 4, 33, "const", 7),
    ]
    for name, rows, cols, kind, seed in cases:
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(rows, cols, generator=g)
        if kind == "bf16":
            x = x.to(torch.bfloat16).float()
        elif kind == "relu":
            x = x.relu()
        elif kind == "const":
            x = torch.full((rows, cols), 0.75)
            x[1] = -2.5
            x[2, ::3] = 1.0
        packed, offset, scale = fallback.pack_affine_rows(x)
        out[f"{name}__x"] = x.numpy()
        out[f"{name}__bits"] = packed.numpy()
        out[f"{name}__offset"] = offset.numpy()
        out[f"{name}__scale"] = scale.numpy()
    return out


def _product_cases(fallback) -> dict:
    out = {}
    shapes = [(17, 13, 5), (64, 64, 32), (128, 96, 40), (33, 8, 7)]
    for i, (rows, cols, samples) in enumerate(shapes):
        g = torch.Generator().manual_seed(100 + i)
        coord = torch.randint(-127, 128, (rows, cols), generator=g, dtype=torch.int32).to(torch.int8)
        packed = fallback.pack_coordinate(coord)
        x = torch.randn(samples, cols, generator=g)
        scale = torch.rand(rows, generator=g) + 0.5
        bias = torch.randn(rows, generator=g)
        dy = torch.randn(samples, rows, generator=g)
        xbits, xoff, xscale = fallback.pack_affine_rows(torch.randn(samples, cols, generator=g))
        mat = torch.randn(rows, cols, generator=g)
        key = f"s{i}"
        out[f"{key}__shape"] = np.array([rows, cols, samples], dtype=np.int64)
        out[f"{key}__coord"] = coord.numpy()
        out[f"{key}__packed"] = packed.numpy()
        out[f"{key}__x"] = x.numpy()
        out[f"{key}__scale"] = scale.numpy()
        out[f"{key}__bias"] = bias.numpy()
        out[f"{key}__dy"] = dy.numpy()
        out[f"{key}__xbits"] = xbits.numpy()
        out[f"{key}__xscale"] = xscale.numpy()
        out[f"{key}__mat"] = mat.numpy()
        out[f"{key}__linear"] = fallback.packed_linear_affine(x, packed, scale, bias, cols).numpy()
        out[f"{key}__transpose"] = fallback.packed_transpose(dy, packed, cols, row_scale=scale).numpy()
        out[f"{key}__evidence"] = fallback.evidence_from_packed(dy, xbits, cols, row_scale=xscale).numpy()
        out[f"{key}__row_inner"] = fallback.packed_row_inner(mat, packed, cols).numpy()
    return out


def _update_cases(fallback) -> dict:
    """Seeded coordinate steps: first step from fresh state, then a second."""

    out = {}
    cases = [
        # name, rows, cols, block, seed, step, lr, evidence scale
        ("u16x32", 16, 32, 64, 7, 3, 1.0, 1.0),
        ("u24x40", 24, 40, 64, 7, 3, 1.0, 1.0),
        ("u8x8", 8, 8, 64, 1, 0, 4.0, 1.0),
        ("u12x20", 12, 20, 64, 99, 5, 4.0, 1.0),
        ("u96x160", 96, 160, 256, 17, 5, 1.0, 1e-3),
        ("u256x512", 256, 512, 256, 1_000_004, 0, 1.0, 3e-2),
        ("u64x200", 64, 200, 256, 2**31 + 11, 9, 2.0, 10.0),
        # learning rates that are not powers of two: the step size is
        # reciprocal(rms) * lr there, which one division would not reproduce
        ("u48x96lr3", 48, 96, 64, 5, 2, 0.3, 1.0),
        ("u128x256lr7", 128, 256, 256, 23, 70, 0.7, 0.1),
        ("u40x72lr1", 40, 72, 64, 3_000_010, 11, 0.1, 5.0),
    ]
    for idx, (name, rows, cols, block, seed, step, lr, mag) in enumerate(cases):
        g = torch.Generator().manual_seed(1000 + idx)
        coord = torch.randint(-127, 128, (rows, cols), generator=g, dtype=torch.int32).to(torch.int8)
        blocks = (rows * cols + block - 1) // block
        state = {
            "coordinate": coord.clone(),
            "packed": fallback.pack_coordinate(coord),
            "moment_q": torch.zeros(rows, cols, dtype=torch.int8),
            "moment_scale": torch.full((blocks,), 1 / 127, dtype=torch.float16),
            "row_v": torch.zeros(rows, dtype=torch.float16),
            "col_v": torch.zeros(cols, dtype=torch.float16),
        }
        common = dict(beta1=0.9, beta2=0.99, update_clip=2.0, coordinate_lr=lr,
                      block_size=block, seed=seed)
        for phase in range(2):
            evidence = torch.randn(rows, cols, generator=g) * mag
            key = f"{name}_p{phase}"
            for k, v in state.items():
                out[f"{key}__in_{k}"] = v.numpy().copy()
            out[f"{key}__evidence"] = evidence.numpy().copy()
            out[f"{key}__params"] = np.array(
                [0.9, 0.99, 2.0, lr, block, seed, step + phase], dtype=np.float64)
            flips = fallback.coordinate_update(
                evidence.clone(), state["coordinate"], state["packed"], state["moment_q"],
                state["moment_scale"], state["row_v"], state["col_v"], step=step + phase,
                **common,
            )
            for k, v in state.items():
                out[f"{key}__out_{k}"] = v.numpy().copy()
            out[f"{key}__flips"] = np.array(flips, dtype=np.int64)
    return out


def _update_case_large(fallback) -> dict:
    """A 1024 x 1024 surface, first step from fresh state then a second one
    (block 256): reductions over 1024 columns, rows and 4096 blocks, the
    length at which the fp32 reduction-order band would show.  The evidence
    values are bf16-representable fp32 (they compress; the step's own
    arithmetic is fp32 throughout)."""

    out = {}
    rows = cols = 1024
    block, seed, step, lr = 256, 77, 1, 1.0
    g = torch.Generator().manual_seed(4096)
    coord = torch.randint(-127, 128, (rows, cols), generator=g, dtype=torch.int32).to(torch.int8)
    blocks = (rows * cols + block - 1) // block
    state = {
        "coordinate": coord.clone(),
        "packed": fallback.pack_coordinate(coord),
        "moment_q": torch.zeros(rows, cols, dtype=torch.int8),
        "moment_scale": torch.full((blocks,), 1 / 127, dtype=torch.float16),
        "row_v": torch.zeros(rows, dtype=torch.float16),
        "col_v": torch.zeros(cols, dtype=torch.float16),
    }
    for phase in range(2):
        evidence = (torch.randn(rows, cols, generator=g) * 0.05).to(torch.bfloat16).float()
        key = f"u1024x1024_p{phase}"
        if phase == 0:  # the second step starts from the first one's outputs (not stored twice)
            for k, v in state.items():
                out[f"{key}__in_{k}"] = v.numpy().copy()
        out[f"{key}__evidence"] = evidence.numpy().copy()
        out[f"{key}__params"] = np.array([0.9, 0.99, 2.0, lr, block, seed, step + phase], dtype=np.float64)
        flips = fallback.coordinate_update(
            evidence.clone(), state["coordinate"], state["packed"], state["moment_q"], state["moment_scale"],
            state["row_v"], state["col_v"], beta1=0.9, beta2=0.99, update_clip=2.0, coordinate_lr=lr,
            block_size=block, seed=seed, step=step + phase)
        for k, v in state.items():
            out[f"{key}__out_{k}"] = v.numpy().copy()
        out[f"{key}__flips"] = np.array(flips, dtype=np.int64)
    return out


def main(argv: list[str]) -> None:
    root = Path(argv[1] if len(argv) > 1 else "/root/reference")
    fallback, stream = _load_reference(root)
    torch.set_num_threads(1)
    np.savez_compressed(HERE / "hash.npz", **_hash_vectors(stream))
    np.savez_compressed(HERE / "pack_affine.npz", **_affine_cases(fallback))
    np.savez_compressed(HERE / "products.npz", **_product_cases(fallback))
    np.savez_compressed(HERE / "coordinate_update.npz", **_update_cases(fallback))
    np.savez_compressed(HERE / "coordinate_update_1024.npz", **_update_case_large(fallback))
    for path in sorted(HERE.glob("*.npz")):
        print(f"{path.name}: {path.stat().st_size} bytes")


if __name__ == "__main__":
    main(sys.argv)
