"""Benchmark of the binary-linear hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]

Headline workload: a Llama-3-8B-shaped SwiGLU MLP,
d=4096, ffn=14336, gate/up/down all QSTE, bf16, 16384 tokens of N(0,1)
activations, seeded int8 coordinates U{-127..127}, row scales |N(0,1)|*0.01,
upstream gradient N(0,1).  One step = forward of the three layers (with the
1-bit activation encoding), backward (input gradient, evidence, scale
gradient) and the coordinate step of all three surfaces, which runs inside
backward as in the reference.  The MLP runs as qste_amd.nn.swiglu_mlp, one
autograd node: its forward values equal the three layers with torch's
F.silu(g) * u between them bit for bit; its backward runs the gate and up
layers as one layer of 2 * ffn rows (their input gradient as one product
with one rounding, their evidence as one product of seven full rounds of
tiles).  The same step with the layers
called one by one is reported as ``step_layer_by_layer_ms`` (the fused gate
qste_amd.nn.swiglu between them) and ``step_torch_gate_ms`` (torch's silu
and mul), and the node's step once the optimizer is past step 64 (where the
coordinate step forms the momentum speculatively in its U^2 pass, which
saves a pass over the evidence for surfaces whose clip is idle and costs
one where it still engages) as ``step_past_64_ms``.  ``value`` = 6 * T * sum(R*C) / step time
of the steps timed from a fresh optimizer.

Alongside, measured live with HIP events on the stream the kernels run on:
each GEMM kind at the gate-layer shape (the dominant kernel is reported as
``roofline``), torch.matmul (hipBLASLt) on dense bf16 operands of the same
shapes for comparison, the coordinate step of one 14336 x 4096 surface (HBM), and
the skinny-M decode GEMV of config 5 (K=8192, N=28672, M in {1, 4, 16}) over
rotated weight copies larger than the 256 MB Infinity Cache, the packed
activation kernels at the MLP's hidden shape, and the step times of config 2
(ReLU MLP, d=1024, 8192 tokens) and config 3 (GPT-2 small, batch 8 x 1024,
AdamW + QSTEOptimizer).  The CPU
baseline is the reference's CPU algorithm (oracle/cpu_baseline.py) timed on
this host on a token sample of the same layers.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

MFMA_BF16_PEAK = 2.5e15  # dense, FLOP/s
HBM_PEAK = 8.0e12        # B/s
METRIC = "binary-linear fwd+bwd TFLOP/s + % MFMA peak at d=4096; decode GEMV HBM GB/s"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--tokens", type=int, default=16384)
    ap.add_argument("--d", type=int, default=4096)
    ap.add_argument("--ffn", type=int, default=14336)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip per-kernel, step and GEMV timing")
    ap.add_argument("--no-configs", action="store_true", help="skip the config 2 and config 3 step lines")
    ap.add_argument("--configs-only", action="store_true",
                    help="only the config 2 and config 3 step lines (for a kernel profile of those workloads)")
    ap.add_argument("--pmc-calibrate", action="store_true",
                    help="one launch of each GEMM kind at the gate-layer shape, one coordinate step there "
                         "(fresh, then steady), one decode GEMV at M = 1, 4, 16, and a plain device copy of "
                         "COPY_BYTES, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs")
    return ap.parse_args()


COPY_BYTES = 256 << 20  # the known-size copy the traffic counters are scaled by
TRAFFIC_FILE = ROOT / "profiles" / "gemm_traffic.txt"


def read_traffic():
    """HBM bytes per launch of each GEMM kind, from the committed counter summary.

    The file's `traffic <kind> <bytes>` lines are FETCH_SIZE + WRITE_SIZE per
    dispatch, scaled by what the same counters read for a plain copy of known
    size (the summary states the command and the factor)."""

    out = {}
    if TRAFFIC_FILE.exists():
        for line in TRAFFIC_FILE.read_text().splitlines():
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic":
                out[parts[1]] = float(parts[2])
    return out


def pmc_calibrate(T, d, ffn, device):
    import torch

    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=device).fill_(7)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    kernels_t, _ = gemm_kernels(T, d, ffn, device, iters=1)
    # one coordinate step at the gate shape, fresh then steady (in that
    # order: their dispatches are told apart by position in the trace)
    for steady in (False, True):
        fn, _, _ = step_state(ffn, d, device, steady)
        fn()
        torch.cuda.synchronize()
    # one decode launch at each M, each on a weight copy of its own
    from qste_amd import kernels

    K, N = 8192, 28672
    gen = torch.Generator(device=device).manual_seed(1)
    for M in (1, 4, 16):
        w = torch.randint(0, 256, (N, K // 8), generator=gen, device=device, dtype=torch.int32).to(torch.uint8)
        s = torch.randn(N, generator=gen, device=device).abs_().mul_(0.02)
        x = torch.randn(M, K, generator=gen, device=device).to(torch.bfloat16)
        torch.cuda.synchronize()
        kernels.packed_linear_affine(x, w, s, None, K)
        torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "gemm_shape": [T, ffn, d], "kernels": kernels_t,
                      "step_shape": [ffn, d], "decode_shape": [N, K]}), flush=True)


def make_layer(rows, cols, seed, device, scale_std=0.01):
    import torch

    import qste_amd as qste

    g = torch.Generator(device=device).manual_seed(seed)
    coord = torch.randint(-127, 128, (rows, cols), generator=g, device=device, dtype=torch.int32).to(torch.int8)
    scale = torch.randn(rows, generator=g, device=device).abs_().mul_(scale_std).clamp_min_(1e-6)
    surface = qste.Surface.from_state(coord, scale.log())
    return qste.QSTELinear(surface, None)


class SwiGLU:
    """down(silu(gate(x)) * up(x)) over three binary layers, run as
    ``mode`` says:

    * "node": qste_amd.nn.swiglu_mlp -- the MLP as one autograd node (the
      gate and up layers' backward as one call over both: their input
      gradients as one product, their evidence as one);
    * "gate": the layers one by one with qste_amd.nn.swiglu between them
      (one kernel each way, the down layer's encoding made by that kernel);
    * "torch": the layers one by one with torch's F.silu and mul.

    All three compute the same forward values; "gate" and "torch" the same
    gradients bit for bit; "node" the same evidence and scale gradients up
    to the order some split-K tiles are summed in, and the input gradient
    rounded once instead of three times."""

    def __init__(self, d, ffn, device, mode="node"):
        import torch.nn as nn

        self.gate = make_layer(ffn, d, 11, device)
        self.up = make_layer(ffn, d, 21, device)
        self.down = make_layer(d, ffn, 31, device)
        self.modules = nn.ModuleList([self.gate, self.up, self.down])
        self.mode = mode

    def __call__(self, x):
        import torch.nn.functional as F

        import qste_amd as qste

        if self.mode == "node":
            return qste.nn.swiglu_mlp(x, self.gate, self.up, self.down)
        if self.mode == "gate":
            return self.down(qste.nn.swiglu(self.gate(x), self.up(x)))
        return self.down(F.silu(self.gate(x)) * self.up(x))


def cfg1_workload(device, base=0):
    """Config 1: one QSTE Linear 2048 -> 2048 in fp32 on 256 tokens.

    Seeded on the CPU (torch.Generator, seeds base+0..3) and copied over:
    x ~ N(0,1) [256, 2048] (s0); coordinates U{-127..127} (s1); row scales
    |N(0,1)| * 0.02 (s2) held as log_scale = ln(scale); bias 0; target
    ~ N(0,1) [256, 2048] (s3).  Returns (layer, x, target) on the device."""

    import torch

    import qste_amd as qste

    def gen(k):
        return torch.Generator().manual_seed(base + k)

    x = torch.randn(256, 2048, generator=gen(0))
    coord = torch.randint(-127, 128, (2048, 2048), generator=gen(1), dtype=torch.int32).to(torch.int8)
    scale = torch.randn(2048, generator=gen(2)).abs_().mul_(0.02).clamp_min_(1e-6)
    target = torch.randn(256, 2048, generator=gen(3))
    surface = qste.Surface.from_state(coord.to(device), scale.log().to(device))
    layer = qste.QSTELinear(surface, torch.zeros(2048, device=device))
    return layer, x.to(device), target.to(device)


def cfg1_step_gpu(layer, x, target, coords):
    """Forward, MSE against the target, backward (the coordinate step runs
    inside it), then QSTEOptimizer.step; returns the flips."""

    import torch.nn.functional as F

    F.mse_loss(layer(x), target).backward()
    return coords.step()


def cfg1_lines(device, cpu: bool):
    """Config 1 timed on the GPU and, as the CPU anchor, on the host's cores
    with the port of the reference's CPU backend (all of config 1, fp32)."""

    import qste_amd as qste

    layer, x, target = cfg1_workload(device)
    coords = qste.QSTEOptimizer([layer.surface])
    ms = timed_wall(lambda: cfg1_step_gpu(layer, x, target, coords), 20, warmup=3)
    flop = 6.0 * 256 * 2048 * 2048
    out = {"workload": "cfg1 QSTE Linear 2048->2048 fp32, 256 tokens, fwd+MSE+bwd+coordinate step",
           "gpu_ms_per_step": round(ms, 4), "gpu_tflops": round(flop / ms / 1e9, 3)}
    if cpu:
        from oracle import cpu_baseline as cb

        threads = cb.set_threads(cb.default_threads())
        xs = x.cpu()
        tg = target.cpu()
        layer_cpu = cb.Surface(layer.surface.coordinate.cpu().numpy(), layer.scale.detach().cpu().numpy())
        cb.cfg1_step(xs, tg, layer_cpu, 0)
        iters, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 10.0 and iters < 2000:
            cb.cfg1_step(xs, tg, layer_cpu, iters + 1)
            iters += 1
        secs = (time.perf_counter() - t0) / iters
        out.update({"cpu_ms_per_step": round(secs * 1e3, 3), "cpu_tflops": round(flop / secs / 1e12, 4),
                    "cpu_threads": threads, "cpu_model": cb.cpu_model(), "cpu_iterations": iters,
                    "cpu_kind": "port of the reference's cpu.cpp (tile sign expansion + torch fp32 GEMM, "
                                "OpenMP encoding and 4-phase step)"})
    return out


def relu_mlp(d=1024, ratio=4, device="cuda"):
    """Config 2: fc1 d -> ratio*d, ReLU, fc2 back, both QSTE, bf16.

    Each layer follows config 1's recipe with its own seeds (layer i: 10i+1
    coordinates U{-127..127}, 10i+2 row scales |N(0,1)| * 0.02, bias 0),
    built on the CPU and moved over; the ReLU between them is the packed
    one-bit ReLU that ``convert`` puts in (it keeps one bit per element for
    backward)."""

    import torch
    import torch.nn as nn

    import qste_amd as qste

    def layer(i, rows, cols):
        gc = torch.Generator().manual_seed(10 * i + 1)
        gs = torch.Generator().manual_seed(10 * i + 2)
        coord = torch.randint(-127, 128, (rows, cols), generator=gc, dtype=torch.int32).to(torch.int8)
        scale = torch.randn(rows, generator=gs).abs_().mul_(0.02).clamp_min_(1e-6)
        surface = qste.Surface.from_state(coord.to(device), scale.log().to(device))
        return qste.QSTELinear(surface, torch.zeros(rows, device=device))

    model = nn.Sequential(layer(0, ratio * d, d), qste.nn.ReLU(), layer(1, d, ratio * d))
    return model.to(device=device, dtype=torch.bfloat16)


class GPT2Small:
    """Config 3: a GPT-2-small-shaped decoder (12 layers, d=768, 12 heads, MLP
    ratio 4, vocab 50257, context 1024, tied embedding), random init, bf16.
    Only the MLPs are converted to QSTE (their tanh-GELU becomes the packed
    one); attention stays float bf16: torch's fused causal attention (flash
    or memory-efficient kernels only -- the unfused math path is excluded,
    so a missing fused kernel is an error rather than a silent fallback)."""

    def __new__(cls, device="cuda", layers=12, d=768, heads=12, vocab=50257, context=1024):
        import torch
        import torch.nn as nn
        import torch.nn.functional as F
        from torch.nn.attention import SDPBackend, sdpa_kernel

        import qste_amd as qste

        class Block(nn.Module):
            def __init__(self):
                super().__init__()
                self.ln1 = nn.LayerNorm(d)
                self.qkv = nn.Linear(d, 3 * d)
                self.proj = nn.Linear(d, d)
                self.ln2 = nn.LayerNorm(d)
                self.mlp = nn.Sequential(nn.Linear(d, 4 * d), nn.GELU(approximate="tanh"), nn.Linear(4 * d, d))

            def attention(self, x):
                b, s, _ = x.shape
                q, k, v = self.qkv(x).split(d, dim=-1)
                q, k, v = (t.reshape(b, s, heads, d // heads).transpose(1, 2) for t in (q, k, v))
                with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                    y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
                return self.proj(y.transpose(1, 2).reshape(b, s, d))

            def forward(self, x):
                x = x + self.attention(self.ln1(x))
                return x + self.mlp(self.ln2(x))

        class Model(nn.Module):
            def __init__(self):
                super().__init__()
                self.wte = nn.Embedding(vocab, d)
                self.wpe = nn.Embedding(context, d)
                self.blocks = nn.ModuleList(Block() for _ in range(layers))
                self.ln_f = nn.LayerNorm(d)

            def forward(self, ids):
                pos = torch.arange(ids.shape[1], device=ids.device)
                x = self.wte(ids) + self.wpe(pos)
                for block in self.blocks:
                    x = block(x)
                return F.linear(self.ln_f(x), self.wte.weight)

        torch.manual_seed(0)
        model = Model()
        for module in model.modules():  # GPT-2's initialisation
            if isinstance(module, (nn.Linear, nn.Embedding)):
                nn.init.normal_(module.weight, 0.0, 0.02)
            if isinstance(module, nn.Linear) and module.bias is not None:
                nn.init.zeros_(module.bias)
        qste.convert(model, include=["blocks.*.mlp.*"])
        return model.to(device=device, dtype=torch.bfloat16)


def in_step_times(step, T, d, ffn, steps=3):
    """Per-call time of the layers' products inside the training step: HIP
    events recorded on the current stream around every operator call that
    runs them, over ``steps`` steps (events do not synchronize, so the step
    runs as it does untimed).  Kinds: "forward" (packed_linear_affine, one
    product), "backward_call" (linear_backward with the input gradient: two
    products), "evidence_call" (linear_backward without it: the evidence
    alone), "backward_call_gate_up" (the MLP node's one call for the gate
    and up layers: their two evidence products and their summed input
    gradient, four products)."""

    import torch

    from qste_amd import kernels

    records = []
    names = ("packed_linear_affine", "linear_backward")
    originals = {n: getattr(kernels, n) for n in names}

    def kind_of(name, args, kwargs):
        if name == "packed_linear_affine":
            return "forward", 1
        if args[0].shape[-1] == 2 * ffn:
            return ("backward_call_gate_up", 4) if kwargs.get("need_input", True) else ("evidence_call_gate_up", 2)
        return ("backward_call", 2) if kwargs.get("need_input", True) else ("evidence_call", 1)

    def wrap(name, fn):
        def timed(*args, **kwargs):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            out = fn(*args, **kwargs)
            b.record()
            records.append((kind_of(name, args, kwargs), a, b))
            return out
        return timed

    for n in names:
        setattr(kernels, n, wrap(n, originals[n]))
    try:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
    finally:
        for n in names:
            setattr(kernels, n, originals[n])
    flop = 2.0 * T * ffn * d  # one product at any of the three shapes
    out = {}
    for kind in ("forward", "backward_call", "evidence_call", "backward_call_gate_up", "evidence_call_gate_up"):
        times = [a.elapsed_time(b) for (k, _), a, b in records if k == kind]
        if not times:
            continue
        products = next(p for (k, p), _, _ in records if k == kind)
        ms = sum(times) / len(times)
        out[kind] = {"ms": round(ms, 4), "calls": len(times), "tflops": round(products * flop / ms / 1e9, 2),
                     "frac_of_mfma_peak": round(products * flop / (ms * 1e-3) / MFMA_BF16_PEAK, 4)}
    return out


def config_steps(device):
    """Configs 2 and 3 (fwd+bwd+step), reported beside the headline."""

    import torch
    import torch.nn.functional as F

    import qste_amd as qste

    out = {}
    # config 2: 8192 tokens through the ReLU MLP, upstream gradient N(0,1)
    model = relu_mlp(device=device)
    coords = qste.QSTEOptimizer(model)
    g = torch.Generator(device=device).manual_seed(0)
    x = torch.randn(8192, 1024, generator=g, device=device).to(torch.bfloat16).requires_grad_(True)
    dy = torch.randn(8192, 1024, generator=g, device=device).to(torch.bfloat16)

    def step2():
        x.grad = None  # both layers form their input gradient (the FLOPs counted)
        model(x).backward(dy)
        coords.step()

    ms, mean, worst = timed_median(step2, 15)
    flop = 6.0 * 8192 * (2 * 4096 * 1024)
    out["cfg2_relu_mlp"] = {"ms_per_step": round(ms, 3), "mean_ms": round(mean, 3), "max_ms": round(worst, 3),
                            "tflops": round(flop / ms / 1e9, 2),
                            "frac_of_mfma_peak": round(flop / (ms * 1e-3) / MFMA_BF16_PEAK, 4),
                            "tokens": 8192, "d": 1024, "ffn": 4096,
                            "timing": "median (mean, max) of 15 steps, each host-clocked and synchronized"}
    del model, coords, x, dy
    # config 3: GPT-2 small, batch 8 x 1024 random ids, AdamW + QSTEOptimizer
    model = GPT2Small(device=device)
    adam = torch.optim.AdamW(list(qste.continuous_parameters(model)), lr=1e-4)
    coords = qste.QSTEOptimizer(model)
    ids = torch.randint(0, 50257, (8, 1024), generator=g, device=device)

    def step3():
        logits = model(ids[:, :-1])
        F.cross_entropy(logits.reshape(-1, logits.shape[-1]).float(), ids[:, 1:].reshape(-1)).backward()
        adam.step()
        coords.step()
        adam.zero_grad(set_to_none=True)

    ms, mean, worst = timed_median(step3, 10, warmup=3)
    tokens = 8 * 1023
    mlp_flop = 6.0 * tokens * 12 * (2 * 3072 * 768)
    out["cfg3_gpt2_small"] = {"ms_per_step": round(ms, 3), "mean_ms": round(mean, 3), "max_ms": round(worst, 3),
                              "tokens_per_s": round(tokens / ms * 1e3, 1),
                              "mlp_fwd_bwd_flop": mlp_flop, "batch": 8, "seq": 1024,
                              "timing": "median (mean, max) of 10 steps, each host-clocked and synchronized",
                              "note": "whole training step; MLPs QSTE with packed tanh-GELU, attention and head bf16 (SDPA flash/efficient)"}
    return out


def timed_wall(fn, iters, warmup=2):
    """Average milliseconds of ``fn`` by the host clock, synchronized around."""

    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / iters * 1e3


def timed_median(fn, iters, warmup=2):
    """Median milliseconds of ``fn`` over ``iters`` calls, each timed by the
    host clock between synchronizations (steps that end in a host read of
    the flip count synchronize anyway; the median keeps a host stall in one
    step out of a host-bound config's figure), with the mean and maximum of
    the same per-step times."""

    import statistics

    import torch

    for _ in range(warmup):
        fn()
    times = []
    for _ in range(iters):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(times), statistics.mean(times), max(times)


def timed_events(fn, iters, stream=None, warm=3):
    """Average milliseconds of ``fn`` over ``iters`` calls, by HIP events,
    after ``warm`` untimed calls (the first launches after the GPU idled
    while inputs were built run up to 20% slower, at lower clocks)."""

    import torch

    stream = stream or torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    for _ in range(max(1, warm)):
        fn()
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(iters):
        fn()
    stop.record(stream)
    stop.synchronize()
    return start.elapsed_time(stop) / iters


def gemm_kernels(T, d, ffn, device, iters=5):
    """Per-launch time of each product kind at the gate-layer shape."""

    import torch

    from qste_amd import kernels

    g = torch.Generator(device=device).manual_seed(7)
    x = torch.randn(T, d, generator=g, device=device).to(torch.bfloat16)
    dy = torch.randn(T, ffn, generator=g, device=device).to(torch.bfloat16)
    layer = make_layer(ffn, d, 11, device)
    packed = layer.surface.packed_sign.data
    scale = layer.scale.detach().float()
    xbits, off, xs = kernels.pack_affine_rows(x)
    flop = 2.0 * T * ffn * d
    out = {}
    runs = {
        "forward": lambda: kernels.packed_linear_affine(x, packed, scale, None, d),
        "dgrad": lambda: kernels.packed_transpose(dy, packed, d, row_scale=scale),
        "evidence": lambda: kernels.evidence_from_packed(dy, xbits, d, row_scale=xs),
    }
    for name, fn in runs.items():
        ms = timed_events(fn, iters)
        out[name] = {"ms": round(ms, 4), "tflops": round(flop / ms / 1e9, 2),
                     "frac_of_mfma_peak": round(flop / (ms * 1e-3) / MFMA_BF16_PEAK, 4)}
    # the training path's backward of one layer: one C-ABI call running dX
    # and the evidence (one launch or two, by the shape's plan) plus the
    # column sums and whatever sign transposes or combine pass the plan needs
    # (two products' FLOPs)
    ms = timed_events(lambda: kernels.linear_backward(dy, xbits, off, xs, packed, scale, d, need_bias=False), iters)
    out["backward_call"] = {"ms": round(ms, 4), "tflops": round(2 * flop / ms / 1e9, 2),
                            "frac_of_mfma_peak": round(2 * flop / (ms * 1e-3) / MFMA_BF16_PEAK, 4)}
    # the same forward on fp16 operands (fp16 MFMA, same dense peak)
    x16 = x.to(torch.float16)
    ms = timed_events(lambda: kernels.packed_linear_affine(x16, packed, scale, None, d), iters)
    out["forward_fp16"] = {"ms": round(ms, 4), "tflops": round(flop / ms / 1e9, 2),
                           "frac_of_mfma_peak": round(flop / (ms * 1e-3) / MFMA_BF16_PEAK, 4)}
    return out, flop


def fp32_products(device, T=8192, rows=4096, cols=4096, iters=5):
    """The three products on fp32 operands (bf16 limbs on the MFMA path),
    against torch's fp32 matmul of the dense expanded signs: the reference's
    own route for fp32 inputs (cuda.py:1531-1597)."""

    import torch

    from qste_amd import kernels

    g = torch.Generator(device=device).manual_seed(9)
    x = torch.randn(T, cols, generator=g, device=device)
    dy = torch.randn(T, rows, generator=g, device=device)
    layer = make_layer(rows, cols, 13, device)
    packed = layer.surface.packed_sign.data
    scale = layer.scale.detach().float()
    xbits, off, xs = kernels.pack_affine_rows(x)
    flop = 2.0 * T * rows * cols
    out = {"shape": [T, rows, cols]}
    runs = {
        "forward": lambda: kernels.packed_linear_affine(x, packed, scale, None, cols),
        "dgrad": lambda: kernels.packed_transpose(dy, packed, cols, row_scale=scale),
        "evidence": lambda: kernels.evidence_from_packed(dy, xbits, cols, row_scale=xs),
    }
    for name, fn in runs.items():
        ms = timed_events(fn, iters)
        out[name] = {"ms": round(ms, 4), "tflops": round(flop / ms / 1e9, 2)}
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        w = kernels.unpack_rows(packed, cols, dtype=torch.float32)
        ms = timed_events(lambda: torch.mm(x, w.t()), iters)
        out["torch_fp32_mm"] = {"ms": round(ms, 4), "tflops": round(flop / ms / 1e9, 2)}
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    return out


def vendor_dense(T, d, ffn, device, iters=5):
    """torch.matmul (hipBLASLt) on dense bf16 operands of each product's shape,
    as the products store them: the practical GEMM rate of this box, for
    comparison with the packed-sign kernels (which also expand the signs)."""

    import torch

    g = torch.Generator(device=device).manual_seed(3)
    x = torch.randn(T, d, generator=g, device=device).to(torch.bfloat16)
    dy = torch.randn(T, ffn, generator=g, device=device).to(torch.bfloat16)
    w = torch.randn(ffn, d, generator=g, device=device).to(torch.bfloat16)
    runs = {
        "forward": lambda: torch.matmul(x, w.t()),
        "dgrad": lambda: torch.matmul(dy, w),
        "evidence": lambda: torch.matmul(dy.t(), x),
    }
    flop = 2.0 * T * ffn * d
    out = {}
    for name, fn in runs.items():
        ms = timed_events(fn, iters)
        out[name] = {"ms": round(ms, 4), "tflops": round(flop / ms / 1e9, 2)}
    return out


def step_state(rows, cols, device, steady: bool):
    """A surface's coordinate-step operands at the gate shape.

    fresh: zero second moments and momentum, as at step 0 (the clip engages,
    so every pass runs).  steady: the state a long run settles into -- second
    moments at the evidence's mean square, int8 momentum with block scales of
    a unit-RMS update -- stepped at step 100, where the normalized update's
    RMS is about 1 and the clip (2.0) stays idle."""

    import torch

    from qste_amd import kernels

    g = torch.Generator(device=device).manual_seed(5)
    ev = torch.randn(rows, cols, generator=g, device=device).mul_(0.01)
    coord = torch.randint(-127, 128, (rows, cols), generator=g, device=device, dtype=torch.int32).to(torch.int8)
    packed = kernels.pack_coordinate(coord)
    blocks = (rows * cols + 255) // 256
    if steady:
        mq = torch.randint(-127, 128, (rows, cols), generator=g, device=device, dtype=torch.int32).to(torch.int8)
        ms_ = torch.full((blocks,), 3.0 / 127, dtype=torch.float16, device=device)
        rv = torch.full((rows,), 1e-4, dtype=torch.float16, device=device)
        cv = torch.full((cols,), 1e-4, dtype=torch.float16, device=device)
    else:
        mq = torch.zeros_like(coord)
        ms_ = torch.full((blocks,), 1 / 127, dtype=torch.float16, device=device)
        rv = torch.zeros(rows, dtype=torch.float16, device=device)
        cv = torch.zeros(cols, dtype=torch.float16, device=device)
    flips = torch.empty((), dtype=torch.int64, device=device)
    step = 100 if steady else 0

    def fn():
        kernels.coordinate_update(ev, coord, packed, mq, ms_, rv, cv, beta1=0.9, beta2=0.99, update_clip=2.0,
                                  coordinate_lr=1.0, block_size=256, seed=1, step=step, flips=flips)

    def divisor():
        """One more step through the C entry with a workspace of our own, whose
        scalars block (sqrt mean row statistic, clip divisor, step size,
        momentum RMS) is read back: the clip divisor it ran with."""

        lib = kernels._lib.load()
        need = lib.qste_coordinate_update_workspace_bytes(rows, cols, 256)
        at = lib.qste_coordinate_update_scalars_offset(rows, cols, 256)
        work = torch.empty(need, dtype=torch.uint8, device=device)
        rc = lib.qste_coordinate_update(
            ev.data_ptr(), coord.data_ptr(), packed.data_ptr(), mq.data_ptr(), ms_.data_ptr(), rv.data_ptr(),
            cv.data_ptr(), rows, cols, 0.9, 0.99, 2.0, 1.0, 256, 1, step, None, flips.data_ptr(), None,
            work.data_ptr(), need, torch.cuda.current_stream(device).cuda_stream)
        kernels._lib.check(rc, "coordinate_update")
        return float(work[at:at + 16].view(torch.float32)[1].item())

    return fn, blocks, divisor


def step_bandwidth(rows, cols, device):
    """Coordinate step of one rows x cols surface, fresh and steady, each with
    the clip divisor it ran with (1.0: the clip is idle)."""

    out = {}
    for kind in ("fresh", "steady"):
        fn, blocks, divisor = step_state(rows, cols, device, kind == "steady")
        # each call steps the state on: one untimed call keeps the timed ones
        # near the state described (the fresh clip divisor 1.92 by the seventh)
        ms = timed_events(fn, 5, warm=1)
        nbytes = rows * cols * (4 + 2 + 2) + rows * ((cols + 7) // 8) + 4 * blocks + 4 * (rows + cols)
        out[kind] = {"rows": rows, "cols": cols, "ms": round(ms, 4), "algorithmic_bytes": nbytes,
                     "gbps": round(nbytes / ms / 1e6, 1),
                     "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / HBM_PEAK, 4),
                     "clip_divisor": divisor()}
    return out


def packed_activation_bandwidth(T, ffn, device):
    """HBM rate of the packed-activation kernels on the MLP's hidden [T, ffn] bf16."""

    import torch

    from qste_amd import kernels

    g = torch.Generator(device=device).manual_seed(7)
    h = torch.randn(T, ffn, generator=g, device=device).to(torch.bfloat16)
    grad = torch.randn(T, ffn, generator=g, device=device).to(torch.bfloat16)
    n = T * ffn
    out = {}

    def rate(name, fn, nbytes):
        ms = timed_events(fn, 5)
        out[name] = {"ms": round(ms, 4), "algorithmic_bytes": nbytes, "gbps": round(nbytes / ms / 1e6, 1),
                     "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / HBM_PEAK, 4)}

    # SiLU value + int8 derivative + fp32 row scale: read x, write y and the payload
    rate("silu_forward", lambda: kernels.smooth_activation(h, "silu"), n * (2 + 2 + 1) + 4 * T)
    _, payload, scale = kernels.smooth_activation(h, "silu")
    # grad * (payload * scale): read grad and payload, write the input gradient
    rate("smooth_backward", lambda: kernels.smooth_backward(grad, payload, scale), n * (2 + 1 + 2) + 4 * T)
    # ReLU value + bit mask; its backward reads grad and bits, writes the gradient
    rate("relu_forward", lambda: kernels.masked_activation(h, kernels.MASK_CLAMP), n * (2 + 2) + n // 8)
    _, bits = kernels.masked_activation(h, kernels.MASK_CLAMP)
    rate("relu_backward", lambda: kernels.masked_backward(grad, bits, ffn), n * (2 + 2) + n // 8)
    return out


def decode_gemv(device, K=8192, N=28672, copies=10):
    import torch

    from qste_amd import kernels

    g = torch.Generator(device=device).manual_seed(1)
    pb = K // 8
    weights = [torch.randint(0, 256, (N, pb), generator=g, device=device, dtype=torch.int32).to(torch.uint8)
               for _ in range(copies)]
    scales = [torch.randn(N, generator=g, device=device).abs_().mul_(0.02) for _ in range(copies)]
    res = {}
    reps = 5
    for name, M, dtype in (("M1", 1, torch.bfloat16), ("M4", 4, torch.bfloat16), ("M16", 16, torch.bfloat16),
                           ("fp16_M1", 1, torch.float16), ("fp16_M16", 16, torch.float16)):
        x = torch.randn(M, K, generator=g, device=device).to(dtype)

        def sweep():
            for i in range(copies):
                kernels.packed_linear_affine(x, weights[i], scales[i], None, K)

        # a few microseconds per launch is less than the host needs to issue
        # one through Python, so the launches are captured once and replayed
        # back to back from a graph
        sweep()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                sweep()
        ms = timed_events(graph.replay, 4) / (reps * copies)
        nbytes = N * pb + 4 * N + 2 * M * K + 2 * M * N
        res[name] = {"us": round(ms * 1e3, 2), "algorithmic_bytes": nbytes,
                        "gbps": round(nbytes / ms / 1e6, 1),
                        "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / HBM_PEAK, 4),
                        "timing": f"graph replay of {reps * copies} launches over {copies} weight copies"}
        del graph
    # the floor: a plain streaming read of the same weight copies, replayed
    # from a graph the same way (every kernel that reads these bytes once,
    # launch included, takes at least this long)
    def reads():
        for i in range(copies):
            kernels.stream_read(weights[i])

    reads()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            reads()
    ms = timed_events(graph.replay, 4) / (reps * copies)
    nbytes = N * pb
    res["read_floor"] = {"us": round(ms * 1e3, 2), "bytes": nbytes, "gbps": round(nbytes / ms / 1e6, 1),
                         "timing": f"graph replay of {reps * copies} qste_stream_read launches over the "
                                   f"{copies} weight copies"}
    del graph
    # back-to-back empty launches in the same harness: the fixed cost per launch
    empty = torch.empty(16, dtype=torch.uint8, device=device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps * copies):
            kernels.stream_read(empty, groups=1)
    ms = timed_events(graph.replay, 4) / (reps * copies)
    res["launch_floor_us"] = round(ms * 1e3, 2)
    del graph
    return res


def device_report(device, T, d, ffn):
    """What the runtime reports (compute units, maximum clocks), the shader
    clock one wave measures at idle, and the clock rocm-smi reads while the
    evidence product runs back to back (the chip is power-limited under the
    GEMMs, so their clock is below the maximum)."""

    import subprocess
    import threading

    import torch

    from qste_amd import kernels

    info = kernels.device_info(device)
    out = {"arch": getattr(torch.cuda.get_device_properties(device), "gcnArchName", "?").split(":")[0],
           "cus": info["cus"], "max_sclk_mhz": info["max_sclk_mhz"], "mclk_mhz": info["mclk_mhz"],
           "lds_per_cu": info["lds_per_cu"], "sclk_idle_probe_mhz": round(kernels.measured_sclk_mhz(device), 1)}
    smi = "/opt/rocm/bin/rocm-smi"
    if not os.path.exists(smi):
        out["sclk_under_gemm_mhz"] = None
        return out
    g = torch.Generator(device=device).manual_seed(11)
    dy = torch.randn(T, ffn, generator=g, device=device).to(torch.bfloat16)
    xs = torch.randn(T, d, generator=g, device=device).to(torch.bfloat16)
    packed_x, _, x_scale = kernels.pack_affine_rows(xs)
    samples = []
    stop = threading.Event()

    def sample():
        while not stop.is_set():
            try:
                res = subprocess.run([smi, "--showclocks", "--json"], capture_output=True, text=True, timeout=10)
                data = json.loads(res.stdout)
                for card in data.values():
                    for key, val in card.items():
                        if "sclk" in key.lower() and "mhz" in str(val).lower():
                            samples.append(float(str(val).strip("()Mhz ").split("Mhz")[0].strip("(")))
            except Exception:
                return

    # the evidence product (the dominant GEMM kind) back to back for ~2 s
    run = lambda: kernels.evidence_from_packed(dy, packed_x, d, row_scale=x_scale)  # noqa: E731
    run()
    torch.cuda.synchronize()
    th = threading.Thread(target=sample, daemon=True)
    t0 = time.perf_counter()
    th.start()
    launches = 0
    while time.perf_counter() - t0 < 2.0:
        for _ in range(50):
            run()
        launches += 50
        torch.cuda.synchronize()
    stop.set()
    th.join(timeout=15)
    busy = sorted(samples)
    out["sclk_under_gemm_mhz"] = {"samples": len(busy), "min": busy[0] if busy else None,
                                  "median": busy[len(busy) // 2] if busy else None,
                                  "max": busy[-1] if busy else None,
                                  "load": f"{launches} evidence products at {ffn} x {d} x {T} tokens, sampled by "
                                          "rocm-smi --showclocks"}
    return out


def memory_bandwidth(device, pair_bytes=256 << 20, pairs=3):
    """Measured HBM rates with buffers rotated over more than the 256 MB
    Infinity Cache: a device copy (torch copy_, read + write bytes) and a
    plain streaming read (qste_stream_read)."""

    import torch

    from qste_amd import kernels

    src = [torch.empty(pair_bytes, dtype=torch.uint8, device=device).fill_(i + 1) for i in range(pairs)]
    dst = [torch.empty(pair_bytes, dtype=torch.uint8, device=device) for _ in range(pairs)]
    reps = 4

    def copy_all():
        for i in range(pairs):
            dst[i].copy_(src[i])

    ms = timed_events(copy_all, reps) / pairs
    read_ms = timed_events(lambda: [kernels.stream_read(t) for t in src + dst], reps) / (2 * pairs)
    return {"copy": {"gbps": round(2 * pair_bytes / ms / 1e6, 1), "bytes_per_copy": pair_bytes,
                     "rotation": f"{pairs} pairs of {pair_bytes >> 20} MiB"},
            "read": {"gbps": round(pair_bytes / read_ms / 1e6, 1), "bytes_per_read": pair_bytes,
                     "rotation": f"{2 * pairs} buffers of {pair_bytes >> 20} MiB"}}


def cpu_baseline(d, ffn, tokens=16384, warm_tokens=512):
    """Config 4 on this host's cores with the port of the reference's CPU
    backend (oracle/cpu_baseline.py): packed signs expanded one tile at a time
    + torch's fp32 GEMMs, OpenMP encodings and four-phase coordinate steps.

    One whole training step at the full token count: the three forwards with
    their encodings, the SwiGLU, every backward product (each layer's input
    gradient included) and the three coordinate steps on the evidence that
    backward produced, after one warm-up pass of the products on
    ``warm_tokens`` tokens.  ``value`` is config 4's FLOPs over that time."""

    import numpy as np
    import torch

    from oracle import cpu_baseline as cb

    threads = cb.set_threads(cb.default_threads())
    rng = np.random.default_rng(0)
    g = torch.Generator().manual_seed(0)
    shapes = ((ffn, d), (ffn, d), (d, ffn))
    layers = []
    for rows, cols in shapes:
        coord = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
        scale = (np.abs(rng.standard_normal(rows)) * 0.01).astype(np.float32)
        layers.append(cb.Surface(coord, scale))
    cb.swiglu_products(torch.randn(warm_tokens, d, generator=g), torch.randn(warm_tokens, d, generator=g),
                       layers)  # warm the BLAS and the thread pool
    x = torch.randn(tokens, d, generator=g)
    dy = torch.randn(tokens, d, generator=g)
    t0 = time.perf_counter()
    evidence = cb.swiglu_products(x, dy, layers)
    t_products = time.perf_counter() - t0
    t1 = time.perf_counter()
    for k, (layer, ev) in enumerate(zip(layers, evidence)):
        layer.step(ev, seed=1 + 1_000_003 * k, step=0)  # the step consumes its evidence as scratch
    t_step = time.perf_counter() - t1
    secs = t_products + t_step
    flop = 6.0 * tokens * (2 * ffn * d + d * ffn)
    return {"value": round(flop / secs / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "cpu_model": cb.cpu_model(), "seconds_per_step": round(secs, 3),
            "sample": f"one whole cfg4 SwiGLU step (d={d}, ffn={ffn}, {tokens} tokens, fp32): forward, backward "
                      f"products {t_products:.2f} s, the three coordinate steps {t_step:.2f} s, on {threads} "
                      f"threads, after a warm-up pass of the products on {warm_tokens} tokens"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch

    import qste_amd as qste

    if not torch.cuda.is_available():
        print("bench.py needs the GPU", file=sys.stderr)
        sys.exit(2)
    device = torch.device("cuda:0")
    T, d, ffn = args.tokens, args.d, args.ffn
    if args.pmc_calibrate:
        pmc_calibrate(T, d, ffn, device)
        return
    if args.configs_only:
        print(json.dumps({"configs": config_steps(device)}), flush=True)
        return

    mlp = SwiGLU(d, ffn, device)
    coords = qste.QSTEOptimizer(list(qste.surfaces(mlp.modules)))
    g = torch.Generator(device=device).manual_seed(0)
    # the block's input takes a gradient, as inside a network: every layer
    # forms its input gradient, so the step does the 6*T*sum(R*C) FLOPs counted
    x = torch.randn(T, d, generator=g, device=device).to(torch.bfloat16).requires_grad_(True)
    g4 = torch.Generator(device=device).manual_seed(4)
    dy = torch.randn(T, d, generator=g4, device=device).to(torch.bfloat16)

    def step():
        x.grad = None
        y = mlp(x)
        y.backward(dy)
        return coords.step()

    def packed_step():
        x.grad = None
        with qste.packed_activations():
            y = mlp(x)
        y.backward(dy)
        return coords.step()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    secs = (time.perf_counter() - t0) / max(1, args.steps)
    flop = 6.0 * T * (2 * ffn * d + d * ffn)
    value = flop / secs / 1e12

    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(secs * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations and gradients, U{-127..127} int8 coordinates)",
        "config": {"workload": "cfg4 Llama-3-8B SwiGLU MLP fwd+bwd+coordinate step",
                   "tokens": T, "d": d, "ffn": ffn, "layers": 3, "flop_per_step": flop,
                   "gate": "qste_amd.nn.swiglu_mlp: the MLP as one autograd node (forward values equal to the "
                           "layers with F.silu(g) * u bit for bit; the gate and up layers' backward as one call "
                           "over both); the layers one by one are step_layer_by_layer_ms (fused gate) and "
                           "step_torch_gate_ms (torch's silu and mul)"},
        "frac_of_mfma_peak": round(flop / secs / MFMA_BF16_PEAK, 4),
    }
    if not args.no_extras:
        kernels_t, kflop = gemm_kernels(T, d, ffn, device)
        dominant = max((k for k in kernels_t if k in ("forward", "dgrad", "evidence")),
                       key=lambda k: kernels_t[k]["ms"])
        dk = kernels_t[dominant]
        traffic = read_traffic().get(dominant)
        launches = {"forward": "wide_kernel<A_ROWS_M, B_BITS_ALONG_K, EPI_FORWARD>",
                    "dgrad": "wide_kernel<A_ROWS_M, B_BITS_ALONG_N, EPI_PLAIN>",
                    "evidence": "evidence_split_kernel + evidence_combine_kernel (the last, partial round of "
                                "tiles split over K, then summed)"}
        line["roofline"] = {"bound": "mfma", "kernel": dominant, "achieved": dk["tflops"],
                            "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                            "frac": round(dk["tflops"] * 1e12 / MFMA_BF16_PEAK, 4),
                            "traffic": None if traffic is None else int(traffic),
                            "launches": launches[dominant]}
        # the same products inside the training step (the chip is power-limited
        # there, so they run slower than back to back in isolation)
        line["in_step"] = in_step_times(step, T, d, ffn)
        if "backward_call" in line["in_step"]:
            line["roofline"]["in_step_backward_call_frac"] = line["in_step"]["backward_call"]["frac_of_mfma_peak"]
        line["roofline"]["isolated_backward_call_frac"] = kernels_t["backward_call"]["frac_of_mfma_peak"]
        line["kernels"] = kernels_t
        line["device"] = device_report(device, T, d, ffn)
        line["memory_bandwidth"] = memory_bandwidth(device)
        line["vendor_dense_bf16_gemm"] = vendor_dense(T, d, ffn, device)
        line["fp32_products"] = fp32_products(device)
        line["coordinate_step"] = step_bandwidth(ffn, d, device)
        line["decode_gemv"] = decode_gemv(device)
        line["packed_activations"] = packed_activation_bandwidth(T, ffn, device)
        # the same step with the layers called one by one: with the fused
        # gate between them, and with torch's silu and mul (what a model
        # written F.silu(gate(x)) * up(x) runs)
        for mode, key in (("gate", "step_layer_by_layer_ms"), ("torch", "step_torch_gate_ms")):
            mlp.mode = mode
            step()
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            for _ in range(3):
                step()
            torch.cuda.synchronize()
            line[key] = round((time.perf_counter() - t1) / 3 * 1e3, 3)
        # and with the SiLU retaining its int8 derivative (qste.packed_activations())
        packed_step()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(3):
            packed_step()
        torch.cuda.synchronize()
        line["packed_activations"]["step_ms"] = round((time.perf_counter() - t1) / 3 * 1e3, 3)
        mlp.mode = "node"
        # The headline times the optimizer's steps W .. W+K-1 from a fresh
        # state, where the clip engages and the coordinate step forms the
        # momentum in a pass of its own.  Past step 64 the U^2 pass forms
        # the momentum too, which saves a pass over the evidence wherever
        # the clip is idle.  The same step timed there (the steps in
        # between untimed):
        while coords.step_number < 64:
            step()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(5):
            step()
        torch.cuda.synchronize()
        line["step_past_64_ms"] = round((time.perf_counter() - t1) / 5 * 1e3, 3)
        if not args.no_configs:
            line["configs"] = config_steps(device)
    line["cfg1"] = cfg1_lines(device, cpu=not args.no_cpu_baseline)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(d, ffn, T)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
