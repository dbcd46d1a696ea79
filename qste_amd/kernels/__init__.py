"""The operator layer: QSTE's ``qste.kernels`` API on gfx950 HIP kernels.

Same names, arguments, return values and error behaviour as the reference's
dispatch layer (``src/qste/kernels/loader.py:247-368``), for tensors on a
ROCm device.  Every call goes to ``libqste_hip.so`` through its C ABI
(``include/qste_hip.h``) on torch's current stream.  There is no CPU or
pure-torch path: a tensor that is not on the GPU, or a missing library, is an
error (``RuntimeError``), never a silent fallback.

Outputs are allocated through torch's caching allocator, as are the
workspaces the C entry points ask for; the library itself never allocates.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib
from ._lib import KernelError

_DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

__all__ = [
    "KernelError",
    "apply_bits",
    "masked_activation",
    "masked_backward",
    "pack_bits",
    "smooth_activation",
    "smooth_backward",
    "unpack_bits",
    "coordinate_update",
    "cuda_available",
    "embedding_backward",
    "packed_embedding",
    "evidence_from_packed",
    "linear_backward",
    "native_available",
    "pack_affine_rows",
    "pack_coordinate",
    "packed_linear_affine",
    "packed_row_inner",
    "packed_transpose",
    "status",
    "swiglu_backward",
    "swiglu_forward",
    "unpack_rows",
]


# ---------------------------------------------------------------------------
# plumbing
# ---------------------------------------------------------------------------


def _require_gpu(*tensors: Tensor) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"qste_amd kernels run on the GPU only; got a tensor on {t.device} "
                "(move the model to the ROCm device first)"
            )
        if device is None:
            device = t.device
        elif t.device != device:
            raise RuntimeError(f"tensors on different devices: {device} and {t.device}")
    if device is None:
        raise RuntimeError("no tensor argument to place the kernel on")
    return device


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    """The device's current HIP stream as an address (torch's current-stream
    query without building a Stream object where torch offers it)."""

    if _RAW_STREAM is not None and device.index is not None:
        return _RAW_STREAM(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def _dtype_code(t: Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32, float16 or bfloat16") from None


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _packed_width(columns: int) -> int:
    return (int(columns) + 7) // 8


def _check_packed(packed: Tensor, columns: int, rows: int | None = None) -> Tensor:
    if packed.dtype != torch.uint8 or packed.dim() != 2:
        raise ValueError("packed signs must be a rank-2 uint8 tensor")
    if packed.shape[1] != _packed_width(columns):
        raise ValueError(
            f"packed sign width {packed.shape[1]} does not match {columns} columns "
            f"(expected {_packed_width(columns)})"
        )
    if rows is not None and packed.shape[0] != rows:
        raise ValueError(f"packed signs have {packed.shape[0]} rows, expected {rows}")
    return packed.contiguous()


def _f32(t: Tensor | None) -> Tensor | None:
    """``t`` as contiguous fp32 (a new tensor unless it already is one).

    Bind the result to a name that lives until the C call returns: a
    temporary passed straight to ``_ptr`` is freed before the launch, and the
    caching allocator hands its block to the next allocation."""

    if t is None:
        return None
    return t.detach().to(torch.float32).contiguous()


def _aligned(t: Tensor) -> Tensor:
    """Contiguous, with the 16-byte start the vector paths need."""

    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _rows2d(t: Tensor, what: str) -> Tensor:
    if t.dim() != 2:
        raise ValueError(f"{what} expects a rank-2 tensor")
    return _aligned(t)


def _workspace(nbytes: int, device: torch.device) -> Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def native_available() -> bool:
    """Whether the HIP library loads (it does not need a GPU to load)."""

    try:
        _lib.load()
        return True
    except KernelError:
        return False


def cuda_available() -> bool:
    return torch.cuda.is_available() and native_available()


def status() -> dict:
    """Whether the HIP library is built and loadable, and why not if not."""

    ok = native_available()
    return {
        "native": ok,
        "library": str(_lib.LIB_PATH),
        "version": _lib.load().qste_version() if ok else None,
        "failure": _lib.failure(),
        "gpu": torch.cuda.is_available(),
    }


def stream_read(src: Tensor, groups: int | None = None) -> None:
    """A plain streaming read of ``src``'s bytes (measurement probe, no
    counterpart in the reference): the floor for any kernel reading them once."""

    device = _require_gpu(src)
    if not src.is_contiguous() or src.numel() * src.element_size() % 16:
        raise ValueError("stream_read needs a contiguous tensor of a multiple of 16 bytes")
    props = torch.cuda.get_device_properties(device)
    groups = int(groups or 4 * props.multi_processor_count)
    sink = torch.empty(groups * 256, dtype=torch.int32, device=device)
    lib = _lib.load()
    _lib.check(lib.qste_stream_read(_ptr(src), src.numel() * src.element_size(), _ptr(sink), groups,
                                    _stream(device)), "stream_read")


def device_info(device=None) -> dict:
    """What the runtime reports for ``device``: compute units, maximum shader
    clock and memory clock (MHz), LDS bytes per compute unit."""

    import ctypes

    device = torch.device(device or "cuda")
    out = (ctypes.c_int64 * 4)()
    with torch.cuda.device(device):
        _lib.check(_lib.load().qste_device_info(ctypes.cast(out, ctypes.c_void_p)), "device_info")
    return {"cus": int(out[0]), "max_sclk_mhz": out[1] / 1000.0, "mclk_mhz": out[2] / 1000.0,
            "lds_per_cu": int(out[3])}


def measured_sclk_mhz(device=None, spins: int = 1 << 18) -> float:
    """Shader clock one wave sees right now, in MHz: s_memtime cycles over
    s_memrealtime (100 MHz) ticks across a dependent integer loop."""

    device = torch.device(device or "cuda")
    out = torch.zeros(3, dtype=torch.int64, device=device)
    lib = _lib.load()
    _lib.check(lib.qste_clock_probe(_ptr(out), int(spins), _stream(device)), "clock_probe")
    cycles, ticks, _ = (int(v) for v in out.cpu().tolist())
    return cycles / ticks * 100.0 if ticks > 0 else float("nan")


def profile(device=None) -> str:
    """One line: what this build runs on ``device`` (reference
    ``kernels.profile(device).describe()``, src/qste/kernels/device.py:85-91).

    Nothing is autotuned: the kernels are written for gfx950 and take their
    grid sizes from the compute-unit count the runtime reports.  The line
    names the device and architecture, that count, the shader clock (the
    maximum the runtime reports and the one a wave measures now), HBM and LDS
    sizes, the library version, and which kernel each operator takes."""

    device = torch.device(device) if device is not None else torch.device(
        "cuda" if torch.cuda.is_available() else "cpu")
    version = _lib.load().qste_version() if native_available() else None
    if device.type != "cuda":
        return (f"{device} [no QSTE kernels: qste_amd runs on gfx950 GPUs only]  "
                f"library={'libqste_hip v%d' % version if version is not None else 'not built'}")
    props = torch.cuda.get_device_properties(device)
    arch = getattr(props, "gcnArchName", "?").split(":")[0]
    info = device_info(device)
    now_mhz = measured_sclk_mhz(device)
    return (f"{props.name} [{arch}]  cus={info['cus']}  "
            f"sclk={info['max_sclk_mhz']:.0f}MHz max / {now_mhz:.0f}MHz measured  "
            f"hbm={props.total_memory / 2**30:.0f}GiB  lds={info['lds_per_cu'] / 1024:.0f}KiB/CU  "
            f"library=libqste_hip v{version}  "
            "(products: bf16/fp16 MFMA 256x256 tiles, fp32 as three bf16 limbs; decode M<=16: biased-operand "
            "MFMA; coordinate step: one launch for columns % 2048 == 0, else six)")


# ---------------------------------------------------------------------------
# operators (reference: src/qste/kernels/loader.py:247-368)
# ---------------------------------------------------------------------------


def pack_coordinate(coordinate: Tensor) -> Tensor:
    """Sign bits of an int8 coordinate matrix, LSB first (fallback.py:91-92)."""

    device = _require_gpu(coordinate)
    if coordinate.dtype != torch.int8 or coordinate.dim() != 2:
        raise ValueError("pack_coordinate expects a rank-2 int8 tensor")
    coordinate = coordinate.contiguous()
    rows, cols = coordinate.shape
    packed = torch.empty(rows, _packed_width(cols), dtype=torch.uint8, device=device)
    code = _lib.load().qste_pack_coordinate(
        _ptr(coordinate), _ptr(packed), rows, cols, _stream(device))
    _lib.check(code, "pack_coordinate")
    return packed


def unpack_rows(packed: Tensor, columns: int, *, dtype: torch.dtype | None = None,
                row_scale: Tensor | None = None) -> Tensor:
    """+-1 matrix of the packed signs (fallback.py:27-29)."""

    dtype = dtype or torch.float32
    device = _require_gpu(packed, row_scale)
    packed = _check_packed(packed, columns)
    out = torch.empty(packed.shape[0], int(columns), dtype=dtype, device=device)
    row_scale_f32 = _f32(row_scale)  # held until the launch is queued
    code = _lib.load().qste_unpack_rows(
        _ptr(packed), _ptr(row_scale_f32), _ptr(out), _dtype_code(out), packed.shape[0],
        int(columns), _stream(device))
    _lib.check(code, "unpack_rows")
    return out


def pack_affine_rows(values: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """(bits, offset, scale) of each row: x ~ offset + scale * sign(x - offset).

    fallback.py:77-88. Arithmetic in fp32 on the dtype's values.  offset and
    scale are rows 0 and 1 of one fp32 [2, rows] tensor (``stacked_pair``).
    """

    device = _require_gpu(values)
    if values.dim() != 2:
        raise ValueError("pack_affine_rows expects a rank-2 tensor")
    values = values.contiguous()
    rows, cols = values.shape
    if cols == 0:
        raise ValueError("pack_affine_rows needs at least one column")
    packed = torch.empty(rows, _packed_width(cols), dtype=torch.uint8, device=device)
    # rows 0 and 1 of one [2, rows] tensor: the layout a saved encoding keeps
    offset, scale = torch.empty(2, rows, dtype=torch.float32, device=device).unbind(0)
    code = _lib.load().qste_pack_affine_rows(
        _ptr(values), _dtype_code(values), _ptr(packed), _ptr(offset), _ptr(scale), rows, cols,
        _stream(device))
    _lib.check(code, "pack_affine_rows")
    return packed, offset, scale


def stacked_pair(offset: Tensor, scale: Tensor) -> Tensor:
    """``torch.stack((offset, scale))``, without a copy when the two are rows
    0 and 1 of one [2, n] tensor (as ``pack_affine_rows`` returns them)."""

    base = offset._base
    n = offset.numel()
    if (base is not None and scale._base is base and base.dim() == 2 and base.shape[0] == 2
            and base.shape[1] == n and base.is_contiguous() and offset.dtype == scale.dtype == base.dtype
            and offset.data_ptr() == base.data_ptr()
            and scale.data_ptr() == base.data_ptr() + n * base.element_size()):
        return base
    return torch.stack((offset, scale))


def packed_linear_affine(inputs: Tensor, packed: Tensor, scale: Tensor, bias: Tensor | None,
                         columns: int) -> Tensor:
    """``(x @ sign^T) * scale + bias`` in the input dtype (fallback.py:95-108)."""

    device = _require_gpu(inputs, packed, scale, bias)
    if inputs.shape[-1] != columns:
        raise ValueError(f"activation width {inputs.shape[-1]} does not match {columns} columns")
    packed = _check_packed(packed, columns)
    rows = packed.shape[0]
    if scale.numel() != rows:
        raise ValueError("scale must have one entry per output row")
    if bias is not None and bias.numel() != rows:
        raise ValueError("bias must have one entry per output row")
    flat = inputs.reshape(-1, columns).contiguous()
    out = torch.empty(flat.shape[0], rows, dtype=inputs.dtype, device=device)
    scale_f32 = _f32(scale)  # held until the launch is queued
    bias_f32 = _f32(bias)  # held until the launch is queued
    lib = _lib.load()
    # fp32 runs its product through bf16 limbs on the MFMA path, in a
    # workspace; products with few output tiles split K there
    nbytes = lib.qste_packed_linear_affine_workspace_bytes(flat.shape[0], rows, int(columns), _dtype_code(flat))
    if nbytes:
        work = _workspace(nbytes, device)
        code = lib.qste_packed_linear_affine_ws(
            _ptr(flat), _dtype_code(flat), _ptr(packed), _ptr(scale_f32), _ptr(bias_f32),
            _ptr(out), flat.shape[0], rows, int(columns), _ptr(work), work.numel(), _stream(device))
    else:
        code = lib.qste_packed_linear_affine(
            _ptr(flat), _dtype_code(flat), _ptr(packed), _ptr(scale_f32), _ptr(bias_f32),
            _ptr(out), flat.shape[0], rows, int(columns), _stream(device))
    _lib.check(code, "packed_linear_affine")
    return out.view(*inputs.shape[:-1], rows)


def packed_transpose(inputs: Tensor, packed: Tensor, columns: int,
                     row_scale: Tensor | None = None) -> Tensor:
    """``inputs @ (row_scale * sign)`` in the input dtype (fallback.py:111-123)."""

    device = _require_gpu(inputs, packed, row_scale)
    packed = _check_packed(packed, columns)
    rows = packed.shape[0]
    if inputs.shape[-1] != rows:
        raise ValueError(f"transpose width {inputs.shape[-1]} does not match {rows} rows")
    if row_scale is not None and row_scale.numel() != rows:
        raise ValueError("transpose row scale must have one entry per packed row")
    flat = inputs.reshape(-1, rows).contiguous()
    out = torch.empty(flat.shape[0], int(columns), dtype=inputs.dtype, device=device)
    row_scale_f32 = _f32(row_scale)  # held until the launch is queued
    lib = _lib.load()
    nbytes = (lib.qste_packed_transpose_workspace_bytes(flat.shape[0], rows, int(columns), _dtype_code(flat))
              if row_scale_f32 is not None else 0)
    if nbytes:
        work = _workspace(nbytes, device)
        code = lib.qste_packed_transpose_ws(
            _ptr(flat), _dtype_code(flat), _ptr(packed), _ptr(row_scale_f32), _ptr(out),
            flat.shape[0], rows, int(columns), _ptr(work), work.numel(), _stream(device))
    else:
        code = lib.qste_packed_transpose(
            _ptr(flat), _dtype_code(flat), _ptr(packed), _ptr(row_scale_f32), _ptr(out),
            flat.shape[0], rows, int(columns), _stream(device))
    _lib.check(code, "packed_transpose")
    return out.view(*inputs.shape[:-1], int(columns))


def evidence_from_packed(grad: Tensor, packed: Tensor, columns: int,
                         row_scale: Tensor | None = None) -> Tensor:
    """``grad^T @ (row_scale * sign(x))`` as fp32 [rows, columns] (fallback.py:126-138)."""

    device = _require_gpu(grad, packed, row_scale)
    if grad.dim() != 2:
        raise ValueError("evidence grad must be a rank-2 tensor")
    packed = _check_packed(packed, columns)
    samples, rows = grad.shape
    if packed.shape[0] != samples:
        raise ValueError("evidence grad and packed activations disagree on sample count")
    if row_scale is not None and row_scale.numel() != samples:
        raise ValueError("evidence row scale must have one entry per sample")
    grad = grad.contiguous()
    out = torch.empty(rows, int(columns), dtype=torch.float32, device=device)
    row_scale_f32 = _f32(row_scale)  # held until the launch is queued
    lib = _lib.load()
    nbytes = lib.qste_evidence_from_packed_workspace_bytes_dtype(samples, rows, int(columns), _dtype_code(grad))
    work = _workspace(nbytes, device) if nbytes else None
    code = lib.qste_evidence_from_packed(
        _ptr(grad), _dtype_code(grad), _ptr(packed), _ptr(row_scale_f32), _ptr(out), samples,
        rows, int(columns), _ptr(work), 0 if work is None else work.numel(), _stream(device))
    _lib.check(code, "evidence_from_packed")
    return out


def packed_row_inner(matrix: Tensor, packed: Tensor, columns: int) -> Tensor:
    """``sum_c matrix[r, c] * sign[r, c]`` (fallback.py:141-148)."""

    device = _require_gpu(matrix, packed)
    if matrix.dim() != 2 or matrix.shape[1] != columns:
        raise ValueError("row inner shape mismatch")
    packed = _check_packed(packed, columns, matrix.shape[0])
    m = matrix.detach().to(torch.float32).contiguous()
    out = torch.empty(m.shape[0], dtype=torch.float32, device=device)
    code = _lib.load().qste_packed_row_inner(
        _ptr(m), _ptr(packed), _ptr(out), m.shape[0], int(columns), _stream(device))
    _lib.check(code, "packed_row_inner")
    return out.to(matrix.dtype)


def linear_backward(grad: Tensor, packed_x: Tensor, x_offset: Tensor, x_scale: Tensor,
                    packed_w: Tensor, scale: Tensor, columns: int, *, need_bias: bool,
                    need_input: bool = True, offset_dot: Tensor | None = None):
    """All of ``QSTELinearFn.backward``'s products in one call (functional.py:173-194).

    Returns ``(grad_input [samples, columns] in grad's dtype or None,
    evidence fp32 [rows, columns] already multiplied by the row scale,
    grad_scale fp32 [rows], grad_bias fp32 [rows] or None)``.  With
    ``need_input=False`` the input-gradient product is not computed (autograd
    asks for no gradient of the layer's input) and grad_input is None.
    ``offset_dot`` (fp32 [rows], ``sum_t grad[t, r] * x_offset[t]`` summed as
    this call sums it, e.g. by ``swiglu_backward_sums``) spares the call that
    pass over ``grad``; it is ignored when a bias gradient is formed.
    """

    device = _require_gpu(grad, packed_x, x_offset, x_scale, packed_w, scale)
    grad = grad.contiguous()
    samples, rows = grad.shape
    packed_w = _check_packed(packed_w, columns, rows)
    packed_x = _check_packed(packed_x, columns, samples)
    lib = _lib.load()
    dx = torch.empty(samples, int(columns), dtype=grad.dtype, device=device) if need_input else None
    evidence = torch.empty(rows, int(columns), dtype=torch.float32, device=device)
    grad_scale = torch.empty(rows, dtype=torch.float32, device=device)
    grad_bias = torch.empty(rows, dtype=torch.float32, device=device) if need_bias else None
    nbytes = lib.qste_linear_backward_workspace_bytes_dtype(samples, rows, int(columns), _dtype_code(grad))
    work = _workspace(nbytes, device)
    x_offset_f32 = _f32(x_offset)  # held until the launch is queued
    x_scale_f32 = _f32(x_scale)  # held until the launch is queued
    scale_f32 = _f32(scale)  # held until the launch is queued
    if offset_dot is not None:
        if offset_dot.dtype != torch.float32 or offset_dot.numel() != rows or offset_dot.device != device:
            raise ValueError("offset_dot must be fp32 [rows] on the layer's device")
        offset_dot = offset_dot.contiguous()
        code = lib.qste_linear_backward_offset_dot(
            _ptr(grad), _dtype_code(grad), _ptr(packed_x), _ptr(x_offset_f32), _ptr(x_scale_f32),
            _ptr(packed_w), _ptr(scale_f32), _ptr(dx), _ptr(evidence), _ptr(grad_scale),
            _ptr(grad_bias), _ptr(offset_dot), samples, rows, int(columns), _ptr(work), work.numel(),
            _stream(device))
    else:
        code = lib.qste_linear_backward(
            _ptr(grad), _dtype_code(grad), _ptr(packed_x), _ptr(x_offset_f32), _ptr(x_scale_f32),
            _ptr(packed_w), _ptr(scale_f32), _ptr(dx), _ptr(evidence), _ptr(grad_scale),
            _ptr(grad_bias), samples, rows, int(columns), _ptr(work), work.numel(), _stream(device))
    _lib.check(code, "linear_backward")
    return dx, evidence, grad_scale, grad_bias


def coordinate_update(
    gradient: Tensor,
    coordinate: Tensor,
    packed: Tensor,
    moment_q: Tensor,
    moment_scale: Tensor,
    row_v: Tensor,
    col_v: Tensor,
    *,
    beta1: float,
    beta2: float,
    update_clip: float,
    coordinate_lr: float,
    block_size: int,
    seed: int,
    step,
    flips: Tensor | None = None,
    update_enabled: Tensor | None = None,
):
    """One fused coordinate step (fallback.py:158-242; GPU signature cuda.py:1705-1729).

    Returns the flip count as an int, or -- when ``flips`` (a device int64
    tensor) is given -- writes it there without a host synchronization and
    returns that tensor. ``step`` may be a device int64 scalar (read at run
    time, for graph replay). ``update_enabled`` (device uint8) gates every
    state write. ``gradient`` is read, not modified.
    """

    device = _require_gpu(gradient, coordinate, packed, moment_q, moment_scale, row_v, col_v)
    if int(block_size) <= 0:
        raise ValueError("momentum block size must be positive")
    gradient = gradient.detach().to(torch.float32).contiguous()
    rows, cols = gradient.shape
    for name, t, dt in (("coordinate", coordinate, torch.int8), ("packed", packed, torch.uint8),
                        ("moment_q", moment_q, torch.int8), ("moment_scale", moment_scale, torch.float16),
                        ("row_v", row_v, torch.float16), ("col_v", col_v, torch.float16)):
        if t.dtype != dt:
            raise ValueError(f"{name} must be {dt}, got {t.dtype}")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous (it is updated in place)")
    if coordinate.shape != gradient.shape or moment_q.shape != gradient.shape:
        raise ValueError("coordinate state shape mismatch")
    if packed.shape != (rows, _packed_width(cols)):
        raise ValueError("packed sign shape mismatch")
    blocks = (rows * cols + block_size - 1) // block_size
    if moment_scale.numel() != blocks:
        raise ValueError("momentum scale shape mismatch")
    if row_v.numel() != rows or col_v.numel() != cols:
        raise ValueError("factored statistics shape mismatch")

    step_device = None
    step_value = 0
    if torch.is_tensor(step):
        if step.device != device or step.dtype != torch.int64:
            raise ValueError("a tensor step must be an int64 scalar on the surface's device")
        step_device = step
    else:
        step_value = int(step)
    enabled = None
    if update_enabled is not None:
        enabled = update_enabled.to(device=device, dtype=torch.uint8).contiguous()
    out = flips
    if out is None or out.dtype != torch.int64 or out.device != device:
        out_dev = torch.empty((), dtype=torch.int64, device=device)
    else:
        out_dev = out

    lib = _lib.load()
    nbytes = lib.qste_coordinate_update_workspace_bytes(rows, cols, int(block_size))
    work = _workspace(nbytes, device)
    wrap = lambda v: ((int(v) + (1 << 63)) % (1 << 64)) - (1 << 63)  # noqa: E731
    code = lib.qste_coordinate_update(
        _ptr(gradient), _ptr(coordinate), _ptr(packed), _ptr(moment_q), _ptr(moment_scale),
        _ptr(row_v), _ptr(col_v), rows, cols, float(beta1), float(beta2), float(update_clip),
        float(coordinate_lr), int(block_size), wrap(seed), wrap(step_value), _ptr(step_device),
        _ptr(out_dev), _ptr(enabled), _ptr(work), work.numel(), _stream(device))
    _lib.check(code, "coordinate_update")
    if flips is None:
        return int(out_dev.item())
    if out_dev is not flips:
        flips.copy_(out_dev)
    return flips


# ---------------------------------------------------------------------------
# packed activations (reference: loader.py:256-273, src/qste/nn.py)
# ---------------------------------------------------------------------------

# kinds of masked_activation / smooth_activation (include/qste_hip.h)
MASK_CLAMP, MASK_LEAKY, MASK_INTERVAL = 0, 1, 2
SMOOTH_KINDS = {
    "gelu": 0, "gelu_tanh": 1, "silu": 2, "tanh": 3, "sigmoid": 4, "elu": 5, "celu": 6,
    "selu": 7, "softplus": 8, "mish": 9, "hardswish": 10, "relu_square": 11, "provided": 12,
}


def pack_bits(mask: Tensor) -> Tensor:
    """One bit per element of a rank-2 mask, LSB first (fallback.py:32-47)."""

    device = _require_gpu(mask)
    if mask.dim() != 2:
        raise ValueError("packing expects a rank-2 tensor")
    if mask.dtype == torch.bool:
        mask = mask.contiguous().view(torch.uint8)
    elif mask.dtype != torch.uint8:
        mask = (mask != 0).view(torch.uint8)
    mask = _aligned(mask)
    rows, cols = mask.shape
    packed = torch.empty(rows, _packed_width(cols), dtype=torch.uint8, device=device)
    code = _lib.load().qste_pack_bits(_ptr(mask), _ptr(packed), rows, cols, _stream(device))
    _lib.check(code, "pack_bits")
    return packed


def unpack_bits(packed: Tensor, columns: int, *, dtype: torch.dtype | None = None) -> Tensor:
    """0/1 matrix of packed bits, pad columns dropped (fallback.py:50-54)."""

    dtype = dtype or torch.float32
    device = _require_gpu(packed)
    packed = _check_packed(packed, columns)
    out = torch.empty(packed.shape[0], int(columns), dtype=dtype, device=device)
    code = _lib.load().qste_unpack_bits(
        _ptr(packed), _ptr(out), _dtype_code(out), packed.shape[0], int(columns), _stream(device))
    _lib.check(code, "unpack_bits")
    return out


def apply_bits(values: Tensor, packed: Tensor, columns: int) -> Tensor:
    """``values`` where the bit is set, zero where it is not (fallback.py:57-70)."""

    return masked_backward(values, packed, columns)


def masked_backward(grad: Tensor, packed: Tensor, columns: int, *, inside: float = 1.0,
                    outside: float = 0.0) -> Tensor:
    """Backward of a one-bit activation (src/qste/nn.py:133-136, 168-181, 278-282, 364-368).

    ``kept = bit ? grad : 0``; ``kept * inside`` when ``outside == 0``, else
    ``grad * outside + kept * (inside - outside)``, each product rounded to
    the dtype like the reference's tensor expressions.
    """

    device = _require_gpu(grad, packed)
    grad = _rows2d(grad, "masked_backward")
    rows, cols = grad.shape
    if cols != columns:
        raise ValueError(f"value width {cols} does not match {columns} columns")
    packed = _check_packed(packed, columns, rows)
    out = torch.empty_like(grad)
    code = _lib.load().qste_masked_backward(
        _ptr(grad), _dtype_code(grad), _ptr(packed), _ptr(out), rows, cols, float(inside),
        float(outside), float(inside - outside), _stream(device))
    _lib.check(code, "masked_backward")
    return out


def masked_activation(x: Tensor, kind: int, *, lower: float = 0.0, upper: float | None = None,
                      slope: float = 0.0, want_output: bool = True) -> tuple[Tensor | None, Tensor]:
    """Forward of a one-bit activation and its packed mask, in one pass.

    ``x`` is rank 2; returns ``(output or None, packed)``.
    """

    device = _require_gpu(x)
    x = _rows2d(x, "masked_activation")
    rows, cols = x.shape
    out = torch.empty_like(x) if (want_output and kind != MASK_INTERVAL) else None
    packed = torch.empty(rows, _packed_width(cols), dtype=torch.uint8, device=device)
    code = _lib.load().qste_masked_activation(
        _ptr(x), _dtype_code(x), int(kind), float(lower), float(0.0 if upper is None else upper),
        0 if upper is None else 1, float(slope), _ptr(out), _ptr(packed), rows, cols,
        _stream(device))
    _lib.check(code, "masked_activation")
    return out, packed


def smooth_activation(x: Tensor | None, kind: str, param: float = 0.0, *,
                      output: Tensor | None = None,
                      derivative: Tensor | None = None) -> tuple[Tensor | None, Tensor, Tensor]:
    """Smooth activation with its row-quantized derivative (src/qste/nn.py:487-502).

    ``x`` rank 2.  When ``output`` is given it holds f(x) already and is read;
    otherwise f(x) is computed and returned.  ``kind == "provided"`` quantizes
    ``derivative`` (fp32) instead.  Returns ``(output, payload, scale)``:
    payload int8 (uint8 for ``relu_square``) ``[rows, cols]``, scale fp32 ``[rows]``.
    """

    code_kind = SMOOTH_KINDS[kind]
    if kind == "provided":
        device = _require_gpu(derivative)
        derivative = _rows2d(derivative.float(), "smooth_activation")
        rows, cols = derivative.shape
        dtype_code, x_ptr, y_ptr, y_given = 0, None, None, 0
        out = None
    else:
        device = _require_gpu(x, output)
        x = _rows2d(x, "smooth_activation")
        rows, cols = x.shape
        dtype_code = _dtype_code(x)
        if output is not None:
            output = _rows2d(output, "smooth_activation")
            if output.shape != x.shape or output.dtype != x.dtype:
                raise ValueError("output must match the input's shape and dtype")
            out, y_given = output, 1
        else:
            out, y_given = torch.empty_like(x), 0
        x_ptr, y_ptr = _ptr(x), _ptr(out)
    payload = torch.empty(rows, cols, dtype=torch.uint8 if kind == "relu_square" else torch.int8,
                          device=device)
    scale = torch.empty(rows, dtype=torch.float32, device=device)
    code = _lib.load().qste_smooth_activation(
        x_ptr, dtype_code, code_kind, float(param), y_ptr, y_given, _ptr(derivative),
        _ptr(payload), _ptr(scale), rows, cols, _stream(device))
    _lib.check(code, "smooth_activation")
    return out, payload, scale


def smooth_backward(grad: Tensor, payload: Tensor, scale: Tensor) -> Tensor:
    """``grad * (payload * scale)`` per row (src/qste/nn.py:504-507, 325-330)."""

    device = _require_gpu(grad, payload, scale)
    grad = _rows2d(grad, "smooth_backward")
    rows, cols = grad.shape
    if payload.shape != grad.shape or scale.shape != (rows,):
        raise ValueError("payload/scale do not match the gradient's shape")
    payload = _aligned(payload)
    out = torch.empty_like(grad)
    scale_f32 = _f32(scale)  # held until the launch is queued
    code = _lib.load().qste_smooth_backward(
        _ptr(grad), _dtype_code(grad), _ptr(payload), 1 if payload.dtype == torch.uint8 else 0,
        _ptr(scale_f32), _ptr(out), rows, cols, _stream(device))
    _lib.check(code, "smooth_backward")
    return out


# ---------------------------------------------------------------------------
# the SwiGLU gate (no counterpart in the reference)
# ---------------------------------------------------------------------------


def swiglu_forward(gate: Tensor, up: Tensor, *, encode: bool = False):
    """``silu(gate) * up`` with torch's roundings, in one pass.

    Returns ``(out, encoding)``; with ``encode`` the encoding is
    ``(packed, offset, scale)`` of ``out``'s rows as ``pack_affine_rows``
    gives them (last dimension = row), else None.
    """

    device = _require_gpu(gate, up)
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError("gate and up must have the same shape and dtype")
    g, u = _aligned(gate), _aligned(up)
    cols = int(g.shape[-1]) if g.dim() else 1
    rows = g.numel() // cols if cols else 0
    out = torch.empty_like(g)
    packed = offset = scale = None
    if encode:
        packed = torch.empty(rows, _packed_width(cols), dtype=torch.uint8, device=device)
        offset, scale = torch.empty(2, rows, dtype=torch.float32, device=device).unbind(0)
    code = _lib.load().qste_swiglu_forward(
        _ptr(g), _ptr(u), _dtype_code(g), _ptr(out), _ptr(packed), _ptr(offset), _ptr(scale), rows, cols,
        _stream(device))
    _lib.check(code, "swiglu_forward")
    return out, ((packed, offset, scale) if encode else None)


def swiglu_backward(grad: Tensor, gate: Tensor, up: Tensor) -> tuple[Tensor, Tensor]:
    """``(grad_gate, grad_up)`` of ``silu(gate) * up`` with torch's roundings."""

    device = _require_gpu(grad, gate, up)
    if not (grad.shape == gate.shape == up.shape) or not (grad.dtype == gate.dtype == up.dtype):
        raise ValueError("grad, gate and up must have the same shape and dtype")
    dh, g, u = _aligned(grad), _aligned(gate), _aligned(up)
    dg, du = torch.empty_like(g), torch.empty_like(g)
    code = _lib.load().qste_swiglu_backward(
        _ptr(dh), _ptr(g), _ptr(u), _dtype_code(g), _ptr(dg), _ptr(du), g.numel(), _stream(device))
    _lib.check(code, "swiglu_backward")
    return dg, du


def swiglu_backward_sums(grad: Tensor, gate: Tensor, up: Tensor, offset_gate: Tensor,
                         offset_up: Tensor, *, side_by_side: bool = False):
    """``swiglu_backward`` of [rows, cols] operands plus ``sums`` fp32 [2, cols]:
    ``sum_t grad_gate[t] * offset_gate[t]`` and ``sum_t grad_up[t] * offset_up[t]``,
    each what ``linear_backward`` would sum from that gradient and offset
    (its ``offset_dot``).  Returns ``(grad_gate, grad_up, sums)``.

    With ``side_by_side`` (16-bit dtypes, cols a multiple of 8) both
    gradients go into one [rows, 2 cols] tensor, grad_gate in its first
    cols columns and grad_up in the rest, and the call returns ``(grads,
    sums)``: two layers that read one input then run their backward as one
    ``linear_backward`` over ``grads`` and their concatenated signs
    (``qste_swiglu_backward_sums_into``)."""

    device = _require_gpu(grad, gate, up, offset_gate, offset_up)
    if not (grad.shape == gate.shape == up.shape) or not (grad.dtype == gate.dtype == up.dtype):
        raise ValueError("grad, gate and up must have the same shape and dtype")
    if grad.dim() != 2:
        raise ValueError("swiglu_backward_sums expects rank-2 operands")
    rows, cols = grad.shape
    offs = []
    for name, o in (("offset_gate", offset_gate), ("offset_up", offset_up)):
        if o.dtype != torch.float32 or o.numel() != rows:
            raise ValueError(f"{name} must be fp32 [rows]")
        offs.append(o.contiguous())
    dh, g, u = _aligned(grad), _aligned(gate), _aligned(up)
    sums = torch.empty(2, cols, dtype=torch.float32, device=device)
    lib = _lib.load()
    work = _workspace(lib.qste_swiglu_backward_sums_workspace_bytes(rows, cols), device)
    if side_by_side:
        both = torch.empty(rows, 2 * cols, dtype=g.dtype, device=device)
        code = lib.qste_swiglu_backward_sums_into(
            _ptr(dh), _ptr(g), _ptr(u), _dtype_code(g), _ptr(both), _ptr(offs[0]), _ptr(offs[1]), _ptr(sums),
            rows, cols, _ptr(work), work.numel(), _stream(device))
        _lib.check(code, "swiglu_backward_sums")
        return both, sums
    dg, du = torch.empty_like(g), torch.empty_like(g)
    code = lib.qste_swiglu_backward_sums(
        _ptr(dh), _ptr(g), _ptr(u), _dtype_code(g), _ptr(dg), _ptr(du), _ptr(offs[0]), _ptr(offs[1]),
        _ptr(sums), rows, cols, _ptr(work), work.numel(), _stream(device))
    _lib.check(code, "swiglu_backward_sums")
    return dg, du, sums


def row_scale(log_scale: Tensor, lo: float, hi: float) -> tuple[Tensor, Tensor]:
    """``(clamp(exp(log_scale), lo, hi), exp(log_scale))`` in log_scale's
    dtype (fp32, fp16 or bf16), one launch (surface.py:84-85), rounded as
    torch's ``exp().clamp()`` on that dtype."""

    device = _require_gpu(log_scale)
    ls = log_scale.detach().contiguous()
    scale, e = torch.empty_like(ls), torch.empty_like(ls)
    code = _lib.load().qste_row_scale(_ptr(ls), _dtype_code(ls), _ptr(scale), _ptr(e), ls.numel(), float(lo),
                                      float(hi), _stream(device))
    _lib.check(code, "row_scale")
    return scale, e


def row_scale_backward(exp_value: Tensor, grad: Tensor, lo: float, hi: float) -> Tensor:
    """Gradient of ``row_scale`` at log_scale: ``(lo <= e <= hi ? grad : 0) * e``,
    in e's dtype (grad is taken in that dtype)."""

    device = _require_gpu(exp_value, grad)
    if grad.shape != exp_value.shape:
        raise ValueError("row_scale_backward takes operands of one shape")
    e, g = exp_value.contiguous(), grad.to(exp_value.dtype).contiguous()
    out = torch.empty_like(e)
    code = _lib.load().qste_row_scale_backward(_ptr(e), _ptr(g), _dtype_code(e), _ptr(out), e.numel(), float(lo),
                                               float(hi), _stream(device))
    _lib.check(code, "row_scale_backward")
    return out


# ---------------------------------------------------------------------------
# binary embedding (reference: cuda.py:1691-1702, functional.py:260-287)
# ---------------------------------------------------------------------------


def _check_ids(ids: Tensor, rows: int) -> Tensor:
    flat = ids.reshape(-1).to(torch.int64).contiguous()
    if flat.numel():
        lo, hi = torch.stack(torch.aminmax(flat)).tolist()  # one reduction, one copy to the host
    if flat.numel() and (lo < 0 or hi >= rows):
        raise IndexError(f"embedding id out of range for {rows} rows")
    return flat


def packed_embedding(ids: Tensor, packed: Tensor, scale: Tensor, columns: int) -> Tensor:
    """``sign(packed[ids]) * scale[ids]``, shape ``ids.shape + (columns,)``, in scale's dtype.

    fallback.py:151-155.
    """

    device = _require_gpu(ids, packed, scale)
    packed = _check_packed(packed, columns)
    rows = packed.shape[0]
    if scale.shape != (rows,):
        raise ValueError(f"scale has shape {tuple(scale.shape)}, expected ({rows},)")
    flat = _check_ids(ids, rows)
    out_dtype = scale.dtype if scale.dtype in _DTYPES else torch.float32
    out = torch.empty(flat.numel(), int(columns), dtype=out_dtype, device=device)
    scale_f32 = _f32(scale)  # held until the launch is queued
    code = _lib.load().qste_packed_embedding(
        _ptr(flat), flat.numel(), _ptr(packed), _ptr(scale_f32), _ptr(out), _dtype_code(out), rows,
        int(columns), _stream(device))
    _lib.check(code, "packed_embedding")
    return out.view(*ids.shape, int(columns)).to(scale.dtype)


def embedding_backward(ids: Tensor, grad: Tensor, packed: Tensor, scale: Tensor,
                       columns: int) -> tuple[Tensor, Tensor]:
    """``(evidence, grad_scale)`` of an embedding (functional.py:274-286).

    ``evidence = zeros(R, C).index_add_(0, ids, grad) * scale[r]`` (fp32,
    token-order sums) and ``grad_scale = row_inner(index_add_, signs)``.
    """

    device = _require_gpu(ids, grad, packed, scale)
    packed = _check_packed(packed, columns)
    rows = packed.shape[0]
    flat = _check_ids(ids, rows)
    g = grad.reshape(-1, int(columns)).contiguous()
    if g.shape[0] != flat.numel():
        raise ValueError("gradient rows do not match the number of ids")
    evidence = torch.empty(rows, int(columns), dtype=torch.float32, device=device)
    grad_scale = torch.empty(rows, dtype=torch.float32, device=device)
    lib = _lib.load()
    ws = _workspace(lib.qste_embedding_backward_workspace_bytes(flat.numel(), rows), device)
    scale_f32 = _f32(scale)  # held until the launch is queued
    code = lib.qste_embedding_backward(
        _ptr(flat), flat.numel(), _ptr(g), _dtype_code(g), _ptr(packed), _ptr(scale_f32),
        _ptr(evidence), _ptr(grad_scale), rows, int(columns), _ptr(ws), ws.numel(), _stream(device))
    _lib.check(code, "embedding_backward")
    return evidence, grad_scale
