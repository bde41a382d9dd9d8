"""torch-facing wrappers over the C ABI (device memory and streams only).

Every function here launches HIP kernels from ``librepresentax_amd.so`` on
torch's current stream. Tensors must live on a ROCm device; there is no CPU
implementation, and a missing library or a CPU tensor raises.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _native as nat

BF16 = torch.bfloat16
F32 = torch.float32


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# torch's current-stream handle without building a Stream object (a few
# microseconds per call on the small-M path, where the kernels take ~10)
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _raw_stream(device: torch.device) -> int:
    if _RAW_STREAM is not None:
        return int(_RAW_STREAM(_device_index(device)))
    return int(torch.cuda.current_stream(device).cuda_stream)


def _stream(device: torch.device) -> int:
    return _raw_stream(device)


def _dtype_code(dtype: torch.dtype) -> int:
    if dtype == BF16:
        return nat.DTYPE_BF16
    if dtype == F32:
        return nat.DTYPE_F32
    raise TypeError(f"unsupported dtype {dtype}; expected float32 or bfloat16")


def _on_device(*tensors: torch.Tensor | None) -> torch.device:
    device = None
    index = -1
    for t in tensors:
        if t is None:
            continue
        i = t.get_device()  # -1 off the GPU
        if i < 0:
            raise RuntimeError(
                "representax_amd kernels run on ROCm devices only; got a tensor on "
                f"{t.device}"
            )
        if device is None:
            device = t.device
            index = i
        elif i != index:
            raise RuntimeError("all operands must be on the same device")
    if device is None:
        raise RuntimeError("no device tensor given")
    nat.load()
    return device


# One scratch buffer per (device, stream), grown on demand. A stream runs its
# calls one after another, so consecutive calls may share it; calls on other
# streams get their own. Calls made under graph capture get a buffer of their
# own from the graph's memory pool, since a graph keeps its buffer for every
# replay.
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def _workspace(nbytes: int, device: torch.device, stream: int | None = None) -> torch.Tensor:
    """``stream``: the device's current raw stream when the caller has it."""

    nbytes = max(int(nbytes), 1)
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    index = _device_index(device)
    key = (index, _raw_stream(device) if stream is None else stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=torch.device("cuda", index))
        _WORKSPACES[key] = ws
    return ws


def _round16(nbytes: int) -> int:
    return -(-int(nbytes) // 16) * 16


def _workspace_with_tails(nbytes: int, tails, device: torch.device,
                          stream: int | None = None) -> tuple[torch.Tensor, list[int]]:
    """The call's scratch (its first ``nbytes``, which the library is given)
    followed by one 16-byte aligned region per entry of ``tails`` (bytes):
    ``(buffer, [address of each region])``."""

    head = _round16(max(int(nbytes), 1))
    ws = _workspace(head + sum(_round16(t) for t in tails), device, stream)
    addrs, at = [], ws.data_ptr() + head
    for t in tails:
        addrs.append(at)
        at += _round16(t)
    return ws, addrs


def release_workspaces() -> None:
    """Drop the cached per-stream scratch buffers (back to torch's allocator)."""

    _WORKSPACES.clear()


def _aligned(t: torch.Tensor | None) -> torch.Tensor | None:
    """Dense and 16-byte aligned (the vectorized kernels' contract); copies
    only views that are not."""

    if t is None:
        return None
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _as(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return t if t.dtype == dtype else t.to(dtype)


def _u16(t: torch.Tensor) -> torch.Tensor:
    """View bf16/int16/uint16 storage as uint16 bit patterns."""

    if t.dtype == torch.uint16:
        return t
    if t.dtype in (BF16, torch.int16):
        return t.view(torch.uint16)
    raise TypeError(f"expected 16-bit bit patterns, got {t.dtype}")


def _ready(index: int, tensors) -> list[int] | None:
    """The addresses of ``tensors`` when each is on device ``index``, dense
    and 16-byte aligned (the form the kernels take as is); None otherwise."""

    ptrs = []
    for t in tensors:
        p = t.data_ptr()
        if p & 15 or t.get_device() != index or not t.is_contiguous():
            return None
        ptrs.append(p)
    return ptrs


def _bias_ready(bias_bits, index: int):
    """(ok, address) of optional bias bits already in the kernels' form:
    uint16, on device ``index``, dense."""

    if bias_bits is None:
        return True, None
    if bias_bits.dtype != torch.uint16 or bias_bits.get_device() != index or not bias_bits.is_contiguous():
        return False, None
    return True, bias_bits.data_ptr()


def group_arg(group_size: int | None, k: int) -> int:
    return 0 if group_size is None or group_size == k else int(group_size)


def _shape_error(what: str, got, want) -> ValueError:
    return ValueError(f"{what}: shape {tuple(got)}, expected {tuple(want)}")


def _lora_dims(x2d, packed, scale_bits, lora_a, lora_b, group_size, bias_bits=None):
    """``(m, k, n, r)`` of an INT4 + LoRA call after checking that every
    operand has the extent the kernels will read: packed ``[N, ceil(K/2)]``
    uint8, N * (K / G) scale values (N for one scale per row), A ``[r, K]``,
    B ``[N, r]`` and N bias values. The C ABI takes plain pointers and sizes,
    so a mismatched tensor would be read past its end; this raises
    ``ValueError`` before any launch. (Written for host time: each torch
    attribute is read once.)"""

    xs = x2d.shape
    if len(xs) != 2:
        raise ValueError(f"x must be 2-D [M, K], got shape {tuple(xs)}")
    m, k = xs
    n, r = _weight_dims(k, packed, scale_bits, lora_a, lora_b, group_size, bias_bits)
    return m, k, n, r


def _weight_dims(k, packed, scale_bits, lora_a, lora_b, group_size, bias_bits=None):
    """``(n, r)`` of an INT4 + LoRA weight with K inputs, after the extent
    checks of ``_lora_dims``."""

    ps = packed.shape
    if packed.dtype != torch.uint8 or len(ps) != 2:
        raise ValueError(f"packed weight must be uint8 [N, ceil(K/2)], got {packed.dtype} "
                         f"{tuple(ps)}")
    n, pc = ps
    if pc != (k + 1) // 2:
        raise _shape_error("packed weight", ps, (n, (k + 1) // 2))
    g = 0 if group_size is None or group_size == k else group_size
    groups = k // g if g > 0 and k % g == 0 else 1
    if scale_bits.numel() != n * groups:
        raise _shape_error("scale_bits", scale_bits.shape, (n, groups))
    sa = lora_a.shape
    if len(sa) != 2 or sa[1] != k:
        raise _shape_error("lora_a", sa, ("r", k))
    r = sa[0]
    if lora_b.shape != (n, r):
        raise _shape_error("lora_b", lora_b.shape, (n, r))
    if bias_bits is not None and bias_bits.numel() != n:
        raise _shape_error("bias", bias_bits.shape, (n,))
    return n, r


def _check_extent(name: str, t, shape) -> None:
    if t is not None and tuple(t.shape) != tuple(shape):
        raise _shape_error(name, t.shape, shape)


# ---------------------------------------------------------------------------
# Kernel-variant knobs and the device error word
# ---------------------------------------------------------------------------
TUNING_KNOBS = {
    "int4_tile": nat.TUNE_INT4_TILE,
    "bf16_tile": nat.TUNE_BF16_TILE,
    "fp8_tile": nat.TUNE_FP8_TILE,
    "skinny_tile": nat.TUNE_SKINNY_TILE,
    "skinny2": nat.TUNE_SKINNY2,
    "skinny2_one": nat.TUNE_SKINNY2_ONE,
    "spin_limit": nat.TUNE_SPIN_LIMIT,
    "gemm_band": nat.TUNE_GEMM_BAND,
    "dx_packed": nat.TUNE_DX_PACKED,
    "rank_blocks": nat.TUNE_RANK_BLOCKS,
    "rank_nt_u": nat.TUNE_RANK_NT_U,
    "fp8_splits": nat.TUNE_FP8_SPLITS,
    "fp8_pair": nat.TUNE_FP8_PAIR,
}


def get_tuning(knob: str) -> int:
    return int(nat.load().rpx_get_tuning(TUNING_KNOBS[knob]))


def set_tuning(knob: str, value: int) -> int:
    """Force a kernel variant for later calls (process-wide); returns the
    previous value. ``ValueError`` for an unknown value."""

    code = TUNING_KNOBS[knob]
    previous = get_tuning(knob)
    nat.call("rpx_set_tuning", code, int(value))
    return previous


class tuning:
    """Context manager: ``with ops.tuning(int4_tile=10): ...`` sets knobs for
    the block and restores their previous values afterwards."""

    def __init__(self, **knobs: int):
        self._knobs = knobs
        self._saved: dict[str, int] = {}

    def __enter__(self):
        for name, value in self._knobs.items():
            self._saved[name] = set_tuning(name, value)
        return self

    def __exit__(self, *exc):
        for name, value in self._saved.items():
            set_tuning(name, value)
        return False


def check_device_errors(device: torch.device | None = None) -> int:
    """Synchronize the current stream and raise ``DeviceError`` if a kernel
    reported an expired bounded wait since the last check (its outputs then
    hold NaN); returns the raw bits otherwise (0)."""

    nat.load()
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    flags = ctypes.c_uint32(0)
    with torch.cuda.device(dev):
        nat.call("rpx_check_device_errors", _stream(dev), ctypes.byref(flags))
    return int(flags.value)


# ---------------------------------------------------------------------------
# INT4 codec
# ---------------------------------------------------------------------------
def int4_pack(weight: torch.Tensor, group_size: int | None = None):
    """Quantize ``weight[*, N, K]`` -> ``(packed uint8[*, N, ceil(K/2)], scale_bits)``.

    ``scale_bits`` is ``uint16[*, N]`` (one bf16 scale per row, the reference
    scheme) or ``uint16[*, N, K/G]`` with ``group_size=G``.
    """

    device = _on_device(weight)
    *stack, n, k = weight.shape
    w = weight.contiguous()
    if w.dtype not in (F32, BF16):
        w = w.to(F32)
    rows = int(math.prod(stack)) * n if stack else n
    packed = torch.empty((*stack, n, (k + 1) // 2), dtype=torch.uint8, device=device)
    g = group_arg(group_size, k)
    scale_shape = (*stack, n) if g == 0 else (*stack, n, k // g)
    scales = torch.empty(scale_shape, dtype=torch.uint16, device=device)
    nat.call("rpx_int4_pack", _ptr(w), _dtype_code(w.dtype), rows, k, g, _ptr(packed),
             _ptr(scales), _stream(device))
    return packed, scales


def int4_dequant(packed: torch.Tensor, scale_bits: torch.Tensor, input_size: int,
                 group_size: int | None = None) -> torch.Tensor:
    """``bf16[*, N, K]`` dequantized weight, bit-exact ``bf16(q * s)``."""

    device = _on_device(packed, scale_bits)
    *stack, n, pc = packed.shape
    k = int(input_size)
    if pc != (k + 1) // 2:
        raise ValueError("packed width does not match input_size")
    rows = int(math.prod(stack)) * n if stack else n
    out = torch.empty((*stack, n, k), dtype=BF16, device=device)
    nat.call("rpx_int4_dequant", _ptr(packed.contiguous()), _ptr(_u16(scale_bits).contiguous()),
             rows, k, group_arg(group_size, k), _ptr(out), _stream(device))
    return out


def int4_merge(packed, scale_bits, lora_a, lora_b, *, alpha: float, rank: int, input_size: int,
               group_size: int | None = None) -> torch.Tensor:
    """float32 ``f32(W_b) + (B @ A) * (alpha / rank)`` for one ``[N, K]`` slice."""

    k = int(input_size)
    n, _ = _weight_dims(k, packed, scale_bits, lora_a, lora_b, group_size)
    if lora_a.shape[0] != int(rank):
        raise _shape_error("lora_a", lora_a.shape, (int(rank), k))
    device = _on_device(packed, scale_bits, lora_a, lora_b)
    out = torch.empty((n, k), dtype=F32, device=device)
    nat.call("rpx_int4_merge", _ptr(packed.contiguous()), _ptr(_u16(scale_bits).contiguous()),
             _ptr(lora_a.to(F32).contiguous()), _ptr(lora_b.to(F32).contiguous()), n, k,
             group_arg(group_size, k), int(rank), float(alpha / rank), _ptr(out),
             _stream(device))
    return out


# ---------------------------------------------------------------------------
# INT4 + LoRA linear
# ---------------------------------------------------------------------------
def _forward_ready(fast, x2d, packed, scale_bits, a, b, scaling, group_size, bias_bits, need_h):
    """int4lora_forward through the fast binding when every operand is
    already in the kernels' form (one device, dense, 16-byte aligned, A and B
    in x's dtype, uint16 scale and bias bits): one pass over the operands
    instead of a check and a conversion each, which is most of a small-M
    call's host time. None otherwise; the general path then converts, copies
    or raises."""

    dt = x2d.dtype
    if a.dtype != dt or b.dtype != dt or scale_bits.dtype != torch.uint16:
        return None
    m, k, n, r = _lora_dims(x2d, packed, scale_bits, a, b, group_size, bias_bits)
    index = x2d.get_device()
    ptrs = _ready(index, (x2d, packed, scale_bits, a, b))
    ok, pb = _bias_ready(bias_bits, index)
    if index < 0 or ptrs is None or not ok:
        return None
    code = _dtype_code(dt)
    g = group_arg(group_size, k)
    device = x2d.device
    y = torch.empty((m, n), dtype=dt, device=device)
    stream = _stream(device)
    ws_bytes = fast.int4lora_forward_workspace(m, n, k, g, r, code)
    if need_h:
        h = torch.empty((m, r), dtype=dt, device=device)
        ws = _workspace(ws_bytes, device, stream)
        ws_bytes, h_ptr = ws.numel(), h.data_ptr()
    else:
        h = None
        ws, (h_ptr,) = _workspace_with_tails(ws_bytes, (m * r * dt.itemsize,), device, stream)
    nat.check(fast.int4lora_forward(ptrs[0], code, m, k, ptrs[1], ptrs[2], n, g, pb, ptrs[3],
                                    ptrs[4], r, float(scaling), y.data_ptr(), h_ptr,
                                    ws.data_ptr(), ws_bytes, stream))
    return y, h


def int4lora_forward(x2d, packed, scale_bits, lora_a_c, lora_b_c, *, scaling: float,
                     group_size: int | None = None, bias_bits=None, need_h: bool = True):
    """Return ``(y [M, N], h [M, r])`` in x's compute dtype.

    ``need_h=False`` (inference: no backward will read h) returns
    ``(y, None)``: the kernels still form h, in the call's scratch, and only
    y is allocated."""

    fast = nat.fast()
    if fast is not None:
        out = _forward_ready(fast, x2d, packed, scale_bits, lora_a_c, lora_b_c, scaling,
                             group_size, bias_bits, need_h)
        if out is not None:
            return out
    m, k, n, r = _lora_dims(x2d, packed, scale_bits, lora_a_c, lora_b_c, group_size, bias_bits)
    device = _on_device(x2d, packed, scale_bits, lora_a_c, lora_b_c, bias_bits)
    dt = x2d.dtype
    code = _dtype_code(dt)
    x2d = _aligned(x2d)
    a = _aligned(_as(lora_a_c, dt))
    b = _aligned(_as(lora_b_c, dt))
    y = torch.empty((m, n), dtype=dt, device=device)
    h = torch.empty((m, r), dtype=dt, device=device) if need_h else None
    g = group_arg(group_size, k)
    bias = None if bias_bits is None else _u16(bias_bits).contiguous()
    packed = _aligned(packed)
    scale_bits = _aligned(_u16(scale_bits))
    fast = nat.fast()
    stream = _stream(device)
    if fast is not None:
        ws_bytes = fast.int4lora_forward_workspace(m, n, k, g, r, code)
    else:
        ws_bytes = nat.query("rpx_int4lora_forward_workspace", m, n, k, g, r, code)
    if need_h:
        ws = _workspace(ws_bytes, device, stream)
        ws_bytes, h_ptr = ws.numel(), h.data_ptr()
    else:
        ws, (h_ptr,) = _workspace_with_tails(ws_bytes, (m * r * dt.itemsize,), device, stream)
    if fast is not None:
        nat.check(fast.int4lora_forward(
            x2d.data_ptr(), code, m, k, packed.data_ptr(), scale_bits.data_ptr(), n, g, _ptr(bias),
            a.data_ptr(), b.data_ptr(), r, float(scaling), y.data_ptr(), h_ptr,
            ws.data_ptr(), ws_bytes, stream))
    else:
        nat.call("rpx_int4lora_forward", _ptr(x2d), code, m, k, _ptr(packed), _ptr(scale_bits), n,
                 g, _ptr(bias), _ptr(a), _ptr(b), r, float(scaling), _ptr(y), h_ptr, _ptr(ws),
                 ws_bytes, stream)
    return y, h


# Up to this many rows, int4lora_forward_multi takes all of its outputs from
# one allocation: at small M a call costs more host time than GPU time, and
# one allocator call in place of two per projection is a large share of it.
# The outputs then share one storage, which lives until the last of them is
# freed (a few KB per projection at these sizes).
SHARED_OUTPUT_ROWS = 64
# fields per projection in the fast binding's flat tuple
PROJECTION_FIELDS = 11


def _dense_views(m: int, cols, dtype: torch.dtype, device: torch.device) -> list[torch.Tensor]:
    """``[t [m, c] for c in cols]`` as dense views of one allocation, each
    starting on a 16-byte boundary."""

    per16 = 16 // dtype.itemsize
    offsets, total = [], 0
    for c in cols:
        offsets.append(total)
        total += -(-m * c // per16) * per16
    buf = torch.empty(total, dtype=dtype, device=device)
    return [buf.as_strided((m, c), (c, 1), o) for c, o in zip(cols, offsets)]


def _multi_ready(fast, x2d, projections, need_h):
    """int4lora_forward_multi through the fast binding at M <= 64 when every
    operand is already in the kernels' form (as for ``_forward_ready``);
    None otherwise."""

    dt = x2d.dtype
    if x2d.dim() != 2 or x2d.shape[0] > SHARED_OUTPUT_ROWS:
        return None
    index = x2d.get_device()
    px = _ready(index, (x2d,))
    if index < 0 or px is None:
        return None
    m, k = x2d.shape
    flat, dims = [], []
    for packed, scale_bits, a, b, scaling, group_size, bias_bits in projections:
        if a.dtype != dt or b.dtype != dt or scale_bits.dtype != torch.uint16:
            return None
        _, _, n, r = _lora_dims(x2d, packed, scale_bits, a, b, group_size, bias_bits)
        ptrs = _ready(index, (packed, scale_bits, a, b))
        ok, pb = _bias_ready(bias_bits, index)
        if ptrs is None or not ok:
            return None
        dims.append((n, r))
        # y's and h's addresses (the last two fields) are filled in below;
        # the size query reads the shapes only
        flat += (ptrs[0], ptrs[1], n, group_arg(group_size, k), pb, ptrs[2], ptrs[3], r,
                 float(scaling), 0, 0)
    code = _dtype_code(dt)
    device = x2d.device
    if need_h:
        views = _dense_views(m, [c for nr in dims for c in nr], dt, device)
        ys, hs = views[0::2], views[1::2]
    else:
        ys, hs = _dense_views(m, [n for n, _ in dims], dt, device), [None] * len(dims)
    stream = _stream(device)
    ws_bytes = fast.int4lora_forward_multi_workspace(m, k, tuple(flat), code)
    if need_h:
        ws = _workspace(ws_bytes, device, stream)
        ws_bytes = ws.numel()
        h_ptrs = [h.data_ptr() for h in hs]
    else:
        ws, h_ptrs = _workspace_with_tails(ws_bytes, [m * r * dt.itemsize for _, r in dims],
                                           device, stream)
    for i, (y, h_ptr) in enumerate(zip(ys, h_ptrs)):
        flat[PROJECTION_FIELDS * i + 9] = y.data_ptr()
        flat[PROJECTION_FIELDS * i + 10] = h_ptr
    nat.check(fast.int4lora_forward_multi(px[0], code, m, k, tuple(flat), ws.data_ptr(), ws_bytes,
                                          stream))
    return list(zip(ys, hs))


def int4lora_forward_multi(x2d, projections, need_h: bool = True):
    """Several INT4 + LoRA projections of one input: ``projections`` is a
    sequence of ``(packed, scale_bits, lora_a_c, lora_b_c, scaling,
    group_size, bias_bits)``; returns ``[(y, h), ...]`` as
    ``int4lora_forward`` gives for each (``h`` None with ``need_h=False``).
    At small M (bf16, M <= 4, one rank) they run in one pair of launches."""

    projections = list(projections)
    count = len(projections)
    fast = nat.fast() if count <= 16 else None
    if fast is not None:
        out = _multi_ready(fast, x2d, projections, need_h)
        if out is not None:
            return out
    tensors = [x2d]
    for p in projections:
        tensors += [p[0], p[1], p[2], p[3], p[6]]
        _lora_dims(x2d, p[0], p[1], p[2], p[3], p[5], p[6])
    device = _on_device(*tensors)
    m, k = x2d.shape
    dt = x2d.dtype
    code = _dtype_code(dt)
    x2d = _aligned(x2d)
    table = None if fast is not None else (nat.Int4LoraProjection * count)()
    dims = [(p[0].shape[-2], p[2].shape[0]) for p in projections]
    if m <= SHARED_OUTPUT_ROWS:
        if need_h:
            views = _dense_views(m, [c for nr in dims for c in nr], dt, device)
            ys, hs = views[0::2], views[1::2]
        else:
            ys, hs = _dense_views(m, [n for n, _ in dims], dt, device), [None] * count
    else:
        ys = [torch.empty((m, n), dtype=dt, device=device) for n, _ in dims]
        hs = [torch.empty((m, r), dtype=dt, device=device) if need_h else None for _, r in dims]
    flat = []
    keep = []
    for i, (packed, scale_bits, lora_a_c, lora_b_c, scaling, group_size, bias_bits) in enumerate(projections):
        n, r = dims[i]
        a = _aligned(_as(lora_a_c, dt))
        b = _aligned(_as(lora_b_c, dt))
        pk = _aligned(packed)
        sc = _aligned(_u16(scale_bits))
        bias = None if bias_bits is None else _u16(bias_bits).contiguous()
        keep += [a, b, pk, sc, bias]
        # h's address (the last field) is filled in below once the scratch
        # is known; the size queries read the shapes only
        fields = (pk.data_ptr(), sc.data_ptr(), n, group_arg(group_size, k), _ptr(bias),
                  a.data_ptr(), b.data_ptr(), r, float(scaling), ys[i].data_ptr(),
                  0 if hs[i] is None else hs[i].data_ptr())
        if fast is not None:
            flat += fields
        else:
            table[i] = nat.Int4LoraProjection(*fields)
    stream = _stream(device)
    if fast is not None:
        ws_bytes = fast.int4lora_forward_multi_workspace(m, k, tuple(flat), code)
    else:
        ws_bytes = nat.query("rpx_int4lora_forward_multi_workspace", m, k, count, table, code)
    if need_h:
        ws = _workspace(ws_bytes, device, stream)
        ws_bytes = ws.numel()
    else:
        ws, h_ptrs = _workspace_with_tails(ws_bytes, [m * r * dt.itemsize for _, r in dims],
                                           device, stream)
        for i, h_ptr in enumerate(h_ptrs):
            if fast is not None:
                flat[PROJECTION_FIELDS * i + PROJECTION_FIELDS - 1] = h_ptr
            else:
                table[i].h = h_ptr
    if fast is not None:
        nat.check(fast.int4lora_forward_multi(x2d.data_ptr(), code, m, k, tuple(flat),
                                              ws.data_ptr(), ws_bytes, stream))
    else:
        nat.call("rpx_int4lora_forward_multi", _ptr(x2d), code, m, k, count, table, _ptr(ws),
                 ws_bytes, stream)
    del keep
    return list(zip(ys, hs))


def int4lora_backward(grad, x2d, packed, scale_bits, lora_a_c, lora_b_c, h, *, scaling: float,
                      group_size: int | None = None):
    """Return ``(dx [M, K], dA f32 [r, K], dB f32 [N, r])``."""

    m, k, n, r = _lora_dims(x2d, packed, scale_bits, lora_a_c, lora_b_c, group_size)
    _check_extent("grad", grad, (m, n))
    _check_extent("h", h, (m, r))
    device = _on_device(grad, x2d, packed, scale_bits, lora_a_c, lora_b_c, h)
    dt = x2d.dtype
    code = _dtype_code(dt)
    grad = _aligned(grad.to(dt))
    a = _aligned(_as(lora_a_c, dt))
    b = _aligned(_as(lora_b_c, dt))
    dx = torch.empty((m, k), dtype=dt, device=device)
    d_a = torch.empty((r, k), dtype=F32, device=device)
    d_b = torch.empty((n, r), dtype=F32, device=device)
    g = group_arg(group_size, k)
    ws_bytes = nat.query("rpx_int4lora_backward_workspace", m, n, k, g, r, code)
    ws = _workspace(ws_bytes, device)
    nat.call("rpx_int4lora_backward", _ptr(grad), _ptr(_aligned(x2d)), code, m, k,
             _ptr(_aligned(packed)), _ptr(_aligned(_u16(scale_bits))), n, g, _ptr(a),
             _ptr(b), r, float(scaling), _ptr(h.contiguous()), _ptr(dx), _ptr(d_a), _ptr(d_b),
             _ptr(ws), ws.numel(), _stream(device))
    return dx, d_a, d_b


ACTIVATIONS = {"gelu": nat.ACT_GELU, "silu_mul": nat.ACT_SILU_MUL, "add": nat.ACT_ADD}


def int4lora_forward_act(x2d, packed, scale_bits, lora_a_c, lora_b_c, *, activation: str,
                         scaling: float, group_size: int | None = None, bias_bits=None,
                         gate=None):
    """The FFN's up projection with its activation fused into the GEMM's
    epilogue: ``(y, z, h)`` with z the linear's output, y = gelu(z)
    (``"gelu"``) or silu(gate) * z (``"silu_mul"``, gate [M, N])."""

    act = ACTIVATIONS[activation]
    m, k, n, r = _lora_dims(x2d, packed, scale_bits, lora_a_c, lora_b_c, group_size, bias_bits)
    _check_extent("gate", gate, (m, n))
    device = _on_device(x2d, packed, scale_bits, lora_a_c, lora_b_c, bias_bits, gate)
    dt = x2d.dtype
    code = _dtype_code(dt)
    x2d = _aligned(x2d)
    a = _aligned(_as(lora_a_c, dt))
    b = _aligned(_as(lora_b_c, dt))
    gate = None if gate is None else _aligned(gate.to(dt))
    y = torch.empty((m, n), dtype=dt, device=device)
    z = torch.empty((m, n), dtype=dt, device=device)
    h = torch.empty((m, r), dtype=dt, device=device)
    g = group_arg(group_size, k)
    ws = _workspace(nat.query("rpx_int4lora_forward_workspace", m, n, k, g, r, code), device)
    bias = None if bias_bits is None else _u16(bias_bits).contiguous()
    nat.call("rpx_int4lora_forward_act", _ptr(x2d), code, m, k, _ptr(_aligned(packed)),
             _ptr(_aligned(_u16(scale_bits))), n, g, _ptr(bias), _ptr(a), _ptr(b), r,
             float(scaling), act, _ptr(gate), _ptr(y), _ptr(z), _ptr(h), _ptr(ws), ws.numel(),
             _stream(device))
    return y, z, h


def int4lora_backward_act(grad, x2d, packed, scale_bits, lora_a_c, lora_b_c, h, *,
                          activation: str, z, gate=None, scaling: float,
                          group_size: int | None = None):
    """The FFN's down projection backward followed by the activation's:
    ``(dz, dgate or None, dA f32, dB f32)``; x2d is the down projection's
    input, z (and gate) the activation's forward operands. With
    ``activation="add"`` it is any linear's backward whose input gradient is
    added to ``z``, the gradient accumulated so far for a shared input."""

    act = ACTIVATIONS[activation]
    m, k, n, r = _lora_dims(x2d, packed, scale_bits, lora_a_c, lora_b_c, group_size)
    _check_extent("grad", grad, (m, n))
    _check_extent("h", h, (m, r))
    _check_extent("z", z, (m, k))
    _check_extent("gate", gate, (m, k))
    device = _on_device(grad, x2d, packed, scale_bits, lora_a_c, lora_b_c, h, z, gate)
    dt = x2d.dtype
    code = _dtype_code(dt)
    grad = _aligned(grad.to(dt))
    a = _aligned(_as(lora_a_c, dt))
    b = _aligned(_as(lora_b_c, dt))
    z = _aligned(z.to(dt))
    gate = None if gate is None else _aligned(gate.to(dt))
    dz = torch.empty((m, k), dtype=dt, device=device)
    dgate = torch.empty((m, k), dtype=dt, device=device) if act == nat.ACT_SILU_MUL else None
    d_a = torch.empty((r, k), dtype=F32, device=device)
    d_b = torch.empty((n, r), dtype=F32, device=device)
    g = group_arg(group_size, k)
    ws = _workspace(nat.query("rpx_int4lora_backward_workspace", m, n, k, g, r, code), device)
    nat.call("rpx_int4lora_backward_act", _ptr(grad), _ptr(_aligned(x2d)), code, m, k,
             _ptr(_aligned(packed)), _ptr(_aligned(_u16(scale_bits))), n, g, _ptr(a),
             _ptr(b), r, float(scaling), _ptr(h.contiguous()), act, _ptr(z), _ptr(gate),
             _ptr(dz), _ptr(dgate), _ptr(d_a), _ptr(d_b), _ptr(ws), ws.numel(), _stream(device))
    return dz, dgate, d_a, d_b


class Int4LoRALinearFn(torch.autograd.Function):
    """Autograd node of the fused INT4 + LoRA linear on 2-D activations.

    Inputs are the activations, the LoRA compute views (differentiable; their
    gradients are the bf16-rounded products returned in the views' dtype)
    and the frozen integer leaves.
    """

    @staticmethod
    def forward(ctx, x2d, lora_a_c, lora_b_c, packed, scale_bits, bias_bits, scaling, group_size):
        y, h = int4lora_forward(x2d, packed, scale_bits, lora_a_c, lora_b_c, scaling=scaling,
                                group_size=group_size, bias_bits=bias_bits)
        ctx.save_for_backward(x2d, lora_a_c, lora_b_c, packed, scale_bits, h)
        ctx.scaling = scaling
        ctx.group_size = group_size
        return y

    @staticmethod
    def backward(ctx, grad_y):
        x2d, lora_a_c, lora_b_c, packed, scale_bits, h = ctx.saved_tensors
        dx, d_a, d_b = int4lora_backward(grad_y, x2d, packed, scale_bits, lora_a_c, lora_b_c, h,
                                         scaling=ctx.scaling, group_size=ctx.group_size)
        return (dx, d_a.to(lora_a_c.dtype), d_b.to(lora_b_c.dtype), None, None, None, None, None)


def int4lora_forward_promoted(x2d, packed, scale_bits, lora_a, lora_b, *, scaling: float,
                              group_size: int | None = None, bias_bits=None):
    """No precision policy, bf16 ``x`` and float32 masters: ``(y f32 [M, N],
    h f32 [M, r])`` with the base product in bf16 and the adapter promoted
    to float32, as ``jnp.matmul`` does in the reference."""

    device = _on_device(x2d, packed, scale_bits, lora_a, lora_b, bias_bits)
    if x2d.dtype != BF16 or lora_a.dtype != F32 or lora_b.dtype != F32:
        raise TypeError("the promoted INT4 + LoRA linear takes bf16 x and float32 masters")
    m, k, n, r = _lora_dims(x2d, packed, scale_bits, lora_a, lora_b, group_size, bias_bits)
    x2d = _aligned(x2d)
    y = torch.empty((m, n), dtype=F32, device=device)
    h = torch.empty((m, r), dtype=F32, device=device)
    g = group_arg(group_size, k)
    ws = _workspace(nat.query("rpx_int4lora_forward_promoted_workspace", m, n, k, g, r), device)
    bias = None if bias_bits is None else _aligned(_u16(bias_bits))
    nat.call("rpx_int4lora_forward_promoted", _ptr(x2d), m, k, _ptr(_aligned(packed)),
             _ptr(_aligned(_u16(scale_bits))), n, g, _ptr(bias), _ptr(_aligned(lora_a)),
             _ptr(_aligned(lora_b)), r, float(scaling), _ptr(y), _ptr(h), _ptr(ws), ws.numel(),
             _stream(device))
    return y, h


def int4lora_backward_promoted(grad, x2d, packed, scale_bits, lora_a, lora_b, h, *,
                               scaling: float, group_size: int | None = None):
    """``(dx bf16 [M, K], dA f32 [r, K], dB f32 [N, r])`` of the promoted
    forward, from the float32 output gradient."""

    m, k, n, r = _lora_dims(x2d, packed, scale_bits, lora_a, lora_b, group_size)
    _check_extent("grad", grad, (m, n))
    _check_extent("h", h, (m, r))
    device = _on_device(grad, x2d, packed, scale_bits, lora_a, lora_b, h)
    grad = _aligned(grad.to(F32))
    dx = torch.empty((m, k), dtype=BF16, device=device)
    d_a = torch.empty((r, k), dtype=F32, device=device)
    d_b = torch.empty((n, r), dtype=F32, device=device)
    g = group_arg(group_size, k)
    ws = _workspace(nat.query("rpx_int4lora_backward_promoted_workspace", m, n, k, g, r), device)
    nat.call("rpx_int4lora_backward_promoted", _ptr(grad), _ptr(_aligned(x2d)), m, k,
             _ptr(_aligned(packed)), _ptr(_aligned(_u16(scale_bits))), n, g,
             _ptr(_aligned(lora_a)), _ptr(_aligned(lora_b)), r, float(scaling),
             _ptr(_aligned(h)), _ptr(dx), _ptr(d_a), _ptr(d_b), _ptr(ws), ws.numel(),
             _stream(device))
    return dx, d_a, d_b


class Int4LoRAPromotedFn(torch.autograd.Function):
    """Autograd node of the promoted INT4 + LoRA linear (no policy, bf16
    activations, float32 masters): float32 output, bf16 input gradient,
    float32 master gradients."""

    @staticmethod
    def forward(ctx, x2d, lora_a, lora_b, packed, scale_bits, bias_bits, scaling, group_size):
        y, h = int4lora_forward_promoted(x2d, packed, scale_bits, lora_a, lora_b,
                                         scaling=scaling, group_size=group_size,
                                         bias_bits=bias_bits)
        ctx.save_for_backward(x2d, lora_a, lora_b, packed, scale_bits, h)
        ctx.scaling = scaling
        ctx.group_size = group_size
        return y

    @staticmethod
    def backward(ctx, grad_y):
        x2d, lora_a, lora_b, packed, scale_bits, h = ctx.saved_tensors
        dx, d_a, d_b = int4lora_backward_promoted(grad_y, x2d, packed, scale_bits, lora_a, lora_b,
                                                  h, scaling=ctx.scaling,
                                                  group_size=ctx.group_size)
        return dx, d_a, d_b, None, None, None, None, None


class Int4LoRAGeluMLPFn(torch.autograd.Function):
    """``down(gelu(up(x)))`` over two INT4 + LoRA linears with the GELU in
    the up projection's GEMM epilogue and its backward in the down
    projection's dx epilogue (bert/model.py:249).

    Per linear: LoRA compute views (a, b), then packed, scale_bits,
    bias_bits, scaling, group_size.
    """

    @staticmethod
    def forward(ctx, x2d, up_a, up_b, down_a, down_b, up_packed, up_scales, up_bias, up_scaling,
                up_group, down_packed, down_scales, down_bias, down_scaling, down_group):
        act, z, h_up = int4lora_forward_act(x2d, up_packed, up_scales, up_a, up_b,
                                            activation="gelu", scaling=up_scaling,
                                            group_size=up_group, bias_bits=up_bias)
        y, h_down = int4lora_forward(act, down_packed, down_scales, down_a, down_b,
                                     scaling=down_scaling, group_size=down_group,
                                     bias_bits=down_bias)
        ctx.save_for_backward(x2d, up_a, up_b, down_a, down_b, up_packed, up_scales, down_packed,
                              down_scales, z, act, h_up, h_down)
        ctx.cfg = (up_scaling, up_group, down_scaling, down_group)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        (x2d, up_a, up_b, down_a, down_b, up_packed, up_scales, down_packed, down_scales, z, act,
         h_up, h_down) = ctx.saved_tensors
        up_scaling, up_group, down_scaling, down_group = ctx.cfg
        dz, _, d_down_a, d_down_b = int4lora_backward_act(
            grad_y, act, down_packed, down_scales, down_a, down_b, h_down, activation="gelu",
            z=z, scaling=down_scaling, group_size=down_group)
        dx, d_up_a, d_up_b = int4lora_backward(dz, x2d, up_packed, up_scales, up_a, up_b, h_up,
                                               scaling=up_scaling, group_size=up_group)
        return (dx, d_up_a.to(up_a.dtype), d_up_b.to(up_b.dtype), d_down_a.to(down_a.dtype),
                d_down_b.to(down_b.dtype)) + (None,) * 10


class Int4LoRASwiGLUMLPFn(torch.autograd.Function):
    """``down(silu(gate(x)) * up(x))`` over three INT4 + LoRA linears with
    the gated product in the up projection's GEMM epilogue and its backward
    (both the up and the gate gradients) in the down projection's dx
    epilogue (qwen3_vl/text.py:202-203)."""

    @staticmethod
    def forward(ctx, x2d, gate_a, gate_b, up_a, up_b, down_a, down_b, gate_packed, gate_scales,
                gate_bias, gate_scaling, gate_group, up_packed, up_scales, up_bias, up_scaling,
                up_group, down_packed, down_scales, down_bias, down_scaling, down_group):
        g, h_gate = int4lora_forward(x2d, gate_packed, gate_scales, gate_a, gate_b,
                                     scaling=gate_scaling, group_size=gate_group,
                                     bias_bits=gate_bias)
        act, u, h_up = int4lora_forward_act(x2d, up_packed, up_scales, up_a, up_b,
                                            activation="silu_mul", scaling=up_scaling,
                                            group_size=up_group, bias_bits=up_bias, gate=g)
        y, h_down = int4lora_forward(act, down_packed, down_scales, down_a, down_b,
                                     scaling=down_scaling, group_size=down_group,
                                     bias_bits=down_bias)
        ctx.save_for_backward(x2d, gate_a, gate_b, up_a, up_b, down_a, down_b, gate_packed,
                              gate_scales, up_packed, up_scales, down_packed, down_scales, g, u,
                              act, h_gate, h_up, h_down)
        ctx.cfg = (gate_scaling, gate_group, up_scaling, up_group, down_scaling, down_group)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        (x2d, gate_a, gate_b, up_a, up_b, down_a, down_b, gate_packed, gate_scales, up_packed,
         up_scales, down_packed, down_scales, g, u, act, h_gate, h_up, h_down) = ctx.saved_tensors
        gate_scaling, gate_group, up_scaling, up_group, down_scaling, down_group = ctx.cfg
        du, dg, d_down_a, d_down_b = int4lora_backward_act(
            grad_y, act, down_packed, down_scales, down_a, down_b, h_down, activation="silu_mul",
            z=u, gate=g, scaling=down_scaling, group_size=down_group)
        dx_up, d_up_a, d_up_b = int4lora_backward(du, x2d, up_packed, up_scales, up_a, up_b, h_up,
                                                  scaling=up_scaling, group_size=up_group)
        # the gate projection's input gradient is added to the up projection's
        # in the dx GEMM's epilogue
        dx, _, d_gate_a, d_gate_b = int4lora_backward_act(
            dg, x2d, gate_packed, gate_scales, gate_a, gate_b, h_gate, activation="add", z=dx_up,
            scaling=gate_scaling, group_size=gate_group)
        return (dx, d_gate_a.to(gate_a.dtype), d_gate_b.to(gate_b.dtype),
                d_up_a.to(up_a.dtype), d_up_b.to(up_b.dtype), d_down_a.to(down_a.dtype),
                d_down_b.to(down_b.dtype)) + (None,) * 15


class Int4LoRASharedInputFn(torch.autograd.Function):
    """Several INT4 + LoRA linears of one input (the q / k / v projections):
    the forward runs them as one multi-projection call (their adapters'
    down-projections in one pass over the input, then one GEMM each); in the
    backward every input
    gradient after the first is added to the running sum in its dx GEMM's
    epilogue (bf16, in projection order) instead of by a separate pass.

    Arguments: x2d, the count n, the n pairs of LoRA compute views, then per
    linear packed, scale_bits, bias_bits, scaling, group_size.
    """

    @staticmethod
    def forward(ctx, x2d, n, *args):
        views = args[:2 * n]
        leaves = args[2 * n:]
        outs, hs = [], []
        if x2d.dim() == 2 and x2d.shape[0] > SHARED_OUTPUT_ROWS:
            # one call: the projections' h = x A^T come from one pass over x
            # where the ranks allow, and each output is its own allocation
            pairs = int4lora_forward_multi(
                x2d, [(leaves[5 * i], leaves[5 * i + 1], views[2 * i], views[2 * i + 1],
                       leaves[5 * i + 3], leaves[5 * i + 4], leaves[5 * i + 2]) for i in range(n)])
            outs = [y for y, _ in pairs]
            hs = [h for _, h in pairs]
        else:
            for i in range(n):
                packed, scales, bias, scaling, group = leaves[5 * i:5 * i + 5]
                y, h = int4lora_forward(x2d, packed, scales, views[2 * i], views[2 * i + 1],
                                        scaling=scaling, group_size=group, bias_bits=bias)
                outs.append(y)
                hs.append(h)
        ctx.n = n
        ctx.cfg = [(leaves[5 * i + 3], leaves[5 * i + 4]) for i in range(n)]
        ctx.save_for_backward(x2d, *views, *[leaves[5 * i] for i in range(n)],
                              *[leaves[5 * i + 1] for i in range(n)], *hs)
        return tuple(outs)

    @staticmethod
    def backward(ctx, *grads):
        n = ctx.n
        saved = ctx.saved_tensors
        x2d = saved[0]
        views = saved[1:1 + 2 * n]
        packed = saved[1 + 2 * n:1 + 3 * n]
        scales = saved[1 + 3 * n:1 + 4 * n]
        hs = saved[1 + 4 * n:1 + 5 * n]
        dx = None
        dviews = []
        for i in range(n):
            a, b = views[2 * i], views[2 * i + 1]
            scaling, group = ctx.cfg[i]
            g = grads[i] if grads[i] is not None else torch.zeros(
                (x2d.shape[0], packed[i].shape[-2]), dtype=x2d.dtype, device=x2d.device)
            if dx is None:
                dx, d_a, d_b = int4lora_backward(g, x2d, packed[i], scales[i], a, b, hs[i],
                                                 scaling=scaling, group_size=group)
            else:
                dx, _, d_a, d_b = int4lora_backward_act(
                    g, x2d, packed[i], scales[i], a, b, hs[i], activation="add", z=dx,
                    scaling=scaling, group_size=group)
            dviews += [d_a.to(a.dtype), d_b.to(b.dtype)]
        return (dx, None, *dviews) + (None,) * (5 * n)


# ---------------------------------------------------------------------------
# Fused in-batch MNR loss
# ---------------------------------------------------------------------------
class MNRLossFn(torch.autograd.Function):
    """In-batch multiple-negatives ranking loss with query i's positive at
    document i (src/representax/tasks/retrieval/mnr.py:48-52,132-158,
    338-341): f32 casts, row normalisation, scaled cosine logits, row
    log-sum-exp and the mean over queries in one fused forward, and its
    gradient in one launch."""

    @staticmethod
    def forward(ctx, queries, documents, scale: float):
        device = _on_device(queries, documents)
        if queries.dim() != 2 or documents.dim() != 2:
            raise ValueError("query and document embeddings must be matrices")
        if queries.shape[1] != documents.shape[1]:
            raise ValueError("query and document embedding dimensions must match")
        if isinstance(scale, bool) or not math.isfinite(float(scale)) or float(scale) <= 0:
            raise ValueError("scale must be finite and positive")
        # each set is cast to float32 on its own (mnr.py:48-52): mixed
        # bf16 / f32 inputs run the f32 kernel on exact upcasts, so neither
        # set is rounded to the other's dtype first
        dtype = queries.dtype if queries.dtype == documents.dtype else F32
        q = queries.to(dtype).contiguous()
        d = documents.to(dtype).contiguous()
        nq, dim = q.shape
        nd = d.shape[0]
        nbytes = nat.query("rpx_mnr_saved_bytes", nq, nd, dim)
        if nbytes == 0:
            raise ValueError("fused MNR loss needs 1 <= queries <= documents <= 8192 and "
                             "1 <= dim <= 4096 (query i's positive is document i)")
        saved = torch.empty(nbytes // 4, dtype=F32, device=device)
        loss = torch.empty((), dtype=F32, device=device)
        nat.call("rpx_mnr_forward", _ptr(q), _ptr(d), _dtype_code(dtype), nq, nd, dim,
                 float(scale), _ptr(loss), _ptr(saved), nbytes, _stream(device))
        ctx.save_for_backward(saved)
        ctx.shape = (nq, nd, dim, float(scale), dtype, queries.dtype, documents.dtype)
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        (saved,) = ctx.saved_tensors
        nq, nd, dim, scale, dtype, q_dtype, d_dtype = ctx.shape
        device = saved.device
        g = grad_loss.to(F32).contiguous().reshape(1)
        dq = torch.empty((nq, dim), dtype=dtype, device=device)
        dd = torch.empty((nd, dim), dtype=dtype, device=device)
        nat.call("rpx_mnr_backward", _ptr(g), _ptr(saved), saved.numel() * 4, nq, nd, dim, scale,
                 _ptr(dq), _ptr(dd), _dtype_code(dtype), _stream(device))
        return dq.to(q_dtype), dd.to(d_dtype), None


def mnr_loss(queries: torch.Tensor, documents: torch.Tensor, scale: float = 20.0) -> torch.Tensor:
    """Scalar f32 loss; differentiable in both embedding sets (f32 or bf16)."""

    return MNRLossFn.apply(queries, documents, scale)


# ---------------------------------------------------------------------------
# FP8
# ---------------------------------------------------------------------------
FORMATS = {"e4m3fn": nat.FP8_E4M3FN, "e5m2": nat.FP8_E5M2}


def _fmt(fmt: str | int) -> int:
    return FORMATS[fmt] if isinstance(fmt, str) else int(fmt)


def fp8_scale(t: torch.Tensor, fmt: str = "e4m3fn") -> torch.Tensor:
    """``float32[1]`` scale ``max(max|t| / fmax, FLT_MIN)``."""

    device = _on_device(t)
    t = t.contiguous()
    out = torch.empty(1, dtype=F32, device=device)
    ws = _workspace(nat.query("rpx_fp8_scale_workspace", t.numel()), device)
    nat.call("rpx_fp8_scale", _ptr(t), _dtype_code(t.dtype), t.numel(), _fmt(fmt), _ptr(out),
             _ptr(ws), ws.numel(), _stream(device))
    return out


def fp8_cast(t: torch.Tensor, scale: torch.Tensor, fmt: str = "e4m3fn", *, rowmajor=True,
             transposed=False):
    """Codes of a 2-D tensor: ``(out [R, C] or None, out_t [C, R] or None)``."""

    device = _on_device(t, scale)
    rows, cols = t.shape
    out = torch.empty((rows, cols), dtype=torch.uint8, device=device) if rowmajor else None
    out_t = torch.empty((cols, rows), dtype=torch.uint8, device=device) if transposed else None
    nat.call("rpx_fp8_cast", _ptr(t), _dtype_code(t.dtype), rows, cols, t.stride(0), t.stride(1),
             _ptr(scale), _fmt(fmt), _ptr(out), _ptr(out_t), _stream(device))
    return out, out_t


def fp8_encode_selfcheck(fmt: str, first: int = 0, count: int = 1 << 31, blocks: int = 4096,
                         device="cuda"):
    """Mismatches between the cast kernels' encoder and the integer encoder
    over f32 patterns [first, first+count) and their negations:
    ``(count, lowest mismatching pattern or None)``."""

    dev = torch.device(device)
    nat.load()
    counts = torch.zeros(blocks, dtype=torch.int32, device=dev)
    firsts = torch.zeros(blocks, dtype=torch.int32, device=dev)
    nat.call("rpx_fp8_encode_selfcheck", _fmt(fmt), int(first), int(count), _ptr(counts),
             _ptr(firsts), blocks, _stream(dev))
    c = counts.cpu().numpy().view("uint32").astype("int64").sum()
    f = firsts.cpu().numpy().view("uint32").min()
    return int(c), (None if f == 0xFFFFFFFF else int(f))


def fp8_gemm(a_codes, fmt_a, scale_a, b_codes, fmt_b, scale_b, out_dtype=BF16):
    """``((a [M,K] . b [N,K]^T) * s_a) * s_b`` -> ``[M, N]``."""

    if a_codes.dim() != 2 or b_codes.dim() != 2 or a_codes.shape[1] != b_codes.shape[1]:
        raise ValueError(f"fp8 GEMM needs a [M, K] and b [N, K] codes; got {tuple(a_codes.shape)} "
                         f"and {tuple(b_codes.shape)}")
    if a_codes.element_size() != 1 or b_codes.element_size() != 1:
        raise ValueError("fp8 GEMM operands are one-byte codes")
    device = _on_device(a_codes, b_codes, scale_a, scale_b)
    m, k = a_codes.shape
    n = b_codes.shape[0]
    out = torch.empty((m, n), dtype=out_dtype, device=device)
    ws = _workspace(nat.query("rpx_fp8_gemm_workspace", m, n, k), device)
    nat.call("rpx_fp8_gemm", _ptr(a_codes.contiguous()), _fmt(fmt_a), _ptr(scale_a),
             _ptr(b_codes.contiguous()), _fmt(fmt_b), _ptr(scale_b), m, n, k, _ptr(out),
             _dtype_code(out_dtype), _ptr(ws), ws.numel(), _stream(device))
    return out


def _dense_2d(t: torch.Tensor) -> torch.Tensor:
    """A 2-D tensor whose storage is dense (row-major or its transpose)."""

    if t.is_contiguous() or t.t().is_contiguous():
        return t
    return t.contiguous()


def _check_fp8_operands(left, right) -> None:
    """The reference's per-tensor scale is ``max(|t|)`` over each operand
    (precision.py:133-135), a max-reduction with no identity: it raises on
    an empty operand, so any zero among M, K, N is an error here too."""

    if left.dim() != 2 or right.dim() != 2 or left.shape[1] != right.shape[0]:
        raise ValueError(f"fp8 linear needs left [M, K] and right [K, N]; got "
                         f"{tuple(left.shape)} and {tuple(right.shape)}")
    m, k = left.shape
    n = right.shape[1]
    if m == 0 or n == 0 or k == 0:
        raise ValueError(f"fp8 linear: empty operand (M={m}, K={k}, N={n}); the per-tensor "
                         "amax of an empty tensor is undefined")


def fp8_linear_forward(left, right, out_dtype=BF16, save_codes=False):
    """``(out [M, N], scales f32[2], codes)`` for ``left [M,K] . right [K,N]``.

    With ``save_codes`` the same cast pass also returns the backward's operand
    codes ``(left codes [M, K], right codes [K, N])``; otherwise ``codes`` is
    None. ``ValueError`` for an empty operand, as in the reference.
    """

    _check_fp8_operands(left, right)
    device = _on_device(left, right)
    left = left.contiguous()
    right = _dense_2d(right)
    m, k = left.shape
    n = right.shape[1]
    out = torch.empty((m, n), dtype=out_dtype, device=device)
    scales = torch.empty(2, dtype=F32, device=device)
    codes = None
    if save_codes:
        codes = (torch.empty((m, k), dtype=torch.uint8, device=device),
                 torch.empty((k, n), dtype=torch.uint8, device=device))
    ws = _workspace(nat.query("rpx_fp8_linear_forward_workspace", m, n, k), device)
    nat.call("rpx_fp8_linear_forward", _ptr(left), _dtype_code(left.dtype), m, k, _ptr(right),
             _dtype_code(right.dtype), n, right.stride(0), right.stride(1), _ptr(out),
             _dtype_code(out_dtype), _ptr(scales), _ptr(codes[0] if codes else None),
             _ptr(codes[1] if codes else None), _ptr(ws), ws.numel(), _stream(device))
    return out, scales, codes


def _grad_buffers(m, k, n, dtype, right_t, need_left, need_right, device):
    d_left = torch.empty((m, k), dtype=dtype, device=device) if need_left else None
    d_right = None
    if need_right:
        d_right = torch.empty((n, k) if right_t else (k, n), dtype=dtype, device=device)
    return d_left, d_right


def fp8_linear_backward(left, right, grad, scales, *, need_left=True, need_right=True):
    """``(d_left [M,K] or None, d_right [K,N] or None)`` in the operand dtypes,
    re-quantizing the bf16 operands with the forward's scales."""

    if left.dim() != 2 or right.dim() != 2 or left.shape[1] != right.shape[0]:
        raise ValueError(f"fp8 linear needs left [M, K] and right [K, N]; got "
                         f"{tuple(left.shape)} and {tuple(right.shape)}")
    _check_extent("grad", grad, (left.shape[0], right.shape[1]))
    if scales.numel() != 2:
        raise _shape_error("scales", scales.shape, (2,))
    device = _on_device(left, right, grad, scales)
    left = left.contiguous()
    right = _dense_2d(right)
    grad = grad.contiguous()
    m, k = left.shape
    n = right.shape[1]
    if left.dtype != right.dtype:
        raise TypeError("fp8 linear backward expects operands of one dtype")
    right_t = not right.is_contiguous()  # a transposed weight view gets a [N, K] gradient
    d_left, d_right = _grad_buffers(m, k, n, left.dtype, right_t, need_left, need_right, device)
    if m == 0 or n == 0 or k == 0:
        for t in (d_left, d_right):
            if t is not None:
                t.zero_()
    elif need_left or need_right:
        ws = _workspace(nat.query("rpx_fp8_linear_backward_workspace", m, n, k), device)
        nat.call("rpx_fp8_linear_backward", _ptr(left), _dtype_code(left.dtype), _ptr(right),
                 _dtype_code(right.dtype), m, k, n, right.stride(0), right.stride(1), _ptr(grad),
                 _dtype_code(grad.dtype), _ptr(scales), _ptr(d_left), _ptr(d_right),
                 1 if right_t else 0, _dtype_code(left.dtype), _ptr(ws), ws.numel(),
                 _stream(device))
    if d_right is not None and right_t:
        d_right = d_right.t()
    return d_left, d_right


def fp8_linear_backward_codes(codes, scales, grad, *, k, dtype, right_transposed,
                              need_left=True, need_right=True):
    """Backward from the codes saved by ``fp8_linear_forward(save_codes=True)``."""

    left_c, right_c = codes
    if grad.dim() != 2:
        raise ValueError(f"grad must be 2-D [M, N], got shape {tuple(grad.shape)}")
    _check_extent("saved left codes", left_c, (grad.shape[0], k))
    _check_extent("saved right codes", right_c, (k, grad.shape[1]))
    if scales.numel() != 2:
        raise _shape_error("scales", scales.shape, (2,))
    device = _on_device(left_c, right_c, grad, scales)
    grad = grad.contiguous()
    m, n = grad.shape
    d_left, d_right = _grad_buffers(m, k, n, dtype, right_transposed, need_left, need_right,
                                    device)
    if m == 0 or n == 0 or k == 0:
        for t in (d_left, d_right):
            if t is not None:
                t.zero_()
    elif need_left or need_right:
        ws = _workspace(nat.query("rpx_fp8_linear_backward_workspace", m, n, k), device)
        nat.call("rpx_fp8_linear_backward_codes", _ptr(left_c), _ptr(right_c), _ptr(scales), m, k,
                 n, _ptr(grad), _dtype_code(grad.dtype), _ptr(d_left), _ptr(d_right),
                 1 if right_transposed else 0, _dtype_code(dtype), _ptr(ws), ws.numel(),
                 _stream(device))
    if d_right is not None and right_transposed:
        d_right = d_right.t()
    return d_left, d_right


def fp8_linear_backward_gemms(g_codes, s_grad, left_codes, s_left, right_codes, s_right, *, k,
                              dtype, right_transposed, need_left=True, need_right=True):
    """The backward's two products from the gradient's codes (e5m2
    ``g_codes`` [M, N]) and the forward's operand codes (``left_codes``
    [M, K], ``right_codes`` [K, N]), each scale a one-element float32 tensor:
    ``(d_left [M, K] or None, d_right or None)`` as in
    ``fp8_linear_backward_codes``. For callers that quantize the gradient
    themselves (delayed scaling)."""

    m, n = g_codes.shape
    _check_extent("left codes", left_codes, (m, k))
    _check_extent("right codes", right_codes, (k, n))
    device = _on_device(g_codes, left_codes, right_codes, s_grad)
    d_left, d_right = _grad_buffers(m, k, n, dtype, True, need_left, need_right, device)
    if m == 0 or n == 0 or k == 0:
        for t in (d_left, d_right):
            if t is not None:
                t.zero_()
    elif need_left or need_right:
        ws = _workspace(nat.query("rpx_fp8_linear_backward_gemms_workspace", m, n, k), device)
        nat.call("rpx_fp8_linear_backward_gemms", _ptr(g_codes), _ptr(s_grad), _ptr(left_codes),
                 _ptr(s_left), _ptr(right_codes), _ptr(s_right), m, k, n, _ptr(d_left),
                 _ptr(d_right), 1, _dtype_code(dtype), _ptr(ws), ws.numel(), _stream(device))
    if d_right is not None:
        # computed as [N, K]; the [K, N] gradient of a natural right operand
        # is its transpose, made contiguous
        d_right = d_right.t() if right_transposed else d_right.t().contiguous()
    return d_left, d_right


# ---------------------------------------------------------------------------
# Delayed-scale fp8 (state: precision.DelayedScaling)
# ---------------------------------------------------------------------------
def _delayed_outputs(t, rowmajor, transposed):
    rows, cols = t.shape
    out = torch.empty((rows, cols), dtype=torch.uint8, device=t.device) if rowmajor else None
    out_t = torch.empty((cols, rows), dtype=torch.uint8, device=t.device) if transposed else None
    return out, out_t


def fp8_cast_delayed(t: torch.Tensor, state, slot: int, fmt: str = "e4m3fn", *, rowmajor=True,
                     transposed=False):
    """Saturating codes of a 2-D tensor under ``state.scales[slot]``, recording
    ``max|t|`` into the slot's pending maxima: ``(out [R, C] or None, out_t
    [C, R] or None)``."""

    device = _on_device(t, state.scales)
    out, out_t = _delayed_outputs(t, rowmajor, transposed)
    nat.call("rpx_fp8_cast_delayed", _ptr(t), _dtype_code(t.dtype), t.shape[0], t.shape[1],
             t.stride(0), t.stride(1), _fmt(fmt), _ptr(state.scales), _ptr(state.amax_pending),
             state.n_slots, int(slot), _ptr(out), _ptr(out_t), _stream(device))
    return out, out_t


def fp8_cast_delayed2(t0: torch.Tensor, slot0: int, t1: torch.Tensor, slot1: int, state,
                      fmt: str = "e4m3fn", *, rowmajor=True, transposed=False):
    """Two ``fp8_cast_delayed`` casts of one dtype in one launch:
    ``((out0, out0_t), (out1, out1_t))``. ``rowmajor`` and ``transposed``
    are a bool for both tensors or a pair, one per tensor."""

    device = _on_device(t0, t1, state.scales)
    if t0.dtype != t1.dtype:
        raise TypeError("fp8_cast_delayed2 casts two tensors of one dtype")
    rm = rowmajor if isinstance(rowmajor, tuple) else (rowmajor, rowmajor)
    tr = transposed if isinstance(transposed, tuple) else (transposed, transposed)
    o0, o0t = _delayed_outputs(t0, rm[0], tr[0])
    o1, o1t = _delayed_outputs(t1, rm[1], tr[1])
    nat.call("rpx_fp8_cast_delayed2", _ptr(t0), t0.shape[0], t0.shape[1], t0.stride(0),
             t0.stride(1), int(slot0), _ptr(o0), _ptr(o0t), _ptr(t1), t1.shape[0], t1.shape[1],
             t1.stride(0), t1.stride(1), int(slot1), _ptr(o1), _ptr(o1t), _dtype_code(t0.dtype),
             _fmt(fmt), _ptr(state.scales), _ptr(state.amax_pending), state.n_slots,
             _stream(device))
    return (o0, o0t), (o1, o1t)


def fp8_scale_update(state) -> None:
    """The once-per-step update of every slot's scale: pending maxima go to
    the history row at the cursor, scales are recomputed from the history and
    the cursor advances (one launch)."""

    device = _on_device(state.scales)
    nat.call("rpx_fp8_scale_update", _ptr(state.scales), _ptr(state.fmax),
             _ptr(state.amax_pending), _ptr(state.amax_history), _ptr(state.cursor),
             state.n_slots, state.history_len, _stream(device))


def fp8_delayed_pending_words() -> int:
    nat.load()
    return int(nat.query("rpx_fp8_delayed_pending_words"))


def _gemm_into(a, fmt_a, scale_a, b, fmt_b, scale_b, out):
    """``out = ((a . b^T) * scale_a) * scale_b`` on fp8 codes (the two scales
    are applied in this order whatever operand they belong to)."""

    m, k = a.shape
    n = b.shape[0]
    ws = _workspace(nat.query("rpx_fp8_gemm_workspace", m, n, k), out.device)
    nat.call("rpx_fp8_gemm", _ptr(a), _fmt(fmt_a), _ptr(scale_a), _ptr(b), _fmt(fmt_b),
             _ptr(scale_b), m, n, k, _ptr(out), _dtype_code(out.dtype), _ptr(ws), ws.numel(),
             _stream(out.device))
    return out


class Fp8DelayedLinearFn(torch.autograd.Function):
    """``left [M, K] @ right [K, N]`` with delayed fp8 scales: e4m3 operands in
    the forward and an e5m2 gradient in the backward, as in the dynamic
    ``Fp8LinearFn``, but each operand is cast once with the scale its slot
    holds (saturating) while its amax is recorded for the next update. The
    slots are (left, right, grad)."""

    @staticmethod
    def forward(ctx, left, right, out_dtype, state, slots):
        _check_fp8_operands(left, right)
        _on_device(left, right)
        left = left.contiguous()
        right = _dense_2d(right)
        m, k = left.shape
        n = right.shape[1]
        s_l, s_r, s_g = (state.scales[i:i + 1] for i in slots)
        out = torch.empty((m, n), dtype=out_dtype, device=left.device)
        need = left.requires_grad or right.requires_grad
        # left -> codes [M, K] (this product's, and d_right's read along the
        # tokens); right [K, N] -> codes [N, K] for this product (+ [K, N] for
        # d_left); one launch
        (ql, _), (qrt, qr) = fp8_cast_delayed2(left, slots[0], right.t(), slots[1], state,
                                               "e4m3fn", rowmajor=True, transposed=(False, need))
        _gemm_into(ql, "e4m3fn", s_l, qrt, "e4m3fn", s_r, out)
        if need:
            ctx.save_for_backward(ql, qr, s_l, s_r, s_g)
            ctx.state = state
            ctx.g_slot = slots[2]
            ctx.dtype = left.dtype
            ctx.right_t = not right.is_contiguous()
        return out

    @staticmethod
    def backward(ctx, grad):
        ql, qr, s_l, s_r, s_g = ctx.saved_tensors
        grad = grad.contiguous()
        k = ql.shape[1]
        need_l, need_r = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        qg, _ = fp8_cast_delayed(grad, ctx.state, ctx.g_slot, "e5m2", rowmajor=True,
                                 transposed=False)
        if not (need_l or need_r):
            return None, None, None, None, None
        d_left, d_right = fp8_linear_backward_gemms(qg, s_g, ql, s_l, qr, s_r, k=k,
                                                    dtype=ctx.dtype,
                                                    right_transposed=ctx.right_t,
                                                    need_left=need_l, need_right=need_r)
        return d_left, d_right, None, None, None


class Fp8LinearFn(torch.autograd.Function):
    """``_fp8_linear_dot`` (precision.py:173-221): e4m3 forward, e5m2 backward.

    The output is produced directly in ``out_dtype`` (the reference computes
    float32 and the caller casts it to the activation dtype; rounding once
    from the float32 epilogue value is the same result). The residuals are the
    operands' e4m3 codes and scales, which are exactly what the reference's
    backward recomputes from its bf16 residuals.
    """

    @staticmethod
    def forward(ctx, left, right, out_dtype):
        need = left.requires_grad or right.requires_grad
        out, scales, codes = fp8_linear_forward(left, right, out_dtype, save_codes=need)
        if need:
            ctx.save_for_backward(scales, *codes)
            ctx.k = left.shape[1]
            ctx.dtype = left.dtype
            ctx.right_t = not _dense_2d(right).is_contiguous()
        return out

    @staticmethod
    def backward(ctx, grad):
        scales, left_c, right_c = ctx.saved_tensors
        d_left, d_right = fp8_linear_backward_codes(
            (left_c, right_c), scales, grad, k=ctx.k, dtype=ctx.dtype,
            right_transposed=ctx.right_t, need_left=ctx.needs_input_grad[0],
            need_right=ctx.needs_input_grad[1])
        return d_left, d_right, None
