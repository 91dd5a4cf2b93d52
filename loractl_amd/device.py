"""Torch-facing calls into libloractl_rocm.so.

PyTorch is only the device-memory and stream plumbing here: tensors are
allocated by torch on the GPU and their device pointers are handed to the C
ABI, which launches the hand-written gfx950 kernels on torch's current
stream. There is no CPU or eager-torch fallback: a missing library, a CPU
tensor or an unsupported shape raises.
"""

from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib as L

class Context:
    """One lrq_ctx per (device, stream), shared by every thread that runs on
    that stream.

    The library's workspace (split partials, t and u, the LoRA reductions)
    is ordered by the context's stream. Keying contexts by stream means two
    streams never share a workspace, and autograd's backward, which runs on
    the forward's stream but on another thread, finds the same context (and
    the workspace ``reserve`` sized). A lock serialises the host side of the
    calls of one context (argument checks, the error message, the
    workspace's growth)."""

    def __init__(self, device: int, stream: int):
        self.lib = L.load()
        h = ctypes.c_void_p()
        rc = self.lib.lrq_create(device, ctypes.byref(h))
        if rc != 0:
            raise L.LrqError(rc, f"lrq_create(device={device}) failed")
        self.h = h
        self.device = device
        self.stream = stream
        self.lock = threading.RLock()
        self.call("lrq_set_stream", ctypes.c_void_p(stream))

    def __del__(self):
        try:
            if getattr(self, "h", None):
                self.lib.lrq_destroy(self.h)
        except Exception:
            pass

    def check(self, rc: int, what: str):
        if rc != 0:
            msg = self.lib.lrq_last_error(self.h).decode(errors="replace")
            raise L.LrqError(rc, f"{what}: {msg}")

    def call(self, name: str, *args):
        """Call ``name(ctx, *args)`` under the context's lock; raise on error."""
        with self.lock:
            self.check(getattr(self.lib, name)(self.h, *args), name)


_ctx_lock = threading.Lock()
_ctxs: dict = {}


def context(device: Optional[int] = None) -> Context:
    """The context of ``device`` (default: the current one) and torch's
    current stream on it."""
    if device is None:
        device = torch.cuda.current_device()
    stream = torch.cuda.current_stream(device).cuda_stream
    key = (device, stream)
    with _ctx_lock:
        c = _ctxs.get(key)
        if c is None:
            c = _ctxs[key] = Context(device, stream)
    return c


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _need(t: torch.Tensor, dtype: torch.dtype, name: str, shape=None):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (no CPU fallback)")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


@dataclass
class PackedWeight:
    """A frozen base weight in device memory, file layout [d_out, d_in].

    int4: ``data`` uint8 [n, k/2] (nibbles q+8, low nibble = even k) and
    ``scales`` f32 [n, k/group]. int8: ``data`` int8 [n, k] and ``scales``
    f32 [n, k/group]. fp8: ``data`` uint8 e4m3fn [n, k] and ``scales`` f32
    [n] (per_channel) or [1]. ``bias`` optional f32 [n].
    """

    fmt: int
    n: int
    k: int
    data: torch.Tensor
    scales: torch.Tensor
    group: int = 0
    per_channel: bool = False
    bias: Optional[torch.Tensor] = None
    layout: int = L.LRQ_LAYOUT_ROWS

    def desc(self) -> L.LrqWeight:
        return L.LrqWeight(
            format=self.fmt,
            group=self.group,
            n=self.n,
            k=self.k,
            data=self.data.data_ptr(),
            scales=self.scales.data_ptr(),
            per_channel=int(self.per_channel),
            layout=self.layout,
            bias=None if self.bias is None else self.bias.data_ptr(),
        )

    @property
    def device(self) -> torch.device:
        return self.data.device

    @property
    def blocked(self) -> bool:
        return self.layout == L.LRQ_LAYOUT_BLOCKED

    def with_bias(self, bias: Optional[torch.Tensor]) -> "PackedWeight":
        return PackedWeight(self.fmt, self.n, self.k, self.data, self.scales, self.group,
                            self.per_channel, bias, self.layout)


def compute_weight(w: PackedWeight) -> PackedWeight:
    """The blocked form the fused kernels read. A row-layout weight is re-laid
    in place, once: ``w`` then holds the blocked data and scales, and its
    row-layout tensors are released, so a frozen weight occupies 2x its
    packed bytes (the row and transposed sections), not 3x. ``dequant`` reads
    either layout."""
    if not w.blocked:
        b = block(w)
        w.data, w.scales, w.layout = b.data, b.scales, b.layout
    return w


# ------------------------------------------------------------------ formats
def block(w: PackedWeight) -> PackedWeight:
    """Re-lay a row-layout weight into the blocked layout the fused kernels read."""
    if w.blocked:
        return w
    ctx = context(w.device.index)
    db = ctypes.c_int64()
    ns = ctypes.c_int64()
    grouped = w.fmt != L.LRQ_FMT_FP8
    rc = ctx.lib.lrq_weight_blocked_size(w.fmt, w.n, w.k, w.group if grouped else 64,
                                         ctypes.byref(db), ctypes.byref(ns))
    ctx.check(rc, "lrq_weight_blocked_size")
    data = torch.empty((db.value,), dtype=torch.uint8, device=w.device)
    if grouped:
        scales = torch.empty((ns.value,), dtype=torch.float32, device=w.device)
    else:
        scales = w.scales
    d = w.desc()
    ctx.call("lrq_weight_block", ctypes.byref(d), _ptr(data), _ptr(scales))
    return PackedWeight(w.fmt, w.n, w.k, data, scales, w.group, w.per_channel, w.bias, L.LRQ_LAYOUT_BLOCKED)


def quantize_int4(w: torch.Tensor, group: int) -> PackedWeight:
    """quantize_linear_weight at Q4S (src/quant.rs:74-82) on the GPU."""
    _need(w, torch.float32, "w")
    n, k = w.shape
    ctx = context(w.device.index)
    packed = torch.empty((n, k // 2), dtype=torch.uint8, device=w.device)
    scales = torch.empty((n, max(k // group, 0) if group > 0 else 0), dtype=torch.float32, device=w.device)
    ctx.call("lrq_quantize_int4", _ptr(w), n, k, group, _ptr(packed), _ptr(scales))
    return PackedWeight(L.LRQ_FMT_INT4, n, k, packed, scales, group=group)


def quantize_int8(w: torch.Tensor, group: int) -> PackedWeight:
    """quantize_linear_weight at Q8S (src/quant.rs:74-82 with the Int8 value of
    src/quant.rs:156-162) on the GPU: int8 q [n, k] and f32 scales [n, k/group]."""
    _need(w, torch.float32, "w")
    n, k = w.shape
    ctx = context(w.device.index)
    q = torch.empty((n, k), dtype=torch.int8, device=w.device)
    scales = torch.empty((n, max(k // group, 0) if group > 0 else 0), dtype=torch.float32, device=w.device)
    ctx.call("lrq_quantize_int8", _ptr(w), n, k, group, _ptr(q), _ptr(scales))
    return PackedWeight(L.LRQ_FMT_INT8, n, k, q, scales, group=group)


def requantize_fp8_int4(w: PackedWeight, group: int) -> PackedWeight:
    """An fp8 weight (e4m3fn bytes and scale) as int4 at Q4S on the GPU: the
    f32 values LUT[byte] * scale (src/fp8.rs:306-318) quantized like
    ``quantize_int4`` (src/quant.rs:74-82), without an f32 copy."""
    if w.fmt != L.LRQ_FMT_FP8:
        raise ValueError("requantize_fp8_int4 needs an fp8 weight")
    if w.layout != L.LRQ_LAYOUT_ROWS:
        raise ValueError("requantize_fp8_int4 reads the row layout of the fp8 bytes")
    n, k = w.n, w.k
    ctx = context(w.data.device.index)
    packed = torch.empty((n, k // 2), dtype=torch.uint8, device=w.data.device)
    scales = torch.empty((n, max(k // group, 0) if group > 0 else 0), dtype=torch.float32, device=w.data.device)
    ctx.call("lrq_requantize_fp8_int4", _ptr(w.data), _ptr(w.scales), int(w.per_channel), n, k, group,
             _ptr(packed), _ptr(scales))
    return PackedWeight(L.LRQ_FMT_INT4, n, k, packed, scales, group=group, bias=w.bias)


def quantize_fp8(w: torch.Tensor, per_channel: bool) -> PackedWeight:
    """fp8 e4m3fn repack (reference/fp8_reference.py:83-91) on the GPU."""
    _need(w, torch.float32, "w")
    n, k = w.shape
    ctx = context(w.device.index)
    data = torch.empty((n, k), dtype=torch.uint8, device=w.device)
    scales = torch.empty((n if per_channel else 1,), dtype=torch.float32, device=w.device)
    ctx.call("lrq_quantize_fp8", _ptr(w), n, k, int(per_channel), _ptr(data), _ptr(scales))
    return PackedWeight(L.LRQ_FMT_FP8, n, k, data, scales, per_channel=per_channel)


def dequant(w: PackedWeight) -> torch.Tensor:
    """f32 [n, k] dequantized weight (bit-exact with the CPU definition)."""
    ctx = context(w.device.index)
    out = torch.empty((w.n, w.k), dtype=torch.float32, device=w.device)
    d = w.desc()
    ctx.call("lrq_dequant", ctypes.byref(d), _ptr(out))
    return out


def dequant_bf16(w: PackedWeight) -> torch.Tensor:
    """The bf16 matrix-core operand (bf16(q*s) for int4, the fp8 value for fp8)."""
    ctx = context(w.device.index)
    out = torch.empty((w.n, w.k), dtype=torch.bfloat16, device=w.device)
    d = w.desc()
    ctx.call("lrq_dequant_bf16", ctypes.byref(d), _ptr(out))
    return out


# ------------------------------------------------------------------ linear
def quant_matmul_t(x: torch.Tensor, w: PackedWeight) -> torch.Tensor:
    """y[m, n] = x[m, k] . dequant(w)^T (+ bias): QuantBackend::quant_matmul_t."""
    _need(x, torch.bfloat16, "x")
    m = x.shape[0]
    if x.dim() != 2 or x.shape[1] != w.k:
        raise ValueError(f"x must be [m, {w.k}], got {tuple(x.shape)}")
    ctx = context(x.device.index)
    y = torch.empty((m, w.n), dtype=torch.bfloat16, device=x.device)
    d = compute_weight(w).desc()
    ctx.call("lrq_quant_matmul_t", ctypes.byref(d), _ptr(x), m, _ptr(y))
    return y


def quant_matmul_t_bwd(dy: torch.Tensor, w: PackedWeight) -> torch.Tensor:
    """dx[m, k] = dy[m, n] . dequant(w): QuantMatmulT::backward."""
    _need(dy, torch.bfloat16, "dy")
    m = dy.shape[0]
    if dy.dim() != 2 or dy.shape[1] != w.n:
        raise ValueError(f"dy must be [m, {w.n}], got {tuple(dy.shape)}")
    ctx = context(dy.device.index)
    dx = torch.empty((m, w.k), dtype=torch.bfloat16, device=dy.device)
    d = compute_weight(w).desc()
    ctx.call("lrq_quant_matmul_t_bwd", ctypes.byref(d), _ptr(dy), m, _ptr(dx))
    return dx


def lora_fwd(x: torch.Tensor, w: PackedWeight, a: torch.Tensor, b: torch.Tensor, scaling: float,
             y: Optional[torch.Tensor] = None, t: Optional[torch.Tensor] = None):
    """Fused site forward. x bf16 [m,k], a bf16 [k,r], b bf16 [r,n] -> (y [m,n], t [m,r])."""
    _need(x, torch.bfloat16, "x")
    m = x.shape[0]
    r = a.shape[1]
    _need(a, torch.bfloat16, "A", (w.k, r))
    _need(b, torch.bfloat16, "B", (r, w.n))
    ctx = context(x.device.index)
    if y is None:
        y = torch.empty((m, w.n), dtype=torch.bfloat16, device=x.device)
    if t is None:
        t = torch.empty((m, r), dtype=torch.bfloat16, device=x.device)
    d = compute_weight(w).desc()
    ctx.call("lrq_lora_fwd", ctypes.byref(d), _ptr(x), m, _ptr(a), _ptr(b), r, float(scaling), _ptr(y), _ptr(t))
    return y, t


def lora_fwd_noalloc(x: torch.Tensor, w: PackedWeight, a: torch.Tensor, b: torch.Tensor, scaling: float,
                     y: torch.Tensor, t: torch.Tensor):
    """``lora_fwd`` through ``lrq_lora_fwd_noalloc``: the library allocates
    nothing (its workspace is a fixed per-GPU scratch array); the caller
    passes every output, and ``w`` must already be blocked. Calls that
    overlap on one GPU race on that array."""
    _need(x, torch.bfloat16, "x")
    m = x.shape[0]
    r = a.shape[1]
    _need(a, torch.bfloat16, "A", (w.k, r))
    _need(b, torch.bfloat16, "B", (r, w.n))
    _need(y, torch.bfloat16, "y", (m, w.n))
    _need(t, torch.bfloat16, "t", (m, r))
    if not w.blocked:
        raise ValueError("lora_fwd_noalloc takes a blocked weight (compute_weight) — blocking allocates")
    ctx = context(x.device.index)
    d = w.desc()
    ctx.call("lrq_lora_fwd_noalloc", ctypes.byref(d), _ptr(x), m, _ptr(a), _ptr(b), r, float(scaling), _ptr(y),
             _ptr(t))
    return y, t


def lora_bwd(x: torch.Tensor, dy: torch.Tensor, w: PackedWeight, a: torch.Tensor, b: torch.Tensor,
             scaling: float, t: torch.Tensor, need_dx: bool = True, need_da: bool = True,
             need_db: bool = True, out=None):
    """Fused site backward -> (dx bf16 [m,k] | None, dA f32 [k,r] | None, dB f32 [r,n] | None)."""
    _need(dy, torch.bfloat16, "dy")
    _need(x, torch.bfloat16, "x")
    _need(t, torch.bfloat16, "t")
    m = dy.shape[0]
    r = a.shape[1]
    _need(a, torch.bfloat16, "A", (w.k, r))
    _need(b, torch.bfloat16, "B", (r, w.n))
    ctx = context(dy.device.index)
    if out is not None:
        dx, da, db = out
    else:
        dx = torch.empty((m, w.k), dtype=torch.bfloat16, device=dy.device) if need_dx else None
        da = torch.empty((w.k, r), dtype=torch.float32, device=dy.device) if need_da else None
        db = torch.empty((r, w.n), dtype=torch.float32, device=dy.device) if need_db else None
    d = compute_weight(w).desc()
    ctx.call("lrq_lora_bwd", ctypes.byref(d), _ptr(x), _ptr(dy), m, _ptr(a), _ptr(b), r, float(scaling),
             _ptr(t), _ptr(dx), _ptr(da), _ptr(db))
    return dx, da, db


# ------------------------------------------------------------------ profiling
def profile_enable(on: bool, device: Optional[int] = None):
    ctx = context(device)
    ctx.call("lrq_profile_enable", int(on))


def profile_reset(device: Optional[int] = None):
    ctx = context(device)
    ctx.call("lrq_profile_reset")


def profile_read(device: Optional[int] = None) -> dict:
    """{kernel name: (total ms, launches)} for every kernel id."""
    ctx = context(device)
    out = {}
    for kid in range(ctx.lib.lrq_profile_count()):
        ms = ctypes.c_double()
        n = ctypes.c_int64()
        ctx.call("lrq_profile_read", kid, ctypes.byref(ms), ctypes.byref(n))
        out[ctx.lib.lrq_profile_name(kid).decode()] = (ms.value, n.value)
    return out


def sync(device: Optional[int] = None):
    """Wait for torch's current stream and raise ``LrqError`` if a few-token
    kernel flagged a failure on the device since the last check (an
    epilogue whose bounded wait for t or u ran out; it wrote NaN outputs).
    The library clears the flag and resets its counters when it reports it.
    A training step calls this once, after reading its loss."""
    context(device).call("lrq_sync")


def debug_force_wait_timeout(on: bool):
    """Test hook: make later few-token launches give up their wait for t
    (the failure path ``sync`` reports). Never on in a real run."""
    L.load().lrq_debug_force_wait_timeout(int(on))


GEMM_PATHS = {"planned": 0, "large": 1, "mid64": 2, "mid128": 3, "mid64s": 4, "mid128s": 5}


def debug_gemm_path(path: str):
    """Tuning and test hook: force the kernel the fused products of m > 16
    tokens take in this process ("planned", "large": the 256-token tiles,
    split in depth when too few, "mid64" / "mid128": 64-row tiles of 64 or
    128 tokens, with depth ranges as planned, "mid64s" / "mid128s": the same
    with at least two depth ranges where the depth allows). Every path
    computes the same products."""
    L.load().lrq_debug_gemm_path(GEMM_PATHS[path])


def probe_stream_read(t: torch.Tensor):
    """Read every byte of the contiguous device tensor ``t`` once (a plain
    streaming read, for timing the box's read rate)."""
    if not t.is_cuda or not t.is_contiguous():
        raise ValueError("probe_stream_read takes a contiguous GPU tensor")
    context(t.device.index).call("lrq_probe_stream_read", _ptr(t), t.numel() * t.element_size())


def profile_relaunch(kernel: str, n: int, ctx: Optional[Context] = None, on_stream=None):
    """Repeat the last launch of ``kernel`` (a profiler name such as
    "fwd_main" or "bwd_dx") on ``ctx`` (default: the current stream's
    context) ``n`` times with the same arguments, to time that kernel alone.
    ``on_stream`` (a torch stream) issues the repeats there instead of on the
    context's stream, e.g. to capture them into a graph."""
    ctx = ctx if ctx is not None else context()
    names = [ctx.lib.lrq_profile_name(i).decode() for i in range(ctx.lib.lrq_profile_count())]
    kid = names.index(kernel)
    with ctx.lock:
        if on_stream is not None:
            ctx.call("lrq_set_stream", ctypes.c_void_p(on_stream.cuda_stream))
        try:
            ctx.call("lrq_profile_relaunch", kid, n)
        finally:
            if on_stream is not None:
                ctx.call("lrq_set_stream", ctypes.c_void_p(ctx.stream))


def reserve(m: int, n: int, k: int, r: int, device: Optional[int] = None):
    ctx = context(device)
    ctx.call("lrq_reserve", m, n, k, r)
