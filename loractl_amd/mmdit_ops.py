"""The double-stream block's glue kernels, through libloractl_mmdit.so:
attention inputs (``attn_prep``), the modulated RMSNorm (``modnorm``) and the
gated residual's gradient (``gated_residual``).

``attn_prep(qkv_txt, qkv_img, rope, heads)`` takes the two streams' QKV
linear outputs (``[l, 3h]`` rows ``[q | k | v]``) and returns q, k, v as
``[L, heads, head_dim]`` bf16 over the joint text-then-image sequence, with
q and k each RMS-normalised per head and rotated by RoPE — the reference's
head split, QK-norm and ``apply_rope`` (``mmdit.rs:599-619``, ``ZRmsNorm``
``:307-330`` with its frozen zero gain, ``apply_rope`` ``:385-399``) as one
kernel, and its gradient as one more. Loading never falls back to torch: a
missing library or symbol raises.
"""

from __future__ import annotations

import ctypes
import os
from typing import Tuple

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libloractl_mmdit.so")

_vp, _i64, _i32, _f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
SIGNATURES = {
    "lmd_last_error": ([], ctypes.c_char_p),
    "lmd_colsum_groups": ([_i64], _i64),
    "lmd_modnorm_fwd": ([_vp, _i64, _i32, _vp, _vp, _f32, _vp, _vp, _vp], _i32),
    "lmd_modnorm_bwd": ([_vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i32),
    "lmd_gated_residual_bwd": ([_vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp], _i32),
    "lmd_gated_residual_fwd": ([_vp, _vp, _i64, _i32, _vp, _vp, _vp], _i32),
    "lmd_gelu_tanh_fwd": ([_vp, _i64, _vp, _vp], _i32),
    "lmd_gelu_tanh_bwd": ([_vp, _vp, _i64, _vp, _vp], _i32),
    "lmd_attn_prep_fwd": ([_vp, _i64, _vp, _i64, _i32, _i32, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _vp], _i32),
    "lmd_attn_prep_bwd": ([_vp, _vp, _vp, _vp, _i64, _vp, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp], _i32),
}
_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed ({rc}): {load().lmd_last_error().decode()}")


def rope_tables(L: int, head_dim: int, device, theta: float = 10000.0) -> Tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin) f32 ``[L, head_dim / 2]``: pair (2j, 2j+1) of position p
    turns by ``p * theta^(-2j / head_dim)``; the angles are formed in f64."""
    inv = theta ** (-torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim)
    ang = torch.arange(L, dtype=torch.float64)[:, None] * inv[None]
    return (torch.cos(ang).float().contiguous().to(device), torch.sin(ang).float().contiguous().to(device))


def _ptr(t):
    return t.data_ptr() if t is not None and t.numel() > 0 else None


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class _AttnPrep(torch.autograd.Function):
    @staticmethod
    def forward(ctx, qkv_txt, qkv_img, cos, sin, heads: int, eps: float):
        lt, li = qkv_txt.shape[0], qkv_img.shape[0]
        h = qkv_img.shape[1] // 3
        hd = h // heads
        if qkv_txt.shape[1] != 3 * h or h % heads or cos.shape != (lt + li, hd // 2) or sin.shape != cos.shape:
            raise ValueError(f"attn_prep: shapes {tuple(qkv_txt.shape)} {tuple(qkv_img.shape)} "
                             f"{tuple(cos.shape)} do not fit {heads} heads")
        for t in (qkv_txt, qkv_img):
            if t.dtype != torch.bfloat16 or not t.is_contiguous() or not t.is_cuda:
                raise ValueError("attn_prep: qkv rows must be contiguous bf16 on the GPU")
        L = lt + li
        dev = qkv_img.device
        q = torch.empty(L, heads, hd, device=dev, dtype=torch.bfloat16)
        k = torch.empty_like(q)
        v = torch.empty_like(q)
        rstd = torch.empty(2, L, heads, device=dev, dtype=torch.float32)
        _check(load().lmd_attn_prep_fwd(_ptr(qkv_txt), lt, _ptr(qkv_img), li, heads, hd, cos.data_ptr(),
                                        sin.data_ptr(), eps, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                        rstd.data_ptr(), _stream(dev)), "lmd_attn_prep_fwd")
        ctx.save_for_backward(qkv_txt, qkv_img, cos, sin, rstd)
        ctx.heads = heads
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk, dv):
        qkv_txt, qkv_img, cos, sin, rstd = ctx.saved_tensors
        lt, li = qkv_txt.shape[0], qkv_img.shape[0]
        hd = qkv_img.shape[1] // 3 // ctx.heads
        dq, dk, dv = (g.to(torch.bfloat16).contiguous() for g in (dq, dk, dv))
        dt = torch.empty_like(qkv_txt)
        di = torch.empty_like(qkv_img)
        _check(load().lmd_attn_prep_bwd(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), _ptr(qkv_txt), lt,
                                        _ptr(qkv_img), li, ctx.heads, hd, cos.data_ptr(), sin.data_ptr(),
                                        rstd.data_ptr(), _ptr(dt), _ptr(di), _stream(qkv_img.device)),
               "lmd_attn_prep_bwd")
        return dt, di, None, None, None, None


def attn_prep(qkv_txt: torch.Tensor, qkv_img: torch.Tensor, rope: Tuple[torch.Tensor, torch.Tensor], heads: int,
              eps: float = 1e-5):
    """q, k, v ``[L, heads, head_dim]`` bf16 (text tokens first) from the two
    streams' QKV rows, differentiable in both."""
    cos, sin = rope
    return _AttnPrep.apply(qkv_txt, qkv_img, cos, sin, heads, eps)


def _rows(x: torch.Tensor, vec: torch.Tensor, what: str):
    h = x.shape[-1]
    if x.dtype != torch.bfloat16 or vec.dtype != torch.bfloat16 or not x.is_cuda:
        raise ValueError(f"{what}: bf16 tensors on the GPU expected")
    if vec.numel() != h or not vec.is_contiguous():
        raise ValueError(f"{what}: the vector must be one contiguous row of {h}")
    return x.reshape(-1, h).contiguous(), h


class _ModNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, scale, shift, eps: float):
        x2, h = _rows(x, scale, "modnorm")
        if shift.numel() != h or shift.dtype != torch.bfloat16 or not shift.is_contiguous():
            raise ValueError("modnorm: shift must be one contiguous bf16 row")
        rows = x2.shape[0]
        out = torch.empty_like(x2)
        rstd = torch.empty(rows, device=x2.device, dtype=torch.float32)
        _check(load().lmd_modnorm_fwd(x2.data_ptr(), rows, h, scale.data_ptr(), shift.data_ptr(), eps,
                                      out.data_ptr(), rstd.data_ptr(), _stream(x2.device)), "lmd_modnorm_fwd")
        ctx.save_for_backward(x2, scale, rstd)
        ctx.shapes = (x.shape, scale.shape, shift.shape)
        return out.view(x.shape)

    @staticmethod
    def backward(ctx, dh):
        x2, scale, rstd = ctx.saved_tensors
        rows, h = x2.shape
        dh2 = dh.to(torch.bfloat16).reshape(rows, h).contiguous()
        dx = torch.empty_like(x2)
        dscale = torch.empty(h, device=x2.device, dtype=torch.bfloat16)
        dshift = torch.empty_like(dscale)
        part = torch.empty(load().lmd_colsum_groups(rows) * 2 * h, device=x2.device, dtype=torch.float32)
        _check(load().lmd_modnorm_bwd(dh2.data_ptr(), x2.data_ptr(), rows, h, scale.data_ptr(), rstd.data_ptr(),
                                      dx.data_ptr(), dscale.data_ptr(), dshift.data_ptr(), part.data_ptr(),
                                      _stream(x2.device)), "lmd_modnorm_bwd")
        xs, ss, hs = ctx.shapes
        return dx.view(xs), dscale.view(ss), dshift.view(hs), None


class _GatedResidual(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, gate, o):
        o2, h = _rows(o, gate, "gated_residual")
        if x.shape != o.shape or x.dtype != torch.bfloat16:
            raise ValueError("gated_residual: x must be bf16 with the shape of o")
        x2 = x.reshape(-1, h).contiguous()
        rows = o2.shape[0]
        y = torch.empty_like(x2)
        _check(load().lmd_gated_residual_fwd(x2.data_ptr(), o2.data_ptr(), rows, h, gate.data_ptr(), y.data_ptr(),
                                             _stream(o2.device)), "lmd_gated_residual_fwd")
        ctx.save_for_backward(o2, gate)
        ctx.shapes = (o.shape, gate.shape)
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        o2, gate = ctx.saved_tensors
        rows, h = o2.shape
        dy2 = dy.to(torch.bfloat16).reshape(rows, h).contiguous()
        do = torch.empty_like(o2)
        dgate = torch.empty(h, device=o2.device, dtype=torch.bfloat16)
        part = torch.empty(load().lmd_colsum_groups(rows) * h, device=o2.device, dtype=torch.float32)
        _check(load().lmd_gated_residual_bwd(dy2.data_ptr(), o2.data_ptr(), rows, h, gate.data_ptr(), do.data_ptr(),
                                             dgate.data_ptr(), part.data_ptr(), _stream(o2.device)),
               "lmd_gated_residual_bwd")
        os_, gs = ctx.shapes
        return dy, dgate.view(gs), do.view(os_)


class _GeluTanh(torch.autograd.Function):
    @staticmethod
    def forward(ctx, u):
        if u.dtype != torch.bfloat16 or not u.is_cuda or u.numel() % 8:
            raise ValueError("gelu_tanh: a bf16 GPU tensor of a multiple of 8 elements expected")
        u2 = u.contiguous()
        g = torch.empty_like(u2)
        _check(load().lmd_gelu_tanh_fwd(u2.data_ptr(), u2.numel(), g.data_ptr(), _stream(u2.device)),
               "lmd_gelu_tanh_fwd")
        ctx.save_for_backward(u2)
        return g

    @staticmethod
    def backward(ctx, dg):
        (u,) = ctx.saved_tensors
        dg2 = dg.to(torch.bfloat16).contiguous()
        du = torch.empty_like(u)
        _check(load().lmd_gelu_tanh_bwd(dg2.data_ptr(), u.data_ptr(), u.numel(), du.data_ptr(), _stream(u.device)),
               "lmd_gelu_tanh_bwd")
        return du


def gelu_tanh(u: torch.Tensor) -> torch.Tensor:
    """``u (1 + tanh(sqrt(2/pi) (u + 0.044715 u^3))) / 2``, the MLP activation
    of the FLUX-style blocks (``F.gelu(u, approximate="tanh")``), in f32 with
    one rounding; forward and gradient are one kernel each."""
    return _GeluTanh.apply(u)


def modnorm(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """``(scale + 1) * x / sqrt(mean(x^2) + eps) + shift`` per row of x
    (``mmdit.rs:857-870``: ZRmsNorm with its frozen zero gain, then the
    block's pre/post modulation), differentiable in x, scale and shift."""
    return _ModNorm.apply(x, scale, shift, eps)


def gated_residual(x: torch.Tensor, gate: torch.Tensor, o: torch.Tensor) -> torch.Tensor:
    """``x + gate * o`` (``mmdit.rs:860-869``), gate one row broadcast over
    the rows of o; the forward is one kernel, the gradient in gate and o
    another."""
    return _GatedResidual.apply(x, gate, o)
