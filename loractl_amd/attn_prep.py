"""Attention inputs of a double-stream block, through libloractl_mmdit.so.

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
