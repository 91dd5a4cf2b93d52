"""LoRA factors and the fused quantized-base site op.

``LoraDelta`` mirrors ``crates/loractl-core/src/lora.rs:154-204``: a base-free
low-rank update ``scaling * B(A(dropout(x)))`` with ``A`` ``[d_in, rank]`` and
``B`` ``[rank, d_out]`` in burn's layout, ``rank`` clamped to at least 1,
``scaling = alpha / rank``, ``A`` Kaiming-uniform (burn's ``LinearConfig``
default, bound ``1/sqrt(d_in)``) and ``B`` zero, so a fresh delta is an exact
no-op (lora.rs:113-137).

``QuantLoraLinear`` is the drop-in for ``site()`` when the base is quantized
and a delta is registered (mmdit.rs:526-536 + adapters.rs:75-85): one fused
forward ``y = x . dequant(wq)^T (+bias) + s . (x . A) . B`` and a 3-parent
backward (x, A, B; the frozen weight never gets a gradient) that runs in
libloractl_rocm.so. Dropout must be 0 on this path (the block-checkpointed
trainer already refuses p > 0: diffusion_trainer.rs:342-348).
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import device as D


class LoraDelta(torch.nn.Module):
    def __init__(self, d_input: int, d_output: int, rank: int, alpha: float, dropout_prob: float = 0.0,
                 device=None, dtype=torch.float32):
        super().__init__()
        rank = max(int(rank), 1)
        bound = 1.0 / math.sqrt(d_input) if d_input > 0 else 0.0
        a = torch.empty((d_input, rank), device=device, dtype=dtype).uniform_(-bound, bound)
        self.lora_a = torch.nn.Parameter(a)
        self.lora_b = torch.nn.Parameter(torch.zeros((rank, d_output), device=device, dtype=dtype))
        self.scaling = float(alpha) / rank
        self.dropout_prob = float(dropout_prob)
        self.rank = rank
        self.bf16_cache = None  # [A, B] in bf16 while LoraAdapters.cached_factors() is open

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """The plain (unfused) delta, for sites whose base is not quantized."""
        if self.dropout_prob > 0 and self.training:
            x = torch.nn.functional.dropout(x, self.dropout_prob, True)
        return (x @ self.lora_a.to(x.dtype)) @ self.lora_b.to(x.dtype) * self.scaling


class _QuantLoraFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x2: torch.Tensor, a: torch.Tensor, b: torch.Tensor, wq: D.PackedWeight, scaling: float,
                factors=None):
        xb = x2.to(torch.bfloat16).contiguous()
        if factors is None:
            ab = a.detach().to(torch.bfloat16).contiguous()
            bb = b.detach().to(torch.bfloat16).contiguous()
        else:
            ab, bb = factors
        y, t = D.lora_fwd(xb, wq, ab, bb, scaling)
        ctx.save_for_backward(xb, ab, bb, t)
        ctx.wq = wq
        ctx.scaling = scaling
        ctx.dtypes = (x2.dtype, a.dtype, b.dtype)
        return y.to(x2.dtype)

    @staticmethod
    def backward(ctx, gy: torch.Tensor):
        xb, ab, bb, t = ctx.saved_tensors
        need_dx, need_da, need_db = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        dyb = gy.to(torch.bfloat16).contiguous()
        dx, da, db = D.lora_bwd(xb, dyb, ctx.wq, ab, bb, ctx.scaling, t, need_dx, need_da, need_db)
        xd, ad, bd = ctx.dtypes
        return (dx.to(xd) if dx is not None else None, da.to(ad) if da is not None else None,
                db.to(bd) if db is not None else None, None, None, None)


def quant_lora_linear(x: torch.Tensor, wq: D.PackedWeight, delta: LoraDelta,
                      bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused ``base(x) + delta(x)`` for a quantized base; x is ``[.., d_in]``."""
    if delta.dropout_prob > 0 and delta.training:
        raise ValueError("compute.backend rocm fuses the LoRA delta and supports adapter dropout 0 only")
    if delta.rank > 64:
        raise ValueError(f"compute.backend rocm supports LoRA rank <= 64, got {delta.rank}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    w = wq if bias is None else wq.with_bias(bias.float().contiguous())
    cache = getattr(delta, "bf16_cache", None)  # (A, B) in bf16 inside LoraAdapters.cached_factors()
    y = _QuantLoraFn.apply(x2, delta.lora_a, delta.lora_b, w, delta.scaling, tuple(cache) if cache else None)
    return y.reshape(*lead, wq.n)
