"""Frozen-base quantization on the ROCm backend — the host mirror of
``crates/loractl-core/src/quant.rs``.

Same names, argument meaning and error behaviour as the reference:

- ``QUANT_BLOCK`` / ``quant_scheme`` (quant.rs:47-67): per-block symmetric
  scheme with an f32 scale; the block size is a parameter here (32 is the
  reference's, 64 the benchmark configs').
- ``quantize_linear_weight`` (quant.rs:74-82): quantizes one ``[d_out, d_in]``
  weight; a ``d_in`` that does not divide into blocks is a programmer error
  and raises (the reference panics with the same message).
- ``dequant_chunk_rows`` / ``quantize_linear_weight_chunked``
  (quant.rs:102-150): the balanced row-chunk layout, a pure function.
- ``quant_value`` (quant.rs:156-162).
- ``quant_matmul_t`` (quant.rs:172-178, the Autodiff override
  ``QuantMatmulT`` at quant.rs:210-263): ``x . dequant(wq)^T`` with the weight
  as a constant; the backward re-dequantizes from packed storage and gives
  ``grad_x = grad . dequant(wq)`` and no weight gradient.

The compute runs in libloractl_rocm.so on the GPU; there is no CPU path.
Both values of the knob are built: ``Q4S`` (int4, packed nibbles) and
``Q8S`` (int8 bytes), each with f32 block scales.
"""

from __future__ import annotations

import enum
from dataclasses import dataclass
from typing import List, Optional

import torch

from . import device as D

QUANT_BLOCK = 32
DEFAULT_DEQUANT_CHUNK_MIB = 512  # crates/loractl-core/src/config.rs:688


class QuantValue(enum.Enum):
    Q8S = "q8s"
    Q4S = "q4s"


class Quant(enum.Enum):
    """The ``compute.quant`` config knob (config.rs:635-676)."""

    NONE = "none"
    INT8 = "int8"
    INT4 = "int4"

    @classmethod
    def parse(cls, s: str) -> "Quant":
        key = s.strip().lower()
        for q in cls:
            if q.value == key:
                return q
        raise ValueError(f"unknown quant {s!r}: expected one of none, int8, int4")


def quant_value(q: Quant) -> Optional[QuantValue]:
    return {Quant.NONE: None, Quant.INT8: QuantValue.Q8S, Quant.INT4: QuantValue.Q4S}[q]


@dataclass(frozen=True)
class QuantScheme:
    value: QuantValue
    block: tuple
    param: str = "F32"
    mode: str = "Symmetric"


def quant_scheme(value: QuantValue, group: int = QUANT_BLOCK) -> QuantScheme:
    return QuantScheme(value=value, block=(1, group))


def _check_block(d_out: int, d_in: int, group: int):
    if d_in % group != 0:
        raise AssertionError(
            f"linear weight [{d_out}, {d_in}]: the input dim must be a multiple of the quant block ({group})"
        )


def quantize_linear_weight(weight: torch.Tensor, value: QuantValue = QuantValue.Q4S,
                           group: int = QUANT_BLOCK) -> D.PackedWeight:
    """Quantize one file-layout ``[d_out, d_in]`` f32 weight on the GPU."""
    d_out, d_in = weight.shape
    _check_block(d_out, d_in, group)
    if group & (group - 1):
        raise ValueError(f"compute.backend rocm needs a power-of-two quant block, got {group}")
    # quantize in the interchange row layout, keep the blocked layout the fused kernels read
    return D.block(_quantize(weight.float().contiguous(), value, group))


def _quantize(w32: torch.Tensor, value: QuantValue, group: int) -> D.PackedWeight:
    """One f32 ``[d_out, d_in]`` weight at ``value`` in the row layout."""
    if value is QuantValue.Q8S:
        return D.quantize_int8(w32, group)
    return D.quantize_int4(w32, group)


def dequant_chunk_rows(d_out: int, d_in: int, chunk_bytes: int) -> List[int]:
    full = d_out * d_in * 4
    if chunk_bytes == 0 or full <= chunk_bytes or d_out <= 1:
        return [d_out]
    max_rows = max(chunk_bytes // (d_in * 4), 1)
    n_chunks = -(-d_out // max_rows)
    base, rem = divmod(d_out, n_chunks)
    return [base + 1 if i < rem else base for i in range(n_chunks)]


def quantize_linear_weight_chunked(weight: torch.Tensor, value: QuantValue = QuantValue.Q4S,
                                   chunk_bytes: int = DEFAULT_DEQUANT_CHUNK_MIB << 20,
                                   group: int = QUANT_BLOCK) -> List[D.PackedWeight]:
    """Row chunks in the interchange row layout (QuantLinear joins and blocks them)."""
    d_out, d_in = weight.shape
    _check_block(d_out, d_in, group)
    rows = dequant_chunk_rows(d_out, d_in, chunk_bytes)
    out, start = [], 0
    for r in rows:
        out.append(_quantize(weight[start:start + r].float().contiguous(), value, group))
        start += r
    return out


def concat_chunks(chunks: List[D.PackedWeight]) -> D.PackedWeight:
    """Join row chunks along d_out into one packed weight (the fused kernels
    never materialise the f32 transient the chunking exists to bound)."""
    if len(chunks) == 1:
        return chunks[0]
    c0 = chunks[0]
    if any(c.fmt != c0.fmt or c.k != c0.k or c.group != c0.group for c in chunks):
        raise ValueError("row chunks of one weight must share format, d_in and block")
    if c0.fmt == D.L.LRQ_FMT_FP8 and any(c.per_channel != c0.per_channel for c in chunks):
        raise ValueError("fp8 row chunks must share the scale kind")
    if any(c.blocked for c in chunks):
        raise ValueError("row chunks are joined in the row layout; block the joined weight afterwards")
    data = torch.cat([c.data for c in chunks], 0).contiguous()
    if c0.fmt == D.L.LRQ_FMT_FP8 and not c0.per_channel:
        if any(not torch.equal(c.scales, c0.scales) for c in chunks):
            raise ValueError("scalar-scale fp8 chunks with different scales cannot be joined")
        scales = c0.scales
    else:
        scales = torch.cat([c.scales for c in chunks], 0).contiguous()
    return D.PackedWeight(c0.fmt, sum(c.n for c in chunks), c0.k, data, scales, c0.group, c0.per_channel)


class QuantMatmulT(torch.autograd.Function):
    """``x . dequant(wq)^T`` with ``wq`` a constant (quant.rs:210-263)."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, wq: D.PackedWeight):
        ctx.wq = wq
        ctx.in_dtype = x.dtype
        y = D.quant_matmul_t(x.to(torch.bfloat16).contiguous(), wq)
        return y.to(x.dtype)

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        dx = D.quant_matmul_t_bwd(grad.to(torch.bfloat16).contiguous(), ctx.wq)
        return dx.to(ctx.in_dtype), None


class QuantBackend:
    """``QuantBackend`` (quant.rs:172-178) for ``compute.backend: rocm``."""

    @staticmethod
    def quant_matmul_t(x: torch.Tensor, wq: D.PackedWeight) -> torch.Tensor:
        if not isinstance(wq, D.PackedWeight):
            raise TypeError("quant_matmul_t requires a quantized weight — see quantize_linear_weight")
        return QuantMatmulT.apply(x, wq)


quant_matmul_t = QuantBackend.quant_matmul_t
