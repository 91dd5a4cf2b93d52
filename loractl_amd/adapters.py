"""Adapter injection and the quantized site seam — the host mirror of
``crates/loractl-core/src/adapters.rs`` and the quant arm of
``crates/loractl-core/src/mmdit.rs:413-536``.

- ``LoraAdapters.get/apply`` (adapters.rs:57-86): a name-keyed set of deltas
  looked up by module path by a linear scan; ``apply`` returns
  ``base_out + delta(x)`` or ``base_out`` unchanged.
- ``build_adapters`` (adapters.rs:116-145): the first matching regex target
  per site decides rank/alpha overrides; registration follows site order;
  an invalid pattern raises immediately.
- ``QuantLinear`` / ``BaseLinear`` (mmdit.rs:413-520): row chunks in file
  layout concatenated along d_out, optional full-precision bias, leading dims
  flattened to ``[n, d_in]`` and restored.
- ``site`` (mmdit.rs:526-536): base + delta. When the base is quantized and a
  delta is registered, the pair runs as ONE fused op in libloractl_rocm.so;
  otherwise the reference's two-step semantics apply unchanged.
"""

from __future__ import annotations

import contextlib
import re
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import torch

from . import device as D
from .lora import LoraDelta, quant_lora_linear
from .quant import (DEFAULT_DEQUANT_CHUNK_MIB, QUANT_BLOCK, QuantBackend, QuantValue, concat_chunks,
                    quantize_linear_weight_chunked)


@dataclass
class TargetSpec:
    pattern: str
    rank: Optional[int] = None
    alpha: Optional[float] = None


@dataclass
class LoraConfig:
    rank: int = 16
    alpha: float = 16.0
    dropout: float = 0.0
    targets: List[TargetSpec] = field(default_factory=list)


@dataclass
class LoraSite:
    path: str
    d_in: int
    d_out: int


class LoraAdapters(torch.nn.Module):
    def __init__(self, deltas: Sequence[LoraDelta], targets: Sequence[str]):
        super().__init__()
        if len(deltas) != len(targets):
            raise ValueError("deltas and targets must be in lockstep")
        self.deltas = torch.nn.ModuleList(deltas)
        self.targets = list(targets)

    def get(self, path: str) -> Optional[LoraDelta]:
        for i, t in enumerate(self.targets):
            if t == path:
                return self.deltas[i]
        return None

    def apply(self, path: str, x: torch.Tensor, base_out: torch.Tensor) -> torch.Tensor:
        delta = self.get(path)
        return base_out + delta(x) if delta is not None else base_out

    @contextlib.contextmanager
    def cached_factors(self):
        """Inside the block the fused sites use bf16 copies of every delta's
        factors, made once on entry, for passes whose factors do not change
        between them (a step's capture and replay). Changing a factor inside
        the block is not seen by the fused sites."""
        params = [p for d in self.deltas for p in (d.lora_a, d.lora_b)]
        casts = [torch.empty(p.shape, dtype=torch.bfloat16, device=p.device) for p in params]
        with torch.no_grad():
            torch._foreach_copy_(casts, params)  # all factors in a few multi-tensor launches
        for i, d in enumerate(self.deltas):
            d.bf16_cache = casts[2 * i:2 * i + 2]
        try:
            yield self
        finally:
            for d in self.deltas:
                d.bf16_cache = None


def build_adapters(sites: Sequence[LoraSite], cfg: LoraConfig, device=None) -> LoraAdapters:
    compiled = []
    for spec in cfg.targets:
        try:
            compiled.append((re.compile(spec.pattern), spec))
        except re.error as e:
            raise ValueError(f"invalid LoRA target pattern {spec.pattern!r}: {e}") from e
    deltas, targets = [], []
    for site_ in sites:
        for rx, spec in compiled:
            if rx.search(site_.path):
                rank = spec.rank if spec.rank is not None else cfg.rank
                alpha = spec.alpha if spec.alpha is not None else cfg.alpha
                deltas.append(LoraDelta(site_.d_in, site_.d_out, rank, alpha, cfg.dropout, device=device))
                targets.append(site_.path)
                break
    return LoraAdapters(deltas, targets)


class QuantLinear:
    """Frozen quantized linear (src/mmdit.rs:413-444): the reference keeps a
    ``Vec`` of packed row chunks in file layout ``[rows_i, d_in]``,
    concatenated along d_out. The chunks are joined once into one weight in
    the blocked layout the fused kernels read, and only that is kept (the
    row-layout chunks are released, so the weight holds 2x its packed bytes:
    the blocked row and transposed sections); ``chunk_rows`` records the
    chunking."""

    def __init__(self, weight: List[D.PackedWeight], bias: Optional[torch.Tensor] = None):
        if not weight:
            raise ValueError("QuantLinear holds at least one chunk")
        self.chunk_rows = [c.n for c in weight]
        joined = weight[0] if len(weight) == 1 else concat_chunks(list(weight))
        self._joined = D.compute_weight(joined)
        self.bias = bias

    @property
    def d_in(self) -> int:
        return self._joined.k

    @property
    def d_out(self) -> int:
        return self._joined.n

    @property
    def packed(self) -> D.PackedWeight:
        return self._joined

    def dequantized_weight(self) -> torch.Tensor:
        """Diagnostics only: the full f32 [d_out, d_in] weight."""
        return D.dequant(self._joined)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1])
        w = self._joined if self.bias is None else self._joined.with_bias(self.bias.float().contiguous())
        y = QuantBackend.quant_matmul_t(x2, w)
        return y.reshape(*lead, self.d_out)


class PlainLinear:
    """The unquantized frozen base in burn layout: weight [d_in, d_out], x.W (+b)."""

    def __init__(self, weight: torch.Tensor, bias: Optional[torch.Tensor] = None):
        self.weight = weight
        self.bias = bias

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = x @ self.weight.to(x.dtype)
        return y + self.bias.to(x.dtype) if self.bias is not None else y


BaseLinear = (PlainLinear, QuantLinear)


def quantize_field(base, value: QuantValue = QuantValue.Q4S, chunk_bytes: int = DEFAULT_DEQUANT_CHUNK_MIB << 20,
                   group: int = QUANT_BLOCK):
    """One base site quantized (src/mmdit.rs:1266-1280): a ``PlainLinear``
    whose burn-layout ``[d_in, d_out]`` weight is block-aligned becomes a
    ``QuantLinear`` (the weight transposed to file layout ``[d_out, d_in]``,
    then quantized as row chunks under ``chunk_bytes``; the bias is kept); a
    ``QuantLinear``, or a ``PlainLinear`` whose ``d_in`` is not a multiple of
    the reference's quant block (32), is returned unchanged. So is one whose
    ``d_out`` is not a multiple of 8, which the fused kernels cannot write:
    it runs as the reference's Plain arm. A caller-chosen ``group`` that does
    not divide an aligned ``d_in`` raises, as the reference's quantizer panics
    (src/quant.rs:76-80)."""
    if not isinstance(base, PlainLinear):
        return base
    d_in, d_out = base.weight.shape
    if d_in % QUANT_BLOCK != 0 or d_out % 8 != 0:
        return base
    chunks = quantize_linear_weight_chunked(base.weight.t().contiguous(), value, chunk_bytes, group)
    return QuantLinear(chunks, base.bias)


def into_quantized(sites: dict, value: QuantValue = QuantValue.Q4S,
                   chunk_bytes: int = DEFAULT_DEQUANT_CHUNK_MIB << 20, group: int = QUANT_BLOCK) -> dict:
    """``Mmdit::into_quantized_chunked`` (src/mmdit.rs:1134-1158) over a
    ``{site path: base}`` map: every base through ``quantize_field``."""
    return {path: quantize_field(b, value, chunk_bytes, group) for path, b in sites.items()}


def site(adapters: Optional[LoraAdapters], path: str, base, x: torch.Tensor) -> torch.Tensor:
    """Run a base linear at an injectable site, adding any registered delta."""
    if adapters is None:
        return base.forward(x)
    delta = adapters.get(path)
    if delta is not None and isinstance(base, QuantLinear):
        return quant_lora_linear(x, base.packed, delta, base.bias)
    return adapters.apply(path, x, base.forward(x))
