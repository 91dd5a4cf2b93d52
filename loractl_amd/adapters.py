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

import re
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import torch

from . import device as D
from .lora import LoraDelta, quant_lora_linear
from .quant import QuantBackend, concat_chunks


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
    """Frozen quantized linear: packed row chunks in file layout [d_out, d_in]."""

    def __init__(self, weight: List[D.PackedWeight], bias: Optional[torch.Tensor] = None):
        if not weight:
            raise ValueError("QuantLinear holds at least one chunk")
        self.weight = list(weight)
        self.bias = bias
        if len(self.weight) == 1:
            self._joined = D.compute_weight(self.weight[0])
        else:
            self._joined = D.block(concat_chunks(self.weight))

    @property
    def d_in(self) -> int:
        return self.weight[0].k

    @property
    def d_out(self) -> int:
        return sum(c.n for c in self.weight)

    @property
    def packed(self) -> D.PackedWeight:
        return self._joined

    def dequantized_weight(self) -> torch.Tensor:
        """Diagnostics only: the full f32 [d_out, d_in] weight."""
        return torch.cat([D.dequant(c) for c in self.weight], 0)

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


def site(adapters: Optional[LoraAdapters], path: str, base, x: torch.Tensor) -> torch.Tensor:
    """Run a base linear at an injectable site, adding any registered delta."""
    if adapters is None:
        return base.forward(x)
    delta = adapters.get(path)
    if delta is not None and isinstance(base, QuantLinear):
        return quant_lora_linear(x, base.packed, delta, base.bias)
    return adapters.apply(path, x, base.forward(x))
