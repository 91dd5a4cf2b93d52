"""fp8 e4m3fn frozen bases on the ROCm backend — the host mirror of the
decode half of ``crates/loractl-core/src/fp8.rs``.

- ``ScaleKind`` classification (fp8.rs:58-68, fp8.rs:109-234): a
  ``<name>_scale`` sidecar of shape ``[]`` or ``[1]`` is one scalar, shape
  ``[out_features]`` (weight axis 0) is per output channel, anything else is
  a hard error naming the tensor.
- ``fp8_weight`` keeps the raw e4m3fn bytes on the GPU and decodes them
  inside the fused kernels (``LUT[byte] * scale``, fp8.rs:306-318, applied
  in the f32 epilogue along d_out); ``dequant`` gives the f32 tensor the
  reference's lazy snapshot would materialise.
- ``quantize_fp8`` is the repack encoder of reference/fp8_reference.py:83-91
  (no counterpart in the crate) with saturation at +-448.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import device as D


def fp8_weight(name: str, data: torch.Tensor, scale: torch.Tensor,
               bias: Optional[torch.Tensor] = None) -> D.PackedWeight:
    """Wrap an e4m3fn weight ``[out, in]`` and its f32 ``scale`` sidecar."""
    if data.dim() != 2:
        raise ValueError(f"fp8 tensor '{name}' must be 2-D [out, in], got {tuple(data.shape)}")
    if data.dtype not in (torch.uint8, getattr(torch, "float8_e4m3fn", torch.uint8)):
        raise ValueError(f"fp8 tensor '{name}' must hold e4m3fn bytes, got {data.dtype}")
    if scale.dtype != torch.float32:
        raise ValueError(f"scale sidecar '{name}_scale' must be F32, got {scale.dtype}")
    n, k = data.shape
    shape = tuple(scale.shape)
    if shape in ((), (1,)):
        per_channel = False
    elif shape == (n,):
        per_channel = True
    else:
        raise ValueError(
            f"scale sidecar '{name}_scale' has shape {list(shape)}: expected [] / [1] (scalar) or [{n}] "
            "(per output channel)"
        )
    raw = data.view(torch.uint8) if data.dtype != torch.uint8 else data
    return D.PackedWeight(D.L.LRQ_FMT_FP8, n, k, raw.contiguous(), scale.reshape(-1).contiguous(),
                          per_channel=per_channel, bias=bias)


def quantize_fp8(w: torch.Tensor, per_channel: bool) -> D.PackedWeight:
    return D.quantize_fp8(w.float().contiguous(), per_channel)


def dequant(w: D.PackedWeight) -> torch.Tensor:
    return D.dequant(w)
