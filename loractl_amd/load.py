"""Scaled-fp8 safetensors checkpoints onto the GPU: the on-device load path
for frozen bases (src/fp8.rs:86-234, src/diffusion_trainer.rs:1094-1267).

The reference maps the file, classifies every key from the header alone,
then decodes each fp8 tensor on the host to an f32 snapshot
(``LUT[byte] * scale``), which the quantized load pass re-quantizes to int4
one tensor at a time (src/diffusion_trainer.rs:1143-1169). Here the bytes
go to the device as they are and either stay e4m3fn (the fused kernels
decode them in registers) or are re-quantized to int4 by one kernel
(``lrq_requantize_fp8_int4``), with no f32 copy of the weight anywhere.

Classification follows src/fp8.rs:86-198, in its order, with its errors:

1. a ``scaled_fp8`` marker or any ``*.scale_weight`` key: the legacy
   ComfyUI format, refused;
2. every ``F8_E4M3`` tensor needs an F32 ``<name>_scale`` sidecar of shape
   ``[]``/``[1]`` (scalar) or ``[out]`` (per output channel, not ``[0]``);
   sidecars are consumed;
3. a ``*.weight_scale`` key without its fp8 base is an orphan, refused;
4. ``*.comfy_quant`` and ``*.input_scale`` are dropped;
5. other tensors pass through with their dtype (the 12 dtypes of
   src/fp8.rs:368-384); any other dtype is refused.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Union

import torch

from . import device as D
from . import fp8 as F

# src/fp8.rs:368-384
PASSTHROUGH_DTYPES = ("F64", "F32", "F16", "BF16", "I64", "I32", "I16", "I8", "U64", "U32", "U8", "BOOL")
DROPPED_SUFFIXES = (".comfy_quant", ".input_scale")


@dataclass
class Fp8Checkpoint:
    """What ``classify_fp8_checkpoint`` found: fp8 weights (name -> per
    output channel scale or not), pass-through tensors and dropped keys."""

    path: str
    fp8: Dict[str, bool] = field(default_factory=dict)
    plain: List[str] = field(default_factory=list)
    dropped: List[str] = field(default_factory=list)


def _header(path: str):
    from safetensors import safe_open

    out = {}
    with safe_open(path, framework="pt") as f:
        for name in f.keys():
            sl = f.get_slice(name)
            out[name] = (sl.get_dtype(), list(sl.get_shape()))
    return out


def classify_fp8_checkpoint(path: str) -> Fp8Checkpoint:
    """Classify every key of a scaled-fp8 checkpoint from its header alone
    (src/fp8.rs:109-198); raises ``ValueError`` naming the tensor."""
    header = _header(path)
    names = sorted(header)
    for name in names:
        if name == "scaled_fp8" or name.endswith(".scale_weight"):
            raise ValueError(
                f"scaled-fp8 checkpoint {path} uses the legacy ComfyUI 'scaled fp8' quant format "
                f"('scaled_fp8' marker / '.scale_weight' keys, found '{name}'): not supported — "
                "re-export with per-tensor '<name>.weight_scale' sidecars")
    ck = Fp8Checkpoint(path)
    consumed = set()
    for name in names:
        dtype, wshape = header[name]
        if dtype != "F8_E4M3":
            continue
        scale_name = f"{name}_scale"
        if scale_name not in header:
            raise ValueError(f"fp8 tensor '{name}' has no '{scale_name}' sidecar in {path}")
        sdtype, sshape = header[scale_name]
        if sdtype != "F32":
            raise ValueError(f"'{scale_name}' dtype {sdtype} — expected F32 (in {path})")
        if sshape in ([], [1]):
            per_channel = False
        elif len(sshape) == 1 and wshape and sshape[0] == wshape[0]:
            if sshape[0] == 0:
                raise ValueError(f"'{scale_name}' is empty ([0]) for weight '{name}' {wshape} in {path}")
            per_channel = True
        else:
            out = wshape[0] if wshape else 0
            raise ValueError(
                f"'{scale_name}' shape {sshape} is neither scalar ([]/[1]) nor per-output-channel ([{out}]) "
                f"for weight '{name}' {wshape} in {path}")
        ck.fp8[name] = per_channel
        consumed.add(scale_name)
    for name in names:
        dtype, _ = header[name]
        if name in consumed or dtype == "F8_E4M3":
            continue
        if name.endswith(".weight_scale"):
            base = name[: -len("_scale")]
            raise ValueError(f"'{name}' has no fp8 base weight '{base}' in {path}")
        if name.endswith(DROPPED_SUFFIXES):
            ck.dropped.append(name)
            continue
        if dtype not in PASSTHROUGH_DTYPES:
            raise ValueError(f"'{name}' has unsupported dtype {dtype} in {path}")
        ck.plain.append(name)
    return ck


def load_fp8_checkpoint(path: str, device: Union[str, torch.device], quant: Optional[str] = None,
                        group: int = 64) -> Dict[str, Union[D.PackedWeight, torch.Tensor]]:
    """Load a scaled-fp8 checkpoint onto ``device``.

    Each 2-D fp8 weight becomes a ``PackedWeight``: e4m3fn as stored
    (``quant=None``) or int4 at Q4S with ``group`` (``quant="int4"``),
    re-quantized on the device from the bytes. A weight whose input dim is
    not a multiple of 32 (or, for int4, of the group) cannot feed the fused
    kernels and comes back as its f32 values, as the reference keeps such
    sites plain (src/mmdit.rs:1266-1280). Pass-through tensors keep their
    dtype; dropped keys are absent."""
    if quant not in (None, "int4"):
        raise ValueError(f"quant must be None or 'int4', got {quant!r}")
    ck = classify_fp8_checkpoint(path)
    from safetensors import safe_open

    device = torch.device(device)
    out: Dict[str, Union[D.PackedWeight, torch.Tensor]] = {}
    with safe_open(path, framework="pt") as f:
        for name in sorted(ck.fp8):
            data = f.get_tensor(name).view(torch.uint8).to(device)
            scale = f.get_tensor(f"{name}_scale").to(device)
            aligned = data.dim() == 2 and data.shape[1] % 32 == 0 and (quant is None or data.shape[1] % group == 0)
            if not aligned:
                vals = data.view(torch.float8_e4m3fn).float()
                out[name] = vals * (scale.reshape(-1, *([1] * (vals.dim() - 1))) if ck.fp8[name] else scale.reshape(()))
                continue
            w = F.fp8_weight(name, data, scale)
            out[name] = D.requantize_fp8_int4(w, group) if quant == "int4" else w
        for name in ck.plain:
            out[name] = f.get_tensor(name).to(device)
    return out
