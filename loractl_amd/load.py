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
from .quant import DEFAULT_DEQUANT_CHUNK_MIB, QUANT_BLOCK

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


def fused_aligned(d_out: int, d_in: int) -> bool:
    """Whether a ``[d_out, d_in]`` base can be quantized and fed to the fused
    kernels: ``d_in`` a multiple of the reference's quant block (32; a site
    that is not stays Plain, src/mmdit.rs:1266-1280) and ``d_out`` a multiple
    of 8 (the fused kernels write 16-byte output runs)."""
    return d_in % QUANT_BLOCK == 0 and d_out % 8 == 0


def _check_group(name: str, d_in: int, group: int):
    if group < QUANT_BLOCK or group & (group - 1):
        raise ValueError(f"quant block {group} must be a power of two >= {QUANT_BLOCK}")
    if d_in % group != 0:
        raise ValueError(
            f"'{name}': input dim {d_in} is a multiple of {QUANT_BLOCK} but not of the chosen quant block "
            f"{group}; use a block that divides it (the reference's is {QUANT_BLOCK})")


def load_fp8_checkpoint(path: str, device: Union[str, torch.device], quant: Optional[str] = None,
                        group: int = QUANT_BLOCK) -> Dict[str, Union[D.PackedWeight, torch.Tensor]]:
    """Load a scaled-fp8 checkpoint onto ``device``.

    Each 2-D fp8 weight becomes a ``PackedWeight``: e4m3fn as stored
    (``quant=None``), int4 at Q4S with ``group`` (``quant="int4"``; the
    reference's load pass always uses QUANT_BLOCK = 32), re-quantized on the
    device from the bytes, or int8 at Q8S (``quant="int8"``), quantized from
    the weight's f32 values on the device (one f32 copy of one weight at a
    time, as the reference's pass holds on the host). A weight whose input dim is not a multiple of 32
    stays plain, as the reference keeps such sites (src/mmdit.rs:1266-1280),
    and so does one whose output dim is not a multiple of 8, which the fused
    kernels cannot write: both come back as their f32 values. A caller-chosen
    group that does not divide an aligned weight's input dim raises.
    Pass-through tensors keep their dtype; dropped keys are absent."""
    if quant not in (None, "int4", "int8"):
        raise ValueError(f"quant must be None, 'int4' or 'int8', got {quant!r}")
    ck = classify_fp8_checkpoint(path)
    from safetensors import safe_open

    device = torch.device(device)
    out: Dict[str, Union[D.PackedWeight, torch.Tensor]] = {}
    with safe_open(path, framework="pt") as f:
        for name in sorted(ck.fp8):
            data = f.get_tensor(name).view(torch.uint8).to(device)
            scale = f.get_tensor(f"{name}_scale").to(device)
            aligned = data.dim() == 2 and fused_aligned(data.shape[0], data.shape[1])
            if aligned and quant is not None:
                _check_group(name, data.shape[1], group)
            if not aligned:
                vals = data.view(torch.float8_e4m3fn).float()
                out[name] = vals * (scale.reshape(-1, *([1] * (vals.dim() - 1))) if ck.fp8[name] else scale.reshape(()))
                continue
            w = F.fp8_weight(name, data, scale)
            if quant == "int4":
                w = D.requantize_fp8_int4(w, group)
            elif quant == "int8":
                w = D.quantize_int8(D.dequant(w), group)
            out[name] = w
        for name in ck.plain:
            out[name] = f.get_tensor(name).to(device)
    return out


def is_fp8_checkpoint(path: str) -> bool:
    """Header-only probe: does any tensor carry F8_E4M3 (src/fp8.rs:74-84)?"""
    return any(dt == "F8_E4M3" for dt, _ in _header(path).values())


@dataclass
class QuantLoadReport:
    """The quant pass's accounting (src/diffusion_trainer.rs:1212-1240)."""

    quantized: int = 0
    left_plain: int = 0
    chunked_sites: int = 0
    total_chunks: int = 0
    plain_sites: List[str] = field(default_factory=list)


def load_quant_checkpoint(path: str, device: Union[str, torch.device], base_paths: List[str],
                          group: int = QUANT_BLOCK, chunk_bytes: int = DEFAULT_DEQUANT_CHUNK_MIB << 20,
                          value=None):
    """The quant pass of ``load_quant_module`` (src/diffusion_trainer.rs:1094-1267)
    for a plain (bf16/f32/f16) or scaled-fp8 safetensors checkpoint, on the
    device: for each frozen-base site in ``base_paths`` (in order), its
    ``<path>.weight`` (file layout ``[d_out, d_in]``) is read, moved to the
    device and quantized at ``value`` (a ``QuantValue``: Q4S int4 by default,
    or Q8S int8) as the row chunks ``dequant_chunk_rows`` prescribes, one
    tensor at a time. A plain weight is widened to f32 first (one f32 copy of
    one chunk's rows at a time). An fp8 weight is quantized from its f32
    values ``LUT[byte] * scale`` (src/fp8.rs:306-318): at Q4S straight from
    the bytes by ``lrq_requantize_fp8_int4`` (no f32 copy), at Q8S through
    the device's f32 decode of the chunk. A base site that an fp8 file
    stores in another float dtype is quantized from its f32 values like a
    plain one. A site whose weight is not block-aligned (``fused_aligned``)
    is left plain: its weight stays in the returned rest, as the reference
    leaves it to the applier. A site missing from the checkpoint raises.

    Everything else goes to the rest as the reference's snapshots give it to
    the applier (src/diffusion_trainer.rs:1106-1112, :1141-1170): fp8
    tensors that are not base sites as their f32 values, other tensors with
    their dtype; dropped fp8 keys are absent.

    Returns ``(quantized, rest, report)``: ``{path: QuantLinear}`` (with the
    site's ``<path>.bias`` as its bias when present), every other tensor by
    key, and the accounting."""
    from safetensors import safe_open

    from .adapters import QuantLinear
    from .quant import QuantValue, dequant_chunk_rows, quantize_linear_weight_chunked

    device = torch.device(device)
    value = QuantValue.Q4S if value is None else value
    report = QuantLoadReport()
    quantized = {}
    ck = classify_fp8_checkpoint(path) if is_fp8_checkpoint(path) else None
    keys = (set(ck.fp8) | set(ck.plain)) if ck is not None else set(_header(path))
    rest = {}
    with safe_open(path, framework="pt") as f:

        def fp8_values(key: str) -> torch.Tensor:
            """The f32 snapshot of an fp8 tensor: LUT[byte] * scale."""
            data = f.get_tensor(key).view(torch.uint8).to(device)
            scale = f.get_tensor(f"{key}_scale").to(device)
            vals = data.view(torch.float8_e4m3fn).float()
            if ck.fp8[key]:
                return vals * scale.reshape(-1, *([1] * (vals.dim() - 1)))
            return vals * scale.reshape(())

        for p in base_paths:
            wkey = f"{p}.weight"
            if wkey not in keys:
                raise ValueError(f"quantized base site {p} has no {wkey} in the checkpoint {path}")
            shape = f.get_slice(wkey).get_shape()
            if len(shape) != 2 or not fused_aligned(shape[0], shape[1]):
                report.left_plain += 1
                report.plain_sites.append(p)
                continue
            _check_group(wkey, shape[1], group)
            if ck is not None and wkey in ck.fp8:
                data = f.get_tensor(wkey).view(torch.uint8).to(device)
                scale = f.get_tensor(f"{wkey}_scale").to(device).reshape(-1)
                per_channel = ck.fp8[wkey]
                chunks, start = [], 0
                for rows in dequant_chunk_rows(shape[0], shape[1], chunk_bytes):
                    w8 = F.fp8_weight(wkey, data[start:start + rows],
                                      scale[start:start + rows] if per_channel else scale)
                    if value is QuantValue.Q8S:
                        chunks.append(D.quantize_int8(D.dequant(w8), group))
                    else:
                        chunks.append(D.requantize_fp8_int4(w8, group))
                    start += rows
                del data, scale
            else:
                w32 = f.get_tensor(wkey).to(device).float()
                chunks = quantize_linear_weight_chunked(w32, value, chunk_bytes, group)
                del w32
            if len(chunks) > 1:
                report.chunked_sites += 1
                report.total_chunks += len(chunks)
            bkey = f"{p}.bias"
            bias = None
            if bkey in keys:
                bias = fp8_values(bkey) if (ck is not None and bkey in ck.fp8) else f.get_tensor(bkey).to(device)
                bias = bias.float()
            quantized[p] = QuantLinear(chunks, bias)
            report.quantized += 1
        taken = {f"{p}.weight" for p in quantized} | {f"{p}.bias" for p in quantized}
        for k in sorted(keys - taken):
            rest[k] = fp8_values(k) if (ck is not None and k in ck.fp8) else f.get_tensor(k).to(device)
    return quantized, rest, report
