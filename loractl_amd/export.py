"""kohya-format adapter interchange for the adapters trained through the
fused path (src/export.rs:47-68, :297-355, :372-449): the same keys,
layouts and checks as the reference, so a file written here loads there and
back.

- keys: ``lora_<path with '.' -> '_'>.lora_down.weight`` = A^T [r, d_in],
  ``.lora_up.weight`` = B^T [d_out, r], ``.alpha`` = scaling * rank as a
  ``[1]`` tensor (src/export.rs:204-209), all F32;
- import checks, in the reference's order and with its messages: a missing
  tensor, a non-F32 tensor, a non-finite value (a corrupt adapter), a shape
  that does not match the configured deltas (a changed rank), an alpha that
  differs from the configured scaling * rank by more than 1e-3.

With metadata, the file also carries the two sd-webui-additional-networks
hashes the reference adds (src/export.rs:211-252, :330-345):
``sshs_model_hash`` = SHA-256 of the tensor-data region and
``sshs_legacy_hash`` = the first 8 hex digits of the SHA-256 of the 64 KiB
at byte 0x100000, both over a serialization whose header holds only the
``ss_*`` metadata. Without metadata no header is written (the reference's
``None`` path, which keeps exports byte-stable).
"""

from __future__ import annotations

import hashlib
import math
import struct
from typing import Dict, Optional, Tuple

import torch

from .adapters import LoraAdapters


def kohya_prefix(path: str) -> str:
    return "lora_" + path.replace(".", "_")


def kohya_keys(path: str):
    p = kohya_prefix(path)
    return f"{p}.lora_down.weight", f"{p}.lora_up.weight", f"{p}.alpha"


LEGACY_OFFSET = 0x100000
LEGACY_LEN = 0x10000


def sd_webui_hashes(buf: bytes) -> Tuple[str, str]:
    """(model hash, legacy hash) of a serialized safetensors buffer
    (src/export.rs:211-252): SHA-256 of everything past the length-prefixed
    JSON header, and the first 8 hex digits of the SHA-256 of the 64 KiB at
    offset 0x100000 (an empty read for a smaller buffer)."""
    (n,) = struct.unpack("<Q", buf[:8])
    model = hashlib.sha256(buf[min(n + 8, len(buf)):]).hexdigest()
    legacy = hashlib.sha256(buf[LEGACY_OFFSET:LEGACY_OFFSET + LEGACY_LEN] if len(buf) > LEGACY_OFFSET else b"")
    return model, legacy.hexdigest()[:8]


def kohya_tensors(adapters: LoraAdapters) -> Dict[str, torch.Tensor]:
    """The kohya tensors of every delta (src/export.rs:297-326)."""
    out = {}
    for delta, target in zip(adapters.deltas, adapters.targets):
        down, up, alpha = kohya_keys(target)
        a = delta.lora_a.detach().float().cpu()  # [d_in, r]
        b = delta.lora_b.detach().float().cpu()  # [r, d_out]
        out[down] = a.t().contiguous()
        out[up] = b.t().contiguous()
        # alpha = scaling * rank, computed in f64 and stored as an f32 [1]
        out[alpha] = torch.tensor([float(delta.scaling) * a.shape[1]], dtype=torch.float32)
    return out


def export_adapters(adapters: LoraAdapters, path: str, metadata: Optional[Dict[str, str]] = None) -> None:
    """Write every delta of ``adapters`` as kohya tensors (src/export.rs:297-355),
    with ``metadata`` plus the sd-webui hash pair in the header when given."""
    from safetensors.torch import save, save_file

    out = kohya_tensors(adapters)
    header = None
    if metadata:
        ss = {k: str(v) for k, v in metadata.items() if k.startswith("ss_")}
        # an empty ss_* subset still serializes an (empty) metadata map, as the
        # reference passes Some(map) to the serializer (src/export.rs:330-336)
        model_hash, legacy_hash = sd_webui_hashes(save(out, metadata=ss))
        header = {k: str(v) for k, v in metadata.items()}
        header["sshs_model_hash"] = model_hash
        header["sshs_legacy_hash"] = legacy_hash
    save_file(out, path, metadata=header)


def import_adapters(adapters: LoraAdapters, path: str) -> int:
    """Load a kohya file written by ``export_adapters`` (or the reference)
    into the configured deltas in place (src/export.rs:372-449); returns the
    number of deltas loaded. Parameters keep their identity (an optimizer
    holding them sees the loaded values)."""
    from safetensors import safe_open

    with safe_open(path, framework="pt") as f:
        keys = set(f.keys())

        def tensor(key):
            if key not in keys:
                raise ValueError(f"adapter export is missing tensor {key}")
            dt = f.get_slice(key).get_dtype()
            if dt != "F32":
                raise ValueError(f"tensor {key} is {dt}, expected F32")
            return f.get_tensor(key)

        def matrix(key):
            t = tensor(key)
            bad = (~torch.isfinite(t)).reshape(-1).nonzero()
            if bad.numel():
                i = int(bad[0])
                raise ValueError(f"tensor {key} is not finite (element {i} is {t.reshape(-1)[i].item()}) — "
                                 "refusing to resume from a corrupt adapter")
            return t

        loaded = []
        for delta, target in zip(adapters.deltas, adapters.targets):
            down, up, alpha_key = kohya_keys(target)
            a = matrix(down).t()
            b = matrix(up).t()
            if tuple(a.shape) != tuple(delta.lora_a.shape) or tuple(b.shape) != tuple(delta.lora_b.shape):
                raise ValueError(
                    f"resume shape mismatch at {target}: file A {list(a.shape)} / B {list(b.shape)} vs configured "
                    f"A {list(delta.lora_a.shape)} / B {list(delta.lora_b.shape)} — did lora.rank change?")
            alpha = float(tensor(alpha_key).reshape(-1)[0])
            expected = float(delta.scaling * delta.lora_a.shape[1])
            if not math.isfinite(alpha) or abs(alpha - expected) > 1e-3:
                raise ValueError(f"resume alpha mismatch at {target}: file {alpha} vs configured {expected} — "
                                 "did lora.alpha change?")
            loaded.append((delta, a, b))
    with torch.no_grad():
        for delta, a, b in loaded:
            delta.lora_a.copy_(a.to(delta.lora_a.dtype))
            delta.lora_b.copy_(b.to(delta.lora_b.dtype))
    return len(adapters.deltas)
