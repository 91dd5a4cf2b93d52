"""AdamW resume sidecar for adapters trained through the fused path — the
host mirror of ``crates/loractl-core/src/resume.rs:60-160, :341-596``.

The adapter export (``export.py``) carries the factors; this file carries
what a lossless resume also needs: AdamW's two moments per factor, its
bias-correction step count, and the trainer's loss-scale state. Same file
format as the reference, so a sidecar written here resumes there and back:

- path: beside the adapter, ``<stem>.optim.safetensors`` (resume.rs:112-120);
- keys: ``<site path>.<lora_down|lora_up>.<exp_avg|exp_avg_sq>`` by site
  path (never by parameter identity), in the factors' own orientation
  (A ``[d_in, rank]``, B ``[rank, d_out]``; no kohya transpose), all F32;
- ``__metadata__``: ``loractl_artifact_kind = optimizer-state``,
  ``loractl_adamw_time`` (one step count for the whole file),
  ``loractl_loss_scale``, ``loractl_clean_streak``, ``loractl_steps_done``.

The optimizer is ``torch.optim.AdamW`` over the deltas' parameters (its
``step`` is the reference's ``time``, ``exp_avg`` / ``exp_avg_sq`` its
moments). AMSGrad state is refused, as the reference refuses
``max_moment_2``. Nothing to save (an optimizer that never stepped) writes
nothing, so an existing sidecar is not clobbered with an empty one.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Dict

import torch

from .adapters import LoraAdapters

ARTIFACT_KIND_KEY = "loractl_artifact_kind"
ARTIFACT_KIND = "optimizer-state"
TIME_KEY = "loractl_adamw_time"
LOSS_SCALE_KEY = "loractl_loss_scale"
CLEAN_STREAK_KEY = "loractl_clean_streak"
STEPS_DONE_KEY = "loractl_steps_done"
# kohya factor name and whether it is the down (A) factor (resume.rs:96)
FACTOR_KEYS = (("lora_down", True), ("lora_up", False))


def moment_key(target: str, suffix: str, kind: str) -> str:
    return f"{target}.{suffix}.{kind}"


def optim_sidecar_path(adapter: str) -> str:
    """``<dir>/<stem>.optim.safetensors`` beside the adapter file."""
    d, name = os.path.split(adapter)
    stem = os.path.splitext(name)[0] if name else "adapter"
    return os.path.join(d, f"{stem or 'adapter'}.optim.safetensors")


@dataclass
class OptimProgress:
    steps_done: int
    loss_scale: float
    clean_streak: int


@dataclass
class OptimRestored:
    params: int
    time: int
    loss_scale: float
    clean_streak: int


def _fmt_f32(v: float) -> str:
    """Rust's ``f32::to_string``: the shortest repr that reads back, with no
    exponent and no trailing ``.0`` for integral values (65536, not 65536.0)."""
    import numpy as np

    return np.format_float_positional(np.float32(v), unique=True, trim="-")


def save_optimizer_state(optim: torch.optim.Optimizer, adapters: LoraAdapters, progress: OptimProgress,
                         path: str) -> None:
    """Write AdamW's per-factor moments plus ``progress`` (resume.rs:375-480)."""
    from safetensors.torch import save_file

    tensors: Dict[str, torch.Tensor] = {}
    time = None
    for delta, target in zip(adapters.deltas, adapters.targets):
        for suffix, is_down in FACTOR_KEYS:
            p = delta.lora_a if is_down else delta.lora_b
            st = optim.state.get(p)
            if not st or "exp_avg" not in st:
                continue  # no update has landed on this factor yet
            if st.get("max_exp_avg_sq") is not None:
                raise ValueError(f"optimizer state at {target}.{suffix} carries an AMSGrad max_exp_avg_sq, which this "
                                 "sidecar does not serialize — enabling amsgrad needs the format extended first")
            step = int(st["step"].item() if torch.is_tensor(st["step"]) else st["step"])
            if time is None:
                time = step
            elif time != step:
                raise ValueError(f"optimizer state is inconsistent: {target}.{suffix} is at step {step} while another "
                                 f"parameter is at step {time} — AdamW's bias correction cannot be recorded as one "
                                 "scalar")
            tensors[moment_key(target, suffix, "exp_avg")] = st["exp_avg"].detach().float().cpu().contiguous()
            tensors[moment_key(target, suffix, "exp_avg_sq")] = st["exp_avg_sq"].detach().float().cpu().contiguous()
    if not tensors:
        return
    header = {
        ARTIFACT_KIND_KEY: ARTIFACT_KIND,
        TIME_KEY: str(time or 0),
        LOSS_SCALE_KEY: _fmt_f32(progress.loss_scale),
        CLEAN_STREAK_KEY: str(int(progress.clean_streak)),
        STEPS_DONE_KEY: str(int(progress.steps_done)),
    }
    d = os.path.dirname(path)
    if d:
        os.makedirs(d, exist_ok=True)
    save_file(tensors, path, metadata=header)


def load_optimizer_state(optim: torch.optim.Optimizer, adapters: LoraAdapters, path: str) -> OptimRestored:
    """Read a sidecar into ``optim`` against the current deltas
    (resume.rs:483-596): every site must be present with matching shapes and
    finite values, or it raises naming the tensor."""
    from safetensors import safe_open

    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
        kind = meta.get(ARTIFACT_KIND_KEY)
        if kind != ARTIFACT_KIND:
            raise ValueError(f"{path} is not a loractl optimizer-state sidecar ({ARTIFACT_KIND_KEY} = "
                             f"{kind!r})")

        def scalar(key, conv):
            try:
                return conv(meta[key])
            except (KeyError, ValueError):
                raise ValueError(f"{path} has no readable {key}") from None

        time = scalar(TIME_KEY, int)
        loss_scale = scalar(LOSS_SCALE_KEY, float)
        clean_streak = scalar(CLEAN_STREAK_KEY, int)
        keys = set(f.keys())

        def matrix(key, expected):
            if key not in keys:
                raise ValueError(f"optimizer state {path} is missing {key}")
            dt = f.get_slice(key).get_dtype()
            if dt != "F32":
                raise ValueError(f"optimizer tensor {key} is {dt}, expected F32")
            t = f.get_tensor(key)
            if list(t.shape) != list(expected):
                raise ValueError(f"optimizer state shape mismatch at {key}: file {list(t.shape)} vs configured "
                                 f"{list(expected)} — did lora.rank or lora.targets change?")
            bad = (~torch.isfinite(t)).reshape(-1).nonzero()
            if bad.numel():
                i = int(bad[0])
                raise ValueError(f"optimizer state {key} is not finite (element {i} is {t.reshape(-1)[i].item()}) — "
                                 "refusing to resume from a corrupt sidecar")
            return t

        loaded = []
        for delta, target in zip(adapters.deltas, adapters.targets):
            for suffix, is_down in FACTOR_KEYS:
                p = delta.lora_a if is_down else delta.lora_b
                m1 = matrix(moment_key(target, suffix, "exp_avg"), p.shape)
                m2 = matrix(moment_key(target, suffix, "exp_avg_sq"), p.shape)
                loaded.append((p, m1, m2))
    for p, m1, m2 in loaded:
        optim.state[p] = {
            "step": torch.tensor(float(time)),
            "exp_avg": m1.to(device=p.device, dtype=p.dtype).contiguous(),
            "exp_avg_sq": m2.to(device=p.device, dtype=p.dtype).contiguous(),
        }
    return OptimRestored(params=len(loaded), time=time, loss_scale=loss_scale, clean_streak=clean_streak)
