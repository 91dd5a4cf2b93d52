"""AdamW resume sidecar (src/resume.rs) on the host: file format, the
reference's refusals, and that a resumed optimizer continues exactly."""

import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from loractl_amd.adapters import LoraAdapters
from loractl_amd.lora import LoraDelta
from loractl_amd.resume import (OptimProgress, load_optimizer_state, optim_sidecar_path, save_optimizer_state)

TARGETS = ["blocks.0.attn.wq", "blocks.0.mlp.w2"]


def _set(seed=0, rank=4):
    torch.manual_seed(seed)
    return LoraAdapters([LoraDelta(16, 24, rank, 8.0), LoraDelta(24, 8, rank, 8.0)], TARGETS)


def _opt(s):
    # burn's AdamWConfig defaults (beta 0.9/0.999, eps 1e-5), weight decay from the config
    return torch.optim.AdamW([p for d in s.deltas for p in (d.lora_a, d.lora_b)], lr=1e-2, eps=1e-5,
                             weight_decay=0.01)


def _steps(s, opt, n, seed):
    g = torch.Generator().manual_seed(seed)
    for _ in range(n):
        opt.zero_grad()
        loss = 0
        for d in s.deltas:
            x = torch.randn(5, d.lora_a.shape[0], generator=g)
            loss = loss + (d(x) ** 2).mean() + (d.lora_b.sum() - 1.0) ** 2
        loss.backward()
        opt.step()


def test_sidecar_path():
    assert optim_sidecar_path("/out/checkpoint-10.safetensors") == "/out/checkpoint-10.optim.safetensors"
    assert optim_sidecar_path("adapter.safetensors") == "adapter.optim.safetensors"


def test_format(tmp_path):
    s = _set()
    opt = _opt(s)
    _steps(s, opt, 3, 1)
    p = str(tmp_path / "a.optim.safetensors")
    save_optimizer_state(opt, s, OptimProgress(steps_done=3, loss_scale=65536.0, clean_streak=2), p)
    with safe_open(p, framework="pt") as f:
        meta = f.metadata()
        keys = set(f.keys())
        m = f.get_tensor("blocks.0.attn.wq.lora_down.exp_avg")
    assert meta == {"loractl_artifact_kind": "optimizer-state", "loractl_adamw_time": "3",
                    "loractl_loss_scale": "65536", "loractl_clean_streak": "2", "loractl_steps_done": "3"}
    assert keys == {f"{t}.{f_}.{k}" for t in TARGETS for f_ in ("lora_down", "lora_up")
                    for k in ("exp_avg", "exp_avg_sq")}
    # the factors' own orientation, A [d_in, rank]
    assert tuple(m.shape) == (16, 4) and torch.equal(m, opt.state[s.deltas[0].lora_a]["exp_avg"])


def test_resume_continues_exactly(tmp_path):
    ref = _set(seed=5)
    opt = _opt(ref)
    _steps(ref, opt, 4, 11)
    snap = {id(p): p.detach().clone() for d in ref.deltas for p in (d.lora_a, d.lora_b)}
    p = str(tmp_path / "c.optim.safetensors")
    save_optimizer_state(opt, ref, OptimProgress(4, 1024.0, 0), p)
    # a fresh process: new deltas (the adapter import restores the factors), new optimizer
    res = _set(seed=99)
    with torch.no_grad():
        for dr, d in zip(res.deltas, ref.deltas):
            dr.lora_a.copy_(snap[id(d.lora_a)])
            dr.lora_b.copy_(snap[id(d.lora_b)])
    opt2 = _opt(res)
    got = load_optimizer_state(opt2, res, p)
    assert (got.params, got.time, got.loss_scale, got.clean_streak) == (4, 4, 1024.0, 0)
    _steps(ref, opt, 3, 12)
    _steps(res, opt2, 3, 12)
    for dr, d in zip(res.deltas, ref.deltas):
        assert torch.equal(dr.lora_a, d.lora_a) and torch.equal(dr.lora_b, d.lora_b)


def test_never_stepped_writes_nothing(tmp_path):
    s = _set()
    p = tmp_path / "n.optim.safetensors"
    save_optimizer_state(_opt(s), s, OptimProgress(0, 1.0, 0), str(p))
    assert not p.exists()


@pytest.mark.parametrize("case,match", [
    ("kind", "not a loractl optimizer-state sidecar"),
    ("missing", "is missing blocks.0.mlp.w2.lora_up.exp_avg_sq"),
    ("shape", "shape mismatch at blocks.0.attn.wq.lora_down.exp_avg"),
    ("nan", "not finite"),
    ("dtype", "expected F32"),
    ("time", "no readable loractl_adamw_time"),
])
def test_refusals(tmp_path, case, match):
    s = _set()
    opt = _opt(s)
    _steps(s, opt, 2, 3)
    p = str(tmp_path / "r.optim.safetensors")
    save_optimizer_state(opt, s, OptimProgress(2, 1.0, 0), p)
    with safe_open(p, framework="pt") as f:
        meta = dict(f.metadata())
        t = {k: f.get_tensor(k) for k in f.keys()}
    if case == "kind":
        meta["loractl_artifact_kind"] = "adapter"
    elif case == "missing":
        del t["blocks.0.mlp.w2.lora_up.exp_avg_sq"]
    elif case == "shape":
        t["blocks.0.attn.wq.lora_down.exp_avg"] = torch.zeros(16, 8)
    elif case == "nan":
        t["blocks.0.attn.wq.lora_up.exp_avg"][0, 1] = float("inf")
    elif case == "dtype":
        t["blocks.0.attn.wq.lora_up.exp_avg"] = t["blocks.0.attn.wq.lora_up.exp_avg"].double()
    else:
        meta["loractl_adamw_time"] = "x"
    save_file(t, p, metadata=meta)
    with pytest.raises(ValueError, match=match):
        load_optimizer_state(_opt(_set()), _set(), p)
