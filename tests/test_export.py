"""kohya adapter interchange (src/export.rs) on the host: keys, layouts and
the import checks of the reference, after its tests/adapter_export.rs."""

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from loractl_amd.adapters import LoraAdapters
from loractl_amd.export import export_adapters, import_adapters, kohya_keys
from loractl_amd.lora import LoraDelta


def _set(rank=4, alpha=8.0, seed=0):
    torch.manual_seed(seed)
    d1 = LoraDelta(16, 24, rank, alpha)
    d2 = LoraDelta(24, 8, rank, alpha)
    with torch.no_grad():
        d1.lora_b.normal_()
        d2.lora_b.normal_()
    return LoraAdapters([d1, d2], ["blocks.0.attn.wq", "blocks.0.mlp.w2"])


def test_keys_and_layouts(tmp_path):
    s = _set()
    p = str(tmp_path / "a.safetensors")
    export_adapters(s, p, {"ss_network_dim": "4"})
    assert kohya_keys("blocks.0.attn.wq") == ("lora_blocks_0_attn_wq.lora_down.weight",
                                              "lora_blocks_0_attn_wq.lora_up.weight", "lora_blocks_0_attn_wq.alpha")
    with safe_open(p, framework="pt") as f:
        assert sorted(f.keys()) == sorted(k for t in s.targets for k in kohya_keys(t))
        assert f.metadata() == {"ss_network_dim": "4"}
        down, up, alpha = (f.get_tensor(k) for k in kohya_keys("blocks.0.attn.wq"))
    d = s.deltas[0]
    assert torch.equal(down, d.lora_a.detach().t())  # [r, d_in]
    assert torch.equal(up, d.lora_b.detach().t())    # [d_out, r]
    assert alpha.shape == () and alpha.item() == 8.0  # scaling * rank


def test_round_trip_is_exact(tmp_path):
    src, dst = _set(seed=1), _set(seed=2)
    p = str(tmp_path / "a.safetensors")
    export_adapters(src, p)
    ids = [id(d.lora_a) for d in dst.deltas]
    assert import_adapters(dst, p) == 2
    for a, b in zip(src.deltas, dst.deltas):
        assert torch.equal(a.lora_a, b.lora_a) and torch.equal(a.lora_b, b.lora_b)
    assert ids == [id(d.lora_a) for d in dst.deltas]


def _rewrite(p, change):
    with safe_open(p, framework="pt") as f:
        t = {k: f.get_tensor(k) for k in f.keys()}
    change(t)
    save_file(t, p)


@pytest.mark.parametrize("case,match", [
    ("missing", "missing tensor lora_blocks_0_attn_wq.lora_up.weight"),
    ("dtype", "expected F32"),
    ("nan", "not finite"),
    ("alpha", "alpha mismatch"),
])
def test_import_checks(tmp_path, case, match):
    s = _set()
    p = str(tmp_path / "a.safetensors")
    export_adapters(s, p)
    up = "lora_blocks_0_attn_wq.lora_up.weight"

    def change(t):
        if case == "missing":
            del t[up]
        elif case == "dtype":
            t[up] = t[up].half()
        elif case == "nan":
            t[up][1, 2] = float("nan")
        else:
            t["lora_blocks_0_attn_wq.alpha"] = torch.tensor(9.0)

    _rewrite(p, change)
    with pytest.raises(ValueError, match=match):
        import_adapters(_set(), p)


def test_rank_change_is_a_shape_mismatch(tmp_path):
    p = str(tmp_path / "a.safetensors")
    export_adapters(_set(rank=4), p)
    with pytest.raises(ValueError, match="did lora.rank change"):
        import_adapters(_set(rank=8, alpha=16.0), p)
