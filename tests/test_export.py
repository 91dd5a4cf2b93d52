"""kohya adapter interchange (src/export.rs) on the host: keys, layouts and
the import checks of the reference, after its tests/adapter_export.rs, and
the reference's own export golden (tests/golden/lora_export.json)."""

import hashlib
import json
import os
import struct

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save, save_file

from loractl_amd.adapters import LoraAdapters
from loractl_amd.export import export_adapters, import_adapters, kohya_keys, kohya_tensors, sd_webui_hashes
from loractl_amd.lora import LoraDelta

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "lora_export.json")


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
        meta = f.metadata()
        down, up, alpha = (f.get_tensor(k) for k in kohya_keys("blocks.0.attn.wq"))
    assert set(meta) == {"ss_network_dim", "sshs_model_hash", "sshs_legacy_hash"}
    assert meta["ss_network_dim"] == "4"
    d = s.deltas[0]
    assert torch.equal(down, d.lora_a.detach().t())  # [r, d_in]
    assert torch.equal(up, d.lora_b.detach().t())    # [d_out, r]
    assert alpha.shape == (1,) and alpha.item() == 8.0  # scaling * rank, a [1] tensor (export.rs:204-209)


def test_export_matches_reference_golden(tmp_path):
    """tests/adapter_export.rs:33-39's fixed constants against the reference's
    golden: key set, [2,4]/[6,2]/[1] shapes, values within 1e-6."""
    g = json.load(open(GOLDEN))
    hp = g["hyperparams"]
    a_init = torch.tensor([0.10, -0.20, 0.30, 0.40, -0.50, 0.60, 0.70, -0.80]).reshape(4, 2)
    b_init = torch.tensor([0.01, -0.02, 0.03, -0.04, 0.05, -0.06, 0.07, -0.08, 0.09, -0.10, 0.11,
                           -0.12]).reshape(2, 6)
    d = LoraDelta(hp["d_in"], hp["d_out"], hp["rank"], hp["alpha"])
    with torch.no_grad():
        d.lora_a.copy_(a_init)
        d.lora_b.copy_(b_init)
    p = str(tmp_path / "adapter.safetensors")
    export_adapters(LoraAdapters([d], [hp["path"]]), p)
    with safe_open(p, framework="pt") as f:
        assert sorted(f.keys()) == sorted(g["kohya_keys"])
        assert f.metadata() is None  # no metadata: no header (the byte-stable golden path)
        down, up, alpha = (f.get_tensor(k) for k in kohya_keys(hp["path"]))
    assert list(alpha.shape) == [1] and abs(alpha.item() - g["alpha_value"]) <= 1e-6
    assert list(down.shape) == g["a_shape"] and list(up.shape) == g["b_shape"]
    np.testing.assert_allclose(down.reshape(-1).numpy(), np.float32(g["a_transposed"]), atol=1e-6, rtol=0)
    np.testing.assert_allclose(up.reshape(-1).numpy(), np.float32(g["b_transposed"]), atol=1e-6, rtol=0)


def test_multi_delta_export_writes_distinct_keys(tmp_path):
    """tests/adapter_export.rs: N deltas give 3N distinct, correctly named tensors."""
    s = LoraAdapters([LoraDelta(4, 6, 2, 8.0), LoraDelta(8, 5, 3, 6.0)],
                     ["transformer.h.0.attn.c_attn", "transformer.h.1.mlp.c_fc"])
    p = str(tmp_path / "a.safetensors")
    export_adapters(s, p)
    with safe_open(p, framework="pt") as f:
        names = set(f.keys())
    assert len(names) == 6 and names == {k for t in s.targets for k in kohya_keys(t)}


def _data_region(buf):
    (n,) = struct.unpack("<Q", buf[:8])
    return buf[8 + n:]


def test_sd_webui_hashes(tmp_path):
    """The model hash is the SHA-256 of the tensor-data region, so it can be
    recomputed from the finished file (whose header is larger); the legacy
    hash reads 64 KiB at 0x100000 of the ss_*-only serialization: an empty
    read below 1 MiB, the real bytes above."""
    small = _set()
    p = str(tmp_path / "small.safetensors")
    export_adapters(small, p, {"ss_network_dim": "4", "modelspec.title": "x"})
    buf = open(p, "rb").read()
    with safe_open(p, framework="pt") as f:
        meta = f.metadata()
    assert meta["sshs_model_hash"] == hashlib.sha256(_data_region(buf)).hexdigest()
    assert meta["sshs_legacy_hash"] == hashlib.sha256(b"").hexdigest()[:8]
    assert meta["modelspec.title"] == "x"
    # user-editable modelspec.* fields do not change a file's identity
    p2 = str(tmp_path / "small2.safetensors")
    export_adapters(small, p2, {"ss_network_dim": "4", "modelspec.title": "other"})
    with safe_open(p2, framework="pt") as f:
        meta2 = f.metadata()
    assert (meta2["sshs_model_hash"], meta2["sshs_legacy_hash"]) == (meta["sshs_model_hash"],
                                                                     meta["sshs_legacy_hash"])
    # above 1 MiB the legacy hash covers real bytes of the ss_*-only buffer
    torch.manual_seed(3)
    big = LoraAdapters([LoraDelta(4096, 4096, 64, 64.0)], ["blocks.0.attn.wq"])
    with torch.no_grad():
        big.deltas[0].lora_b.normal_()
    p3 = str(tmp_path / "big.safetensors")
    export_adapters(big, p3, {"ss_network_dim": "64", "modelspec.title": "y"})
    ref_buf = save(kohya_tensors(big), metadata={"ss_network_dim": "64"})
    assert len(ref_buf) > 0x110000
    with safe_open(p3, framework="pt") as f:
        meta3 = f.metadata()
    assert meta3["sshs_legacy_hash"] == hashlib.sha256(ref_buf[0x100000:0x110000]).hexdigest()[:8]
    assert meta3["sshs_legacy_hash"] != hashlib.sha256(b"").hexdigest()[:8]
    assert (meta3["sshs_model_hash"], meta3["sshs_legacy_hash"]) == sd_webui_hashes(ref_buf)
    assert meta3["sshs_model_hash"] == hashlib.sha256(_data_region(open(p3, "rb").read())).hexdigest()


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
            t["lora_blocks_0_attn_wq.alpha"] = torch.tensor([9.0])

    _rewrite(p, change)
    with pytest.raises(ValueError, match=match):
        import_adapters(_set(), p)


def test_rank_change_is_a_shape_mismatch(tmp_path):
    p = str(tmp_path / "a.safetensors")
    export_adapters(_set(rank=4), p)
    with pytest.raises(ValueError, match="did lora.rank change"):
        import_adapters(_set(rank=8, alpha=16.0), p)


def test_legacy_hash_without_ss_metadata(tmp_path):
    """Metadata with no ss_* key still hashes a serialization that carries a
    metadata map, an empty one: the reference hands the serializer
    Some(map) whenever metadata is given (src/export.rs:330-336), which
    writes '"__metadata__":{}' into the header. Above 1 MiB that header
    length moves the 64 KiB the legacy hash reads, so it differs from the
    hash of a buffer without the map."""
    torch.manual_seed(5)
    big = LoraAdapters([LoraDelta(4096, 4096, 64, 64.0)], ["blocks.0.attn.wq"])
    with torch.no_grad():
        big.deltas[0].lora_b.normal_()
    p = str(tmp_path / "nometa.safetensors")
    export_adapters(big, p, {"modelspec.title": "z"})
    with_map = save(kohya_tensors(big), metadata={})
    without = save(kohya_tensors(big), metadata=None)
    n = struct.unpack("<Q", with_map[:8])[0]
    assert b'"__metadata__":{}' in with_map[8:8 + n]
    assert len(with_map) > 0x110000
    with safe_open(p, framework="pt") as f:
        meta = f.metadata()
    assert meta["sshs_legacy_hash"] == hashlib.sha256(with_map[0x100000:0x110000]).hexdigest()[:8]
    assert meta["sshs_legacy_hash"] != sd_webui_hashes(without)[1]
    assert meta["sshs_model_hash"] == hashlib.sha256(_data_region(open(p, "rb").read())).hexdigest()
