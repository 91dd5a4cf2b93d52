"""The scaled-fp8 checkpoint classification (src/fp8.rs:86-234) on the host,
after the reference's own cases (tests/fp8.rs), on files written here."""

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from loractl_amd.load import classify_fp8_checkpoint

# tests/fp8.rs WEIGHT_5X3: 15 exactly representable e4m3fn values, [5, 3]
WEIGHT_5X3 = [0.5, -0.5, 1.0, 1.5, -1.5, 2.75, -3.0, 448.0, 0.0, 0.001953125, -448.0, 0.25, -2.0, 3.5, -0.0625]


def fp8(shape, vals=None):
    t = torch.zeros(shape, dtype=torch.float32) if vals is None else torch.tensor(vals, dtype=torch.float32).reshape(shape)
    return t.to(torch.float8_e4m3fn)


def write(tmp_path, tensors):
    p = str(tmp_path / "ck.safetensors")
    save_file(tensors, p)
    return p


def test_weight_5x3_is_exact_in_e4m3fn():
    w = torch.tensor(WEIGHT_5X3)
    assert torch.equal(w.to(torch.float8_e4m3fn).float(), w)


def test_scalar_and_per_channel_sidecars(tmp_path):
    p = write(tmp_path, {"blk.w.weight": fp8([5, 3], WEIGHT_5X3), "blk.w.weight_scale": torch.tensor(2.0),
                         "blk.v.weight": fp8([5, 3], WEIGHT_5X3), "blk.v.weight_scale": torch.ones(5),
                         "blk.u.weight": fp8([5, 3], WEIGHT_5X3), "blk.u.weight_scale": torch.ones(1)})
    ck = classify_fp8_checkpoint(p)
    assert ck.fp8 == {"blk.u.weight": False, "blk.v.weight": True, "blk.w.weight": False}
    assert ck.plain == [] and ck.dropped == []  # consumed sidecars are not emitted


@pytest.mark.parametrize("shape", [[3], [5, 1]])
def test_bad_scale_shape_is_hard_error(tmp_path, shape):
    p = write(tmp_path, {"blk.w.weight": fp8([5, 3]), "blk.w.weight_scale": torch.ones(shape)})
    with pytest.raises(ValueError) as e:
        classify_fp8_checkpoint(p)
    msg = str(e.value)
    assert "blk.w.weight_scale" in msg and str(shape) in msg and "[5]" in msg


def test_empty_per_channel_scale_is_hard_error(tmp_path):
    p = write(tmp_path, {"blk.w.weight": fp8([0, 3]), "blk.w.weight_scale": torch.ones(0)})
    with pytest.raises(ValueError, match="empty"):
        classify_fp8_checkpoint(p)


def test_non_f32_scale_is_hard_error(tmp_path):
    p = write(tmp_path, {"blk.w.weight": fp8([5, 3]), "blk.w.weight_scale": torch.ones((), dtype=torch.float16)})
    with pytest.raises(ValueError, match="expected F32") as e:
        classify_fp8_checkpoint(p)
    assert "blk.w.weight_scale" in str(e.value)


def test_fp8_weight_without_scale_is_hard_error(tmp_path):
    p = write(tmp_path, {"blk.w.weight": fp8([5, 3])})
    with pytest.raises(ValueError) as e:
        classify_fp8_checkpoint(p)
    assert "blk.w.weight" in str(e.value) and "blk.w.weight_scale" in str(e.value)


@pytest.mark.parametrize("base", [None, "f32"])
def test_orphan_weight_scale_is_hard_error(tmp_path, base):
    t = {"blk.w.weight_scale": torch.tensor(1.0)}
    if base:
        t["blk.w.weight"] = torch.tensor([1.0, 2.0])
    p = write(tmp_path, t)
    with pytest.raises(ValueError, match="no fp8 base weight") as e:
        classify_fp8_checkpoint(p)
    assert "blk.w.weight_scale" in str(e.value)


@pytest.mark.parametrize("key", ["scaled_fp8", "blk.w.scale_weight"])
def test_legacy_scaled_fp8_is_hard_error(tmp_path, key):
    t = {"blk.w.weight": fp8([2, 2]), "blk.w.weight_scale": torch.tensor(1.0)}
    t[key] = fp8([0]) if key == "scaled_fp8" else torch.ones(1)
    p = write(tmp_path, t)
    with pytest.raises(ValueError, match="legacy ComfyUI"):
        classify_fp8_checkpoint(p)


def test_comfy_quant_and_input_scale_are_dropped(tmp_path):
    p = write(tmp_path, {"blk.w.weight": fp8([2, 2]), "blk.w.weight_scale": torch.tensor(2.0),
                         "blk.w.comfy_quant": torch.zeros(4, dtype=torch.uint8),
                         "blk.w.input_scale": torch.tensor(0.5), "blk.bias": torch.tensor([3.0, -4.0])})
    ck = classify_fp8_checkpoint(p)
    assert sorted(ck.fp8) == ["blk.w.weight"] and ck.plain == ["blk.bias"]
    assert ck.dropped == ["blk.w.comfy_quant", "blk.w.input_scale"]


def test_unsupported_dtype_is_hard_error(tmp_path):
    p = write(tmp_path, {"blk.x": torch.zeros(2, dtype=torch.float8_e5m2)})
    with pytest.raises(ValueError, match="unsupported dtype") as e:
        classify_fp8_checkpoint(p)
    assert "blk.x" in str(e.value)


def test_passthrough_keeps_every_mapped_dtype(tmp_path):
    dts = [torch.float64, torch.float32, torch.float16, torch.bfloat16, torch.int64, torch.int32, torch.int16,
           torch.int8, torch.uint8, torch.bool]
    p = write(tmp_path, {f"t{i}": torch.zeros(3, dtype=dt) for i, dt in enumerate(dts)})
    ck = classify_fp8_checkpoint(p)
    assert ck.plain == sorted(f"t{i}" for i in range(len(dts))) and not ck.fp8


def test_quantize_field_keeps_unaligned_sites_plain():
    """src/mmdit.rs:1266-1280: a Plain whose d_in is not a multiple of 32 is
    left untouched (no device work), as is one whose d_out the fused kernels
    cannot write; a quantized site passes through."""
    from loractl_amd.adapters import PlainLinear, into_quantized, quantize_field
    from loractl_amd.load import fused_aligned

    odd_in = PlainLinear(torch.zeros(16, 64))    # burn [d_in=16, d_out=64]
    odd_out = PlainLinear(torch.zeros(64, 60))   # d_out 60
    assert quantize_field(odd_in) is odd_in and quantize_field(odd_out) is odd_out
    assert into_quantized({"a": odd_in, "b": odd_out}) == {"a": odd_in, "b": odd_out}
    assert fused_aligned(64, 96) and not fused_aligned(64, 80) and not fused_aligned(60, 96)


def test_is_fp8_checkpoint(tmp_path):
    from loractl_amd.load import is_fp8_checkpoint

    p = write(tmp_path, {"a.weight": fp8([2, 2]), "a.weight_scale": torch.tensor(1.0)})
    assert is_fp8_checkpoint(p)
    q = str(tmp_path / "plain.safetensors")
    save_file({"a.weight": torch.zeros(2, 2)}, q)
    assert not is_fp8_checkpoint(q)
