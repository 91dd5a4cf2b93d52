"""Host-side logic of the ROCm backend and the C-ABI surface. CPU only: no
GPU compute call is made here."""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

from loractl_amd import _lib
from loractl_amd.accuracy import RelGate, cosine, rel_deviation
from loractl_amd.adapters import LoraAdapters, LoraConfig, LoraSite, TargetSpec, build_adapters
from loractl_amd.fp8 import fp8_weight
from loractl_amd.lora import LoraDelta
from loractl_amd.quant import Quant, QuantValue, dequant_chunk_rows, quant_value, quantize_linear_weight

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "loractl_rocm.h")


def test_chunk_rows_matches_reference_contract():
    """tests/quant.rs:330-350 against the host mirror."""
    assert dequant_chunk_rows(1000, 96, 0) == [1000]
    assert dequant_chunk_rows(12, 96, 12 * 96 * 4) == [12]
    assert dequant_chunk_rows(12, 96, 96 * 4 * 5) == [4, 4, 4]
    assert dequant_chunk_rows(13, 96, 96 * 4 * 5) == [5, 4, 4]
    assert dequant_chunk_rows(4, 96, 1) == [1, 1, 1, 1]
    for d_out, d_in, b in [(53, 96, 700), (16, 96, 96 * 4 * 3), (7, 32, 200)]:
        assert sum(dequant_chunk_rows(d_out, d_in, b)) == d_out


def test_quant_knob_and_block_guard():
    assert quant_value(Quant.parse("int4")) is QuantValue.Q4S
    assert quant_value(Quant.parse("INT8")) is QuantValue.Q8S
    assert quant_value(Quant.parse("none")) is None
    with pytest.raises(ValueError):
        Quant.parse("int3")
    # non-divisible input dim fails before any device work (quant.rs:76-80)
    with pytest.raises(AssertionError, match="multiple of the quant block"):
        quantize_linear_weight(torch.zeros(4, 33), QuantValue.Q4S, 32)
    # Q8S is built, and like Q4S it has no CPU path: a host tensor raises
    with pytest.raises(ValueError, match="no CPU fallback"):
        quantize_linear_weight(torch.zeros(4, 64), QuantValue.Q8S, 32)


def test_lora_delta_init_contract():
    """lora.rs:113-137, :174-190, tests at lora.rs:229-249."""
    d = LoraDelta(4, 3, 2, 8.0)
    assert tuple(d.lora_a.shape) == (4, 2) and tuple(d.lora_b.shape) == (2, 3)
    assert d.scaling == 4.0
    assert not d.lora_b.detach().any()
    assert d.lora_a.detach().abs().max() <= 0.5  # Kaiming-uniform bound 1/sqrt(4)
    d0 = LoraDelta(4, 3, 0, 8.0)
    assert d0.rank == 1 and d0.scaling == 8.0
    x = torch.randn(5, 4)
    assert torch.equal(d(x), torch.zeros(5, 3))  # zero-B delta is a no-op


def test_build_adapters_routing():
    """adapters.rs:116-145: first matching pattern wins, overrides apply,
    order follows sites, invalid regex raises."""
    sites = [LoraSite("blocks.0.attn.wq", 64, 64), LoraSite("blocks.0.attn.gate", 64, 64),
             LoraSite("blocks.0.mlp.up", 64, 256), LoraSite("blocks.1.attn.wq", 64, 64)]
    cfg = LoraConfig(rank=8, alpha=8.0, targets=[TargetSpec(r"attn\.w[qkv]$", rank=4, alpha=2.0),
                                                 TargetSpec(r"mlp\.")])
    ad = build_adapters(sites, cfg)
    assert ad.targets == ["blocks.0.attn.wq", "blocks.0.mlp.up", "blocks.1.attn.wq"]
    assert ad.get("blocks.0.attn.wq").rank == 4 and ad.get("blocks.0.attn.wq").scaling == 0.5
    assert ad.get("blocks.0.mlp.up").rank == 8
    assert ad.get("blocks.0.attn.gate") is None
    base = torch.randn(2, 64)
    assert ad.apply("blocks.0.attn.gate", torch.randn(2, 64), base) is base
    with pytest.raises(ValueError, match="invalid LoRA target pattern"):
        build_adapters(sites, LoraConfig(targets=[TargetSpec("(")]))
    with pytest.raises(ValueError):
        LoraAdapters([LoraDelta(4, 4, 1, 1.0)], [])


def test_rel_gate_semantics():
    """accuracy.rs tests: band, ceiling, floor, non-finite, peak-normalized."""
    gate = RelGate(0.01, 1e-4, 0.05)
    assert gate.apply(0.015).passed and gate.apply(0.02).passed
    out = gate.apply(0.03)
    assert not out.passed and out.band == 0.02
    loose = RelGate(0.1, 1e-4, 0.05)
    assert not loose.apply(0.08).passed and loose.apply(0.04).passed
    tight = RelGate(1e-8, 1e-4, 0.05)
    assert tight.apply(0.0).band == 1e-4 and tight.apply(5e-5).passed and not tight.apply(2e-4).passed
    assert not gate.apply(float("nan")).passed and not gate.apply(float("inf")).passed
    assert abs(rel_deviation([1.1, 2.0, 4.0], [1.0, 2.0, 4.0]) - 0.1 / 4.0) < 1e-6
    assert rel_deviation([1.0], [1.0, 2.0]) == float("inf")
    assert rel_deviation([], []) == float("inf")
    assert rel_deviation([float("nan")], [1.0]) == float("inf")
    assert cosine([1.0, 0.0], [2.0, 0.0]) == 1.0


def test_fp8_scale_sidecar_classification():
    """fp8.rs:58-68 / :109-234: [] and [1] are scalar, [out] per channel, else an error."""
    b = torch.zeros(5, 32, dtype=torch.uint8)
    assert not fp8_weight("w", b, torch.tensor(0.5)).per_channel
    assert not fp8_weight("w", b, torch.tensor([0.5])).per_channel
    assert fp8_weight("w", b, torch.ones(5)).per_channel
    with pytest.raises(ValueError, match="w_scale"):
        fp8_weight("w", b, torch.ones(32))
    with pytest.raises(ValueError, match="F32"):
        fp8_weight("w", b, torch.ones(5, dtype=torch.float64))


def _declared_symbols():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(lrq_[a-z0-9_]+)\s*\(", txt)))


def test_c_abi_library_exports_every_declared_symbol():
    """libloractl_rocm.so loads on a machine without a GPU and exports exactly
    what include/loractl_rocm.h declares (no compute call is made)."""
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"
    lib = ctypes.CDLL(_lib.LIB_PATH)
    declared = _declared_symbols()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_lib.SIGNATURES), "ctypes binding and header disagree"
    lib.lrq_version.restype = ctypes.c_int
    assert lib.lrq_version() == 1
    lib.lrq_profile_count.restype = ctypes.c_int
    lib.lrq_profile_name.restype = ctypes.c_char_p
    lib.lrq_profile_name.argtypes = [ctypes.c_int]
    names = [lib.lrq_profile_name(i).decode() for i in range(lib.lrq_profile_count())]
    assert "fwd_main" in names and "bwd_dx" in names


def test_mmdit_library_exports_what_its_header_declares():
    """libloractl_mmdit.so (the MMDiT driver's attention-input kernels) loads
    without a GPU and exports exactly include/loractl_mmdit.h's functions,
    each bound in mmdit_ops.SIGNATURES; invalid shapes are refused before
    any launch."""
    from loractl_amd import mmdit_ops

    txt = open(os.path.join(ROOT, "include", "loractl_mmdit.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    declared = set(re.findall(r"\b(lmd_[a-z0-9_]+)\s*\(", txt))
    assert declared == set(mmdit_ops.SIGNATURES)
    lib = mmdit_ops.load()
    for name in declared:
        assert hasattr(lib, name), name
    # head_dim 96 is not supported: refused with a message, no device work
    rc = lib.lmd_attn_prep_fwd(None, 0, None, 4, 2, 96, None, None, 1e-5, None, None, None, None, None)
    assert rc == -1 and b"head_dim" in lib.lmd_last_error()


def test_c_abi_rejects_null_context():
    lib = _lib.load()
    assert lib.lrq_sync(None) == _lib.LRQ_EINVAL
    assert lib.lrq_create(0, None) == _lib.LRQ_EINVAL


def test_gpu_kernels_are_built_for_gfx950_only():
    """The shared library carries gfx950 code objects (hipcc --offload-arch=gfx950)."""
    blob = open(_lib.LIB_PATH, "rb").read()
    assert b"gfx950" in blob
    assert b"gfx942" not in blob and b"sm_" not in blob[:0]


def test_dropout_above_zero_is_refused():
    """lora.rs:44-48 dropout is fused away on this path: p > 0 in training
    raises before any device work (the block-checkpointed trainer refuses it
    too, diffusion_trainer.rs:342-348); so does a rank above the kernels' 64."""
    import torch

    from loractl_amd.lora import LoraDelta, quant_lora_linear

    d = LoraDelta(64, 32, 4, 4.0, dropout_prob=0.1)
    with pytest.raises(ValueError, match="dropout 0 only"):
        quant_lora_linear(torch.zeros(2, 64), None, d)
    big = LoraDelta(64, 32, 65, 65.0)
    with pytest.raises(ValueError, match="rank <= 64"):
        quant_lora_linear(torch.zeros(2, 64), None, big)


def test_quantizer_quotient_without_division(tmp_path):
    """The quantizer kernels (lrq_quant.hip k_quantize) form RN(v / s) as
    fma(r, y, q0) with y = RN(1/s), q0 = RN(v y), r = fma(-q0, s, v), not by
    a division per value. tests/quotient_check.c restates that sequence in C
    and holds it to the correctly rounded division over the kernels' domain
    (every f32 near each rounding threshold, random values, 4000 scales):
    the quotient is equal, and so is its half-away rounding. The GPU tests
    hold the kernels themselves bit-exact against the oracle's division."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    exe = str(tmp_path / "quotient_check")
    src = os.path.join(os.path.dirname(__file__), "quotient_check.c")
    subprocess.run([gcc, "-O2", "-ffp-contract=off", "-o", exe, src, "-lm"], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 differ" in r.stdout and " 0 round differently" in r.stdout
