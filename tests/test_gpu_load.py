"""The on-device load path on the GPU: fp8 checkpoint bytes re-quantized to
int4 by one kernel, bit-exact against the oracle's f32 decode
(src/fp8.rs:306-318) followed by its Q4S quantizer (src/quant.rs:74-82),
and whole checkpoints through load_fp8_checkpoint."""

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import oracle as O
from gpu_helpers import check, to_dev
from loractl_amd import device as D
from loractl_amd import fp8 as F
from loractl_amd.load import load_fp8_checkpoint

pytestmark = pytest.mark.gpu

WEIGHT_5X3 = [0.5, -0.5, 1.0, 1.5, -1.5, 2.75, -3.0, 448.0, 0.0, 0.001953125, -448.0, 0.25, -2.0, 3.5, -0.0625]


def _fp8_case(n, k, per_channel, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    b = rng.integers(0, 256, (n, k), dtype=np.uint8)
    b[(b & 0x7F) == 0x7F] = 0x3C  # no NaN codes
    s = (rng.uniform(0.5, 2.0, n if per_channel else 1) * 1e-3).astype(np.float32)
    return b, s


@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("per_channel", [True, False])
def test_requantize_fp8_int4_bit_exact(cuda, group, per_channel):
    n, k = 72, 384
    b, s = _fp8_case(n, k, per_channel, seed=group + per_channel)
    w8 = F.fp8_weight("w", torch.from_numpy(b).to(cuda), torch.from_numpy(s).to(cuda))
    w4 = D.requantize_fp8_int4(w8, group)
    p_ref, s_ref = O.quantize_int4_packed(O.fp8_dequant(b, s), group)
    assert np.array_equal(w4.data.cpu().numpy(), p_ref)
    assert np.array_equal(w4.scales.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    # the same as the two-step device path through an f32 copy
    w4b = D.quantize_int4(D.dequant(w8), group)
    assert torch.equal(w4.data, w4b.data) and torch.equal(w4.scales, w4b.scales)


def test_requantize_exact_ties(cuda):
    """Half-integer quotients (exact on fp8 input) round half away from zero,
    as the oracle's Q4S does: 7, 6.5 ... 0.5 times a scale, amax 7."""
    halves = [7.0, 6.5, 5.5, 4.5, 3.5, 2.5, 1.5, 0.5]
    row = np.array(halves + [-h for h in halves] + [0.0] * 16, np.float32)  # one run of 32
    w = np.stack([row * 2.0 ** e for e in range(-6, 2)])  # 8 rows, k = 32
    b = torch.tensor(w).to(torch.float8_e4m3fn)
    assert np.array_equal(b.float().numpy(), w)
    s = np.ones(8, np.float32)
    w8 = F.fp8_weight("w", b.view(torch.uint8).to(cuda), torch.from_numpy(s).to(cuda))
    w4 = D.requantize_fp8_int4(w8, 32)
    p_ref, s_ref = O.quantize_int4_packed(w, 32)
    assert np.array_equal(w4.data.cpu().numpy(), p_ref)
    assert np.array_equal(w4.scales.cpu().numpy(), s_ref)
    # closed form: the scale is exactly 2^e, every quotient is the half-integer itself
    got = w4.data.cpu().numpy().astype(np.int64)
    q = np.stack([got & 15, got >> 4], axis=-1).reshape(8, 32) - 8
    want = [7, 7, 6, 5, 4, 3, 2, 1, -7, -7, -6, -5, -4, -3, -2, -1] + [0] * 16
    assert (q == np.array(want)).all()
    assert np.array_equal(w4.scales.cpu().numpy()[:, 0], 2.0 ** np.arange(-6, 2, dtype=np.float32))
    w4f = D.quantize_int4(torch.from_numpy(w).to(cuda), 32)
    assert torch.equal(w4.data, w4f.data)


def test_load_fp8_checkpoint_end_to_end(cuda, tmp_path):
    n, k, M = 64, 256, 24
    b, s = _fp8_case(n, k, True, seed=5)
    bias = np.linspace(-1, 1, n).astype(np.float32)
    path = str(tmp_path / "ck.safetensors")
    save_file({"blk.w.weight": torch.from_numpy(b).view(torch.float8_e4m3fn),
               "blk.w.weight_scale": torch.from_numpy(s), "blk.w.comfy_quant": torch.zeros(2, dtype=torch.uint8),
               "blk.odd.weight": torch.tensor(WEIGHT_5X3).reshape(5, 3).to(torch.float8_e4m3fn),
               "blk.odd.weight_scale": torch.tensor(2.0), "blk.bias": torch.from_numpy(bias)}, path)
    raw = load_fp8_checkpoint(path, cuda)
    q4 = load_fp8_checkpoint(path, cuda, quant="int4", group=64)
    assert sorted(raw) == ["blk.bias", "blk.odd.weight", "blk.w.weight"]
    # fp8 kept as stored: its decode is the reference snapshot, exactly
    wd = O.fp8_dequant(b, s)
    assert np.array_equal(D.dequant(raw["blk.w.weight"]).cpu().numpy(), wd)
    # int4 re-quantized on the device: bit-exact Q4S of that snapshot
    p_ref, s_ref = O.quantize_int4_packed(wd, 64)
    assert np.array_equal(q4["blk.w.weight"].data.cpu().numpy(), p_ref)
    assert np.array_equal(q4["blk.w.weight"].scales.cpu().numpy(), s_ref)
    # an input dim the fused kernels cannot take stays plain f32 (tests/fp8.rs expected values)
    for d in (raw, q4):
        assert torch.equal(d["blk.odd.weight"].cpu(), torch.tensor(WEIGHT_5X3).reshape(5, 3) * 2.0)
        assert torch.equal(d["blk.bias"].cpu(), torch.from_numpy(bias))
    # and the loaded weights drive the fused forward
    rng = np.random.Generator(np.random.PCG64(9))
    x = rng.standard_normal((M, k), dtype=np.float32)
    xb = to_dev(x, cuda)
    xr = xb.float().cpu().numpy()
    y8 = D.quant_matmul_t(xb, raw["blk.w.weight"])
    y4 = D.quant_matmul_t(xb, q4["blk.w.weight"])
    check("y fp8", y8, O.linear_fwd(xr, wd)[0])
    check("y int4", y4, O.linear_fwd(xr, O.dequant_int4(p_ref, s_ref, k, 64))[0])
    # int8 (Q8S) from the same snapshot: bit-exact q and scales, and the fused forward
    q8 = load_fp8_checkpoint(path, cuda, quant="int8", group=64)
    q_ref, s8_ref = O.quantize(wd, 64, 127)
    assert np.array_equal(q8["blk.w.weight"].data.cpu().numpy(), q_ref)
    assert np.array_equal(q8["blk.w.weight"].scales.cpu().numpy(), s8_ref)
    assert torch.equal(q8["blk.odd.weight"].cpu(), torch.tensor(WEIGHT_5X3).reshape(5, 3) * 2.0)
    check("y int8", D.quant_matmul_t(xb, q8["blk.w.weight"]), O.linear_fwd(xr, O.dequant_q(q_ref, s8_ref, 64))[0])


def test_fp8_load_default_block_and_alignment(cuda, tmp_path):
    """The load pass's default block is the reference's QUANT_BLOCK = 32, so a
    d_in of 96 quantizes; a caller-chosen block that does not divide it
    raises; a d_out the fused kernels cannot write (60) stays plain f32."""
    b96, s96 = _fp8_case(64, 96, True, seed=6)
    b60, s60 = _fp8_case(60, 128, False, seed=7)
    path = str(tmp_path / "ck.safetensors")
    save_file({"a.weight": torch.from_numpy(b96).view(torch.float8_e4m3fn), "a.weight_scale": torch.from_numpy(s96),
               "b.weight": torch.from_numpy(b60).view(torch.float8_e4m3fn),
               "b.weight_scale": torch.from_numpy(s60.reshape(()))}, path)
    q = load_fp8_checkpoint(path, cuda, quant="int4")
    p_ref, s_ref = O.quantize_int4_packed(O.fp8_dequant(b96, s96), 32)
    assert q["a.weight"].group == 32
    assert np.array_equal(q["a.weight"].data.cpu().numpy(), p_ref)
    assert np.array_equal(q["a.weight"].scales.cpu().numpy(), s_ref)
    assert isinstance(q["b.weight"], torch.Tensor)
    assert np.array_equal(q["b.weight"].cpu().numpy(), O.fp8_dequant(b60, s60))
    with pytest.raises(ValueError, match="not of the chosen quant block 64"):
        load_fp8_checkpoint(path, cuda, quant="int4", group=64)


def test_load_quant_checkpoint_plain(cuda, tmp_path):
    """Quantize-on-load for a plain checkpoint (src/diffusion_trainer.rs:1143-1169):
    each aligned base site is quantized on the device, bit-exact with the
    oracle's Q4S of its f32 values (bf16 and f32 files), in row chunks when
    the f32 size passes the threshold (the same bytes as whole); unaligned
    sites stay in the rest; a missing site raises."""
    from loractl_amd.load import load_quant_checkpoint

    rng = np.random.Generator(np.random.PCG64(21))
    w_a = (rng.standard_normal((96, 128)) * 0.02).astype(np.float32)      # f32, aligned
    w_b = (rng.standard_normal((40, 64)) * 0.02).astype(np.float32)       # bf16 file, aligned
    w_c = (rng.standard_normal((24, 20)) * 0.02).astype(np.float32)       # d_in 20: stays plain
    bias = np.linspace(-1, 1, 96).astype(np.float32)
    norm = np.ones(8, np.float32)
    path = str(tmp_path / "plain.safetensors")
    save_file({"s.a.weight": torch.from_numpy(w_a), "s.a.bias": torch.from_numpy(bias),
               "s.b.weight": torch.from_numpy(w_b).to(torch.bfloat16), "s.c.weight": torch.from_numpy(w_c),
               "norm.scale": torch.from_numpy(norm)}, path)
    q, rest, rep = load_quant_checkpoint(path, cuda, ["s.a", "s.b", "s.c"], chunk_bytes=96 * 128 * 4 // 3)
    assert (rep.quantized, rep.left_plain, rep.plain_sites) == (2, 1, ["s.c"])
    assert (rep.chunked_sites, rep.total_chunks) == (1, 3) and q["s.a"].chunk_rows == [32, 32, 32]
    assert sorted(rest) == ["norm.scale", "s.c.weight"]
    wb32 = torch.from_numpy(w_b).to(torch.bfloat16).float().numpy()
    for p_, w_ in (("s.a", w_a), ("s.b", wb32)):
        pk, sc = O.quantize_int4_packed(w_, 32)
        assert np.array_equal(q[p_].dequantized_weight().cpu().numpy(), O.dequant_int4(pk, sc, w_.shape[1], 32)), p_
    assert torch.equal(q["s.a"].bias.cpu(), torch.from_numpy(bias)) and q["s.b"].bias is None
    assert torch.equal(rest["s.c.weight"].cpu(), torch.from_numpy(w_c))
    with pytest.raises(ValueError, match="quantized base site s.d has no s.d.weight"):
        load_quant_checkpoint(path, cuda, ["s.a", "s.d"])
    # the same pass at Q8S (the Quant::Int8 knob): bit-exact int8 of the f32 values, same chunks
    from loractl_amd.quant import QuantValue
    q8, _, rep8 = load_quant_checkpoint(path, cuda, ["s.a", "s.b", "s.c"], chunk_bytes=96 * 128 * 4 // 3,
                                        value=QuantValue.Q8S)
    assert (rep8.quantized, rep8.left_plain, rep8.total_chunks) == (2, 1, 3)
    for p_, w_ in (("s.a", w_a), ("s.b", wb32)):
        qq, sc = O.quantize(w_, 32, 127)
        assert np.array_equal(q8[p_].dequantized_weight().cpu().numpy(), O.dequant_q(qq, sc, 32)), p_


@pytest.mark.parametrize("q8", [False, True], ids=["q4s", "q8s"])
def test_load_quant_checkpoint_fp8(cuda, tmp_path, q8):
    """Quantize-on-load for a scaled-fp8 checkpoint (src/diffusion_trainer.rs:1106-1170):
    only the base sites are quantized, from their f32 values LUT[byte] * scale
    (an fp8 base) or widened floats (a base the file stores in bf16), in row
    chunks under the threshold; an fp8 tensor that is not a base site (a
    modulation linear) and an fp8 bias reach the rest as their f32 values,
    other tensors keep their dtype, and the sidecars are consumed."""
    from loractl_amd.load import load_quant_checkpoint
    from loractl_amd.quant import QuantValue

    b_a, s_a = _fp8_case(96, 128, True, seed=31)     # fp8 base, per-channel scale
    b_m, s_m = _fp8_case(64, 128, False, seed=32)    # fp8, not a base site
    b_bias, s_bias = _fp8_case(96, 1, False, seed=33)
    rng = np.random.Generator(np.random.PCG64(34))
    w_b = (rng.standard_normal((40, 64)) * 0.02).astype(np.float32)  # base site stored as bf16
    norm = np.ones(8, np.float32)
    path = str(tmp_path / "fp8.safetensors")
    save_file({"s.a.weight": torch.from_numpy(b_a).view(torch.float8_e4m3fn),
               "s.a.weight_scale": torch.from_numpy(s_a),
               "s.a.bias": torch.from_numpy(b_bias.reshape(96)).view(torch.float8_e4m3fn),
               "s.a.bias_scale": torch.from_numpy(s_bias),
               "mod.weight": torch.from_numpy(b_m).view(torch.float8_e4m3fn),
               "mod.weight_scale": torch.from_numpy(s_m),
               "s.b.weight": torch.from_numpy(w_b).to(torch.bfloat16),
               "norm.scale": torch.from_numpy(norm)}, path)
    value = QuantValue.Q8S if q8 else QuantValue.Q4S
    q, rest, rep = load_quant_checkpoint(path, cuda, ["s.a", "s.b"], chunk_bytes=96 * 128 * 4 // 3, value=value)
    assert (rep.quantized, rep.left_plain, rep.chunked_sites, rep.total_chunks) == (2, 0, 1, 3)
    assert q["s.a"].chunk_rows == [32, 32, 32]
    assert sorted(rest) == ["mod.weight", "norm.scale"]
    assert rest["mod.weight"].dtype == torch.float32
    assert np.array_equal(rest["mod.weight"].cpu().numpy(), O.fp8_dequant(b_m, s_m))
    assert rest["norm.scale"].dtype == torch.float32
    assert np.array_equal(q["s.a"].bias.cpu().numpy(), O.fp8_dequant(b_bias, s_bias).reshape(96))
    wb32 = torch.from_numpy(w_b).to(torch.bfloat16).float().numpy()
    for p_, w_ in (("s.a", O.fp8_dequant(b_a, s_a)), ("s.b", wb32)):
        if q8:
            qq, sc = O.quantize(w_, 32, 127)
            ref = O.dequant_q(qq, sc, 32)
        else:
            pk, sc = O.quantize_int4_packed(w_, 32)
            ref = O.dequant_int4(pk, sc, w_.shape[1], 32)
        assert np.array_equal(q[p_].dequantized_weight().cpu().numpy(), ref), p_


def test_quantize_field_orientation(cuda):
    """quantize_field (src/mmdit.rs:1266-1280): a burn-layout [d_in, d_out]
    weight is transposed to file layout, then quantized; the forward equals
    x . W with W the dequantized burn weight; unaligned d_in stays Plain."""
    from loractl_amd.adapters import PlainLinear, QuantLinear, quantize_field

    rng = np.random.Generator(np.random.PCG64(4))
    wb = (rng.standard_normal((256, 72)) * 0.02).astype(np.float32)  # burn [d_in, d_out]
    base = PlainLinear(torch.from_numpy(wb).to(cuda))
    q = quantize_field(base)
    assert isinstance(q, QuantLinear) and (q.d_in, q.d_out) == (256, 72)
    pk, sc = O.quantize_int4_packed(np.ascontiguousarray(wb.T), 32)
    wdq = O.dequant_int4(pk, sc, 256, 32)
    assert np.array_equal(q.dequantized_weight().cpu().numpy(), wdq)
    x = rng.standard_normal((33, 256), dtype=np.float32)
    xb = to_dev(x, cuda)
    check("y", q.forward(xb), O.linear_fwd(xb.float().cpu().numpy(), wdq)[0])
    odd = PlainLinear(torch.zeros(48, 16, device=cuda))
    assert quantize_field(odd) is odd
