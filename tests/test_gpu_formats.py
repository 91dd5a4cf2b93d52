"""Bit-exact parity of the GPU weight-format kernels with the CPU oracle:
int4 quantize/pack/dequant, int8 quantize/dequant and fp8 e4m3fn
encode/decode."""

import json
import os

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import rng
from loractl_amd import device as D
from loractl_amd._lib import LrqError

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _int4_case(N, K, g, seed):
    w = (rng(seed).standard_normal((N, K)) * 0.5).astype(np.float32)
    if N > 2 and K >= 64:
        w[1, :g] = 0.0                          # an all-zero block
        w[2, :32] = 0.0
        w[2, :6] = [7.0, 2.5, -2.5, 0.5, -0.5, 6.5]  # exact .5 ties at scale 1
    return w


@pytest.mark.parametrize("N,K,g", [(8, 64, 32), (40, 96, 32), (64, 256, 32), (128, 512, 64), (72, 1024, 128),
                                   (3, 2048, 2048)])
def test_quantize_int4_bit_exact(cuda, N, K, g):
    w = _int4_case(N, K, g, seed=N + K)
    wq = D.quantize_int4(torch.from_numpy(w).to(cuda), g)
    p_ref, s_ref = O.quantize_int4_packed(w, g)
    assert np.array_equal(wq.data.cpu().numpy(), p_ref)
    assert np.array_equal(wq.scales.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    dq = D.dequant(wq).cpu().numpy()
    dq_ref = O.dequant_int4(p_ref, s_ref, K, g)
    assert np.array_equal(dq.view(np.uint32), dq_ref.view(np.uint32))
    bf = D.dequant_bf16(wq).view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(bf, O.bf16_bits(dq_ref))


def test_int4_reference_golden_on_gpu(cuda):
    """quant_int4_golden.json dequantized on the GPU equals the torch golden."""
    g = json.load(open(os.path.join(GOLD, "quant_int4_golden.json")))
    w = np.array(g["w"], np.float32)
    wq = D.quantize_int4(torch.from_numpy(w).to(cuda), 32)
    assert np.array_equal(D.dequant(wq).cpu().numpy(), np.array(g["dq"], np.float32))


@pytest.mark.parametrize("N,K,g", [(8, 64, 32), (40, 96, 32), (128, 512, 64), (72, 1024, 128), (3, 2048, 2048)])
def test_quantize_int8_bit_exact(cuda, N, K, g):
    """Q8S (qmax 127): q and scales equal the oracle's quantizer byte for byte
    (ties, all-zero blocks), and so do dequant and the bf16 operand."""
    w = _int4_case(N, K, g, seed=3 * N + K)
    if N > 2 and K >= 64:
        w[2, 6:10] = [127.0, 1.5, -1.5, 63.5]  # exact .5 ties once the block's scale is 1
    wq = D.quantize_int8(torch.from_numpy(w).to(cuda), g)
    q_ref, s_ref = O.quantize(w, g, 127)
    assert wq.data.dtype == torch.int8
    assert np.array_equal(wq.data.cpu().numpy(), q_ref)
    assert np.array_equal(wq.scales.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    dq_ref = O.dequant_q(q_ref, s_ref, g)
    assert np.array_equal(D.dequant(wq).cpu().numpy().view(np.uint32), dq_ref.view(np.uint32))
    bf = D.dequant_bf16(wq).view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(bf, O.bf16_bits(dq_ref))


def test_int8_reference_golden_on_gpu(cuda):
    """quant_int8_golden.json dequantized on the GPU equals the torch golden."""
    g = json.load(open(os.path.join(GOLD, "quant_int8_golden.json")))
    w = np.array(g["w"], np.float32)
    wq = D.quantize_int8(torch.from_numpy(w).to(cuda), g["block"])
    assert np.array_equal(D.dequant(wq).cpu().numpy(), np.array(g["dq"], np.float32))


def test_quantize_int8_rejects_bad_blocks(cuda):
    with pytest.raises(LrqError, match="LRQ_EINVAL"):
        D.quantize_int8(torch.zeros(4, 96, device=cuda), 64)
    with pytest.raises(LrqError, match="LRQ_EINVAL"):
        D.quantize_int8(torch.zeros(4, 96, device=cuda), 48)


def test_quantize_int4_rejects_bad_blocks(cuda):
    with pytest.raises(LrqError, match="LRQ_EINVAL"):
        D.quantize_int4(torch.zeros(4, 96, device=cuda), 64)
    with pytest.raises(LrqError, match="LRQ_EINVAL"):
        D.quantize_int4(torch.zeros(4, 96, device=cuda), 48)


@pytest.mark.parametrize("per_channel", [False, True])
def test_quantize_fp8_bit_exact(cuda, per_channel):
    w = (rng(7).standard_normal((48, 160)) * 0.3).astype(np.float32)
    w[3] = 0.0  # all-zero row: scale clamps to 1e-12
    w[5, 7] = -4.2e-8
    pw = D.quantize_fp8(torch.from_numpy(w).to(cuda), per_channel)
    b_ref, s_ref = O.fp8_quantize(w, per_channel)
    assert np.array_equal(pw.scales.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(pw.data.cpu().numpy(), b_ref)


def test_fp8_encoder_reproduces_reference_fixture_pairs_on_gpu(cuda):
    z = np.load(os.path.join(GOLD, "fp8_pairs.npz"))
    for n in [str(v) for v in z["names"]]:
        key = n.split("=")[0]
        w, want_b, want_s = z[key + "_w"], z[key + "_bytes"], z[key + "_scale"]
        if w.shape[1] % 4:
            continue
        pw = D.quantize_fp8(torch.from_numpy(np.ascontiguousarray(w)).to(cuda), want_s.size > 1)
        assert np.array_equal(pw.scales.cpu().numpy().view(np.uint32), want_s.view(np.uint32)), n
        assert np.array_equal(pw.data.cpu().numpy(), want_b), n


def test_fp8_decode_all_256_bytes(cuda):
    """Every e4m3fn byte decodes to the torch LUT golden (bf16 operand and f32 dequant)."""
    lut = json.load(open(os.path.join(GOLD, "fp8_lut_golden.json")))["lut"]
    data = np.arange(256, dtype=np.uint8).reshape(8, 32)
    scale = np.ones(8, np.float32)
    pw = D.PackedWeight(D.L.LRQ_FMT_FP8, 8, 32, torch.from_numpy(data).to(cuda),
                        torch.from_numpy(scale).to(cuda), per_channel=True)
    f = D.dequant(pw).cpu().numpy().reshape(-1)
    bf = D.dequant_bf16(pw).float().cpu().numpy().reshape(-1)
    for b, want in enumerate(lut):
        if want is None:
            assert np.isnan(f[b]) and np.isnan(bf[b]), hex(b)
        else:
            assert np.float32(want).view(np.uint32) == f[b].view(np.uint32), hex(b)
            assert np.float32(want).view(np.uint32) == bf[b].view(np.uint32), hex(b)


@pytest.mark.parametrize("case", ["scalar", "per_channel", "scale_shape_one"])
def test_fp8_dequant_golden_on_gpu(cuda, case):
    """fp8_dequant_golden.json ([5,3] weights) embedded in a [5,32] weight."""
    c = json.load(open(os.path.join(GOLD, "fp8_dequant_golden.json")))[case]
    b = np.zeros((5, 32), np.uint8)
    b[:, :3] = np.array(c["weight_bytes"], np.uint8).reshape(5, 3)
    scale = np.array(c["scale"], np.float32).reshape(-1)
    pw = D.PackedWeight(D.L.LRQ_FMT_FP8, 5, 32, torch.from_numpy(b).to(cuda), torch.from_numpy(scale).to(cuda),
                        per_channel=scale.size > 1)
    out = D.dequant(pw).cpu().numpy()[:, :3].reshape(-1)
    assert np.array_equal(out.view(np.uint32), np.array(c["expected"], np.float32).view(np.uint32))


@pytest.mark.parametrize("fmt,N,K,g", [("int4", 72, 96, 32), ("int4", 130, 256, 64), ("int4", 64, 512, 128),
                                       ("fp8", 40, 96, 0), ("fp8", 200, 320, 0),
                                       ("int8", 72, 96, 32), ("int8", 130, 256, 64)])
def test_blocked_layout_roundtrip(cuda, fmt, N, K, g):
    """The blocked device layout dequantizes bit-identically to the row layout
    (padding rows and columns included), and places bytes where the layout
    definition says (spot-checked against the row layout)."""
    w = (rng(N * K).standard_normal((N, K)) * 0.3).astype(np.float32)
    t = torch.from_numpy(w).to(cuda)
    rows = {"int4": lambda: D.quantize_int4(t, g), "int8": lambda: D.quantize_int8(t, g),
            "fp8": lambda: D.quantize_fp8(t, True)}[fmt]()
    blk = D.block(rows)
    assert blk.blocked and not rows.blocked
    a = D.dequant(rows).cpu().numpy()
    b = D.dequant(blk).cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert torch.equal(D.dequant_bf16(rows), D.dequant_bf16(blk))
    # layout spot checks: row n, byte j of the row layout sits at block (n/64, k/64)
    KB = (K + 63) // 64
    rb = 32 if fmt == "int4" else 64
    src = rows.data.view(torch.uint8).cpu().numpy()
    dst = blk.data.cpu().numpy()
    for n_, kk in [(0, 0), (N - 1, K - 8), (N // 2, K // 2)]:
        kk -= kk % (2 if fmt == "int4" else 1)
        off = (((n_ // 64) * KB + kk // 64) * 64 + n_ % 64) * rb + ((kk % 64) // 2 if fmt == "int4" else kk % 64)
        assert dst[off] == src[n_, kk // 2 if fmt == "int4" else kk]
    # the transposed section after it: W^T blocked, block (k/64, n/64), rows
    # along k; int4 nibbles hold q (two's complement), byte c of a row holds
    # n = 2c (low) and 2c+1 (high)
    NB = (N + 63) // 64
    t0 = NB * KB * 64 * rb
    assert dst.size == 2 * t0
    for n_, kk in [(0, 0), (N - 1, K - 1), (N // 2 + 1, K // 2 + 3), (N - 2, 1)]:
        off = t0 + ((kk // 64) * NB + n_ // 64) * 64 * rb + (kk % 64) * rb
        if fmt == "int4":
            u = (src[n_, kk // 2] >> (4 * (kk % 2))) & 15  # q + 8 in the row layout
            nib = (dst[off + (n_ % 64) // 2] >> (4 * (n_ % 2))) & 15
            assert nib == (int(u) - 8) & 15
        else:
            assert dst[off + n_ % 64] == src[n_, kk]
    if N % 64:  # padding depth columns of the last block column are zero (N is even here)
        last = dst[t0 + (NB - 1) * 64 * rb:t0 + NB * 64 * rb].reshape(64, rb)
        assert not last[:, ((N % 64) // 2 if fmt == "int4" else N % 64):].any()
    if fmt != "fp8":
        Gp = KB * 64 // g
        allsc = blk.scales.cpu().numpy()
        sc = allsc[:NB * Gp * 64].reshape(NB, Gp, 64)
        ref = rows.scales.cpu().numpy()
        assert np.array_equal(sc[(N - 1) // 64, (K - 1) // g, (N - 1) % 64], ref[N - 1, (K - 1) // g])
        if N % 64:
            assert not sc[NB - 1, :, N % 64:].any()  # padding rows carry scale 0
        # transposed scale table ST [ceil(64 KB / g)][NB*64]: ST[kg][n] = scale(n, kg)
        KGt = (KB * 64 + g - 1) // g
        st = allsc[NB * Gp * 64:].reshape(KGt, NB * 64)
        assert np.array_equal(st[:K // g, :N], ref.T)
        assert not st[:, N:].any() and not st[K // g:].any()
