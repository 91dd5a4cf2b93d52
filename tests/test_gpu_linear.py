"""Parity of the fused quantized LoRA linear (forward and backward) on the GPU,
through the C ABI, against the CPU oracle on identical seeded inputs
(tolerance: rel_deviation <= 1e-2 and cosine >= 0.999 for bf16 outputs),
and at the benchmark configurations' full sizes against a torch fp32 reference built from the
bit-exact dequantized weight."""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import case_inputs, check, gemm_path, to_dev
from loractl_amd import device as D
from loractl_amd._lib import LrqError

pytestmark = pytest.mark.gpu

# (M, K, N, group): ragged M, K % 64 == 32, N not a tile multiple, exact tiles
SHAPES = [(1, 64, 64, 32), (5, 64, 8, 32), (37, 96, 72, 32), (130, 192, 520, 64), (256, 256, 256, 64),
          (300, 320, 264, 64), (513, 512, 392, 128)]


def _weight(w, fmt, g, dev, per_channel=True):
    t = torch.from_numpy(w).to(dev)
    if fmt == "int4":
        wq = D.quantize_int4(t, g)
        p, s = O.quantize_int4_packed(w, g)
        return wq, O.dequant_int4(p, s, w.shape[1], g)
    if fmt == "int8":
        wq = D.quantize_int8(t, g)
        q, s = O.quantize(w, g, 127)
        return wq, O.dequant_q(q, s, g)
    wq = D.quantize_fp8(t, per_channel)
    b, s = O.fp8_quantize(w, per_channel)
    return wq, O.fp8_dequant(b, s)


def _quantize(w, fmt, group, per_channel=True):
    """A device weight of ``fmt`` from an f32 device tensor (int4 / int8 at ``group``)."""
    if fmt == "int4":
        return D.quantize_int4(w, group)
    if fmt == "int8":
        return D.quantize_int8(w, group)
    return D.quantize_fp8(w, per_channel)


@pytest.mark.parametrize("M,K,N,g", SHAPES)
@pytest.mark.parametrize("fmt", ["int4", "fp8", "int8"])
def test_quant_matmul_t_and_bwd(cuda, fmt, M, K, N, g):
    w, x, _, _, dy = case_inputs(M, K, N, 0, seed=M + N)
    wq, wdq = _weight(w, fmt, g, cuda)
    y = D.quant_matmul_t(to_dev(x, cuda), wq)
    dx = D.quant_matmul_t_bwd(to_dev(dy, cuda), wq)
    y_ref, _ = O.linear_fwd(x, wdq)
    dx_ref, _, _ = O.linear_bwd(x, wdq, None, None, 1.0, dy)
    check(f"{fmt} y", y, y_ref)
    check(f"{fmt} dx", dx, dx_ref)


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_quant_matmul_t_reference_golden(cuda, fmt):
    """quant_int4_golden.json / quant_int8_golden.json: y = x . dq^T on the GPU
    within bf16 rounding."""
    import json, os
    g = json.load(open(os.path.join(os.path.dirname(__file__), "golden", f"quant_{fmt}_golden.json")))
    w = np.array(g["w"], np.float32)
    x = np.array(g["x"], np.float32)
    wq = _quantize(torch.from_numpy(w).to(cuda), fmt, 32)
    y = D.quant_matmul_t(to_dev(x, cuda), wq)
    check("golden y", y, np.array(g["y"], np.float32))


@pytest.mark.parametrize("M,K,N,g", SHAPES)
@pytest.mark.parametrize("r", [16, 32])
def test_lora_fwd_bwd_int4(cuda, M, K, N, g, r):
    w, x, a, b, dy = case_inputs(M, K, N, r, seed=3 * M + N + r)
    wq, wdq = _weight(w, "int4", g, cuda)
    s = 16.0 / r
    xd, ad, bd = to_dev(x, cuda), to_dev(a, cuda), to_dev(b, cuda)
    y, t = D.lora_fwd(xd, wq, ad, bd, s)
    dx, da, db = D.lora_bwd(xd, to_dev(dy, cuda), wq, ad, bd, s, t)
    y_ref, t_ref = O.linear_fwd(x, wdq, a, b, s)
    dx_ref, da_ref, db_ref = O.linear_bwd(x, wdq, a, b, s, dy)
    check("t", t, t_ref)
    check("y", y, y_ref)
    check("dx", dx, dx_ref)
    check("dA", da, da_ref)
    check("dB", db, db_ref)
    # the LoRA term itself (y - base) must be right, not just drowned by the base:
    # y and base are each a bf16 rounding (<= 2^-8 relative) of an f32 sum, and
    # the term is t.B with t held in bf16 (<= 2^-8 relative per element), so
    # elementwise |(y - base) - lora| <= 2^-8 (|y| + |base| + |t|.|B|) + f32 slack
    base = D.quant_matmul_t(xd, wq).float().cpu().numpy()
    base_ref = O.linear_fwd(x, wdq)[0]
    lora_ref = y_ref - base_ref
    err = np.abs((y.float().cpu().numpy() - base) - lora_ref)
    bound = (2.0 ** -8 * (np.abs(y_ref) + np.abs(base_ref) + np.abs(t_ref) @ np.abs(b))
             + 1e-4 * np.abs(y_ref).max())
    assert (err <= bound).all(), f"y-base: worst excess {(err - bound).max():.3e}"
    assert np.abs(lora_ref).max() > 1e-2 * np.abs(y_ref).max()  # the case exercises a visible LoRA term


def test_reduced_precision_accuracy_gates(cuda):
    """tests/reduced_precision_accuracy.rs:44-62, :105-155 on the fused
    forward: y = x . dq(w)^T against x . w^T with the unquantized f32 weight,
    on the reference's golden w [8, 64] and x [4, 64] (block 32). int8 and
    int4 each stay within the reference's calibrated band (d <= max(2 d_bar,
    1e-3) and d <= ceil, d the peak-normalized deviation) and are not
    no-ops, and on the same inputs int4 moves the output more than 4x as
    much as int8. x enters as bf16 (the kernels' activation type) on both
    sides; y leaves as bf16, whose rounding the bands absorb."""
    import json, os
    from loractl_amd.accuracy import RelGate, rel_deviation

    gates = {"int8": RelGate(5.8e-3, 1e-3, 2.5e-2), "int4": RelGate(9.4e-2, 1e-3, 2.0e-1)}

    def deviation(fmt, golden):
        g = json.load(open(os.path.join(os.path.dirname(__file__), "golden", golden)))
        w = np.array(g["w"], np.float32)
        xb = to_dev(np.array(g["x"], np.float32), cuda)
        ref = xb.float().cpu().numpy().astype(np.float64) @ w.astype(np.float64).T
        y = D.quant_matmul_t(xb, _quantize(torch.from_numpy(w).to(cuda), fmt, 32))
        return rel_deviation(y.float().cpu().numpy(), ref)

    for fmt in ("int8", "int4"):
        d = deviation(fmt, f"quant_{fmt}_golden.json")
        assert d > 0.0, f"{fmt}: quantization was a no-op"
        gates[fmt].apply(d).expect_pass(f"{fmt} forward")
    d8 = deviation("int8", "quant_int8_golden.json")
    d4 = deviation("int4", "quant_int8_golden.json")
    assert d4 > 4.0 * d8, f"int4 must be markedly coarser than int8: int4 {d4:e} vs int8 {d8:e}"


@pytest.mark.parametrize("M,K,N,g", [SHAPES[0], SHAPES[2], SHAPES[3], SHAPES[6]])
def test_lora_fwd_bwd_int8(cuda, M, K, N, g):
    """The int8 (Q8S) base through the fused forward and backward, few-token
    and large-tile paths, against the oracle on its dequantized weight."""
    r = 16
    w, x, a, b, dy = case_inputs(M, K, N, r, seed=5 * M + N)
    wq, wdq = _weight(w, "int8", g, cuda)
    s = 16.0 / r
    xd, ad, bd = to_dev(x, cuda), to_dev(a, cuda), to_dev(b, cuda)
    y, t = D.lora_fwd(xd, wq, ad, bd, s)
    dx, da, db = D.lora_bwd(xd, to_dev(dy, cuda), wq, ad, bd, s, t)
    y_ref, t_ref = O.linear_fwd(x, wdq, a, b, s)
    dx_ref, da_ref, db_ref = O.linear_bwd(x, wdq, a, b, s, dy)
    check("t", t, t_ref)
    check("y", y, y_ref)
    check("dx", dx, dx_ref)
    check("dA", da, da_ref)
    check("dB", db, db_ref)


@pytest.mark.parametrize("r", [1, 3, 8, 17, 64])
def test_lora_ranks(cuda, r):
    M, K, N, g = 70, 128, 96, 64
    w, x, a, b, dy = case_inputs(M, K, N, r, seed=r, b_sigma=0.05)
    wq, wdq = _weight(w, "int4", g, cuda)
    s = 2.0
    xd, ad, bd = to_dev(x, cuda), to_dev(a, cuda), to_dev(b, cuda)
    y, t = D.lora_fwd(xd, wq, ad, bd, s)
    dx, da, db = D.lora_bwd(xd, to_dev(dy, cuda), wq, ad, bd, s, t)
    y_ref, _ = O.linear_fwd(x, wdq, a, b, s)
    dx_ref, da_ref, db_ref = O.linear_bwd(x, wdq, a, b, s, dy)
    check("y", y, y_ref)
    check("dx", dx, dx_ref)
    check("dA", da, da_ref)
    check("dB", db, db_ref)


@pytest.mark.parametrize("per_channel", [True, False])
def test_lora_fwd_bwd_fp8(cuda, per_channel):
    M, K, N, r = 200, 256, 200, 32
    w, x, a, b, dy = case_inputs(M, K, N, r, seed=17)
    wq, wdq = _weight(w, "fp8", 0, cuda, per_channel)
    xd, ad, bd = to_dev(x, cuda), to_dev(a, cuda), to_dev(b, cuda)
    y, t = D.lora_fwd(xd, wq, ad, bd, 1.0)
    dx, da, db = D.lora_bwd(xd, to_dev(dy, cuda), wq, ad, bd, 1.0, t)
    y_ref, _ = O.linear_fwd(x, wdq, a, b, 1.0)
    dx_ref, da_ref, db_ref = O.linear_bwd(x, wdq, a, b, 1.0, dy)
    check("y", y, y_ref)
    check("dx", dx, dx_ref)
    check("dA", da, da_ref)
    check("dB", db, db_ref)


def test_bias_epilogue(cuda):
    M, K, N = 33, 128, 64
    w, x, _, _, _ = case_inputs(M, K, N, 0, seed=5)
    wq, wdq = _weight(w, "int4", 64, cuda)
    bias = np.linspace(-1, 1, N).astype(np.float32)
    wb = wq.with_bias(torch.from_numpy(bias).to(cuda))
    y = D.quant_matmul_t(to_dev(x, cuda), wb)
    y_ref, _ = O.linear_fwd(x, wdq, bias=bias)
    check("y+bias", y, y_ref)


@pytest.mark.parametrize("path", ["large", "mid64", "mid128", "mid64s", "mid128s"])
@pytest.mark.parametrize("fmt,per_channel", [("int4", True), ("fp8", True), ("fp8", False), ("int8", True)])
def test_split_depth_bias_and_scales(cuda, fmt, per_channel, path):
    """Few output tiles (M = 200, d_out = 3072). On the large tiles the depth
    is split into ranges whose f32 partials a reduction sums, and the bias
    and the forward fp8 channel scales (or the scalar) are applied there,
    once; the mid-size tiles run the whole depth ("mid64s", "mid128s": in
    depth ranges summed in the launch) and apply them in their epilogue."""
    M, K, N, r = 200, 3072, 3072, 16
    g = torch.Generator(device=cuda).manual_seed(7)
    w = torch.randn(N, K, device=cuda, generator=g) * 0.02
    wq = _quantize(w, fmt, 64, per_channel)
    bias = torch.randn(N, device=cuda, generator=g) * 0.1
    wq = wq.with_bias(bias)
    wdq = D.dequant(wq)
    x = torch.randn(M, K, device=cuda, generator=g).to(torch.bfloat16)
    a = ((torch.rand(K, r, device=cuda, generator=g) * 2 - 1) / K ** 0.5).to(torch.bfloat16)
    b = (torch.randn(r, N, device=cuda, generator=g) * 1e-2).to(torch.bfloat16)
    dy = torch.randn(M, N, device=cuda, generator=g).to(torch.bfloat16)
    with gemm_path(path):
        y, t = D.lora_fwd(x, wq, a, b, 0.5)
        dx, _, _ = D.lora_bwd(x, dy, wq, a, b, 0.5, t)
    xf, af, bf, dyf = x.float(), a.float(), b.float(), dy.float()
    y_ref = xf @ wdq.t() + 0.5 * (xf @ af) @ bf + bias
    dx_ref = dyf @ wdq + 0.5 * (dyf @ bf.t()) @ af.t()
    check("y", y, y_ref.cpu().numpy())
    check("dx", dx, dx_ref.cpu().numpy())


@pytest.mark.parametrize("per_channel", [True, False])
def test_fp8_mid_forward_repeats(cuda, per_channel):
    """The fp8 forward's mid-size tiles load no scale in their main loop (the
    channel scales apply in the epilogue), so a stage issues one load fewer
    per block than the other formats, and the counted waits for a stage's
    activation copies must count exactly that. Every mid path's forward,
    three times over, against the fp32 reference and bit-identical across
    the repeats: a count one too high let a wavefront read 8 token rows of
    its stage before their copy landed (16 outputs x 8 tokens wrong, in the
    ragged last token tile, in about a third of the calls)."""
    M, K, N, r = 200, 3072, 3072, 16
    g = torch.Generator(device=cuda).manual_seed(11)
    w = torch.randn(N, K, device=cuda, generator=g) * 0.02
    wq = _quantize(w, "fp8", 64, per_channel)
    wdq = D.dequant(wq)
    x = torch.randn(M, K, device=cuda, generator=g).to(torch.bfloat16)
    a = ((torch.rand(K, r, device=cuda, generator=g) * 2 - 1) / K ** 0.5).to(torch.bfloat16)
    b = (torch.randn(r, N, device=cuda, generator=g) * 1e-2).to(torch.bfloat16)
    xf = x.float()
    y_ref = (xf @ wdq.t() + 0.5 * (xf @ a.float()) @ b.float()).cpu().numpy()
    for path in ("mid64", "mid128", "mid64s", "mid128s"):
        outs = []
        for _ in range(3):
            with gemm_path(path):
                y, _t = D.lora_fwd(x, wq, a, b, 0.5)
            check(f"y {path}", y, y_ref)
            outs.append(y)
        assert all(torch.equal(outs[0], o) for o in outs[1:]), path


@pytest.mark.parametrize("M,r", [(1, 17), (3, 32), (16, 17), (16, 64)])
@pytest.mark.parametrize("fmt,per_channel,group", [("int4", True, 32), ("int4", True, 128), ("fp8", True, 0),
                                                   ("fp8", False, 0), ("int8", True, 32), ("int8", True, 128)])
def test_few_token_input_gradient(cuda, M, r, fmt, per_channel, group):
    """m <= 16: the input gradient streams the transposed section once in
    depth splits (d_out = 2056, ragged past 32 blocks of 64); the transposed
    scales (int4 groups along d_in, fp8 channel scales or the scalar along
    the depth) are applied per value, and u . A^T is added in the reduction;
    u itself (s . dy . B^T) is reduced there too and feeds dA."""
    K, N = 1024, 2056
    g = torch.Generator(device=cuda).manual_seed(11 + M + r)
    w = torch.randn(N, K, device=cuda, generator=g) * 0.02
    wq = _quantize(w, fmt, group, per_channel)
    wdq = D.dequant(wq)
    x = torch.randn(M, K, device=cuda, generator=g).to(torch.bfloat16)
    a = ((torch.rand(K, r, device=cuda, generator=g) * 2 - 1) / K ** 0.5).to(torch.bfloat16)
    b = (torch.randn(r, N, device=cuda, generator=g) * 1e-1).to(torch.bfloat16)
    dy = torch.randn(M, N, device=cuda, generator=g).to(torch.bfloat16)
    y, t = D.lora_fwd(x, wq, a, b, 0.5)
    dx, da, db = D.lora_bwd(x, dy, wq, a, b, 0.5, t)
    dx0 = D.quant_matmul_t_bwd(dy, wq)
    dyf, af, bf = dy.float(), a.float(), b.float()
    u = (0.5 * (dyf @ bf.t())).to(torch.bfloat16).float()
    check("dx", dx, (dyf @ wdq + u @ af.t()).cpu().numpy())
    check("dx base", dx0, (dyf @ wdq).cpu().numpy())
    # u comes out of the input gradient's launches and feeds dA
    check("dA", da, (x.float().t() @ u).cpu().numpy())
    check("dB", db, (t.float().t() @ dyf).cpu().numpy())


def test_zero_b_delta_is_bitwise_no_op(cuda):
    """lora.rs:262-276 on the fused kernel: B = 0 gives exactly the base output."""
    M, K, N, r = 64, 256, 128, 16
    w, x, a, _, _ = case_inputs(M, K, N, r, seed=8)
    wq, _ = _weight(w, "int4", 64, cuda)
    xd = to_dev(x, cuda)
    y, _ = D.lora_fwd(xd, wq, to_dev(a, cuda), torch.zeros(r, N, dtype=torch.bfloat16, device=cuda), 1.0)
    assert torch.equal(y, D.quant_matmul_t(xd, wq))


def test_outputs_are_deterministic(cuda):
    M, K, N, r = 300, 256, 200, 16
    w, x, a, b, dy = case_inputs(M, K, N, r, seed=4)
    wq, _ = _weight(w, "int4", 64, cuda)
    args = (to_dev(x, cuda), wq, to_dev(a, cuda), to_dev(b, cuda), 1.0)
    y1, t1 = D.lora_fwd(*args)
    y2, t2 = D.lora_fwd(*args)
    g1 = D.lora_bwd(args[0], to_dev(dy, cuda), wq, args[2], args[3], 1.0, t1)
    g2 = D.lora_bwd(args[0], to_dev(dy, cuda), wq, args[2], args[3], 1.0, t2)
    assert torch.equal(y1, y2) and torch.equal(t1, t2)
    for u, v in zip(g1, g2):
        assert torch.equal(u, v)


# (M, K, N, r, path): the mid-size passes that keep state in the context's
# counter area (fold groups' arrivals and ready flags, depth-range counters,
# the weight gradients' counters), interleaved with a few-token call and a
# large-tile call that use the same area
INTERLEAVED = [(200, 3072, 2560, 16, "mid64s"), (130, 192, 520, 8, "mid128"), (9, 512, 768, 16, "planned"),
               (513, 512, 392, 16, "mid64"), (256, 2560, 1536, 8, "mid128s"), (300, 1024, 768, 32, "large"),
               (64, 1536, 1024, 16, "mid64")]


def test_interleaved_calls_repeat_bit_for_bit(cuda):
    """Three rounds over differently planned calls, forward and backward,
    each call bit-identical to its first round: every kernel that counts or
    flags across its workgroups leaves the counter area as it found it,
    whatever ran before it."""
    cases = []
    for i, (M, K, N, r, path) in enumerate(INTERLEAVED):
        w, x, a, b, dy = case_inputs(M, K, N, r, seed=50 + i)
        wq, _ = _weight(w, "int4", 64, cuda)
        cases.append((path, wq, to_dev(x, cuda), to_dev(a, cuda), to_dev(b, cuda), to_dev(dy, cuda)))
    first = None
    for rnd in range(3):
        outs = []
        for path, wq, xd, ad, bd, dyd in cases:
            with gemm_path(path):
                y, t = D.lora_fwd(xd, wq, ad, bd, 0.5)
                dx, da, db = D.lora_bwd(xd, dyd, wq, ad, bd, 0.5, t)
            outs.append((y, t, dx, da, db))
        D.sync()
        if first is None:
            first = outs
            continue
        for i, (o1, o2) in enumerate(zip(first, outs)):
            for name, u, v in zip(("y", "t", "dx", "dA", "dB"), o1, o2):
                assert torch.equal(u, v), (rnd, INTERLEAVED[i], name)


def test_shape_errors_are_loud(cuda):
    w = torch.randn(64, 96, device=cuda)
    wq = D.quantize_int4(w, 32)
    with pytest.raises(LrqError, match="LRQ_EINVAL"):
        D.lora_fwd(torch.zeros(4, 96, dtype=torch.bfloat16, device=cuda), wq,
                   torch.zeros(96, 65, dtype=torch.bfloat16, device=cuda),
                   torch.zeros(65, 64, dtype=torch.bfloat16, device=cuda), 1.0)
    bad = D.PackedWeight(wq.fmt, 60, 96, wq.data, wq.scales, group=32)  # d_out % 8 != 0
    with pytest.raises(LrqError, match="multiple of 8"):
        D.quant_matmul_t(torch.zeros(4, 96, dtype=torch.bfloat16, device=cuda), bad)
    with pytest.raises(ValueError):
        D.quant_matmul_t(torch.zeros(4, 96, dtype=torch.float32, device=cuda), wq)


@pytest.mark.parametrize("M,K,N,r,fmt", [(4096, 3072, 12288, 32, "int4"), (1024, 3072, 3072, 16, "int4"),
                                         (4096, 3072, 12288, 32, "fp8"), (16, 3072, 12288, 32, "int4"),
                                         # ragged edges on the large-tile paths (tokens, d_in, d_out)
                                         (4000, 3008, 12280, 16, "int4"), (4000, 3008, 12280, 16, "fp8"),
                                         # the MLP-down shape: 192-row forward tiles, 256-row input-gradient
                                         # tiles (the shapes above take the other pairing), exact and ragged
                                         (4096, 12288, 3072, 32, "int4"), (4000, 12224, 3064, 16, "fp8"),
                                         # split depth (fewer output tiles than CUs): both passes
                                         (256, 3072, 12288, 32, "fp8"), (300, 3008, 12280, 16, "int4"),
                                         # few tokens with a deep d_in (Qwen MLP down): more than 16 t
                                         # slices and 8 reduction splits in the few-token epilogue
                                         (16, 9728, 2560, 16, "int4"), (5, 9728, 2560, 16, "fp8"),
                                         # the int8 base on the same paths: large tiles, ragged edges,
                                         # 192-row tiles, split depth, few tokens
                                         (4096, 3072, 12288, 32, "int8"), (4000, 12224, 3064, 16, "int8"),
                                         (300, 3008, 12280, 16, "int8"), (16, 3072, 12288, 32, "int8"),
                                         (5, 9728, 2560, 16, "int8")])
def test_baseline_shapes_against_torch_fp32(cuda, M, K, N, r, fmt):
    """The benchmark configurations at full size: the fused kernels vs torch fp32 GEMMs over the
    same bf16 inputs and the (bit-exact) dequantized weight."""
    g = torch.Generator(device=cuda).manual_seed(M + N)
    w = torch.randn(N, K, device=cuda, generator=g) * 0.02
    wq = _quantize(w, fmt, 64)
    wdq = D.dequant(wq)
    x = torch.randn(M, K, device=cuda, generator=g).to(torch.bfloat16)
    a = ((torch.rand(K, r, device=cuda, generator=g) * 2 - 1) / K ** 0.5).to(torch.bfloat16)
    b = (torch.randn(r, N, device=cuda, generator=g) * 1e-3).to(torch.bfloat16)
    dy = torch.randn(M, N, device=cuda, generator=g).to(torch.bfloat16)
    y, t = D.lora_fwd(x, wq, a, b, 1.0)
    dx, da, db = D.lora_bwd(x, dy, wq, a, b, 1.0, t)
    xf, af, bf, dyf = x.float(), a.float(), b.float(), dy.float()
    t_ref = xf @ af
    u_ref = dyf @ bf.t()
    y_ref = xf @ wdq.t() + t_ref @ bf
    dx_ref = dyf @ wdq + u_ref @ af.t()
    da_ref = xf.t() @ u_ref
    db_ref = t_ref.t() @ dyf
    for name, got, ref in (("y", y, y_ref), ("dx", dx, dx_ref), ("dA", da, da_ref), ("dB", db, db_ref)):
        check(name, got, ref.cpu().numpy())


# m > 16: ragged token counts (not a multiple of 64 or 128), K % 64 == 32,
# d_out not a multiple of 64, groups 32 to 128
PATH_SHAPES = [(37, 96, 72, 32), (130, 192, 520, 64), (300, 320, 264, 64), (513, 512, 392, 128), (200, 1536, 1280, 64)]


@pytest.mark.parametrize("r", [33, 32, 24, 16, 8])
@pytest.mark.parametrize("path", ["large", "mid64", "mid128", "mid64s", "mid128s"])
@pytest.mark.parametrize("fmt,per_channel", [("int4", True), ("int8", True), ("fp8", True), ("fp8", False)])
@pytest.mark.parametrize("M,K,N,g", PATH_SHAPES)
def test_gemm_paths_against_oracle(cuda, M, K, N, g, fmt, per_channel, path, r):
    """Every kernel path of m > 16 (the 256-token tiles, split in depth where
    they are few, and the 64-row tiles of 64 or 128 tokens) on the same
    inputs: y (with bias), t, dx, dA and dB of the fused site, and the plain
    product and its input gradient, against the f64 oracle. At ranks 8, 16,
    24 and 32 the 64-row tiles form t, u, dA and dB in their own launches; "mid64s"
    and "mid128s" split their depth into ranges where it allows."""
    w, x, a, b, dy = case_inputs(M, K, N, r, seed=7 * M + N + g)
    wq, wdq = _weight(w, fmt, g, cuda, per_channel)
    bias = np.linspace(-0.5, 0.5, N).astype(np.float32)
    wb = wq.with_bias(torch.from_numpy(bias).to(cuda))
    s = 0.75
    xd, ad, bd, dyd = to_dev(x, cuda), to_dev(a, cuda), to_dev(b, cuda), to_dev(dy, cuda)
    with gemm_path(path):
        y, t = D.lora_fwd(xd, wb, ad, bd, s)
        dx, da, db = D.lora_bwd(xd, dyd, wb, ad, bd, s, t)
        y0 = D.quant_matmul_t(xd, wq)
        dx0 = D.quant_matmul_t_bwd(dyd, wq)
    y_ref, t_ref = O.linear_fwd(x, wdq, a, b, s, bias=bias)
    dx_ref, da_ref, db_ref = O.linear_bwd(x, wdq, a, b, s, dy)
    check("y", y, y_ref)
    check("t", t, t_ref)
    check("dx", dx, dx_ref)
    check("dA", da, da_ref)
    check("dB", db, db_ref)
    check("y base", y0, O.linear_fwd(x, wdq)[0])
    check("dx base", dx0, O.linear_bwd(x, wdq, None, None, 1.0, dy)[0])
