"""The few-token forward (m <= 16 takes its own HBM-streaming kernel) against
the CPU oracle on identical seeded inputs, and against the large-m kernel on
the same rows (both round dequantized weights to bf16 and accumulate in f32,
so they agree to f32 summation order)."""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import case_inputs, check, to_dev
from loractl_amd import device as D

pytestmark = pytest.mark.gpu


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


# (fmt, group, per_channel): int4 blocks smaller, equal and larger than the 64-wide step
FORMATS = [("int4", 32, True), ("int4", 64, True), ("int4", 128, True), ("fp8", 0, True), ("fp8", 0, False),
           ("int8", 32, True), ("int8", 128, True)]


@pytest.mark.parametrize("M", [1, 7, 16])
# reduction splits with partials, except (1088, 8192): 128 whole-depth
# workgroups (skinny_plan's rule)
@pytest.mark.parametrize("K,N", [(96, 72), (1088, 520), (3072, 264), (4160, 136), (1088, 8192)])
@pytest.mark.parametrize("fmt,g,pc", FORMATS)
def test_skinny_base_and_lora(cuda, M, K, N, fmt, g, pc):
    if fmt != "fp8" and K % g:
        pytest.skip("int4 and int8 blocks must divide d_in")
    r = 17
    w, x, a, b, _ = case_inputs(M, K, N, r, seed=11 * M + K + N, b_sigma=0.05)
    wq, wdq = _weight(w, fmt, g, cuda, pc)
    xd, ad, bd = to_dev(x, cuda), to_dev(a, cuda), to_dev(b, cuda)
    base = D.quant_matmul_t(xd, wq)
    check(f"{fmt} base", base, O.linear_fwd(x, wdq)[0])
    y, t = D.lora_fwd(xd, wq, ad, bd, 0.5)
    y_ref, t_ref = O.linear_fwd(x, wdq, a, b, 0.5)
    check("t", t, t_ref)
    check("y", y, y_ref)


@pytest.mark.parametrize("r", [1, 16, 33, 64])
@pytest.mark.parametrize("N", [200, 8192])  # splits; whole-depth workgroups
def test_skinny_ranks_and_bias(cuda, r, N):
    M, K, g = 9, 640, 64
    w, x, a, b, _ = case_inputs(M, K, N, r, seed=r, b_sigma=0.05)
    wq, wdq = _weight(w, "int4", g, cuda)
    bias = np.linspace(-1, 1, N).astype(np.float32)
    wb = wq.with_bias(torch.from_numpy(bias).to(cuda))
    y, _ = D.lora_fwd(to_dev(x, cuda), wb, to_dev(a, cuda), to_dev(b, cuda), 2.0)
    y_ref, _ = O.linear_fwd(x, wdq, a, b, 2.0, bias=bias)
    check("y", y, y_ref)


@pytest.mark.parametrize("fmt", ["int4", "fp8", "int8"])
def test_skinny_matches_large_m_kernel(cuda, fmt):
    """Rows 0..15 of a 300-token call (large-m kernel) against the same 16
    tokens alone (few-token kernel). The large-m kernel multiplies bf16(q s);
    the few-token int4 kernel (groups >= 64) multiplies q exactly and scales
    in f32, so the two differ by at most the weight's bf16 rounding (half
    an ulp, 2^-8 relative per weight, int4 only: fp8 values are exact in
    bf16 and both int8 kernels multiply bf16(q s)), the rounding of both outputs and of t to bf16, and f32
    summation order."""
    M, K, N, r = 300, 1024, 328, 32
    w, x, a, b, _ = case_inputs(M, K, N, r, seed=21)
    wq, wdq = _weight(w, fmt, 64, cuda)
    xd, ad, bd = to_dev(x, cuda), to_dev(a, cuda), to_dev(b, cuda)
    y_big, t_big = D.lora_fwd(xd, wq, ad, bd, 1.0)
    y_small, t_small = D.lora_fwd(xd[:16].contiguous(), wq, ad, bd, 1.0)
    tb, ts = t_big[:16].float(), t_small.float()  # split reductions may differ in order
    assert ((tb - ts).abs() <= 2.0 ** -7 * tb.abs() + 1e-6).all()
    yb, ys = y_big[:16].float(), y_small.float()
    xa = xd[:16].float().abs()
    wr = 2.0 ** -8 if fmt == "int4" else 0.0
    bound = (wr * (xa @ torch.from_numpy(np.abs(wdq)).to(cuda).t()) + 2.0 ** -7 * yb.abs()
             + 2.0 ** -7 * (tb.abs() @ bd.float().abs()) + 1e-5 * yb.abs().max())
    assert ((yb - ys).abs() <= bound).all()
    y_ref, _ = O.linear_fwd(x[:16], wdq, a, b, 1.0)
    check("y few-token", y_small, y_ref)
    check("y large-m", y_big[:16], y_ref)


def test_skinny_zero_b_is_bitwise_no_op(cuda):
    M, K, N, r = 4, 256, 128, 16
    w, x, a, _, _ = case_inputs(M, K, N, r, seed=8)
    wq, _ = _weight(w, "int4", 64, cuda)
    xd = to_dev(x, cuda)
    y, _ = D.lora_fwd(xd, wq, to_dev(a, cuda), torch.zeros(r, N, dtype=torch.bfloat16, device=cuda), 1.0)
    assert torch.equal(y, D.quant_matmul_t(xd, wq))


def test_few_token_counters_leave_no_failure_flag(cuda):
    """The single-launch few-token kernels finish through arrival counters
    and a bounded wait for the t slices; after forward and backward calls at
    m <= 16 (with and without LoRA) and a repeat of each, lrq_sync reports no
    timed-out wait, and the repeat reproduces the first result bit for bit
    (the counters were left at zero)."""
    M, K, N, r = 9, 3072, 4096, 32
    w, x, a, b, dy = case_inputs(M, K, N, r, seed=5, b_sigma=0.05)
    wq, _ = _weight(w, "int4", 64, cuda)
    xd, ad, bd, dyd = to_dev(x, cuda), to_dev(a, cuda), to_dev(b, cuda), to_dev(dy, cuda)
    outs = []
    for _ in range(2):
        y, t = D.lora_fwd(xd, wq, ad, bd, 0.5)
        dx, da, db = D.lora_bwd(xd, dyd, wq, ad, bd, 0.5, t)
        base = D.quant_matmul_t(xd, wq)
        gx = D.quant_matmul_t_bwd(dyd, wq)
        outs.append([v.clone() for v in (y, t, dx, da, db, base, gx)])
    D.context().call("lrq_sync")
    for u, v in zip(*outs):
        assert torch.equal(u, v)
