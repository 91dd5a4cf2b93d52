"""Seeded random shapes through the whole LoRA linear, forward and backward.

The other GPU tests pick their shapes by hand (tile edges, ragged tails,
the baseline configurations). Here 120 shapes come from a fixed seed, a
third each in the few-token (m <= 16), mid-size (17 <= m < 1024) and
large (1024 <= m < 4100) token ranges, with d_in any multiple of the
format's block (or of 32 for fp8) up to 4096, d_out any multiple of 8 up to
4096 and any rank 1..64, over int4 and int8 (blocks 32, 64, 128), fp8 with
channel scales and fp8 with one scalar scale. The kernel path is the
planned one, so the planners' choices for odd shapes are exercised too.

Each case checks y, t, dx, dA and dB within the north star's tolerance
(rel_deviation <= 1e-2, cosine >= 0.999; tests/gpu_helpers.py) against an
fp32 torch reference of the same algebra (crates/loractl-core/src/lora.rs:
199-203 and its autodiff: t = s x A and u = s dy B^T held in bf16 as the
kernels hold them, y = x W^T + t B, dx = dy W + u A^T, dA = x^T u,
dB = t^T dy, W the library's dequantized weight, bit-exact with the oracle
in tests/test_gpu_formats.py), and that a repeated backward is bit-identical.
"""

import numpy as np
import pytest
import torch

from gpu_helpers import check
from loractl_amd import device as D

pytestmark = pytest.mark.gpu

FORMATS = ["int4", "int8", "fp8", "fp8-scalar"]


def _cases(n=120, seed=20261202):
    g = np.random.Generator(np.random.PCG64(seed))
    out = []
    for i in range(n):
        regime = i % 3
        lo, hi = [(1, 17), (17, 1024), (1024, 4100)][regime]
        M = int(g.integers(lo, hi))
        fmt = FORMATS[(i // 3) % 4]
        grp = int(g.choice([32, 64, 128])) if fmt in ("int4", "int8") else 0
        unit = max(grp, 32)
        K = unit * int(g.integers(1, 4096 // unit + 1))
        N = 8 * int(g.integers(1, 513))
        r = int(g.integers(1, 65))
        out.append((M, K, N, r, fmt, grp))
    return out


CASES = _cases()


def _quantize(w, fmt, grp):
    if fmt == "int4":
        return D.quantize_int4(w, grp)
    if fmt == "int8":
        return D.quantize_int8(w, grp)
    return D.quantize_fp8(w, fmt == "fp8")


@pytest.mark.parametrize("M,K,N,r,fmt,grp", CASES, ids=[f"m{c[0]}-k{c[1]}-n{c[2]}-r{c[3]}-{c[4]}" + (f"-g{c[5]}" if c[5] else "")
                                                        for c in CASES])
def test_random_shape_forward_backward(cuda, M, K, N, r, fmt, grp):
    g = torch.Generator(device=cuda).manual_seed(M * 131 + K * 7 + N + r)
    w = torch.randn(N, K, device=cuda, generator=g) * 0.02
    wq = _quantize(w, fmt, grp)
    W = D.dequant(wq).float()
    x = torch.randn(M, K, device=cuda, generator=g).to(torch.bfloat16)
    a = ((torch.rand(K, r, device=cuda, generator=g) * 2 - 1) / K ** 0.5).to(torch.bfloat16)
    b = (torch.randn(r, N, device=cuda, generator=g) * 1e-1).to(torch.bfloat16)
    dy = torch.randn(M, N, device=cuda, generator=g).to(torch.bfloat16)
    s = 16.0 / r
    y, t = D.lora_fwd(x, wq, a, b, s)
    dx, da, db = D.lora_bwd(x, dy, wq, a, b, s, t)
    dx2, da2, db2 = D.lora_bwd(x, dy, wq, a, b, s, t)
    D.sync()

    xf, af, bf, dyf = x.float(), a.float(), b.float(), dy.float()
    t_ref = s * xf @ af
    tb = t_ref.to(torch.bfloat16).float()
    u = (s * dyf @ bf.t()).to(torch.bfloat16).float()
    ref = {
        "t": t_ref,
        "y": xf @ W.t() + tb @ bf,
        "dx": dyf @ W + u @ af.t(),
        "dA": xf.t() @ u,
        "dB": tb.t() @ dyf,
    }
    got = {"t": t, "y": y, "dx": dx, "dA": da, "dB": db}
    for name, rv in ref.items():
        check(name, got[name], rv.cpu().numpy())
    assert torch.equal(dx, dx2) and torch.equal(da, da2) and torch.equal(db, db2), "repeated backward differs"


@pytest.mark.parametrize("M,K,N,r,fmt,grp", CASES[::2], ids=[f"m{c[0]}-k{c[1]}-n{c[2]}-r{c[3]}-{c[4]}" +
                                                             (f"-g{c[5]}" if c[5] else "") for c in CASES[::2]])
def test_random_shape_base_bias_and_noalloc(cuda, M, K, N, r, fmt, grp):
    """Every other shape of the sweep without LoRA and with a bias:
    y = x W^T + bias (quant_matmul_t, crates/loractl-core/src/quant.rs's
    QuantBackend::quant_matmul_t), dx = dy W (its backward), and the LoRA
    forward with the bias through lrq_lora_fwd_noalloc, bit-identical to
    lrq_lora_fwd where its fixed scratch holds the shape's workspace (else
    it refuses the shape with LRQ_EINVAL)."""
    from loractl_amd._lib import LrqError

    g = torch.Generator(device=cuda).manual_seed(M * 137 + K * 5 + N + r)
    w = torch.randn(N, K, device=cuda, generator=g) * 0.02
    bias = torch.randn(N, device=cuda, generator=g) * 0.1
    wq = D.compute_weight(_quantize(w, fmt, grp).with_bias(bias))
    W = D.dequant(wq).float()
    x = torch.randn(M, K, device=cuda, generator=g).to(torch.bfloat16)
    a = ((torch.rand(K, r, device=cuda, generator=g) * 2 - 1) / K ** 0.5).to(torch.bfloat16)
    b = (torch.randn(r, N, device=cuda, generator=g) * 1e-1).to(torch.bfloat16)
    dy = torch.randn(M, N, device=cuda, generator=g).to(torch.bfloat16)
    s = 16.0 / r
    y0 = D.quant_matmul_t(x, wq)
    dx0 = D.quant_matmul_t_bwd(dy, wq)
    y1, t1 = D.lora_fwd(x, wq, a, b, s)
    y2, t2 = torch.empty_like(y1), torch.empty_like(t1)
    try:
        D.lora_fwd_noalloc(x, wq, a, b, s, y2, t2)
        noalloc = True
    except LrqError as e:
        assert "scratch" in str(e), str(e)
        noalloc = False
    D.sync()

    xf = x.float()
    tb = (s * xf @ a.float()).to(torch.bfloat16).float()
    check("y base + bias", y0, (xf @ W.t() + bias).cpu().numpy())
    check("dx base", dx0, (dy.float() @ W).cpu().numpy())
    check("y LoRA + bias", y1, (xf @ W.t() + tb @ b.float() + bias).cpu().numpy())
    if noalloc:
        assert torch.equal(y1, y2) and torch.equal(t1, t2), "noalloc forward differs from lrq_lora_fwd"


@pytest.mark.parametrize("M,K,N,r,fmt,grp", [(65536, 1024, 2048, 32, "int4", 64), (259456, 256, 512, 16, "int8", 128),
                                            (259456, 256, 512, 64, "fp8", 0)],
                         ids=["m65536-int4", "m-limit-int8", "m-limit-fp8-r64"])
def test_large_token_counts(cuda, M, K, N, r, fmt, grp):
    """Token counts far past the benchmark's 4096, up to LRQ_MAX_LORA_TOKENS
    itself (259456: the t and u kernels' one arrival counter per 16 tokens
    then fills the counter area to its limit), forward and backward against
    the fp32 reference; dA and dB then reduce over a quarter million
    tokens."""
    from loractl_amd import _lib as L

    assert M <= L.LRQ_MAX_LORA_TOKENS
    g = torch.Generator(device=cuda).manual_seed(M + K + N + r)
    w = torch.randn(N, K, device=cuda, generator=g) * 0.02
    wq = _quantize(w, fmt, grp)
    W = D.dequant(wq).float()
    x = torch.randn(M, K, device=cuda, generator=g).to(torch.bfloat16)
    a = ((torch.rand(K, r, device=cuda, generator=g) * 2 - 1) / K ** 0.5).to(torch.bfloat16)
    b = (torch.randn(r, N, device=cuda, generator=g) * 1e-1).to(torch.bfloat16)
    dy = torch.randn(M, N, device=cuda, generator=g).to(torch.bfloat16)
    s = 16.0 / r
    y, t = D.lora_fwd(x, wq, a, b, s)
    dx, da, db = D.lora_bwd(x, dy, wq, a, b, s, t)
    D.sync()
    xf, af, bf, dyf = x.float(), a.float(), b.float(), dy.float()
    tb = (s * xf @ af).to(torch.bfloat16).float()
    u = (s * dyf @ bf.t()).to(torch.bfloat16).float()
    check("t", t, (s * xf @ af).cpu().numpy())
    check("y", y, (xf @ W.t() + tb @ bf).cpu().numpy())
    check("dx", dx, (dyf @ W + u @ af.t()).cpu().numpy())
    check("dA", da, (xf.t() @ u).cpu().numpy())
    check("dB", db, (tb.t() @ dyf).cpu().numpy())


@pytest.mark.parametrize("M,path", [(5, "planned"), (300, "mid64"), (300, "mid128"), (200, "mid64s"), (2048, "large")])
@pytest.mark.parametrize("grp", [256, 512])
@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_large_quant_blocks(cuda, fmt, grp, M, path):
    """Quant blocks of 256 and 512 (any power of two >= 32 that divides d_in
    is accepted; crates/loractl-core/src/quant.rs's group argument): the
    device quantization and dequantization are bit-exact against the oracle
    (Q4S / Q8S with that block), and every kernel path (few-token, both
    mid-size tiles, depth ranges, large tiles) gives y, t, dx, dA and dB
    within the tolerance. A block then spans four or eight of the kernels'
    64-deep steps, and in the transposed section four or eight 64-row
    block rows share one scale row."""
    import oracle as O
    from gpu_helpers import case_inputs, gemm_path, to_dev

    K, N, r = 2048, 1032, 16
    w, x, a, b, dy = case_inputs(M, K, N, r, seed=M + grp + len(fmt))
    t32 = torch.from_numpy(w).to(cuda)
    if fmt == "int4":
        wq = D.quantize_int4(t32, grp)
        p, sc = O.quantize_int4_packed(w, grp)
        wdq = O.dequant_int4(p, sc, K, grp)
    else:
        wq = D.quantize_int8(t32, grp)
        q, sc = O.quantize(w, grp, 127)
        wdq = O.dequant_q(q, sc, grp)
    assert np.array_equal(D.dequant(wq).cpu().numpy(), wdq), "dequantized weight differs from the oracle"
    xd, ad, bd, dyd = (to_dev(v, cuda) for v in (x, a, b, dy))
    s = 16.0 / r
    with gemm_path(path):
        y, t = D.lora_fwd(xd, wq, ad, bd, s)
        dx, da, db = D.lora_bwd(xd, dyd, wq, ad, bd, s, t)
    D.sync()
    W = torch.from_numpy(wdq).to(cuda)
    xf, af, bf, dyf = xd.float(), ad.float(), bd.float(), dyd.float()
    tb = (s * xf @ af).to(torch.bfloat16).float()
    u = (s * dyf @ bf.t()).to(torch.bfloat16).float()
    check("t", t, (s * xf @ af).cpu().numpy())
    check("y", y, (xf @ W.t() + tb @ bf).cpu().numpy())
    check("dx", dx, (dyf @ W + u @ af.t()).cpu().numpy())
    check("dA", da, (xf.t() @ u).cpu().numpy())
    check("dB", db, (tb.t() @ dyf).cpu().numpy())


@pytest.mark.parametrize("path", ["mid64", "mid128", "mid64s", "mid128s", "large"])
@pytest.mark.parametrize("fmt", FORMATS)
def test_mid_paths_repeat_bit_identical(cuda, fmt, path):
    """The mid-size tiles' pipelines count their copies per stage (one load
    fewer per stage in the fp8 forward, which loads no scales in its loop):
    a miscounted wait lets a wavefront read a stage before its copy lands,
    which shows up in some calls and not others. Forward and backward on
    every mid-size path and format, at a ragged token count (200: three full
    64-token tiles and 8 tokens), five times over: within the tolerance and
    bit-identical across the repeats. "large" at this token count is the
    256-token tiles split in depth, with their partials summed in range
    order by k_split_reduce."""
    M, K, N, r = 200, 3072, 3072, 16
    g = torch.Generator(device=cuda).manual_seed(23)
    w = torch.randn(N, K, device=cuda, generator=g) * 0.02
    wq = _quantize(w, fmt, 64)
    W = D.dequant(wq).float()
    x = torch.randn(M, K, device=cuda, generator=g).to(torch.bfloat16)
    a = ((torch.rand(K, r, device=cuda, generator=g) * 2 - 1) / K ** 0.5).to(torch.bfloat16)
    b = (torch.randn(r, N, device=cuda, generator=g) * 1e-1).to(torch.bfloat16)
    dy = torch.randn(M, N, device=cuda, generator=g).to(torch.bfloat16)
    s = 1.0
    from gpu_helpers import gemm_path

    runs = []
    with gemm_path(path):
        for _ in range(5):
            y, t = D.lora_fwd(x, wq, a, b, s)
            runs.append((y, t) + D.lora_bwd(x, dy, wq, a, b, s, t))
    D.sync()
    xf, af, bf, dyf = x.float(), a.float(), b.float(), dy.float()
    tb = (s * xf @ af).to(torch.bfloat16).float()
    u = (s * dyf @ bf.t()).to(torch.bfloat16).float()
    ref = (xf @ W.t() + tb @ bf, s * xf @ af, dyf @ W + u @ af.t(), xf.t() @ u, tb.t() @ dyf)
    names = ("y", "t", "dx", "dA", "dB")
    for name, got, want in zip(names, runs[0], ref):
        check(f"{name} {path}", got, want.cpu().numpy())
    for i, run in enumerate(runs[1:], 1):
        for name, first, again in zip(names, runs[0], run):
            assert torch.equal(first, again), f"{path} {fmt}: {name} of call {i} differs from call 0"
