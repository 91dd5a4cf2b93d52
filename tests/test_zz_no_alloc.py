"""lrq_lora_fwd_noalloc against lrq_lora_fwd through the C ABI: the same
kernels on a fixed per-GPU scratch array instead of the context's
workspace, so the outputs must be bit-identical, also when a call follows a
larger one that left its own values in the array."""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import case_inputs, gemm_path, to_dev
from loractl_amd import _lib as L
from loractl_amd import device as D

pytestmark = pytest.mark.gpu


def _case(cuda, M, K, N, r, fmt, seed):
    w, x, a, b, _ = case_inputs(M, K, N, r, seed=seed)
    wt = torch.from_numpy(w).to(cuda)
    wq = {"int4": lambda: D.quantize_int4(wt, 64), "int8": lambda: D.quantize_int8(wt, 64),
          "fp8": lambda: D.quantize_fp8(wt, True)}[fmt]()
    wq = D.compute_weight(wq)
    return wq, to_dev(x, cuda), to_dev(a[:, :r], cuda), to_dev(b[:r], cuda)


def _both(cuda, wq, xb, ab, bb, s):
    M, r = xb.shape[0], ab.shape[1]
    y0, t0 = D.lora_fwd(xb, wq, ab, bb, s)
    y1 = torch.full((M, wq.n), float("nan"), dtype=torch.bfloat16, device=cuda)
    t1 = torch.full((M, r), float("nan"), dtype=torch.bfloat16, device=cuda)
    D.lora_fwd_noalloc(xb, wq, ab, bb, s, y1, t1)
    torch.cuda.synchronize()
    return (y0, t0), (y1, t1)


@pytest.mark.parametrize("fmt", ["int4", "fp8", "int8"])
def test_noalloc_matches_lora_fwd_twice(cuda, fmt):
    """Two calls in a row, the second smaller, through each path (large-m
    GEMM with the LoRA side kernels; few-token stream), each bit-identical
    to lrq_lora_fwd."""
    for (M, K, N, r, seed) in ((600, 1024, 2048, 24, 1), (300, 512, 1024, 16, 2), (9, 512, 256, 8, 3),
                               (3, 256, 128, 4, 4)):
        wq, xb, ab, bb = _case(cuda, M, K, N, r, fmt, seed)
        (y0, t0), (y1, t1) = _both(cuda, wq, xb, ab, bb, 0.75)
        assert torch.equal(y0.view(torch.int16), y1.view(torch.int16)), (fmt, M, K, N, r)
        assert torch.equal(t0.view(torch.int16), t1.view(torch.int16)), (fmt, M, K, N, r)
        assert torch.isfinite(y1.float()).all()


def test_noalloc_mid_depth_ranges(cuda):
    """The mid-size tiles with depth ranges (their f32 accumulators summed in
    the launch, t formed by the fold) on the scratch array: two calls, the
    second smaller, each bit-identical to lrq_lora_fwd."""
    with gemm_path("mid64s"):
        for (M, K, N, r, seed) in ((200, 3072, 2560, 16, 6), (150, 2048, 1024, 8, 7)):
            wq, xb, ab, bb = _case(cuda, M, K, N, r, "int4", seed)
            (y0, t0), (y1, t1) = _both(cuda, wq, xb, ab, bb, 0.75)
            assert torch.equal(y0.view(torch.int16), y1.view(torch.int16)), (M, K, N, r)
            assert torch.equal(t0.view(torch.int16), t1.view(torch.int16)), (M, K, N, r)
            assert torch.isfinite(y1.float()).all()


def test_noalloc_against_the_oracle(cuda):
    """And within the north star's tolerance of the f64 oracle."""
    M, K, N, r = 130, 512, 384, 16
    w, x, a, b, _ = case_inputs(M, K, N, r, seed=7)
    wq = D.compute_weight(D.quantize_int4(torch.from_numpy(w).to(cuda), 64))
    y = torch.empty((M, N), dtype=torch.bfloat16, device=cuda)
    t = torch.empty((M, r), dtype=torch.bfloat16, device=cuda)
    D.lora_fwd_noalloc(to_dev(x, cuda), wq, to_dev(a, cuda), to_dev(b, cuda), 1.0, y, t)
    y_ref, _ = O.linear_fwd(x, D.dequant(wq).cpu().numpy(), a, b, 1.0)
    g = y.float().cpu().numpy()
    assert O.rel_deviation(g, y_ref) <= 1e-2 and O.cosine(g, y_ref) >= 0.999


def test_noalloc_rejects_a_shape_beyond_its_scratch(cuda):
    """256 tokens of a 3072 -> 12288 layer on the large tiles split the GEMM
    depth into ranges whose f32 partials (about 50-60 MB) exceed the 32 MiB
    scratch array; the planned path (the 128-token tiles, no partials) runs
    the same shape in the array, bit-identical to lrq_lora_fwd."""
    M, K, N, r = 256, 3072, 12288, 32
    wq, xb, ab, bb = _case(cuda, M, K, N, r, "int4", 5)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=cuda)
    t = torch.empty((M, r), dtype=torch.bfloat16, device=cuda)
    # the array's first 64 KiB hold the few-token kernels' arrival counters
    with gemm_path("large"):
        with pytest.raises(L.LrqError, match=f"more than its fixed {(32 << 20) - (64 << 10)}"):
            D.lora_fwd_noalloc(xb, wq, ab, bb, 1.0, y, t)
    assert L.LRQ_NOALLOC_SCRATCH_BYTES == 32 << 20
    (y0, t0), (y1, t1) = _both(cuda, wq, xb, ab, bb, 1.0)
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    assert torch.equal(t0.view(torch.int16), t1.view(torch.int16))
