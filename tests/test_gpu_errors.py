"""Failure handling of the C ABI on the GPU, each condition forced from the
host so that every kernel still ends normally:

- a few-token epilogue, or a mid-size tile of rank 16, whose bounded wait
  for t (u) runs out (the test hook makes it wait for a stamp that is never
  published, 16 polls): the outputs it owns are NaN, lrq_sync reports the flag once, then clears it
  and resets the counters, and the next calls are exact again;
- a LoRA call past LRQ_MAX_LORA_TOKENS is refused before any launch, and
  one at the limit runs;
- a workspace that grows after a graph was captured on the context keeps
  the old allocation: the graph replays bit-identically to the eager call."""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import case_inputs, check, to_dev
from loractl_amd import _lib as L
from loractl_amd import device as D

pytestmark = pytest.mark.gpu


def _weight(cuda, w, group=64):
    return D.compute_weight(D.quantize_int4(torch.from_numpy(w).to(cuda), group))


@pytest.mark.parametrize(
    "M,K,N,path",
    [(4, 3072, 12288, "planned"), (4, 1024, 4096, "planned"), (192, 1024, 1536, "mid64"), (256, 1152, 1024, "mid128"),
     (200, 3072, 2560, "mid64s")],
    ids=["whole-depth", "splits", "mid64-fold", "mid128-fold", "mid64-ranges-fold"],
)
def test_few_token_wait_timeout_is_reported_and_cleared(cuda, M, K, N, path):
    r = 16
    w, x, a, b, dy = case_inputs(M, K, N, r, seed=7)
    wq = _weight(cuda, w)
    xd, ad, bd, dyd = (to_dev(v, cuda) for v in (x, a, b, dy))
    y0, t0 = D.lora_fwd(xd, wq, ad, bd, 1.0)
    dx0, da0, db0 = D.lora_bwd(xd, dyd, wq, ad, bd, 1.0, t0)
    D.sync()
    D.debug_gemm_path(path)
    D.debug_force_wait_timeout(True)
    try:
        print(f"forced timeout M={M} K={K} N={N} {path}: forward", flush=True)
        y1, _ = D.lora_fwd(xd, wq, ad, bd, 1.0)
        print(f"forced timeout M={M} K={K} N={N} {path}: backward", flush=True)
        dx1, da1, _ = D.lora_bwd(xd, dyd, wq, ad, bd, 1.0, t0)
    finally:
        D.debug_force_wait_timeout(False)
        D.debug_gemm_path("planned")
    with pytest.raises(L.LrqError, match="gave up waiting"):
        D.sync()
    assert bool(torch.isnan(y1.float()).all()) and bool(torch.isnan(dx1.float()).all())
    if path != "planned":  # dA from the same launch, after its own wait for u
        assert bool(torch.isnan(da1).all())
    D.sync()  # reported once: the flag is clear
    # the counters were reset: the same calls are bit-identical to the first
    y2, t2 = D.lora_fwd(xd, wq, ad, bd, 1.0)
    dx2, da2, db2 = D.lora_bwd(xd, dyd, wq, ad, bd, 1.0, t2)
    D.sync()
    for first, again in ((y0, y2), (t0, t2), (dx0, dx2), (da0, da2), (db0, db2)):
        assert torch.equal(first, again)


def test_lora_token_limit(cuda):
    K, N, r = 64, 64, 4
    rng = np.random.Generator(np.random.PCG64(3))
    wq = _weight(cuda, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    a = to_dev(rng.uniform(-0.1, 0.1, (K, r)).astype(np.float32), cuda)
    b = to_dev((rng.standard_normal((r, N)) * 0.01).astype(np.float32), cuda)
    lim = L.LRQ_MAX_LORA_TOKENS
    x = torch.randn(lim + 16, K, device=cuda).to(torch.bfloat16)
    with pytest.raises(L.LrqError, match="at most 259456 tokens"):
        D.lora_fwd(x, wq, a, b, 1.0)
    with pytest.raises(L.LrqError, match="at most 259456 tokens"):
        D.lora_bwd(x, x, wq, a, b, 1.0, torch.zeros(lim + 16, r, device=cuda, dtype=torch.bfloat16))
    xl = x[:lim].contiguous()
    y, t = D.lora_fwd(xl, wq, a, b, 1.0)
    torch.cuda.synchronize()
    rows = np.array([0, 1, lim // 2, lim - 2, lim - 1])
    ri = torch.from_numpy(rows).to(cuda)
    y_ref, t_ref = O.linear_fwd(xl[ri].float().cpu().numpy(), D.dequant(wq).cpu().numpy(),
                                a.float().cpu().numpy(), b.float().cpu().numpy(), 1.0)
    check("y", y[ri], y_ref)
    check("t", t[ri], t_ref)


def test_workspace_growth_keeps_captured_graphs_valid(cuda):
    M, K, N, r = 300, 1024, 2048, 32
    w, x, a, b, _ = case_inputs(M, K, N, r, seed=11)
    wq = _weight(cuda, w)
    xd, ad, bd = (to_dev(v, cuda) for v in (x, a, b))
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    y = torch.empty((M, N), dtype=torch.bfloat16, device=cuda)
    t = torch.empty((M, r), dtype=torch.bfloat16, device=cuda)
    with torch.cuda.stream(stream):
        D.reserve(M, N, K, r)
        y_eager, t_eager = D.lora_fwd(xd, wq, ad, bd, 1.0)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            D.lora_fwd(xd, wq, ad, bd, 1.0, y=y, t=t)
    torch.cuda.synchronize()
    big = (8192, 12288, 3072, 64)
    for i in range(3):
        y.zero_()
        t.zero_()
        if i == 1:
            # the context of the capture stream grows its workspace: the
            # graph still points at the old one, which must stay allocated
            with torch.cuda.stream(stream):
                D.reserve(*big)
                # eager work in the grown workspace between the replays
                D.lora_fwd(xd, wq, ad, bd, 1.0)
            torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_eager) and torch.equal(t, t_eager), f"replay {i}"


# the kernels each pass launches on the 256-token tiles and on the mid-size
# tiles (which form t, u, dA and dB in the GEMM's own launch)
RELAUNCH_PATHS = {
    "large": (("lora_t", "fwd_main"), ("lora_u", "bwd_dx", "lora_dadb")),
    "mid128": (("fwd_main",), ("bwd_dx",)),
}


@pytest.mark.parametrize("path", sorted(RELAUNCH_PATHS))
def test_profile_relaunch_repeats_the_step_launch(cuda, path):
    """lrq_profile_relaunch repeats a context's last launch of one kernel with
    its arguments: while the buffers it reads (the workspace included) hold
    what they held, the outputs it writes come back bit for bit. A kernel
    the pass's latest call did not launch, or one never launched on the
    context, is refused."""
    M, K, N, r = 300, 1024, 2048, 16
    fwd_k, bwd_k = RELAUNCH_PATHS[path]
    w, x, a, b, dy = case_inputs(M, K, N, r, seed=13)
    wq = _weight(cuda, w)
    xd, ad, bd, dyd = (to_dev(v, cuda) for v in (x, a, b, dy))
    D.debug_gemm_path(path)
    try:
        y, t = D.lora_fwd(xd, wq, ad, bd, 1.0)
        torch.cuda.synchronize()
        y_ref, t_ref = y.clone(), t.clone()
        y.zero_()
        D.profile_relaunch("fwd_main", 2)
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref) and torch.equal(t, t_ref)
        for k in {"lora_t", "fwd_main"} - set(fwd_k):
            with pytest.raises(L.LrqError, match=f"no launch of kernel {k}"):
                D.profile_relaunch(k, 1)
        # the backward reuses the workspace slot of the forward's B^T rows for A
        dx, da, db = D.lora_bwd(xd, dyd, wq, ad, bd, 1.0, t)
        torch.cuda.synchronize()
        ref = [v.clone() for v in (dx, da, db)]
        for v in (dx, da, db):
            v.zero_()
        for k in bwd_k:
            D.profile_relaunch(k, 2)
        torch.cuda.synchronize()
        for got, want in zip((dx, da, db), ref):
            assert torch.equal(got, want)
        for k in {"lora_u", "bwd_dx", "lora_dadb"} - set(bwd_k):
            with pytest.raises(L.LrqError, match=f"no launch of kernel {k}"):
                D.profile_relaunch(k, 1)
    finally:
        D.debug_gemm_path("planned")
    other = torch.cuda.Stream()
    with torch.cuda.stream(other):
        with pytest.raises(L.LrqError, match="no launch of kernel fwd_main"):
            D.profile_relaunch("fwd_main", 1)
