"""Two streams at once, and captured graphs replayed on new inputs.

The Python layer keeps one library context per (device, stream), each with
its own workspace and counter area (the few-token, fold and side kernels'
arrival counters, epochs and ready flags live there). Calls on two torch
streams then run concurrently on the GPU; these tests check that nothing
is shared between them by accident: every path (few-token, mid-size with
its in-launch folds, large tiles with the separate side launches), forward
and backward, issued alternately on two streams without waits between
them, gives results bit-identical to the same calls made one at a time.
"""

import pytest
import torch

from loractl_amd import device as D

pytestmark = pytest.mark.gpu

# (m, k, n, r): few-token, mid-size (the fold and the in-launch dA / dB),
# large tiles (separate t, u and dA / dB launches)
SHAPES = [(8, 1024, 2048, 16), (300, 1024, 1032, 32), (2048, 1024, 2048, 32), (200, 2048, 1536, 24)]


def _inputs(cuda, m, k, n, r, seed):
    g = torch.Generator(device=cuda).manual_seed(seed)
    wq = D.compute_weight(D.quantize_int4(torch.randn(n, k, device=cuda, generator=g) * 0.02, 64))
    x = torch.randn(m, k, device=cuda, generator=g).to(torch.bfloat16)
    a = ((torch.rand(k, r, device=cuda, generator=g) * 2 - 1) / k ** 0.5).to(torch.bfloat16)
    b = (torch.randn(r, n, device=cuda, generator=g) * 1e-1).to(torch.bfloat16)
    dy = torch.randn(m, n, device=cuda, generator=g).to(torch.bfloat16)
    return wq, x, a, b, dy


def _site(wq, x, a, b, dy, r):
    s = 16.0 / r
    y, t = D.lora_fwd(x, wq, a, b, s)
    dx, da, db = D.lora_bwd(x, dy, wq, a, b, s, t)
    return y, t, dx, da, db


def test_two_streams_match_one_at_a_time(cuda):
    cases = [(_inputs(cuda, *shp, seed=i + 1), shp[3]) for i, shp in enumerate(SHAPES)]
    ref = [_site(*inp, r) for inp, r in cases]
    torch.cuda.synchronize()
    D.sync()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    outs = []
    for rep in range(3):
        for i, (inp, r) in enumerate(cases):
            for k, st in enumerate(streams):
                with torch.cuda.stream(st):
                    outs.append((i, rep, k, _site(*inp, r)))
    for st in streams:
        with torch.cuda.stream(st):
            D.sync()
    torch.cuda.synchronize()
    names = ("y", "t", "dx", "dA", "dB")
    for i, rep, k, got in outs:
        for name, g_, r_ in zip(names, got, ref[i]):
            assert torch.equal(g_, r_), f"shape {SHAPES[i]} repeat {rep} stream {k}: {name} differs"


@pytest.mark.parametrize("m,k,n,r", SHAPES, ids=["few-token", "mid", "large", "mid-r24"])
def test_captured_forward_backward_replays(cuda, m, k, n, r):
    """A site's forward and backward captured into one graph (the library
    issues only kernel launches there: the workspace is reserved first and
    the counters are kept zero by the kernels, no memset), replayed four
    times with new x and dy written in place before each replay and eager
    calls on another stream in between. Every replay is bit-identical to
    eager calls on the same inputs: no launch carries state (counters,
    epochs, ready flags) from one replay into the next."""
    wq, x, a, b, dy = _inputs(cuda, m, k, n, r, seed=7)
    s = 16.0 / r
    bf = torch.bfloat16
    y, t = torch.empty(m, n, dtype=bf, device=cuda), torch.empty(m, r, dtype=bf, device=cuda)
    dx = torch.empty(m, k, dtype=bf, device=cuda)
    da = torch.empty(k, r, dtype=torch.float32, device=cuda)
    db = torch.empty(r, n, dtype=torch.float32, device=cuda)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        D.reserve(m, n, k, r)
        _site(wq, x, a, b, dy, r)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            D.lora_fwd(x, wq, a, b, s, y=y, t=t)
            D.lora_bwd(x, dy, wq, a, b, s, t, out=(dx, da, db))
    torch.cuda.synchronize()
    g = torch.Generator(device=cuda).manual_seed(99)
    for i in range(4):
        x.copy_(torch.randn(m, k, device=cuda, generator=g).to(bf))
        dy.copy_(torch.randn(m, n, device=cuda, generator=g).to(bf))
        ref = _site(wq, x, a, b, dy, r)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, want in zip(("y", "t", "dx", "dA", "dB"), (y, t, dx, da, db), ref):
            assert torch.equal(got, want), f"replay {i}: {name} differs from the eager call"
    with torch.cuda.stream(stream):
        D.sync()
    D.sync()
