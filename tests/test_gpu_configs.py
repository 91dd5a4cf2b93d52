"""Every site of the benchmark's C3 and C5 configurations on the GPU, through
the C ABI, at full size:

- C3, one synthetic double-stream block's linear set (int4 g64, r = 32):
  QKV 3072 -> 9216, attn-out 3072 -> 3072, MLP 3072 -> 12288 -> 3072,
  adaLN 3072 -> 18432, on the image stream (M = 4096) and the text stream
  (M = 512);
- C5, a Qwen3-style decoder layer (int4 g64, r = 16): q 2560 -> 4096,
  k/v 2560 -> 1024, o 4096 -> 2560, gate/up 2560 -> 9728, down
  9728 -> 2560, at M = 1, 16, 256 and 2048.

At each weight shape the device quantizer and dequantizer are bit-exact
against the oracle (src/quant.rs:74-82, :232). y and dx rows depend only on
the same rows of x and dy, so they are checked against the f64 oracle
(quant.rs:172-178, :221-235 with lora.rs:199-203) on a spread of token
rows; dA and dB reduce over every token and are checked at full size
against fp32 GEMMs over the same bf16 inputs. Tolerance: rel_deviation
<= 1e-2 and cosine >= 0.999 (the north star's bar)."""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import check
from loractl_amd import device as D

pytestmark = pytest.mark.gpu

G = 64
C3_SITES = {"qkv": (3072, 9216), "attn_out": (3072, 3072), "mlp_up": (3072, 12288), "mlp_down": (12288, 3072),
            "adaln": (3072, 18432)}
C5_SITES = {"q": (2560, 4096), "kv": (2560, 1024), "o": (4096, 2560), "gate_up": (2560, 9728),
            "down": (9728, 2560)}

_weights = {}


def _weight(cuda, K, N):
    """The site's weight, quantized on the device and checked bit-exact
    against the oracle once per shape; returns (packed weight, f32 dequant)."""
    key = (K, N)
    if key not in _weights:
        rng = np.random.Generator(np.random.PCG64(K * 7 + N))
        w = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        wq = D.quantize_int4(torch.from_numpy(w).to(cuda), G)
        p_ref, s_ref = O.quantize_int4_packed(w, G)
        assert np.array_equal(wq.data.cpu().numpy(), p_ref), f"packed int4 of [{N}, {K}]"
        assert np.array_equal(wq.scales.cpu().numpy().view(np.uint32), s_ref.view(np.uint32)), f"scales [{N}, {K}]"
        wdq_ref = O.dequant_int4(p_ref, s_ref, K, G)
        wdq = D.dequant(wq)
        assert np.array_equal(wdq.cpu().numpy(), wdq_ref), f"dequant of [{N}, {K}]"
        D.compute_weight(wq)
        _weights.clear()  # keep one shape resident at a time
        _weights[key] = (wq, wdq)
    return _weights[key]


def _site(cuda, K, N, M, r):
    wq, wdq = _weight(cuda, K, N)
    g = torch.Generator(device=cuda).manual_seed(M * 31 + K + N)
    x = torch.randn(M, K, device=cuda, generator=g).to(torch.bfloat16)
    a = ((torch.rand(K, r, device=cuda, generator=g) * 2 - 1) / K ** 0.5).to(torch.bfloat16)
    b = (torch.randn(r, N, device=cuda, generator=g) * 1e-2).to(torch.bfloat16)
    dy = torch.randn(M, N, device=cuda, generator=g).to(torch.bfloat16)
    s = 1.0
    y, t = D.lora_fwd(x, wq, a, b, s)
    dx, da, db = D.lora_bwd(x, dy, wq, a, b, s, t)
    torch.cuda.synchronize()
    # y and dx on a spread of token rows against the f64 oracle
    rows = np.unique(np.linspace(0, M - 1, min(M, 48)).astype(np.int64))
    ri = torch.from_numpy(rows).to(cuda)
    xs = x[ri].float().cpu().numpy()
    dys = dy[ri].float().cpu().numpy()
    af, bf = a.float().cpu().numpy(), b.float().cpu().numpy()
    wdq_np = wdq.cpu().numpy()
    y_ref, t_ref = O.linear_fwd(xs, wdq_np, af, bf, s)
    dx_ref, _, _ = O.linear_bwd(xs, wdq_np, af, bf, s, dys)
    check("y", y[ri], y_ref)
    check("t", t[ri], t_ref)
    check("dx", dx[ri], dx_ref)
    # dA, dB over every token against fp32 GEMMs
    xf, dyf, a32, b32 = x.float(), dy.float(), a.float(), b.float()
    u_ref = (dyf @ b32.t()) * s
    check("dA", da, (xf.t() @ u_ref).cpu().numpy())
    check("dB", db, ((xf @ a32) * s).t().matmul(dyf).cpu().numpy())


@pytest.mark.parametrize("M", [4096, 512], ids=["image", "text"])
@pytest.mark.parametrize("site", list(C3_SITES))
def test_c3_double_stream_block_site(cuda, site, M):
    K, N = C3_SITES[site]
    _site(cuda, K, N, M, 32)


@pytest.mark.parametrize("M", [1, 16, 256, 2048])
@pytest.mark.parametrize("site", list(C5_SITES))
def test_c5_qwen3_site(cuda, site, M):
    K, N = C5_SITES[site]
    _site(cuda, K, N, M, 16)
