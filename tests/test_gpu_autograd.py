"""The torch autograd mirror of the reference seam (QuantBackend,
QuantLinear, site() with LoraAdapters) running on the GPU kernels."""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import check
from loractl_amd.adapters import LoraAdapters, LoraConfig, LoraSite, QuantLinear, TargetSpec, build_adapters, site
from loractl_amd.lora import LoraDelta
from loractl_amd.quant import QuantBackend, QuantValue, quantize_linear_weight, quantize_linear_weight_chunked

pytestmark = pytest.mark.gpu


def test_quant_matmul_t_autograd_grad_x_only(cuda):
    """quant.rs:210-263: y = x . dq^T, grad_x = grad . dq, no weight grad."""
    torch.manual_seed(0)
    w = torch.randn(96, 128, device=cuda) * 0.05
    wq = quantize_linear_weight(w, QuantValue.Q4S, 32)
    wdq = QuantLinear([wq]).dequantized_weight()
    x = torch.randn(40, 128, device=cuda).to(torch.bfloat16).requires_grad_(True)
    y = QuantBackend.quant_matmul_t(x, wq)
    loss = (y.float() * y.float()).sum()
    loss.backward()
    xr = x.detach().float().requires_grad_(True)
    yr = xr @ wdq.t()
    (yr * yr).sum().backward()
    check("y", y, yr.detach().cpu().numpy())
    check("grad_x", x.grad, xr.grad.cpu().numpy())


def test_chunked_quant_linear_equals_whole(cuda):
    """mmdit.rs:483-519: chunks concatenate along d_out; forward bit-identical."""
    torch.manual_seed(1)
    w = torch.randn(96, 64, device=cuda) * 0.1
    whole = QuantLinear([quantize_linear_weight(w, QuantValue.Q4S, 32)])
    chunks = quantize_linear_weight_chunked(w, QuantValue.Q4S, 64 * 4 * 40, 32)
    assert [c.n for c in chunks] == [32, 32, 32]
    chunked = QuantLinear(chunks)
    assert torch.equal(chunked.dequantized_weight(), whole.dequantized_weight())
    x = torch.randn(2, 7, 64, device=cuda).to(torch.bfloat16)
    assert torch.equal(chunked.forward(x), whole.forward(x))
    assert chunked.forward(x).shape == (2, 7, 96)


def test_q8s_chunked_quant_linear_equals_whole(cuda):
    """The Quant::Int8 knob (quant.rs:156-162) through QuantLinear: int8 row
    chunks join to the whole weight bit for bit, and the forward and input
    gradient equal the oracle's on the int8 dequantization."""
    torch.manual_seed(2)
    w = torch.randn(96, 128, device=cuda) * 0.1
    whole = QuantLinear([quantize_linear_weight(w, QuantValue.Q8S, 32)])
    chunked = QuantLinear(quantize_linear_weight_chunked(w, QuantValue.Q8S, 128 * 4 * 40, 32))
    q, sc = O.quantize(w.cpu().numpy(), 32, 127)
    wdq = O.dequant_q(q, sc, 32)
    assert np.array_equal(whole.dequantized_weight().cpu().numpy(), wdq)
    assert torch.equal(chunked.dequantized_weight(), whole.dequantized_weight())
    x = (torch.randn(3, 5, 128, device=cuda) * 0.5).to(torch.bfloat16).requires_grad_(True)
    y = chunked.forward(x)
    assert torch.equal(y, whole.forward(x))
    dy = torch.randn_like(y)
    y.backward(dy)
    xr = x.detach().float().reshape(-1, 128).cpu().numpy()
    check("y", y.reshape(-1, 96), O.linear_fwd(xr, wdq)[0])
    check("grad_x", x.grad.reshape(-1, 128), O.linear_bwd(xr, wdq, None, None, 1.0,
                                                          dy.float().reshape(-1, 96).cpu().numpy())[0])


def test_site_fused_matches_two_step_semantics(cuda):
    """site() with a quantized base and a delta (fused) equals base + delta
    computed from the oracle, and routes gradients to x, A and B only."""
    torch.manual_seed(2)
    d_in, d_out, M = 128, 64, 50
    w = torch.randn(d_out, d_in, device=cuda) * 0.05
    bias = torch.randn(d_out, device=cuda) * 0.1
    base = QuantLinear([quantize_linear_weight(w, QuantValue.Q4S, 64)], bias=bias)
    sites = [LoraSite("blocks.0.attn.wq", d_in, d_out), LoraSite("blocks.0.attn.gate", d_in, d_out)]
    ad = build_adapters(sites, LoraConfig(rank=8, alpha=16.0, targets=[TargetSpec(r"attn\.wq")]), device=cuda)
    delta = ad.get("blocks.0.attn.wq")
    with torch.no_grad():
        delta.lora_b.normal_(0, 0.05)
    x = torch.randn(M, d_in, device=cuda).to(torch.bfloat16).requires_grad_(True)
    y = site(ad, "blocks.0.attn.wq", base, x)
    gy = torch.randn_like(y)
    y.backward(gy)
    # the gate site has no delta: base only, and no LoRA params touched
    y_gate = site(ad, "blocks.0.attn.gate", base, x.detach())
    assert torch.equal(y_gate, base.forward(x.detach()))

    wdq = base.dequantized_weight().cpu().numpy()
    xn = x.detach().float().cpu().numpy()
    an = O.bf16_round(delta.lora_a.detach().cpu().numpy())
    bn = O.bf16_round(delta.lora_b.detach().cpu().numpy())
    dyn = gy.float().cpu().numpy()
    y_ref, _ = O.linear_fwd(xn, wdq, an, bn, delta.scaling, bias=bias.cpu().numpy())
    dx_ref, da_ref, db_ref = O.linear_bwd(xn, wdq, an, bn, delta.scaling, dyn)
    check("y", y, y_ref)
    check("dx", x.grad, dx_ref)
    check("dA", delta.lora_a.grad, da_ref)
    check("dB", delta.lora_b.grad, db_ref)
    assert delta.lora_a.grad.dtype == torch.float32


def test_fused_site_training_step_reduces_loss(cuda):
    """A few SGD steps on the fused site lower an MSE loss (the GPU-smoke
    policy of README.md:294-296: loss decreases)."""
    torch.manual_seed(3)
    d_in, d_out, M = 256, 128, 256
    w = torch.randn(d_out, d_in, device=cuda) * 0.05
    base = QuantLinear([quantize_linear_weight(w, QuantValue.Q4S, 64)])
    delta = LoraDelta(d_in, d_out, 16, 16.0, device=cuda)
    ad = LoraAdapters([delta], ["l"])
    x = torch.randn(M, d_in, device=cuda).to(torch.bfloat16)
    target = torch.randn(M, d_out, device=cuda)
    opt = torch.optim.SGD(delta.parameters(), lr=0.05)
    losses = []
    for _ in range(10):
        opt.zero_grad()
        y = site(ad, "l", base, x)
        loss = ((y.float() - target) ** 2).mean()
        loss.backward()
        opt.step()
        losses.append(loss.item())
    assert losses[-1] < losses[0]
