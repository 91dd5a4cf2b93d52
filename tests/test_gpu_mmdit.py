"""The block-checkpointed MMDiT step driver (C4) on the GPU, on a small
config: the checkpointed step equals the monolithic one (the analogue of
the reference's tests/block_ckpt.rs:237-284: identical loss, matching
gradients at every adapter site), the fused sites agree with an fp32
reference built from the dequantized weights, and AdamW on the adapters
lowers the flow-matching loss."""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import check
from loractl_amd import device as D
from loractl_amd.mmdit_ops import attn_prep, gated_residual, gelu_tanh, modnorm, rope_tables
from loractl_amd.mmdit import (Mmdit, MmditConfig, build_mmdit_adapters, checkpointed_step, flow_batch,
                               monolithic_step)

pytestmark = pytest.mark.gpu

CFG = MmditConfig(hidden=256, heads=4, mlp_ratio=4, layers=3, patch_dim=16, txt_dim=64, tdim=32, group=64,
                  rank=8, alpha=8.0)
IMG, TXT = 96, 32


def _grads(adapters):
    return [(p.grad.detach().clone() if p.grad is not None else None)
            for d in adapters.deltas for p in (d.lora_a, d.lora_b)]


def _zero(adapters):
    for d in adapters.deltas:
        d.lora_a.grad = None
        d.lora_b.grad = None


def test_checkpointed_step_matches_monolithic(cuda):
    model = Mmdit(CFG, cuda, seed=0)
    ad = build_mmdit_adapters(CFG, cuda, seed=1, b_std=0.02)
    batch = flow_batch(CFG, IMG, TXT, cuda, seed=2)
    loss_m = monolithic_step(model, ad, batch, loss_scale=4.0)
    gm = _grads(ad)
    _zero(ad)
    loss_c = checkpointed_step(model, ad, batch, loss_scale=4.0)
    gc = _grads(ad)
    assert np.isfinite(loss_m) and loss_m > 0
    # the capture forward + head is the monolithic forward's kernel sequence
    assert loss_c == loss_m
    paths = CFG.site_paths()
    assert len(gm) == len(gc) == 2 * len(paths)
    last = CFG.layers - 1
    # the last block's text stream after attention feeds nothing the loss
    # reads (the head takes the image tokens): no gradient in the monolithic
    # graph, exact zeros from the checkpointed sweep (seeded with zeros)
    dead = {f"blocks.{last}.txt.{n}" for n in ("out", "up", "down")}
    for path_i, (a, b) in enumerate(zip(gm, gc)):
        path = paths[path_i // 2]
        if path in dead:
            assert a is None and b is not None and not b.abs().max() > 0, path
            continue
        assert a is not None and b is not None, f"missing gradient at {path}"
        assert a.abs().max() > 0, f"zero gradient at {path}"
        # attention's memory-efficient backward accumulates with atomics:
        # equal up to reduction order
        ref = a.cpu().numpy()
        got = b.cpu().numpy()
        assert O.rel_deviation(got, ref) <= 1e-3 and O.cosine(got, ref) >= 0.99999, path


def test_kept_attention_matches_full_replay(cuda):
    """keep_attention (the capture's attention output and log-sum-exp reused
    by the replay) gives the full replay's loss and, up to the attention
    backward's atomic reduction order, its gradients."""
    model = Mmdit(CFG, cuda, seed=3)
    ad = build_mmdit_adapters(CFG, cuda, seed=4, b_std=0.02)
    batch = flow_batch(CFG, IMG, TXT, cuda, seed=5)
    loss_f = checkpointed_step(model, ad, batch, keep_attention=False)
    gf = _grads(ad)
    _zero(ad)
    loss_k = checkpointed_step(model, ad, batch, keep_attention=True)
    gk = _grads(ad)
    assert loss_k == loss_f
    for path_i, (a, b) in enumerate(zip(gf, gk)):
        path = CFG.site_paths()[path_i // 2]
        assert (a is None) == (b is None), path
        if a is None or not a.abs().max() > 0:
            continue
        got, ref = b.cpu().numpy(), a.cpu().numpy()
        assert O.rel_deviation(got, ref) <= 1e-3 and O.cosine(got, ref) >= 0.99999, path


@pytest.mark.parametrize("L,heads,hd", [(160, 4, 128), (96, 2, 64)])
def test_attention_matches_fp32_reference(cuda, L, heads, hd):
    """The block's attention (torch's memory-efficient kernels called on
    [1, L, heads, d]) against softmax(q k^T / sqrt(d)) v in fp32 with fp32
    autograd: output and dq, dk, dv within bf16 rounding, and a kept
    (output, log-sum-exp) pair gives the same output and gradients."""
    from loractl_amd.mmdit import _Attention

    g = torch.Generator(device=cuda).manual_seed(L + hd)
    q, k, v = (torch.randn(1, L, heads, hd, device=cuda, generator=g).to(torch.bfloat16) for _ in range(3))
    do = torch.randn(1, L, heads, hd, device=cuda, generator=g).to(torch.bfloat16)
    qf, kf, vf = (t.float().detach().requires_grad_() for t in (q, k, v))
    s = torch.einsum("blhd,bmhd->bhlm", qf, kf) / hd ** 0.5
    of = torch.einsum("bhlm,bmhd->blhd", s.softmax(-1), vf)
    of.backward(do.float())
    keep = []
    with torch.no_grad():
        _Attention.apply(q, k, v, None, keep)
    for kept in (None, keep[0]):
        qq, kk, vv = (t.detach().requires_grad_() for t in (q, k, v))
        o = _Attention.apply(qq, kk, vv, kept, None)
        o.backward(do)
        check("o", o, of.detach().cpu().numpy())
        for name, got, ref in (("dq", qq.grad, qf.grad), ("dk", kk.grad, kf.grad), ("dv", vv.grad, vf.grad)):
            check(name, got, ref.cpu().numpy())


def test_fused_sites_match_fp32_dequantized_reference(cuda):
    """The same trunk with every site computed as fp32 x . dq(W)^T + s (x A) B
    from the bit-exact dequantized weight: the fused model's prediction is
    within the north star's tolerance of it."""
    model = Mmdit(CFG, cuda, seed=3)
    ad = build_mmdit_adapters(CFG, cuda, seed=4, b_std=0.05)
    img, txt, t, _ = flow_batch(CFG, IMG, TXT, cuda, seed=5)
    with torch.no_grad():
        pred = model.forward(img, txt, t, ad).float()
        wdq = {p: D.dequant(b.packed) for p, b in model.bases.items()}

        def ref_site(adapters, path, base, x):
            d = adapters.get(path)
            xf = x.float().reshape(-1, x.shape[-1])
            y = xf @ wdq[path].t() + (xf @ d.lora_a.float()) @ d.lora_b.float() * d.scaling
            return y.to(x.dtype).reshape(*x.shape[:-1], -1)

        model.site_fn = ref_site
        ref = model.forward(img, txt, t, ad).float()
    g, r = pred.cpu().numpy(), ref.cpu().numpy()
    assert O.rel_deviation(g, r) <= 1e-2 and O.cosine(g, r) >= 0.999


def test_adamw_on_adapters_lowers_the_loss(cuda):
    model = Mmdit(CFG, cuda, seed=6)
    ad = build_mmdit_adapters(CFG, cuda, seed=7)
    batch = flow_batch(CFG, IMG, TXT, cuda, seed=8)
    opt = torch.optim.AdamW([p for d in ad.deltas for p in (d.lora_a, d.lora_b)], lr=5e-3, eps=1e-5,
                            weight_decay=0.0)
    losses = []
    for _ in range(8):
        opt.zero_grad(set_to_none=True)
        losses.append(checkpointed_step(model, ad, batch))
        opt.step()
    assert all(np.isfinite(losses))
    # B starts at zero (lora.rs:123-137), so the first step only moves B
    assert losses[-1] < losses[0] * 0.97, losses
    assert all(b < a for a, b in zip(losses, losses[1:])), losses


def _prep_reference(qkv_txt, qkv_img, cos, sin, heads, eps):
    """The reference's head split, ZRmsNorm (gain 1) and consecutive-pair
    RoPE (mmdit.rs:307-330, :385-399) in f64 on the joint sequence."""
    x = torch.cat([qkv_txt, qkv_img]).double()
    L, h = x.shape[0], x.shape[1] // 3
    hd = h // heads
    q, k, v = x.view(L, 3, heads, hd).unbind(1)
    c, s = cos.double()[:, None, :], sin.double()[:, None, :]

    def norm_rope(t):
        t = t / torch.sqrt(t.pow(2).mean(-1, keepdim=True) + eps)
        x0, x1 = t[..., 0::2], t[..., 1::2]
        return torch.stack((c * x0 - s * x1, s * x0 + c * x1), dim=-1).reshape(L, heads, hd)

    return norm_rope(q), norm_rope(k), v


@pytest.mark.parametrize("lt,li,heads,hd", [(37, 91, 4, 128), (5, 128, 3, 64), (0, 64, 2, 128), (16, 0, 2, 64)])
def test_attn_prep_matches_reference(cuda, lt, li, heads, hd):
    """q, k, v and the gradient of the fused attention-input kernel against
    the f64 reference and its autograd, on ragged streams (one may be
    empty). Forward: within bf16 rounding of the reference; v bit-exact.
    Backward: within bf16 rounding plus 1e-4 of the largest entry."""
    g = torch.Generator(device=cuda).manual_seed(lt * 1000 + li + hd)
    h = heads * hd
    # per-head scales far from 1 so the normalisation matters
    scale = torch.rand(1, 3 * h, device=cuda, generator=g) * 4 + 0.1
    qt = (torch.randn(lt, 3 * h, device=cuda, generator=g) * scale).to(torch.bfloat16)
    qi = (torch.randn(li, 3 * h, device=cuda, generator=g) * scale).to(torch.bfloat16)
    cos, sin = rope_tables(lt + li, hd, cuda)
    eps = 1e-5
    qt.requires_grad_(True)
    qi.requires_grad_(True)
    q, k, v = attn_prep(qt, qi, (cos, sin), heads, eps)
    ref = _prep_reference(qt.detach(), qi.detach(), cos, sin, heads, eps)
    for got, want in zip((q, k), ref[:2]):
        err = (got.double() - want).abs()
        assert bool((err <= want.abs() * 2.0 ** -8 + 1e-6).all()), err.max().item()
    assert torch.equal(v, ref[2].to(torch.bfloat16))
    dq, dk, dv = (torch.randn(lt + li, heads, hd, device=cuda, generator=g).to(torch.bfloat16) for _ in range(3))
    torch.autograd.backward([q, k, v], [dq, dk, dv])
    xt = qt.detach().double().requires_grad_(True)
    xi = qi.detach().double().requires_grad_(True)
    rq, rk, rv = _prep_reference(xt, xi, cos, sin, heads, eps)
    torch.autograd.backward([rq, rk, rv], [dq.double(), dk.double(), dv.double()])
    for got, want in ((qt.grad, xt.grad), (qi.grad, xi.grad)):
        if want.numel() == 0:
            continue
        err = (got.double() - want).abs()
        tol = want.abs() * 2.0 ** -8 + 1e-4 * want.abs().max()
        assert bool((err <= tol).all()), (err - tol).max().item()


def test_rope_tables_closed_form(cuda):
    """Position 0 turns nothing; pair 0 turns by the position in radians; the
    last pair of head_dim 128 by p * 10000^(-126/128)."""
    cos, sin = rope_tables(4096, 128, cuda)
    assert torch.equal(cos[0], torch.ones(64, device=cuda)) and torch.equal(sin[0], torch.zeros(64, device=cuda))
    p = torch.arange(4096, dtype=torch.float64)
    assert torch.allclose(cos[:, 0].double().cpu(), torch.cos(p), atol=1e-7)
    assert torch.allclose(sin[:, 63].double().cpu(), torch.sin(p * 10000.0 ** (-126 / 128)), atol=1e-7)


def _close(got, want, rtol, atol_frac):
    err = (got.double() - want).abs()
    tol = want.abs() * rtol + atol_frac * want.abs().max()
    assert bool((err <= tol).all()), (err - tol).max().item()


@pytest.mark.parametrize("rows,h", [(37, 256), (1000, 3072), (5, 4096), (4096, 3072)])
def test_modnorm_and_gated_residual_match_reference(cuda, rows, h):
    """The modulated RMSNorm ((scale + 1) x / sqrt(mean(x^2) + eps) + shift,
    mmdit.rs:857-870) and the gated residual x + gate o, each against its
    f64 formula and autograd: outputs, dx and d_o within bf16 rounding, the
    column-summed vector gradients within bf16 rounding plus 1e-3 of the
    largest entry; the column sums are bitwise reproducible."""
    g = torch.Generator(device=cuda).manual_seed(rows + h)
    x = (torch.randn(rows, h, device=cuda, generator=g) * 3).to(torch.bfloat16)
    sc = (torch.randn(1, h, device=cuda, generator=g) * 0.5).to(torch.bfloat16)
    sh = (torch.randn(1, h, device=cuda, generator=g) * 0.5).to(torch.bfloat16)
    gt = (torch.randn(1, h, device=cuda, generator=g)).to(torch.bfloat16)
    o = torch.randn(rows, h, device=cuda, generator=g).to(torch.bfloat16)
    dh = torch.randn(rows, h, device=cuda, generator=g).to(torch.bfloat16)
    dy = torch.randn(rows, h, device=cuda, generator=g).to(torch.bfloat16)
    eps = 1e-5

    def norm_grads():
        ls = [t.detach().clone().requires_grad_(True) for t in (x, sc, sh)]
        out = modnorm(*ls, eps)
        out.backward(dh)
        return out.detach(), [t.grad for t in ls]

    def res_grads():
        ls = [t.detach().clone().requires_grad_(True) for t in (x, gt, o)]
        out = gated_residual(*ls)
        out.backward(dy)
        return out.detach(), [t.grad for t in ls]

    hh, (dx, dsc, dsh) = norm_grads()
    xd, scd, shd = (t.double().requires_grad_(True) for t in (x, sc, sh))
    hr = (scd + 1) * xd / torch.sqrt(xd.pow(2).mean(-1, keepdim=True) + eps) + shd
    hr.backward(dh.double())
    _close(hh, hr.detach(), 2.0 ** -8, 1e-6)
    _close(dx, xd.grad, 2.0 ** -8, 1e-4)
    _close(dsc, scd.grad, 2.0 ** -7, 1e-3)
    _close(dsh, shd.grad, 2.0 ** -7, 1e-3)

    y, (gx, dgt, do) = res_grads()
    xr, gd, od = (t.double().requires_grad_(True) for t in (x, gt, o))
    yr = xr + gd * od
    yr.backward(dy.double())
    _close(y, yr.detach(), 2.0 ** -8, 1e-6)
    assert torch.equal(gx, dy)
    _close(do, od.grad, 2.0 ** -8, 1e-6)
    _close(dgt, gd.grad, 2.0 ** -7, 1e-3)

    # again: the same bits
    for a, b in zip([hh, dx, dsc, dsh, y, dgt, do], [*(lambda r: [r[0], *r[1]])(norm_grads()),
                                                   *(lambda r: [r[0], r[1][1], r[1][2]])(res_grads())]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("n", [64, 4096 * 24, 512 * 12288])
def test_gelu_tanh_matches_reference(cuda, n):
    """The MLP's GELU (forward and gradient kernels) against the f64 formula
    u (1 + tanh(sqrt(2/pi) (u + 0.044715 u^3))) / 2 and its autograd within
    bf16 rounding, against torch's F.gelu(approximate="tanh") on the same
    bf16 input within one bf16 ulp (plus 1e-5 where torch's f32 1 + tanh(z)
    cancels, u below about -4; the kernel's u * sigmoid(2z) does not), and
    at zeros and saturation (finite, exact limits)."""
    import torch.nn.functional as F

    g = torch.Generator(device=cuda).manual_seed(n)
    u = (torch.randn(n, device=cuda, generator=g) * 3).to(torch.bfloat16)
    dg = torch.randn(n, device=cuda, generator=g).to(torch.bfloat16)
    ul = u.clone().requires_grad_(True)
    out = gelu_tanh(ul)
    out.backward(dg)
    ud = u.double().requires_grad_(True)
    ref = 0.5 * ud * (1 + torch.tanh((2 / np.pi) ** 0.5 * (ud + 0.044715 * ud ** 3)))
    ref.backward(dg.double())
    _close(out, ref.detach(), 2.0 ** -8, 1e-6)
    _close(ul.grad, ud.grad, 2.0 ** -8, 1e-4)
    tg = F.gelu(u.float(), approximate="tanh").to(torch.bfloat16).float()
    assert bool(((out.float() - tg).abs() <= 2.0 ** -7 * tg.abs() + 1e-5).all())
    ext = torch.tensor([0.0, -0.0, 30.0, -30.0, 1e20, -1e20, 3e38, -3e38], device=cuda).to(torch.bfloat16)
    e = ext.clone().requires_grad_(True)
    o = gelu_tanh(e)
    o.backward(torch.ones_like(e))
    assert torch.equal(o.float().cpu(), torch.tensor([0.0, 0.0, 30.0, 0.0, 0.0, 0.0, 0.0, 0.0]) +
                       torch.where(ext.float().cpu() > 1e19, ext.float().cpu(), torch.zeros(8)))
    assert torch.equal(e.grad.float().cpu(), torch.tensor([0.5, 0.5, 1.0, 0.0, 1.0, 0.0, 1.0, 0.0]))
