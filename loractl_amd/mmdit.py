"""A synthetic double-stream MMDiT and its block-checkpointed LoRA training
step, with every block linear running through the fused quantized LoRA op.

This is the driver of the benchmark's C4 configuration ("MMDiT train
steps/s"): 24 FLUX-style double-stream blocks, hidden 3072, 24 heads of
128, MLP ratio 4, an int4 group-64 frozen base and LoRA r = 32 on every
block linear, AdamW on the adapters only, batch 1 of 4096 image tokens (a
64 x 64 latent in 2 x 2 patches) and 512 text tokens, flow-matching MSE.
The reference's own model is single-stream (``mmdit.rs``); only the linear
sites and the step structure carry over:

- sites: each stream of each block has five quantized linears, all
  injectable (``blocks.{i}.{img,txt}.{mod,qkv,out,up,down}``), run through
  ``site()`` (``mmdit.rs:526-536``), so a registered delta fuses with its
  base in one op;
- ``checkpointed_step`` follows ``block_ckpt.rs:103-207``: a no-grad
  capture forward stores each block's inputs, a small head graph gives the
  loss and the trunk cotangent (the loss scale folded in once), then each
  block is replayed last to first on its own graph, seeded by the incoming
  cotangent, its adapter gradients accumulating on the deltas' parameters;
  the per-site cost is two fused forwards and one fused backward. The
  capture may also keep each block's attention output and log-sum-exp
  (``keep_attention``, about 29 MB per block at 4608 tokens): the replay
  then recomputes q, k and v (its backward needs them) but not the
  attention forward, and the gradients are those of the full replay;
- the flow-matching target follows ``flow.rs``: ``x_t = (1 - t) x0 + t eps``,
  target ``v = eps - x0`` (t = 0 is data), loss ``mean((pred - v)^2)``.

Each stream's pre- and post-attention norms are the reference block's
modulated norm, ``(scale + 1) * ZRmsNorm(x) + shift`` (``mmdit.rs:857-870``,
the norm's gain its frozen zero parameter + 1), and its residuals are gated,
``x + gate * branch``; both run as HIP kernels (``modnorm``,
``gated_residual``), as do the MLP's GELU (``gelu_tanh``) and the attention
input (``attn_prep``: head split, per-head RMSNorm of q and k, RoPE over
the joint text-then-image sequence). The rest around the fused sites is
PyTorch-ROCm (attention through torch's memory-efficient kernels, the
frozen bf16 embedders and head linears): outside the quantized-linear path.
The modulation (adaLN) linears take the conditioning vector, one row per
batch element, as in FLUX.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

from . import device as D
from .adapters import LoraAdapters, QuantLinear, site
from .mmdit_ops import attn_prep, gated_residual, gelu_tanh, modnorm, rope_tables
from .lora import LoraDelta

STREAMS = ("img", "txt")
SITE_NAMES = ("mod", "qkv", "out", "up", "down")


class _Attention(torch.autograd.Function):
    """softmax(q k^T / sqrt(d)) v over the joint sequence with torch's
    memory-efficient attention kernels (``aten::_efficient_attention_forward``
    and ``_backward``) on [1, L, heads, d], the layout they take and the one
    ``attn_prep`` writes. ``kept`` is (out, log-sum-exp) of an earlier forward
    of the same q, k, v, which the call returns instead of running the
    forward again; ``keep`` (a list) receives them from a forward that runs."""

    @staticmethod
    def forward(ctx, q, k, v, kept, keep):
        grad = any(ctx.needs_input_grad[:3])
        if kept is None:
            out, lse = torch.ops.aten._efficient_attention_forward(q, k, v, None, None, None, None, None, 0.0, 0,
                                                                    grad or keep is not None)[:2]
            if keep is not None:
                keep.append((out, lse))
        else:
            out, lse = kept
        if grad:
            ctx.save_for_backward(q, k, v, out, lse)
        return out.detach()

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        # no dropout: the philox state is not read
        zero = torch.zeros((), dtype=torch.int64)
        dq, dk, dv, _ = torch.ops.aten._efficient_attention_backward(
            dout.contiguous(), q, k, v, None, out, None, None, q.shape[1], k.shape[1], lse, 0.0, zero, zero, 0,
            False)
        return dq, dk, dv, None, None


@dataclass
class MmditConfig:
    hidden: int = 3072
    heads: int = 24
    mlp_ratio: int = 4
    layers: int = 24
    patch_dim: int = 64      # 16 latent channels x 2 x 2 patch
    txt_dim: int = 4096      # text-encoder width of the conditioning tokens
    tdim: int = 256          # sinusoidal timestep embedding width
    group: int = 64          # int4 quant block
    rank: int = 32
    alpha: float = 32.0

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    def site_shapes(self) -> Dict[str, Tuple[int, int]]:
        """(d_in, d_out) of each site of one stream of one block."""
        h = self.hidden
        return {"mod": (h, 6 * h), "qkv": (h, 3 * h), "out": (h, h), "up": (h, self.mlp_ratio * h),
                "down": (self.mlp_ratio * h, h)}

    def site_paths(self) -> List[str]:
        return [f"blocks.{i}.{s}.{n}" for i in range(self.layers) for s in STREAMS for n in SITE_NAMES]


def timestep_embedding(t: torch.Tensor, dim: int, max_period: float = 10000.0) -> torch.Tensor:
    """Sinusoidal embedding of ``1000 t`` (the FLUX/SD3 convention), [B, dim] f32."""
    half = dim // 2
    freqs = torch.exp(-math.log(max_period) * torch.arange(half, dtype=torch.float32, device=t.device) / half)
    args = (t.float() * 1000.0)[:, None] * freqs[None]
    return torch.cat([torch.cos(args), torch.sin(args)], dim=-1)


@dataclass
class Capture:
    """What the capture forward keeps (``mmdit.rs:1474-1507``): each block's
    input streams, the conditioning vector, RoPE tables and the trunk output."""

    block_inputs: List[Tuple[torch.Tensor, torch.Tensor]] = field(default_factory=list)
    vec: Optional[torch.Tensor] = None
    rope: Optional[Tuple[torch.Tensor, torch.Tensor]] = None
    attention: list = field(default_factory=list)  # per block (out, log-sum-exp), when kept
    x_img: Optional[torch.Tensor] = None
    x_txt: Optional[torch.Tensor] = None


class Mmdit:
    """The frozen synthetic double-stream denoiser: int4 blocked base weights
    for every block linear, bf16 plain embedders and head."""

    def __init__(self, cfg: MmditConfig, device, seed: int = 0, w_std: float = 0.02):
        self.cfg = cfg
        self.device = torch.device(device)
        self.site_fn = site  # how a block runs its linears: site() (a test may substitute a reference)
        g = torch.Generator(device=self.device).manual_seed(seed)
        h = cfg.hidden

        def plain(d_in, d_out):
            w = (torch.randn(d_out, d_in, device=self.device, generator=g) / math.sqrt(d_in)).to(torch.bfloat16)
            return w, torch.zeros(d_out, device=self.device, dtype=torch.bfloat16)

        self.img_in = plain(cfg.patch_dim, h)
        self.txt_in = plain(cfg.txt_dim, h)
        self.t_in = plain(cfg.tdim, h)
        self.t_out = plain(h, h)
        self.final_mod = plain(h, 2 * h)
        self.final = plain(h, cfg.patch_dim)
        self.bases: Dict[str, QuantLinear] = {}
        for i in range(cfg.layers):
            for s in STREAMS:
                for n, (d_in, d_out) in cfg.site_shapes().items():
                    w = torch.randn(d_out, d_in, device=self.device, generator=g) * w_std
                    self.bases[f"blocks.{i}.{s}.{n}"] = QuantLinear([D.quantize_int4(w, cfg.group)])
                    del w

    # ------------------------------------------------------------ pieces
    @staticmethod
    def _linear(x, wb):
        return F.linear(x, wb[0], wb[1])

    def conditioning(self, t: torch.Tensor) -> torch.Tensor:
        """vec [B, hidden] bf16 from the timestep (frozen)."""
        e = timestep_embedding(t, self.cfg.tdim).to(torch.bfloat16)
        return self._linear(F.silu(self._linear(e, self.t_in)), self.t_out)

    def embed(self, img: torch.Tensor, txt: torch.Tensor):
        return self._linear(img, self.img_in), self._linear(txt, self.txt_in)

    def head(self, x_img: torch.Tensor, vec: torch.Tensor) -> torch.Tensor:
        """The output head (``mmdit.rs:885-887``): modulated norm, then the
        linear back to patches."""
        scale, shift = self._linear(F.silu(vec), self.final_mod).chunk(2, dim=-1)
        return self._linear(modnorm(x_img, scale.contiguous(), shift.contiguous()), self.final)

    def block(self, i: int, x_img: torch.Tensor, x_txt: torch.Tensor, vec: torch.Tensor, rope,
              adapters: Optional[LoraAdapters], kept=None, keep: Optional[list] = None):
        """One double-stream block on [L_img, H] and [L_txt, H] bf16 streams
        (``kept`` / ``keep``: the attention output and log-sum-exp to reuse, or
        a list to append them to; see ``_Attention``)."""
        cfg = self.cfg
        H, nh, hd = cfg.hidden, cfg.heads, cfg.head_dim
        p = f"blocks.{i}"
        site = self.site_fn
        cvec = F.silu(vec)
        mods, qkvs = {}, []
        for s, x in (("txt", x_txt), ("img", x_img)):  # text tokens first in the joint sequence
            m = site(adapters, f"{p}.{s}.mod", self.bases[f"{p}.{s}.mod"], cvec)
            mods[s] = m.chunk(6, dim=-1)
            sh1, sc1 = mods[s][0], mods[s][1]
            h = modnorm(x, sc1, sh1)
            qkvs.append(site(adapters, f"{p}.{s}.qkv", self.bases[f"{p}.{s}.qkv"], h))
        # q, k, v [L, nh, hd] over the joint sequence, q and k RMS-normalised
        # per head and rotated (one kernel over both streams' rows)
        q, k, v = attn_prep(qkvs[0], qkvs[1], rope, nh)
        o = _Attention.apply(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), kept, keep)
        o = o.reshape(-1, H)  # [L, H]
        lt = x_txt.shape[0]
        outs = {}
        for s, x, oo in (("txt", x_txt, o[:lt]), ("img", x_img, o[lt:])):
            _, _, g1, sh2, sc2, g2 = mods[s]
            x = gated_residual(x, g1, site(adapters, f"{p}.{s}.out", self.bases[f"{p}.{s}.out"], oo))
            h2 = modnorm(x, sc2, sh2)
            up = site(adapters, f"{p}.{s}.up", self.bases[f"{p}.{s}.up"], h2)
            x = gated_residual(x, g2, site(adapters, f"{p}.{s}.down", self.bases[f"{p}.{s}.down"],
                                           gelu_tanh(up)))
            outs[s] = x
        return outs["img"], outs["txt"]

    # ------------------------------------------------------------ passes
    def prepare(self, img, txt, t):
        vec = self.conditioning(t)
        x_img, x_txt = self.embed(img, txt)
        rope = rope_tables(x_img.shape[0] + x_txt.shape[0], self.cfg.head_dim, self.device)
        return x_img, x_txt, vec, rope

    def forward(self, img, txt, t, adapters) -> torch.Tensor:
        """The monolithic forward (autograd through every block)."""
        with torch.no_grad():
            x_img, x_txt, vec, rope = self.prepare(img, txt, t)
        for i in range(self.cfg.layers):
            x_img, x_txt = self.block(i, x_img, x_txt, vec, rope, adapters)
        return self.head(x_img, vec)

    @torch.no_grad()
    def forward_capture(self, img, txt, t, adapters, keep_attention: bool = False) -> Capture:
        """Pre-trunk and trunk with no graph, keeping each block's inputs
        (``mmdit.rs:1474-1507``) and, with ``keep_attention``, each block's
        attention output and log-sum-exp."""
        x_img, x_txt, vec, rope = self.prepare(img, txt, t)
        cap = Capture(vec=vec, rope=rope)
        keep = cap.attention if keep_attention else None
        for i in range(self.cfg.layers):
            cap.block_inputs.append((x_img, x_txt))
            x_img, x_txt = self.block(i, x_img, x_txt, vec, rope, adapters, keep=keep)
        cap.x_img, cap.x_txt = x_img, x_txt
        return cap


def build_mmdit_adapters(cfg: MmditConfig, device, seed: int = 1, b_std: float = 0.0) -> LoraAdapters:
    """A delta on every block site (rank/alpha from the config); A is
    Kaiming-uniform and B zero as ``lora.rs:123-137`` (``b_std`` > 0 draws B
    from N(0, b_std) so a fresh set is not a no-op)."""
    torch.manual_seed(seed)
    deltas, targets = [], []
    shapes = cfg.site_shapes()
    for path in cfg.site_paths():
        d_in, d_out = shapes[path.rsplit(".", 1)[1]]
        d = LoraDelta(d_in, d_out, cfg.rank, cfg.alpha, device=device)
        if b_std > 0:
            with torch.no_grad():
                d.lora_b.normal_(0.0, b_std)
        deltas.append(d)
        targets.append(path)
    return LoraAdapters(deltas, targets)


def flow_batch(cfg: MmditConfig, img_tokens: int, txt_tokens: int, device, seed: int = 2):
    """A synthetic flow-matching batch (``flow.rs``): latent patches x0 and
    text embeddings ~ N(0, 1), t ~ U(0, 1), noise eps; returns
    (x_t bf16, txt bf16, t, target f32) with x_t = (1 - t) x0 + t eps and
    the velocity target v = eps - x0."""
    g = torch.Generator(device=device).manual_seed(seed)
    x0 = torch.randn(img_tokens, cfg.patch_dim, device=device, generator=g)
    eps = torch.randn(img_tokens, cfg.patch_dim, device=device, generator=g)
    txt = torch.randn(txt_tokens, cfg.txt_dim, device=device, generator=g).to(torch.bfloat16)
    t = torch.rand(1, device=device, generator=g)
    x_t = ((1 - t) * x0 + t * eps).to(torch.bfloat16)
    return x_t, txt, t, eps - x0


def flow_loss(pred: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    d = pred.float() - target
    return (d * d).mean()


def monolithic_step(model: Mmdit, adapters: LoraAdapters, batch, loss_scale: float = 1.0) -> float:
    """Loss and adapter gradients (on the deltas' ``.grad``) through one
    autograd graph over the whole trunk."""
    img, txt, t, target = batch
    loss = flow_loss(model.forward(img, txt, t, adapters), target)
    (loss * loss_scale).backward()
    value = float(loss.item())
    D.sync()  # a few-token kernel's device-side failure flag, once per step
    return value


def checkpointed_step(model: Mmdit, adapters: LoraAdapters, batch, loss_scale: float = 1.0,
                      keep_attention: bool = False) -> float:
    """One block-checkpointed step (``block_ckpt.rs:103-207``): capture, head
    graph, reverse per-block replay of the whole block, as the reference
    does. Returns the unscaled loss; adapter gradients accumulate on the
    deltas' ``.grad`` (scaled by ``loss_scale``). ``keep_attention=True``
    instead keeps each block's attention output and log-sum-exp from the
    capture for its replay (memory for time: the replay skips the attention
    forward; the gradients are the same)."""
    with adapters.cached_factors():  # the factors stay fixed through capture and replay
        return _checkpointed_step(model, adapters, batch, loss_scale, keep_attention)


def _checkpointed_step(model: Mmdit, adapters: LoraAdapters, batch, loss_scale: float,
                       keep_attention: bool) -> float:
    img, txt, t, target = batch
    cap = model.forward_capture(img, txt, t, adapters, keep_attention)
    # head graph: trunk output re-tracked, loss scale folded into the seed once
    x_img = cap.x_img.detach().requires_grad_()
    loss = flow_loss(model.head(x_img, cap.vec), target)
    (loss * loss_scale).backward()
    g_img = x_img.grad
    g_txt = torch.zeros_like(cap.x_txt)  # the text stream's final output feeds no loss
    del x_img
    # reverse sweep, one standalone graph per block
    for i in reversed(range(model.cfg.layers)):
        xi, xt = (v.detach().requires_grad_() for v in cap.block_inputs[i])
        kept = cap.attention[i] if keep_attention else None
        oi, ot = model.block(i, xi, xt, cap.vec, cap.rope, adapters, kept=kept)
        torch.autograd.backward([oi, ot], [g_img, g_txt])
        g_img, g_txt = xi.grad, xt.grad
        cap.block_inputs[i] = None  # this block's inputs are done
        if keep_attention:
            cap.attention[i] = None
    value = float(loss.item())
    D.sync()  # a few-token kernel's device-side failure flag, once per step
    return value


def mmdit_step_flops(cfg: MmditConfig, img_tokens: int, txt_tokens: int, batch: int = 1,
                     grad_checkpointing: bool = True, mod_at_stream: bool = False) -> Dict[str, float]:
    """The step work model of ``bench.rs:274-311`` for the double-stream
    trunk: dense block projections at 2 d_in d_out per token (the
    modulation linears at one row per batch element), the two attention
    matmuls at 4 L^2 hidden per block over the joint sequence; a frozen
    base's backward costs one forward and attention's two, and block
    checkpointing replays one more forward (x3 projections, x4 attention).
    The LoRA terms are reported apart (``lora``), as the reference excludes
    them. ``mod_at_stream`` counts the modulation linears at the stream's
    token count instead (a work model that treats them like the other
    projections; this model does not run them that way)."""
    shapes = cfg.site_shapes()
    proj = 0.0
    lora = 0.0
    for s, M in (("img", img_tokens * batch), ("txt", txt_tokens * batch)):
        for n, (k, nn) in shapes.items():
            rows = batch if (n == "mod" and not mod_at_stream) else M
            proj += 2.0 * rows * k * nn
            lora += 2.0 * rows * cfg.rank * (k + nn)
    proj *= cfg.layers
    lora *= cfg.layers
    L = img_tokens + txt_tokens
    attn = 4.0 * L * L * cfg.hidden * batch * cfg.layers
    pp = 3.0 if grad_checkpointing else 2.0
    # LoRA: 2 forwards (1 x 2Mr(K+N)) and a backward of 2 x that with ckpt
    lora_total = lora * (2.0 + 2.0) if grad_checkpointing else lora * 3.0
    return {"proj": proj * pp, "attn": attn * (pp + 1.0), "lora": lora_total,
            "total": proj * pp + attn * (pp + 1.0), "fwd_proj": proj, "fwd_attn": attn}
