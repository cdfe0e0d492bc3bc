"""Training-step harness for config 5: a small MLA + MoE language model whose Linear and
expert layers run through the FP8 path.

Test infrastructure, not product code.  The model follows the structure of the
reference's `Cinnamon` (src/model.py:8-146, src/layers.py:14-241, src/attention.py:316-506)
at the sizes of config 5, with three recorded simplifications:

- attention is dense causal with standard RoPE on the decoupled rope channels; the DSA
  indexer and its top-k key mask (src/attention.py:212-314, 379-399) are left out.  The
  attention projections are excluded from FP8 by `convert_to_fp8`'s name rules either way
  ("attn", src/kernels.py:863-867), so the FP8 path sees the same layers;
- the model runs in fp32 (the reference trains under bf16 autocast, src/train.py:344):
  the comparison isolates the FP8 quantization, and fp32 attention avoids torch's bf16
  batched products with transposed right operands, which this GPU pool's operating notes
  report as having faulted its GPUs (not observed here; the bf16-autocast step is untested);
- the DSA KL auxiliary loss is absent with the indexer; the MoE balance loss and the MTP
  loss are kept (src/train.py:355-372).

Two modes share initial weights and data: "fp8" converts the eligible Linears with
`kernels.convert_to_fp8` (src/train.py:696-698) and runs the routed experts through
`layers.GroupedExperts` (FP8 forward and backward); "ref" keeps every layer in fp32 and runs
the routed experts as a per-expert loop (the reference's fallback, src/layers.py:78-87).
"""
from __future__ import annotations

import copy
import math
import time

import torch
import torch.nn as nn
import torch.nn.functional as F


class C5Config:
    d_model = 1024
    n_layers = 8
    vocab_size = 32000
    hidden_dim = 4096      # shared expert hidden; routed hidden = hidden_dim // expert_scale
    expert_scale = 4
    n_heads = 16
    d_ckv = 256
    d_cq = 512
    d_head = 64
    d_v = 64
    d_rope = 64
    n_routed = 16
    n_shared = 1
    top_k = 2
    gamma = 0.001
    balance_alpha = 1e-4
    mtp_depth = 1
    mtp_lambda = 0.3
    rms_eps = 1e-6
    rope_base = 10000.0
    max_seq_len = 1024
    lr = 3e-4
    weight_decay = 0.1
    grad_clip = 1.0

    def __init__(self, **kw):
        for k, v in kw.items():
            if not hasattr(self, k):
                raise AttributeError(k)
            setattr(self, k, v)


class RMSNorm(nn.Module):
    def __init__(self, d, eps):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d))

    def forward(self, x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)).to(x.dtype) * self.weight


def _rope(x, cos, sin):
    """Rotate channel pairs (2i, 2i+1) of x [B, L, H, d] by the position angles."""
    x0, x1 = x[..., 0::2], x[..., 1::2]
    out = torch.stack((x0 * cos - x1 * sin, x0 * sin + x1 * cos), dim=-1)
    return out.flatten(-2)


class MLA(nn.Module):
    """Multi-head latent attention: low-rank query/key-value compression plus decoupled
    rope channels (one shared rope key per position), causal softmax attention."""

    def __init__(self, c: C5Config):
        super().__init__()
        self.h, self.dh, self.dv, self.dr = c.n_heads, c.d_head, c.d_v, c.d_rope
        self.w_dkv = nn.Linear(c.d_model, c.d_ckv, bias=False)
        self.kv_norm = RMSNorm(c.d_ckv, c.rms_eps)
        self.w_uk = nn.Linear(c.d_ckv, c.d_head * c.n_heads, bias=False)
        self.w_uv = nn.Linear(c.d_ckv, c.d_v * c.n_heads, bias=False)
        self.w_dq = nn.Linear(c.d_model, c.d_cq, bias=False)
        self.q_norm = RMSNorm(c.d_cq, c.rms_eps)
        self.w_uq = nn.Linear(c.d_cq, c.d_head * c.n_heads, bias=False)
        self.w_qr = nn.Linear(c.d_cq, c.d_rope * c.n_heads, bias=False)
        self.w_kr = nn.Linear(c.d_model, c.d_rope, bias=False)
        self.qr_norm = RMSNorm(c.d_rope * c.n_heads, c.rms_eps)
        self.kr_norm = RMSNorm(c.d_rope, c.rms_eps)
        self.w_out = nn.Linear(c.d_v * c.n_heads, c.d_model, bias=False)
        inv = c.rope_base ** (-torch.arange(0, c.d_rope, 2, dtype=torch.float64) / c.d_rope)
        ang = torch.outer(torch.arange(c.max_seq_len, dtype=torch.float64), inv)
        self.register_buffer("cos", ang.cos().float(), persistent=False)
        self.register_buffer("sin", ang.sin().float(), persistent=False)
        self.scale = (c.d_head + c.d_rope) ** -0.5

    def forward(self, x):
        B, L, _ = x.shape
        c_kv = self.kv_norm(self.w_dkv(x))
        c_q = self.q_norm(self.w_dq(x))
        cos, sin = self.cos[:L, None, :], self.sin[:L, None, :]
        q = torch.cat((self.w_uq(c_q).view(B, L, self.h, self.dh),
                       _rope(self.qr_norm(self.w_qr(c_q)).view(B, L, self.h, self.dr), cos, sin)), -1)
        kr = _rope(self.kr_norm(self.w_kr(x)).view(B, L, 1, self.dr), cos, sin)
        k = torch.cat((self.w_uk(c_kv).view(B, L, self.h, self.dh), kr.expand(B, L, self.h, self.dr)), -1)
        v = self.w_uv(c_kv).view(B, L, self.h, self.dv)
        o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                           is_causal=True, scale=self.scale)
        return self.w_out(o.transpose(1, 2).reshape(B, L, self.h * self.dv))


class SwiGLU(nn.Module):
    def __init__(self, d, hidden):
        super().__init__()
        self.w1 = nn.Linear(d, hidden, bias=False)
        self.w2 = nn.Linear(d, hidden, bias=False)
        self.w3 = nn.Linear(hidden, d, bias=False)

    def forward(self, x):
        return self.w3(F.silu(self.w1(x)) * self.w2(x))


class LoopExperts(nn.Module):
    """Stacked SwiGLU experts (w12 [E, 2H, D], w3 [E, D, H]) run as a per-expert loop in the
    input dtype: the reference's fallback (src/layers.py:78-87)."""

    def __init__(self, n_experts, d_model, hidden):
        super().__init__()
        self.n_experts, self.d_model = n_experts, d_model
        self.w12 = nn.Parameter(torch.empty(n_experts, 2 * hidden, d_model))
        self.w3 = nn.Parameter(torch.empty(n_experts, d_model, hidden))
        nn.init.normal_(self.w12, std=0.02)
        nn.init.normal_(self.w3, std=0.02)

    def forward(self, sorted_x, starts, ends, max_expert_tokens=None):
        out = torch.zeros(sorted_x.size(0), self.d_model, device=sorted_x.device, dtype=sorted_x.dtype)
        bounds = torch.stack((starts, ends)).tolist()
        for e in range(self.n_experts):
            s, t = bounds[0][e], bounds[1][e]
            if t > s:
                h1, h2 = F.linear(sorted_x[s:t], self.w12[e]).chunk(2, dim=-1)
                out[s:t] = F.linear(F.silu(h1) * h2, self.w3[e])
        return out


class MoE(nn.Module):
    """Shared SwiGLU expert(s) plus top-k sigmoid-gated routed experts with a selection bias
    updated outside the gradient (src/layers.py:90-180)."""

    def __init__(self, c: C5Config):
        super().__init__()
        self.top_k, self.n_routed, self.gamma, self.alpha = c.top_k, c.n_routed, c.gamma, c.balance_alpha
        self.routed_experts = LoopExperts(c.n_routed, c.d_model, c.hidden_dim // c.expert_scale)
        self.shared_experts = nn.ModuleList([SwiGLU(c.d_model, c.hidden_dim) for _ in range(c.n_shared)])
        self.router = nn.Linear(c.d_model, c.n_routed, bias=False)
        self.register_buffer("expert_bias", torch.zeros(c.n_routed))
        self.device_dispatch = False  # FP8 mode: route / dispatch / combine with cinnamon_amd.moe
        # per-layer checks: the top-k choice of a recorded forward (last_top_idx, kept when
        # record_route is set) can be imposed on a later one (route_override)
        self.record_route = False
        self.route_override = None
        self.last_top_idx = None

    def forward(self, x):
        B, L, d = x.shape
        shared = sum(e(x) for e in self.shared_experts)
        scores = torch.sigmoid(self.router(x))
        if self.route_override is not None:
            top_idx = self.route_override
        else:
            _, top_idx = (scores + self.expert_bias).topk(self.top_k, dim=-1)
        if self.record_route:
            self.last_top_idx = top_idx.detach().clone()
        gates = scores.gather(-1, top_idx)
        gates = gates / (gates.sum(-1, keepdim=True) + 1e-9)
        flat = x.reshape(-1, d)
        if self.device_dispatch and x.is_cuda:
            from cinnamon_amd import moe as moe_ops
            routed, counts = moe_ops.routed_experts(self.routed_experts, flat,
                                                    top_idx.reshape(-1, self.top_k),
                                                    gates.reshape(-1, self.top_k))
            routed = routed.to(flat.dtype).view(B, L, d)
        else:
            expert_of, order = top_idx.reshape(-1).sort()
            token = order // self.top_k
            counts = torch.bincount(expert_of, minlength=self.n_routed)
            ends = counts.cumsum(0)
            starts = ends - counts
            out = self.routed_experts(flat[token], starts, ends)
            out = out * gates.reshape(-1)[order][:, None]
            routed = torch.zeros_like(flat).index_add_(0, token, out.to(flat.dtype)).view(B, L, d)
        if self.training:
            with torch.no_grad():
                expected = top_idx.numel() / self.n_routed
                self.expert_bias += torch.where(counts.float() > expected, -self.gamma, self.gamma)
                self.expert_bias.clamp_(-1, 1)
        f = torch.zeros(B, self.n_routed, device=x.device, dtype=x.dtype)
        f.scatter_add_(1, top_idx.reshape(B, -1), torch.ones(B, L * self.top_k, device=x.device, dtype=x.dtype))
        f = f * (self.n_routed / (self.top_k * L))
        p = (scores / (scores.sum(-1, keepdim=True) + 1e-9)).mean(1)
        balance = self.alpha * (f * p).sum(-1).mean()
        return shared + routed, balance


class Block(nn.Module):
    def __init__(self, c: C5Config):
        super().__init__()
        self.rms1 = RMSNorm(c.d_model, c.rms_eps)
        self.rms2 = RMSNorm(c.d_model, c.rms_eps)
        self.attn = MLA(c)
        self.moe = MoE(c)

    def forward(self, x):
        x = x + self.attn(self.rms1(x))
        m, bal = self.moe(self.rms2(x))
        return x + m, bal


class MTP(nn.Module):
    def __init__(self, c: C5Config):
        super().__init__()
        self.norm_h = RMSNorm(c.d_model, c.rms_eps)
        self.norm_emb = RMSNorm(c.d_model, c.rms_eps)
        self.proj = nn.Linear(2 * c.d_model, c.d_model, bias=False)
        self.block = Block(c)

    def forward(self, h, e):
        return self.block(self.proj(torch.cat((self.norm_h(h), self.norm_emb(e)), -1)))


class C5Model(nn.Module):
    def __init__(self, c: C5Config):
        super().__init__()
        self.c = c
        self.embedding = nn.Embedding(c.vocab_size, c.d_model)
        self.layers = nn.ModuleList([Block(c) for _ in range(c.n_layers)])
        self.norm = RMSNorm(c.d_model, c.rms_eps)
        self.lm_head = nn.Linear(c.d_model, c.vocab_size, bias=False)
        self.lm_head.weight = self.embedding.weight
        self.mtp = nn.ModuleList([MTP(c) for _ in range(c.mtp_depth)])
        for name, p in self.named_parameters():
            if "weight" in name and p.dim() >= 2:
                std = 0.02 / math.sqrt(2 * c.n_layers) if name.endswith(("w_out.weight", "w3.weight")) else 0.02
                nn.init.normal_(p, std=std)

    def forward(self, ids):
        emb = self.embedding(ids)
        x, bal = emb, 0.0
        for blk in self.layers:
            x, b = blk(x)
            bal = bal + b
        logits = self.lm_head(self.norm(x))
        mtp_logits, h = [], x
        for depth, m in enumerate(self.mtp, start=1):
            h, b = m(h[:, :-1], emb[:, depth:])
            bal = bal + b
            mtp_logits.append(self.lm_head(self.norm(h)))
        return logits, mtp_logits, bal


def loss_fn(model: C5Model, ids: torch.Tensor):
    """Main next-token loss + lambda * MTP loss + balance loss (src/train.py:355-372)."""
    x, y = ids[:, :-1], ids[:, 1:]
    logits, mtp_logits, bal = model(x)
    main = F.cross_entropy(logits.reshape(-1, logits.size(-1)), y.reshape(-1))
    mtp = [F.cross_entropy(lg.reshape(-1, lg.size(-1)), y[:, d:].reshape(-1))
           for d, lg in enumerate(mtp_logits, start=1)]
    mtp_loss = sum(mtp) / len(mtp) if mtp else 0.0
    return main + model.c.mtp_lambda * mtp_loss + bal, main


def to_fp8(model: C5Model) -> C5Model:
    """The FP8 mode: eligible Linears -> FP8Linear (convert_to_fp8's rules), routed experts ->
    layers.GroupedExperts with the same weights, routed through cinnamon_amd.moe (device
    routing, dispatch fused into the quantization, device combine)."""
    from cinnamon_amd import kernels, layers

    model = copy.deepcopy(model)
    for blk in list(model.layers) + [m.block for m in model.mtp]:
        old = blk.moe.routed_experts
        new = layers.GroupedExperts(old.n_experts, old.d_model, old.w3.shape[2]).to(old.w12.device)
        with torch.no_grad():
            new.w12.copy_(old.w12)
            new.w3.copy_(old.w3)
        blk.moe.routed_experts = new
        blk.moe.device_dispatch = True
    return kernels.convert_to_fp8(model)


def capture_fp8_layer_io(model: C5Model, ids):
    """One forward and backward of the loss through `model` (the fp32 mode), recording for
    every MoE module and every MTP projection its input and the gradient of its output, and
    each MoE module's top-k expert choice.  Returns ({module name: {"x": input, "dout":
    output gradient[, "top_idx": experts]}}, {parameter name: grad})."""
    caps, handles = {}, []

    def hook(name):
        def f(mod, inp, out):
            caps[name] = {"x": inp[0].detach().clone()}
            t = out[0] if isinstance(out, tuple) else out
            t.register_hook(lambda g: caps[name].__setitem__("dout", g.detach().clone()))
        return f

    for n, m in model.named_modules():
        if isinstance(m, MoE) or n.endswith(".proj"):
            handles.append(m.register_forward_hook(hook(n)))
        if isinstance(m, MoE):
            m.record_route = True
    model.train()
    model.zero_grad(set_to_none=True)
    loss, _ = loss_fn(model, ids)
    loss.backward()
    for h in handles:
        h.remove()
    for n, m in model.named_modules():
        if isinstance(m, MoE):
            m.record_route = False
            caps[n]["top_idx"] = m.last_top_idx
    grads = {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}
    return caps, grads


def make_optimizer(model: C5Model):
    """AdamW with decoupled decay on matrices only (src/train.py:180-200)."""
    decay = [p for p in model.parameters() if p.dim() >= 2]
    no_decay = [p for p in model.parameters() if p.dim() < 2]
    return torch.optim.AdamW([{"params": decay, "weight_decay": model.c.weight_decay},
                              {"params": no_decay, "weight_decay": 0.0}], lr=model.c.lr)


def train(model: C5Model, batches, sync=None):
    """One optimizer step per batch; returns ([loss], [main loss], [seconds per step])."""
    opt = make_optimizer(model)
    model.train()
    losses, mains, secs = [], [], []
    for ids in batches:
        if sync:
            sync()
        t0 = time.perf_counter()
        opt.zero_grad(set_to_none=True)
        loss, main = loss_fn(model, ids)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), model.c.grad_clip)
        opt.step()
        losses.append(float(loss.detach()))
        mains.append(float(main.detach()))
        if sync:
            sync()
        secs.append(time.perf_counter() - t0)
    return losses, mains, secs
