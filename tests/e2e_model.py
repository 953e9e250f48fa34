"""KilatTransformer forward, restated to measure the decay path end to end.

A compact restatement of the reference model's forward in its default
configuration (no RoPE, no dropout), full-sequence and with the decode cache,
used by bench.py's end-to-end figure and by the end-to-end parity tests.  Only
the global-decay op is this package's kernel; everything else is plain torch,
as in the reference:

  KilatTransformer.forward   /root/reference/src/kilat/arc/model.py:490-595
  Block / RMSNorm            /root/reference/src/kilat/arc/blocks.py:80-90, 306-406
  KilatAttention.forward     /root/reference/src/kilat/arc/attention.py:241-518
  SwiGLU / DeepSeekMoE       /root/reference/src/kilat/arc/ffn.py:63-112, 232-367, 403-482
  weight init                /root/reference/src/kilat/arc/model.py:71-89

The decay op is pluggable (`decay` below): it takes (lam [H_g], V [B,H_g,N,Dh])
and returns y of V's shape.  `fused_layout=True` hands it the projection's
(B,N,H_g*Dh) buffer viewed as (B,H_g,N,Dh) and takes y back as a view, instead
of the two .contiguous()/reshape copies of attention.py:368,374.

The decode cache (use_cache / past_key_values, model.py:490-560,
blocks.py:306-406, attention.py:299-518) keeps per layer the decay state
(B,H_g,Dh) and the latent KV (B,T,L).  Its two decay operations are pluggable
too (`cache_ops`, see ReferenceDecayCache): `prefill` (the full-sequence op
plus the state seed of attention.py:383-394) and `step` (the incremental
update of attention.py:344-360, with t_pos = the latent cache's length, one
position shared by the batch).

The reference's validate_finite_tensor host checks (model.py:565, ffn.py:112,
365-366) are not repeated: they synchronise with the host and compute nothing.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

DecayFn = Callable[[torch.Tensor, torch.Tensor], torch.Tensor]


class ReferenceDecayCache:
    """The reference's two decode-cache operations of the decay path, in plain torch.

    prefill(decay, lam, V, x_dtype) -> (y, state): the full-sequence op, then
        the state seed the reference computes after it when use_cache is set
        (attention.py:383-394): acc = zeros(B,H,Dh, x.dtype);
        acc = lam * acc + V[:, :, t] for every t.
    step(lam, past_state, v_current, t_pos) -> (out, new_state): the
        incremental update (attention.py:344-360), out of shape (B,H,Dh).
    """

    def prefill(self, decay: DecayFn, lam, V, x_dtype):
        y = decay(lam, V)
        B, H, N, Dh = V.shape
        lam_bc = lam.view(1, H, 1)
        acc = torch.zeros(B, H, Dh, device=V.device, dtype=x_dtype)
        for t in range(N):
            acc = lam_bc * acc + V[:, :, t, :]
        return y, acc

    def step(self, lam, past_state, v_current, t_pos: int):
        H = lam.shape[0]
        lam_bc = lam.view(1, H, 1)
        new_state = lam_bc * past_state + v_current
        z_inc = (1 - lam_bc ** (t_pos + 1)) / (1 - lam_bc + 1e-6)
        return new_state / z_inc, new_state


class KernelDecayCache:
    """The same two operations on this package's HIP kernels: prefill is one
    global_decay_scan launch that returns y and the final state together (the
    seed without the reference's N-step loop), step one decay_step launch for
    the whole batch.  The state is fp32 (B,H,Dh), the type the reference's
    state has once fp32 lam has multiplied it."""

    def prefill(self, decay: DecayFn, lam, V, x_dtype):
        import kilat_amd

        return kilat_amd.global_decay_scan(lam, V, return_final_state=True)

    def step(self, lam, past_state, v_current, t_pos: int):
        import kilat_amd

        return kilat_amd.decay_step(lam, past_state, v_current, t_pos)


@dataclass
class E2EConfig:
    """The reference's KilatConfig fields that shape the forward (model_config.py:67-100)."""

    vocab_size: int = 50000
    n_embd: int = 768
    n_layer: int = 12
    n_head: int = 12
    recall_ratio: float = 0.5
    latent_dim: Optional[int] = None
    ff_mult: float = 8 / 3
    num_experts: int = 8
    active_experts: int = 2
    # Block does not forward num_shared_experts (blocks.py:288-296), so
    # FeedForward's default of 2 shared experts applies (ffn.py:409-413).
    num_shared_experts: int = 2
    aux_loss_coef: float = 0.01
    device_balance_coef: float = 0.001


class RMSNorm(nn.Module):
    """blocks.py:80-90: x / sqrt(mean(x^2) + eps) * weight."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        rms = torch.sqrt(torch.mean(x ** 2, dim=-1, keepdim=True) + self.eps)
        return x / rms * self.weight


class SwiGLU(nn.Module):
    """ffn.py:63-112: down(silu(gate(x)) * up(x)); hidden rounded up to a multiple of 64."""

    def __init__(self, dim: int, ff_mult: float):
        super().__init__()
        hidden = (int(dim * ff_mult) + 63) // 64 * 64
        self.gate = nn.Linear(dim, hidden, bias=False)
        self.up = nn.Linear(dim, hidden, bias=False)
        self.down = nn.Linear(hidden, dim, bias=False)

    def forward(self, x):
        return self.down(F.silu(self.gate(x)) * self.up(x))


class DeepSeekMoE(nn.Module):
    """ffn.py:232-367: shared experts + top-k routed experts (renormalised weights) + aux loss."""

    def __init__(self, cfg: E2EConfig):
        super().__init__()
        d = cfg.n_embd
        self.k = cfg.active_experts
        self.n_routed = cfg.num_experts
        self.aux_loss_coef = cfg.aux_loss_coef
        self.device_balance_coef = cfg.device_balance_coef
        self.router = nn.Linear(d, cfg.num_experts, bias=False)
        self.shared_experts = nn.ModuleList([SwiGLU(d, cfg.ff_mult) for _ in range(cfg.num_shared_experts)])
        self.routed_experts = nn.ModuleList([SwiGLU(d, cfg.ff_mult) for _ in range(cfg.num_experts)])

    def forward(self, x):
        B, S, D = x.shape
        shared = torch.zeros_like(x)
        for e in self.shared_experts:
            shared = shared + e(x)
        xf = x.view(-1, D)
        probs = F.softmax(self.router(xf), dim=-1)
        w, idx = torch.topk(probs, self.k, dim=-1)
        w = w / w.sum(dim=-1, keepdim=True)
        routed = torch.zeros_like(xf)
        for e_i, e in enumerate(self.routed_experts):
            mask = (idx == e_i).any(dim=-1)
            if mask.any():
                out = e(xf[mask])
                pos = (idx[mask] == e_i).float().argmax(dim=-1)
                we = w[mask].gather(1, pos.unsqueeze(1)).squeeze(1)
                routed[mask] += we.unsqueeze(1) * out
        y = (shared.view(-1, D) + routed).view(B, S, D)
        frac = torch.zeros(self.n_routed, device=x.device, dtype=x.dtype)
        for i in range(self.n_routed):
            frac[i] = (idx == i).any(dim=-1).float().mean()
        balance = self.n_routed * (frac * probs.mean(dim=0)).sum()
        device = torch.var(frac) * self.n_routed
        return y, self.aux_loss_coef * balance + self.device_balance_coef * device


class HybridAttention(nn.Module):
    """attention.py:146-239 (layers) and :241-518 (forward, full-sequence and incremental)."""

    def __init__(self, cfg: E2EConfig, decay: DecayFn, fused_layout: bool, cache_ops=None):
        super().__init__()
        self.cache_ops = cache_ops if cache_ops is not None else ReferenceDecayCache()
        d = cfg.n_embd
        self.dh = d // cfg.n_head
        self.n_recall = int(cfg.n_head * cfg.recall_ratio)
        self.n_global = cfg.n_head - self.n_recall
        self.latent = cfg.latent_dim if cfg.latent_dim is not None else d // 4
        self.decay = decay
        self.fused_layout = fused_layout
        self.log_lambda = nn.Parameter(torch.full((self.n_global,), math.log(0.9 / 0.1)))
        self.v_proj_global = nn.Linear(d, self.n_global * self.dh, bias=False)
        self.q_a_proj = nn.Linear(d, self.latent, bias=False)
        self.q_a_norm = nn.LayerNorm(self.latent)
        self.q_b_proj = nn.Linear(self.latent, self.n_recall * self.dh, bias=False)
        self.kv_a_proj = nn.Linear(d, self.latent, bias=False)
        self.kv_a_norm = nn.LayerNorm(self.latent)
        self.kv_b_proj = nn.Linear(self.latent, 2 * self.n_recall * self.dh, bias=False)
        self.gamma_net = nn.Sequential(nn.Linear(2 * d, d), nn.ReLU(), nn.Linear(d, d), nn.Sigmoid())
        self.c_proj = nn.Linear(d, d, bias=False)

    def forward(self, x, past=None, use_cache: bool = False):
        """Returns the output, and with use_cache also the layer's new cache
        (decay state (B,H_g,Dh), latent KV (B,T,L)).  `past` is the layer's
        cache from the previous call; with one new token it takes the
        incremental path (attention.py:310-311)."""
        B, N, _ = x.shape
        Hg, Dh = self.n_global, self.dh
        past_state, past_latent = past if past is not None else (None, None)
        incremental = N == 1 and past is not None
        lam = torch.sigmoid(self.log_lambda)
        vg = self.v_proj_global(x)
        new_state = None
        if incremental and past_state is not None:
            t_pos = past_latent.shape[1] if past_latent is not None else 0  # the cache length (attention.py:357)
            out, new_state = self.cache_ops.step(lam, past_state, vg.view(B, 1, Hg, Dh).squeeze(1), t_pos)
            out_global = out.reshape(B, 1, Hg * Dh)
        else:
            if self.fused_layout:
                V = vg.view(B, N, Hg, Dh).transpose(1, 2)
            else:
                V = vg.view(B, N, Hg, Dh).transpose(1, 2).contiguous()
            if use_cache:
                y, new_state = self.cache_ops.prefill(self.decay, lam, V, x.dtype)
            else:
                y = self.decay(lam, V)
            out_global = y.transpose(1, 2).reshape(B, N, Hg * Dh)
        new_latent = None
        if self.n_recall == 0:
            out_recall = torch.zeros(B, N, 0, device=x.device, dtype=x.dtype)
            if use_cache:
                new_latent = torch.zeros(B, 0, self.latent, device=x.device, dtype=x.dtype)
        else:
            q = self.q_b_proj(self.q_a_norm(self.q_a_proj(x))).view(B, N, self.n_recall, Dh).transpose(1, 2)
            latent = self.kv_a_norm(self.kv_a_proj(x))
            if incremental and past_latent is not None:
                latent = torch.cat([past_latent, latent], dim=1)
            if use_cache:
                new_latent = latent.clone()
            kv = self.kv_b_proj(latent)
            kv = kv.view(B, -1, 2, self.n_recall, Dh).permute(2, 0, 3, 1, 4)
            out_recall = F.scaled_dot_product_attention(q, kv[0], kv[1], is_causal=not incremental)
            if incremental:
                out_recall = out_recall[:, :, -1:, :]
            out_recall = out_recall.transpose(1, 2).reshape(B, N, self.n_recall * Dh)
        combined = torch.cat([out_global, out_recall], dim=-1)  # promotes mixed dtypes, as the reference's cat
        gate = self.gamma_net(torch.cat([x, combined], dim=-1))
        out = self.c_proj(combined * gate)
        if use_cache:
            return out, (new_state, new_latent)
        return out


class Block(nn.Module):
    """blocks.py:306-406: pre-norm attention and MoE residual branches."""

    def __init__(self, cfg: E2EConfig, decay: DecayFn, fused_layout: bool, cache_ops=None):
        super().__init__()
        self.rms1 = RMSNorm(cfg.n_embd)
        self.rms2 = RMSNorm(cfg.n_embd)
        self.attn = HybridAttention(cfg, decay, fused_layout, cache_ops)
        self.mlp = DeepSeekMoE(cfg)

    def forward(self, x, past=None, use_cache: bool = False):
        a = self.attn(self.rms1(x), past, use_cache)
        a, present = a if use_cache else (a, None)
        x = x + a
        f, aux = self.mlp(self.rms2(x))
        return x + f, aux, present


class KilatE2E(nn.Module):
    """model.py:191-257 (layers, tied LM head) and :490-595 (forward -> logits, loss)."""

    def __init__(self, cfg: E2EConfig, decay: DecayFn, fused_layout: bool = False, cache_ops=None):
        super().__init__()
        self.cfg = cfg
        self.wte = nn.Embedding(cfg.vocab_size, cfg.n_embd)
        self.layers = nn.ModuleList([Block(cfg, decay, fused_layout, cache_ops) for _ in range(cfg.n_layer)])
        self.ln_f = RMSNorm(cfg.n_embd)
        self.lm_head = nn.Linear(cfg.n_embd, cfg.vocab_size, bias=False)
        self.wte.weight = self.lm_head.weight
        for m in self.modules():  # model.py:71-89; log_lambda and norms keep their own init
            if isinstance(m, (nn.Linear, nn.Embedding)):
                nn.init.normal_(m.weight, mean=0.0, std=0.02)
                if isinstance(m, nn.Linear) and m.bias is not None:
                    nn.init.zeros_(m.bias)

    def forward(self, input_ids, labels=None, past_key_values=None, use_cache: bool = False):
        """(logits, loss), and with use_cache also the per-layer caches (a tuple
        the next call takes as past_key_values)."""
        x = self.wte(input_ids)
        aux_total = torch.zeros((), device=x.device, dtype=x.dtype)
        pasts = past_key_values if past_key_values is not None else [None] * len(self.layers)
        presents = []
        for block, past in zip(self.layers, pasts):
            x, aux, present = block(x, past, use_cache)
            aux_total = aux_total + aux
            presents.append(present)
        logits = self.lm_head(self.ln_f(x))
        loss = None
        if labels is not None:
            loss = F.cross_entropy(logits[..., :-1, :].contiguous().view(-1, logits.size(-1)),
                                   labels[..., 1:].contiguous().view(-1), ignore_index=-100) + aux_total
        if use_cache:
            return logits, loss, tuple(presents)
        return logits, loss

    def set_decay(self, decay: DecayFn, fused_layout: Optional[bool] = None, cache_ops=None) -> None:
        for block in self.layers:
            block.attn.decay = decay
            if fused_layout is not None:
                block.attn.fused_layout = fused_layout
            if cache_ops is not None:
                block.attn.cache_ops = cache_ops
