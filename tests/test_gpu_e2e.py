"""End-to-end: the KilatTransformer forward restatement (tests/e2e_model.py) with
the decay path on the HIP kernel matches the same model on the CPU with the
oracle's decay (the reference's _cpu_global_decay, triton_ops.py:232-247), on
identical weights and tokens.  Tolerance: logits within 1e-4 relative to their
scale (fp32; the rest of the model runs on different devices)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import kilat_amd
from tests.decay_cases import rel_err
from tests.e2e_model import E2EConfig, KernelDecayCache, KilatE2E
from oracle import decay_oracle as O

pytestmark = pytest.mark.gpu


def tiny():
    return E2EConfig(vocab_size=256, n_embd=64, n_layer=2, n_head=4, num_experts=4, active_experts=2)


def test_e2e_logits_match_cpu_reference_decay(hip_device, kdecay_lib):
    torch.manual_seed(40)
    model = KilatE2E(tiny(), O.global_decay).eval()
    with torch.no_grad():  # vary the decay rates per head so every head differs
        for blk in model.layers:
            blk.attn.log_lambda.copy_(torch.randn_like(blk.attn.log_lambda) + 2.0)
    ids = torch.randint(0, 256, (2, 700), generator=torch.Generator().manual_seed(41))
    with torch.no_grad():
        ref, ref_loss = model(ids, labels=ids)
    model = model.to(hip_device)
    out = {}
    for fused in (False, True):
        print(f"  e2e fused_layout={fused}", flush=True)
        model.set_decay(kilat_amd.triton_global_decay, fused_layout=fused)
        with torch.no_grad():
            logits, loss = model(ids.to(hip_device), labels=ids.to(hip_device))
        torch.cuda.synchronize()
        out[fused] = logits.cpu()
        err = float((logits.cpu() - ref).abs().max() / ref.abs().max())
        assert err <= 1e-4, f"fused={fused}: logits rel err {err:.3e}"
        assert abs(float(loss) - float(ref_loss)) <= 1e-4 * abs(float(ref_loss))
    assert torch.equal(out[False], out[True])  # layout-fused I/O changes no value


def test_e2e_training_gradients_match_cpu_reference_decay(hip_device, kdecay_lib):
    """One training backward through the model: the HIP decay's autograd
    (the chunked scan's backward kernel, dlam chained through the caller's
    sigmoid(log_lambda)) against torch autograd through the oracle on the CPU,
    identical weights and tokens, fp32.  Gradients of every layer's
    log_lambda and value projection within 1e-3 of their scale (the rest of
    the model's backward runs on different devices)."""
    torch.manual_seed(42)
    model = KilatE2E(tiny(), O.global_decay)
    with torch.no_grad():
        for blk in model.layers:
            blk.attn.log_lambda.copy_(torch.randn_like(blk.attn.log_lambda) + 2.0)
    ids = torch.randint(0, 256, (2, 300), generator=torch.Generator().manual_seed(43))
    _, loss = model(ids, labels=ids)
    loss.backward()
    ref = {n: p.grad.clone() for n, p in model.named_parameters() if "log_lambda" in n or "v_proj_global" in n}
    model.zero_grad(set_to_none=True)
    model = model.to(hip_device)
    model.set_decay(kilat_amd.triton_global_decay, fused_layout=True)
    print("  e2e training backward on the GPU", flush=True)
    _, loss_d = model(ids.to(hip_device), labels=ids.to(hip_device))
    loss_d.backward()
    torch.cuda.synchronize()
    assert abs(float(loss_d.detach()) - float(loss.detach())) <= 1e-4 * abs(float(loss.detach()))
    grads = dict(model.named_parameters())
    assert ref and all(grads[n].grad is not None for n in ref)
    for n, r in ref.items():
        gpu = grads[n].grad.cpu()
        err = float((gpu - r).abs().max() / r.abs().max().clamp_min(1e-30))
        assert err <= 1e-3, f"{n}: grad rel err {err:.3e}"


def test_c5_full_config_every_layer_matches_oracle(hip_device, kdecay_lib):
    """The C5 configuration itself: n_embd 768, 12 layers, 12 heads with
    recall_ratio 0.5 (6 decay heads of 64 channels per layer), MoE 8 x top-2
    (+2 shared), vocab 50000, random init, bf16 autocast, B=8 N=1024.  The
    decay op is wrapped to record each layer's (lam, V, y) on the GPU; every
    one of the 12 outputs is checked against the oracle's decay
    (triton_ops.py:232-247) on the same lam and V, to the bf16 tolerance
    (max-abs <= 2e-2), with the reference's glue copies and with the
    layout-fused view (attention.py:319-374)."""
    torch.manual_seed(4)
    cfg = E2EConfig()
    calls = []

    def recording_decay(lam, V):
        y = kilat_amd.triton_global_decay(lam, V)
        calls.append((lam.detach().cpu(), V.detach().cpu(), y.detach().cpu()))
        return y

    model = KilatE2E(cfg, recording_decay).to(hip_device).eval()
    with torch.no_grad():  # a spread of decay rates, up to 0.9999, per head and layer
        for blk in model.layers:
            u = 0.5 + (0.9999 - 0.5) * torch.rand(blk.attn.n_global, dtype=torch.float64)
            blk.attn.log_lambda.copy_(torch.log(u / (1 - u)).float())
    ids = torch.randint(0, cfg.vocab_size, (8, 1024), generator=torch.Generator().manual_seed(44)).to(hip_device)
    logits = {}
    for fused in (False, True):
        calls.clear()
        model.set_decay(recording_decay, fused_layout=fused)
        print(f"  C5 forward fused_layout={fused}", flush=True)
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            lg, _ = model(ids)
        torch.cuda.synchronize()
        logits[fused] = lg.float().cpu()
        assert bool(torch.isfinite(logits[fused]).all())
        assert len(calls) == cfg.n_layer
        for layer, (lam, V, y) in enumerate(calls):
            assert V.shape == (8, 6, 1024, 64) and V.dtype == torch.bfloat16 and y.dtype == torch.bfloat16
            ref = O.global_decay(lam, V)
            err = float((y.double() - ref.double()).abs().max())
            print(f"    layer {layer}: max_abs {err:.3e}", flush=True)
            assert err <= 2e-2, f"fused={fused} layer {layer}: max_abs {err:.3e}"
    # the two layouts feed the decay op the same values and get the same bits back
    assert torch.equal(logits[False], logits[True])


class RecordingKernelCache(KernelDecayCache):
    """KernelDecayCache that keeps every call's inputs and outputs (on the CPU)."""

    def __init__(self):
        self.prefills, self.steps = [], []

    def prefill(self, decay, lam, V, x_dtype):
        y, state = super().prefill(decay, lam, V, x_dtype)
        self.prefills.append((lam.detach().cpu(), V.detach().cpu(), x_dtype, state.detach().cpu()))
        return y, state

    def step(self, lam, past_state, v_current, t_pos):
        past = past_state.detach().cpu()  # before the call: the step may not alias it, but copy first anyway
        out, new_state = super().step(lam, past_state, v_current, t_pos)
        self.steps.append((lam.detach().cpu(), past, v_current.detach().cpu(), t_pos, out.detach().cpu(),
                           new_state.detach().cpu()))
        return out, new_state


def _ulps(a: torch.Tensor, b: torch.Tensor) -> int:
    x = a.float().numpy().view(np.int32).astype(np.int64)
    y = b.float().numpy().view(np.int32).astype(np.int64)
    return int(np.abs(x - y).max())


def test_c5_prefill_then_decode_through_the_cache(hip_device, kdecay_lib):
    """Incremental mode driven the way the reference's caller drives it, at
    the C5 configuration (n_embd 768, 12 layers, 6 decay heads x 64 per
    layer, MoE 8 x top-2, vocab 50000, random init, bf16 autocast, B=8): one
    prefill of N=1024 tokens with use_cache, then 16 tokens decoded one call
    each with the returned cache (model.py:490-560, attention.py:310-394).
    The decay half runs on the HIP kernels: the prefill's seed is the scan's
    final state (one launch with y), each token's update one decay_step
    launch with t_pos = the latent cache's length (attention.py:357), a
    position shared by the batch.  Every layer and every call is checked
    against the oracle on the same inputs:
      - seed: within 1e-5 per stream of attention.py:383-394's loop
        (O.seed_state; the chunked scan reassociates the recurrence), and bit
        for bit with the sequential kernel's final state on the same V;
      - step: the new state bit for bit against attention.py:344-360
        (O.step) from the state the kernel carried in, the output within one
        ulp (the double-precision power inside z), t_pos = 1024 + token.
    16 tokens x 12 layers = 192 steps."""
    torch.manual_seed(4)
    cfg = E2EConfig()
    cache = RecordingKernelCache()
    model = KilatE2E(cfg, kilat_amd.triton_global_decay, fused_layout=True, cache_ops=cache).to(hip_device).eval()
    with torch.no_grad():  # a spread of decay rates, up to 0.9999, per head and layer
        for blk in model.layers:
            u = 0.5 + (0.9999 - 0.5) * torch.rand(blk.attn.n_global, dtype=torch.float64)
            blk.attn.log_lambda.copy_(torch.log(u / (1 - u)).float())
    B, N, T = 8, 1024, 16
    ids = torch.randint(0, cfg.vocab_size, (B, N + T), generator=torch.Generator().manual_seed(45)).to(hip_device)
    print(f"  C5 prefill B={B} N={N} with the cache", flush=True)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        logits, _, past = model(ids[:, :N], use_cache=True)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(logits.float()).all())
        for t in range(T):
            print(f"  C5 decode token {t}", flush=True)
            logits, _, past = model(ids[:, N + t:N + t + 1], past_key_values=past, use_cache=True)
            assert tuple(logits.shape) == (B, 1, cfg.vocab_size)
        torch.cuda.synchronize()
    assert bool(torch.isfinite(logits.float()).all())
    assert len(cache.prefills) == cfg.n_layer and len(cache.steps) == cfg.n_layer * T
    for layer, (lam, V, x_dtype, state) in enumerate(cache.prefills):
        assert V.shape == (B, 6, N, 64) and V.dtype == torch.bfloat16 and x_dtype == torch.float32
        ref = O.seed_state(lam, V, x_dtype)
        assert state.dtype == ref.dtype == torch.float32
        e = rel_err(state.view(B, 6, 1, 64), ref.view(B, 6, 1, 64))
        _, seq = kilat_amd.global_decay_scan(lam.to(hip_device), V.to(hip_device), return_final_state=True,
                                             algorithm="sequential")
        print(f"    layer {layer} seed: rel {e:.2e}, sequential kernel bitwise "
              f"{torch.equal(seq.cpu(), ref)}", flush=True)
        assert e <= 1e-5, f"layer {layer}: seed rel err {e:.3e}"
        assert torch.equal(seq.cpu(), ref), f"layer {layer}: sequential seed differs from attention.py:383-394"
    worst = 0
    for k, (lam, past_state, v, t_pos, out, new_state) in enumerate(cache.steps):
        token, layer = divmod(k, cfg.n_layer)
        assert t_pos == N + token, (token, layer, t_pos)
        ro, rs = O.step(lam, past_state, v, t_pos)
        assert torch.equal(new_state, rs), f"token {token} layer {layer}: state not bit-identical"
        worst = max(worst, _ulps(out, ro))
        assert worst <= 1, f"token {token} layer {layer}: output {worst} ulps from attention.py:344-360"
    # the state each step started from is the one the previous token left (the cache carried it)
    for k in range(cfg.n_layer, len(cache.steps)):
        assert torch.equal(cache.steps[k][1], cache.steps[k - cfg.n_layer][5]), k
    for layer in range(cfg.n_layer):
        assert torch.equal(cache.steps[layer][1], cache.prefills[layer][3]), layer
    print(f"  192 steps: states bit-identical, outputs within {worst} ulp", flush=True)

