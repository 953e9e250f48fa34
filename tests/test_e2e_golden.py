"""The composition tests/e2e_model.py restates, pinned against the reference
KilatTransformer itself: tests/golden/c5_tiny_golden.npz holds the logits the
reference model (model.py:490-595 with blocks.py, attention.py, ffn.py and its
CPU decay path triton_ops.py:232-247) produced for a tiny configuration
(n_embd 64, 2 layers, 4 heads, recall_ratio 0.5, MoE 4 x top-2 + 2 shared,
vocab 256, B=2 N=16), with the weights of the restatement built from a fixed
seed (tests/golden/make_c5_golden.py writes it; the weights are identified by
a checksum, not stored).  This pins the MoE top-k routing and its tie-breaks,
the 2-shared-expert default, the gamma gate, the MLA attention and the
residual structure that the end-to-end figures rely on."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import decay_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "c5_tiny_golden.npz")


def _restatement(decay, cache_ops=None):
    from tests.golden.make_c5_golden import CFG, SEED, weight_checksum
    from tests.e2e_model import E2EConfig, KilatE2E

    torch.manual_seed(SEED)
    model = KilatE2E(E2EConfig(**CFG), decay, cache_ops=cache_ops).eval()
    with torch.no_grad():
        g = torch.Generator().manual_seed(SEED + 1)
        for blk in model.layers:
            blk.attn.log_lambda.copy_(torch.randn(blk.attn.log_lambda.shape, generator=g) + 2.0)
    return model, weight_checksum(model)


def test_restatement_matches_reference_logits_on_cpu():
    d = np.load(GOLDEN)
    model, cks = _restatement(O.global_decay)
    assert cks == pytest.approx(float(d["weight_checksum"]), rel=1e-12), "weights differ from the fixture's"
    ids = torch.from_numpy(d["ids"])
    with torch.no_grad():
        logits, loss = model(ids, labels=ids)
    ref = torch.from_numpy(d["logits"])
    err = float((logits - ref).abs().max() / ref.abs().max())
    assert err <= 1e-6, f"logits rel err {err:.3e}"
    assert float(loss) == pytest.approx(float(d["loss"]), rel=1e-6)


@pytest.mark.gpu
def test_restatement_on_gpu_with_hip_decay_matches_reference_logits(hip_device, kdecay_lib):
    """The same model on the GPU with the decay path on the HIP kernel, both
    layouts, against the reference model's logits (fp32; the chunked scan and
    the GPU's other kernels differ in rounding only)."""
    import kilat_amd

    d = np.load(GOLDEN)
    model, _ = _restatement(kilat_amd.triton_global_decay)
    model = model.to(hip_device)
    ids = torch.from_numpy(d["ids"]).to(hip_device)
    ref = torch.from_numpy(d["logits"])
    for fused in (False, True):
        model.set_decay(kilat_amd.triton_global_decay, fused_layout=fused)
        with torch.no_grad():
            logits, loss = model(ids, labels=ids)
        torch.cuda.synchronize()
        err = float((logits.cpu() - ref).abs().max() / ref.abs().max())
        print(f"  fused_layout={fused}: logits rel err {err:.3e}", flush=True)
        assert err <= 1e-4, f"fused={fused}: logits rel err {err:.3e}"
        assert float(loss) == pytest.approx(float(d["loss"]), rel=1e-4)


def test_restatement_cache_path_matches_reference_on_cpu():
    """The decode cache as the reference's generation loop drives it: a
    prefill with use_cache (the decay state seeded by attention.py:383-394),
    then one token per call through the incremental path (attention.py:
    344-360, t_pos = the latent cache's length).  The restatement with the
    reference's torch operations gives the reference model's own logits of
    every call and every layer's final decay state, bit for bit."""
    from tests.e2e_model import ReferenceDecayCache
    from tests.golden.make_c5_golden import run_with_cache

    d = np.load(GOLDEN)
    model, _ = _restatement(O.global_decay, ReferenceDecayCache())
    pre, steps, states = run_with_cache(model, torch.from_numpy(d["ids"]), reference=False)
    assert torch.equal(pre, torch.from_numpy(d["inc_prefill_logits"]))
    assert torch.equal(steps, torch.from_numpy(d["inc_step_logits"]))
    assert torch.equal(states, torch.from_numpy(d["inc_states"]))


@pytest.mark.gpu
def test_restatement_cache_path_on_gpu_with_hip_kernels(hip_device, kdecay_lib):
    """The same prefill and decode calls on the GPU, the decay path on the HIP
    kernels (the prefill's state from the scan's final state, each token's
    update one decay_step launch), both layouts, against the reference
    model's logits and decay states (fp32)."""
    import kilat_amd
    from tests.e2e_model import KernelDecayCache
    from tests.golden.make_c5_golden import run_with_cache

    d = np.load(GOLDEN)
    model, _ = _restatement(kilat_amd.triton_global_decay, KernelDecayCache())
    model = model.to(hip_device)
    ids = torch.from_numpy(d["ids"]).to(hip_device)
    for fused in (False, True):
        model.set_decay(kilat_amd.triton_global_decay, fused_layout=fused)
        pre, steps, states = run_with_cache(model, ids, reference=False)
        torch.cuda.synchronize()
        for name, got in (("inc_prefill_logits", pre), ("inc_step_logits", steps), ("inc_states", states)):
            ref = torch.from_numpy(d[name])
            err = float((got.cpu() - ref).abs().max() / ref.abs().max())
            print(f"  fused_layout={fused} {name}: rel err {err:.3e}", flush=True)
            assert err <= 1e-4, f"fused={fused} {name}: rel err {err:.3e}"

