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


def _restatement(decay):
    from tests.golden.make_c5_golden import CFG, SEED, weight_checksum
    from tests.e2e_model import E2EConfig, KilatE2E

    torch.manual_seed(SEED)
    model = KilatE2E(E2EConfig(**CFG), decay).eval()
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
