"""Writes tests/golden/c5_tiny_golden.npz: logits of the reference KilatTransformer
on a tiny configuration, to pin the composition that tests/e2e_model.py restates.

Run in the build container only, where the reference is mounted:

    PYTHONDONTWRITEBYTECODE=1 python tests/golden/make_c5_golden.py

It imports the reference's model modules from /root/reference/src by file,
under package stubs that do not execute the reference's package __init__
files (those pull in the trainer, datasets and generation front ends), and
writes nothing into the reference tree.  The weights are not stored: the
restatement (tests.e2e_model.KilatE2E) is built from a fixed torch seed, its
state dict is copied into the reference model by name, and the fixture keeps
a checksum of those weights so the test can tell the same weights were used.
The decay op is the reference's own CPU path (V on the CPU routes
triton_global_decay to _cpu_global_decay, triton_ops.py:305-306).

Fixture: ids [2,16] int64, logits [2,16,256] float32, loss, weight checksum,
and the configuration.  Reference files exercised: model.py:191-257 and
:490-595, blocks.py:80-90 and :306-406, attention.py:146-518,
ffn.py:63-112, :232-367 and :403-482, triton_ops.py:232-330.

The decode cache, as the generation loop drives it (generation_mixin.py:
484-509): a prefill of the first INC_PREFILL tokens with use_cache=True, then
one call per later token with the returned past_key_values (the incremental
path, attention.py:310-360 and :434-491): inc_prefill_logits [2,12,256],
inc_step_logits [4,2,1,256], and inc_states [2 layers, 2, 2, 16], every
layer's decay state after the last step.
"""
from __future__ import annotations

import importlib
import os
import sys
import types

import numpy as np
import torch

sys.dont_write_bytecode = True
HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_SRC = os.environ.get("KILAT_REFERENCE_SRC", "/root/reference/src")
OUT = os.path.join(HERE, "c5_tiny_golden.npz")

SEED = 1234
CFG = dict(vocab_size=256, n_embd=64, n_layer=2, n_head=4, recall_ratio=0.5, num_experts=4, active_experts=2)
B, N = 2, 16
INC_PREFILL = 12  # tokens of the cached prefill; the other N - INC_PREFILL are decoded one at a time


def run_with_cache(model, ids, reference: bool):
    """Prefill ids[:, :INC_PREFILL] with use_cache, then one call per later
    token with the cache: (prefill logits, [step logits], decay states of
    every layer after the last step)."""
    def call(x, past):
        if reference:
            out = model(x, past_key_values=past, use_cache=True, return_dict=True)
            return out.logits.float(), out.past_key_values
        logits, _, presents = model(x, past_key_values=past, use_cache=True)
        return logits.float(), presents

    with torch.no_grad():
        pre, past = call(ids[:, :INC_PREFILL], None)
        steps = []
        for t in range(INC_PREFILL, ids.shape[1]):
            lg, past = call(ids[:, t:t + 1], past)
            steps.append(lg)
    states = torch.stack([layer[0].float() for layer in past])
    return pre, torch.stack(steps), states


def weight_checksum(model: torch.nn.Module) -> float:
    """Sum over parameters of sum(w * position weights): order-sensitive, float64."""
    tot = 0.0
    for name, p in sorted(model.state_dict().items()):
        w = p.detach().double().reshape(-1)
        tot += float((w * torch.linspace(1.0, 2.0, w.numel(), dtype=torch.float64)).sum())
    return tot


def build_restatement():
    sys.path.insert(0, ROOT)
    from tests.e2e_model import E2EConfig, KilatE2E
    from oracle import decay_oracle as O

    torch.manual_seed(SEED)
    model = KilatE2E(E2EConfig(**CFG), O.global_decay).eval()
    with torch.no_grad():  # distinct decay rates per head and layer
        g = torch.Generator().manual_seed(SEED + 1)
        for blk in model.layers:
            blk.attn.log_lambda.copy_(torch.randn(blk.attn.log_lambda.shape, generator=g) + 2.0)
    return model


def import_reference_model():
    """kilat.arc.model from the reference sources, without running the package
    __init__ files: each package is an empty module whose __path__ points at
    the reference directory, so only the modules model.py imports are run."""
    pkgs = ["kilat", "kilat.arc", "kilat.utils", "kilat.configs", "kilat.pipeline", "kilat.pipeline.generation"]
    for name in pkgs:
        mod = types.ModuleType(name)
        mod.__path__ = [os.path.join(REF_SRC, *name.split("."))]
        sys.modules[name] = mod
    model_mod = importlib.import_module("kilat.arc.model")
    config_mod = importlib.import_module("kilat.configs.model_config")
    return model_mod.KilatTransformer, config_mod.KilatConfig


def reference_key_of(ours: str) -> str:
    """tests.e2e_model names -> the reference's (its FeedForward wraps the MoE as .layer)."""
    return ours.replace(".mlp.", ".mlp.layer.", 1) if ".mlp." in ours else ours


def main() -> None:
    ours = build_restatement()
    KilatTransformer, KilatConfig = import_reference_model()
    cfg = KilatConfig(ffn_mode="moe", use_rope=False, use_cache=False, return_dict=True, **CFG)
    ref = KilatTransformer(cfg).eval()
    ref_sd = ref.state_dict()
    mapped = {reference_key_of(k): v for k, v in ours.state_dict().items()}
    missing = sorted(set(ref_sd) - set(mapped))
    extra = sorted(set(mapped) - set(ref_sd))
    if missing or extra:
        raise SystemExit(f"state dict names differ: reference-only {missing}, restatement-only {extra}")
    for k, v in mapped.items():
        if tuple(v.shape) != tuple(ref_sd[k].shape):
            raise SystemExit(f"{k}: shape {tuple(v.shape)} vs reference {tuple(ref_sd[k].shape)}")
    ref.load_state_dict(mapped, strict=True)
    ids = torch.randint(0, CFG["vocab_size"], (B, N), generator=torch.Generator().manual_seed(SEED + 2))
    with torch.no_grad():
        out = ref(ids, labels=ids)
        mine, mine_loss = ours(ids, labels=ids)
    logits = out.logits.float()
    print(f"reference loss {float(out.loss):.6f}; restatement loss {float(mine_loss):.6f}; "
          f"max |logit diff| {float((mine - logits).abs().max()):.3e} (scale {float(logits.abs().max()):.3e})")
    pre, steps, states = run_with_cache(ref, ids, reference=True)
    m_pre, m_steps, m_states = run_with_cache(ours, ids, reference=False)
    print(f"with the cache: prefill max |diff| {float((m_pre - pre).abs().max()):.3e}, steps "
          f"{float((m_steps - steps).abs().max()):.3e}, states {float((m_states - states).abs().max()):.3e}")
    np.savez_compressed(
        OUT, ids=ids.numpy(), logits=logits.numpy(), loss=np.float64(float(out.loss)),
        weight_checksum=np.float64(weight_checksum(ours)), seed=np.int64(SEED),
        config=np.array(repr(sorted(CFG.items()))),
        inc_prefill_logits=pre.numpy(), inc_step_logits=steps.numpy(), inc_states=states.numpy(),
    )
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
