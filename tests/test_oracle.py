"""Pins the CPU oracle (oracle/decay_oracle.py) before anything is checked against it.

Each check is chosen so a plausible mistake in a restatement of
/root/reference/src/kilat/arc/triton_ops.py:232-247 or attention.py:344-394
fails it: closed forms catch a dropped +1e-6 or an exponent off by one, the
fp64 brute force catches wrong indexing or a transposed operand, bit-equality
with the plain-C restatement catches a fused multiply-add or a different power
routine, and test_mutants_are_caught plants such mistakes in copies of the
oracle to prove the checks see them.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from oracle import decay_oracle as O
from tests.decay_cases import assert_rounded_once, c1_inputs, c2_inputs, lam_uniform, ordered_bits, rel_err

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "decay_golden.npz")


def _lam(vals):
    return torch.tensor(vals, dtype=torch.float32)


# --------------------------------------------------------------------------
# Checks, parameterised by the scan under test: fn(lam, V) -> out
# --------------------------------------------------------------------------
def check_constant(fn) -> bool:
    """V = c everywhere: y_t = c (1 - lam + 1e-6) / (1 - lam) for every t."""
    lam = _lam([0.5, 0.9, 0.99])
    V = torch.full((1, 3, 200, 4), 1.5)
    y = fn(lam, V).double()
    l = lam.double().view(1, 3, 1, 1)
    expect = 1.5 * ((1 - l) + 1e-6) / (1 - l)
    return bool(((y - expect).abs() / expect.abs()).max() < 2e-5)


def check_impulse(fn) -> bool:
    """V = delta at t=0: y_t = lam^t (1 - lam + 1e-6) / (1 - lam^(t+1))."""
    lam = _lam([0.3, 0.8, 0.999])
    V = torch.zeros(1, 3, 64, 2)
    V[:, :, 0, :] = 1.0
    y = fn(lam, V).double()
    l = lam.double().view(1, 3, 1, 1)
    t = torch.arange(64, dtype=torch.float64).view(1, 1, 64, 1)
    expect = l**t * ((1 - l) + 1e-6) / (1 - l ** (t + 1))
    return bool(((y - expect).abs() / expect.abs()).max() < 2e-5)


def check_n1(fn) -> bool:
    """N = 1: y_0 = V_0 (1 - lam + 1e-6) / (1 - lam)."""
    g = torch.Generator().manual_seed(5)
    lam = _lam([0.1, 0.6, 0.95])
    V = torch.randn(2, 3, 1, 8, generator=g)
    y = fn(lam, V).double()
    l = lam.double().view(1, 3, 1, 1)
    expect = V.double() * ((1 - l) + 1e-6) / (1 - l)
    return bool(((y - expect).abs() / expect.abs().clamp_min(1e-12)).max() < 2e-6)


def check_bruteforce(fn) -> bool:
    """fp64 dense sum over j <= i, distinct B,H,N,D so transposes cannot hide."""
    g = torch.Generator().manual_seed(6)
    lam = lam_uniform(3, 0.6, 0.999, g)
    V = torch.randn(2, 3, 37, 5, generator=g)
    y = fn(lam, V)
    ref = torch.from_numpy(C.bruteforce_f64(lam.numpy(), V.numpy()))
    return rel_err(y, ref) < 1e-5


def check_c_bitwise(fn) -> bool:
    """Bit-equal to the plain-C restatement (fp32, H < 16)."""
    g = torch.Generator().manual_seed(7)
    lam = lam_uniform(5, 0.5, 0.9999, g)
    V = torch.randn(2, 5, 90, 8, generator=g)
    y = fn(lam, V)
    yc, _ = C.scan_f32(lam.numpy(), V.numpy())
    return np.array_equal(y.numpy().view(np.uint32), yc.view(np.uint32))


CHECKS = [check_constant, check_impulse, check_n1, check_bruteforce, check_c_bitwise]


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_oracle_passes(check):
    assert check(O.global_decay)


# --------------------------------------------------------------------------
# Planted mistakes (in copies of the oracle, on the CPU)
# --------------------------------------------------------------------------
def _mutant(kind):
    def fn(lam, V):
        B, H, N, D = V.shape
        out = torch.zeros_like(V)
        lam_b = lam.view(1, H, 1)
        if kind == "heads_reversed":
            lam_b = lam.flip(0).view(1, H, 1)
        state = torch.zeros(B, H, D, dtype=V.dtype)
        for t in range(N):
            if kind == "fused":
                state = (lam_b.double() * state.double() + V[:, :, t, :].double()).float()
            else:
                state = lam_b * state + V[:, :, t, :]
            e = t if kind == "exponent_t" else t + 1
            eps = 0.0 if kind == "no_eps" else 1e-6
            z = (1.0 - lam_b**e) / (1.0 - lam_b + eps)
            if kind == "exp_log_pow":  # the Triton variant's power: exp(e * log(lam + 1e-9))
                z = (1.0 - torch.exp(e * torch.log(lam_b + 1e-9))) / (1.0 - lam_b + eps)
            out[:, :, t, :] = state / z
        return out

    return fn


@pytest.mark.parametrize("kind", ["exponent_t", "no_eps", "heads_reversed", "fused", "exp_log_pow"])
def test_mutants_are_caught(kind):
    fn = _mutant(kind)
    failed = [c.__name__ for c in CHECKS if not c(fn)]
    assert failed, f"mutant {kind} passed every check"


# --------------------------------------------------------------------------
# Identities between the oracle's functions and edge behaviour
# --------------------------------------------------------------------------
def test_torch_and_c_scan_bitwise_c1_shape():
    lam, V = c1_inputs(B=1, N=256)
    y, s = O.scan(lam, V)
    yc, sc = C.scan_f32(lam.numpy(), V.numpy())
    assert np.array_equal(y.numpy().view(np.uint32), yc.view(np.uint32))
    assert np.array_equal(s.numpy().view(np.uint32), sc.view(np.uint32))


def test_causality_and_independence():
    lam, V = c1_inputs(B=2, N=64, H=3, D=8)
    y0 = O.global_decay(lam, V)
    V2 = V.clone()
    V2[1, 2, 40, 3] += 10.0
    y1 = O.global_decay(lam, V2)
    diff = (y0 != y1)
    assert not diff[:, :, :40].any()
    assert not diff[0].any() and not diff[1, :2].any()
    assert diff[1, 2, 40:, 3].all()
    assert not diff[1, 2, :, [0, 1, 2, 4, 5, 6, 7]].any()


def test_linearity():
    g = torch.Generator().manual_seed(8)
    lam = lam_uniform(2, 0.5, 0.99, g)
    V1 = torch.randn(1, 2, 50, 4, generator=g)
    V2 = torch.randn(1, 2, 50, 4, generator=g)
    y = O.global_decay(lam, 2.0 * V1 - 0.5 * V2)
    ylin = 2.0 * O.global_decay(lam, V1) - 0.5 * O.global_decay(lam, V2)
    assert rel_err(y, ylin) < 1e-5


def test_step_continues_the_scan_bitwise():
    lam, V = c1_inputs(B=2, N=41, H=3, D=8)
    _, s_t = O.scan(lam, V[:, :, :40])
    out, ns = O.step(lam, s_t, V[:, :, 40], 40)
    y_all, s_all = O.scan(lam, V)
    assert torch.equal(ns, s_all)
    assert torch.equal(out, y_all[:, :, 40])


def test_step_per_sequence_matches_scalar_rows():
    g = torch.Generator().manual_seed(9)
    lam = lam_uniform(3, 0.5, 0.99, g)
    s = torch.randn(3, 3, 4, generator=g)
    v = torch.randn(3, 3, 4, generator=g)
    out, ns = O.step(lam, s, v, [2, 9, 300])
    for b, tp in enumerate([2, 9, 300]):
        ob, nb = O.step(lam, s[b : b + 1], v[b : b + 1], tp)
        assert torch.equal(out[b : b + 1], ob) and torch.equal(ns[b : b + 1], nb)


def test_c_step_bitwise():
    g = torch.Generator().manual_seed(10)
    lam = lam_uniform(4, 0.5, 0.9999, g)
    s = torch.randn(3, 4, 8, generator=g) * 3
    v = torch.randn(3, 4, 8, generator=g).to(torch.bfloat16).float()
    for tp in (0, 1, 2, 3, 57, [0, 5, 4096]):
        out, ns = O.step(lam, s, v, tp)
        oc, nc = C.step_f32(lam.numpy(), s.numpy(), v.numpy(), tp)
        assert np.array_equal(out.numpy().view(np.uint32), oc.view(np.uint32)), tp
        assert np.array_equal(ns.numpy().view(np.uint32), nc.view(np.uint32)), tp


def test_seed_state_is_scan_final_state():
    lam, V = c1_inputs(B=2, N=77, H=3, D=8)
    assert torch.equal(O.seed_state(lam, V, torch.float32), O.scan(lam, V)[1])
    Vb = V.to(torch.bfloat16)
    assert torch.equal(O.seed_state(lam, Vb, torch.float32), O.scan(lam, Vb)[1])


def test_split_scan_with_carry_is_bitwise_whole():
    lam, V = c1_inputs(B=1, N=90, H=3, D=8)
    y, s = O.scan(lam, V)
    y1, s1 = O.scan(lam, V[:, :, :33])
    y2, s2 = O.scan(lam, V[:, :, 33:], init_state=s1, t_offset=33)
    assert torch.equal(torch.cat([y1, y2], 2), y) and torch.equal(s2, s)


def test_bf16_promotes_to_fp32_state():
    lam, V = c1_inputs(B=1, N=20, H=2, D=8)
    Vb = V.to(torch.bfloat16)
    y, s = O.scan(lam, Vb)
    y32, s32 = O.scan(lam, Vb.float())
    assert s.dtype == torch.float32 and torch.equal(s, s32)
    assert y.dtype == torch.bfloat16 and torch.equal(y, y32.to(torch.bfloat16))


def test_lambda_edges():
    V = torch.randn(1, 2, 5, 4, generator=torch.Generator().manual_seed(11))
    V[0, 1, 0, 0] = 0.0
    y = O.global_decay(torch.tensor([0.0, 1.0]), V)
    # lam = 0: z = 1 / (1 + 1e-6f) at every t
    z0 = torch.tensor(1.0) / (torch.tensor(1.0) + 1e-6)
    assert torch.equal(y[0, 0], V[0, 0] / z0)
    # lam = 1: z = 0, so s/0 = +-inf, 0/0 = nan
    assert torch.isnan(y[0, 1, 0, 0])
    assert torch.isinf(y[0, 1, 1:]).all() and torch.isinf(y[0, 1, 0, 1:]).all()


def test_golden_fixtures_reproduce():
    d = np.load(GOLDEN)

    def t(name, bf16=False):
        a = d[name]
        if bf16:
            return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
        return torch.from_numpy(a.copy())

    out, fin = O.scan(t("scan_f32_lam"), t("scan_f32_V"))
    assert torch.equal(out, t("scan_f32_out")) and torch.equal(fin, t("scan_f32_final"))
    out, fin = O.scan(t("scan_bf16_lam"), t("scan_bf16_V", True))
    assert torch.equal(out, t("scan_bf16_out", True)) and torch.equal(fin, t("scan_bf16_final"))
    out, fin = O.scan(t("scan_init_lam"), t("scan_init_V"), init_state=t("scan_init_init"),
                      t_offset=int(d["scan_init_offset"]))
    assert torch.equal(out, t("scan_init_out")) and torch.equal(fin, t("scan_init_final"))
    out, fin = O.scan(t("edge_lam"), t("edge_V"))
    assert torch.equal(torch.isnan(out), torch.isnan(t("edge_out")))
    m = ~torch.isnan(out)
    assert torch.equal(out[m], t("edge_out")[m])
    out, ns = O.step(t("step_lam"), t("step_state"), t("step_v", True), int(d["step_tpos_scalar"]))
    assert torch.equal(out, t("step_out")) and torch.equal(ns, t("step_new_state"))
    out, ns = O.step(t("step_lam"), t("step_state"), t("step_v", True), [int(x) for x in d["step_tpos"]])
    assert torch.equal(out, t("step_out_vec")) and torch.equal(ns, t("step_new_state_vec"))


# --------------------------------------------------------------------------
# Gradients of the oracle (torch autograd through the restatement of
# triton_ops.py:240-246) -- the reference for the GPU backward.
# --------------------------------------------------------------------------
def _loss(lam, V, gy, init=None, gfin=None, t_offset=0):
    y, fin = O.scan(lam, V, init_state=init, t_offset=t_offset)
    total = (y * gy).sum()
    if gfin is not None:
        total = total + (fin * gfin).sum()
    return total


def test_oracle_grad_dv_closed_form():
    """dL/dV_t = sum_{k>=t} lam^(k-t) gy_k / z_k (fp64, brute force)."""
    g = torch.Generator().manual_seed(30)
    lam = lam_uniform(3, 0.5, 0.999, g).double()
    V = torch.randn(2, 3, 23, 4, generator=g, dtype=torch.float64, requires_grad=True)
    gy = torch.randn(2, 3, 23, 4, generator=g, dtype=torch.float64)
    _loss(lam, V, gy).backward()
    l = lam.view(1, 3, 1, 1)
    t = torch.arange(23, dtype=torch.float64)
    z = ((1 - l ** (t.view(1, 1, 23, 1) + 1)) / ((1 - l) + 1e-6))
    u = gy / z
    ref = torch.zeros_like(u)
    for ti in range(23):
        for k in range(ti, 23):
            ref[:, :, ti] += l[:, :, 0] ** (k - ti) * u[:, :, k]
    assert torch.allclose(V.grad, ref, rtol=1e-12, atol=1e-12)


def test_oracle_grad_dlam_and_init_finite_difference():
    """Autograd dlam and d(init) against central differences (fp64)."""
    g = torch.Generator().manual_seed(31)
    lam = lam_uniform(2, 0.6, 0.99, g).double().requires_grad_(True)
    V = torch.randn(1, 2, 30, 3, generator=g, dtype=torch.float64)
    init = torch.randn(1, 2, 3, generator=g, dtype=torch.float64, requires_grad=True)
    gy = torch.randn(1, 2, 30, 3, generator=g, dtype=torch.float64)
    gfin = torch.randn(1, 2, 3, generator=g, dtype=torch.float64)
    _loss(lam, V, gy, init, gfin, t_offset=4).backward()
    eps = 1e-6
    for h in range(2):
        lp, lm = lam.detach().clone(), lam.detach().clone()
        lp[h] += eps
        lm[h] -= eps
        fd = (_loss(lp, V, gy, init.detach(), gfin, 4) - _loss(lm, V, gy, init.detach(), gfin, 4)) / (2 * eps)
        assert abs(float(fd) - float(lam.grad[h])) <= 1e-6 * max(1.0, abs(float(fd)))
    ip, im = init.detach().clone(), init.detach().clone()
    ip[0, 1, 2] += eps
    im[0, 1, 2] -= eps
    fd = (_loss(lam.detach(), V, gy, ip, gfin, 4) - _loss(lam.detach(), V, gy, im, gfin, 4)) / (2 * eps)
    assert abs(float(fd) - float(init.grad[0, 1, 2])) <= 1e-6 * max(1.0, abs(float(fd)))


@pytest.mark.parametrize("case", ["plain", "init_gfin_offset"])
def test_adjoint_grads_match_autograd(case):
    """scan_grads_f64 (the adjoint recurrence, for lengths autograd's graph
    cannot hold) against fp64 autograd through the scan restatement, which the
    two tests above pin to a closed form and to finite differences."""
    g = torch.Generator().manual_seed(32)
    lam = lam_uniform(3, 0.5, 0.999, g)
    V = torch.randn(2, 3, 41, 5, generator=g)
    gy = torch.randn(2, 3, 41, 5, generator=g)
    init = gfin = None
    t_offset = 0
    if case != "plain":
        init = torch.randn(2, 3, 5, generator=g)
        gfin = torch.randn(2, 3, 5, generator=g)
        t_offset = 7
    lam64 = lam.double().requires_grad_(True)
    V64 = V.double().requires_grad_(True)
    init64 = init.double().requires_grad_(True) if init is not None else None
    _loss(lam64, V64, gy.double(), init64, gfin.double() if gfin is not None else None, t_offset).backward()
    dv, dl, di = O.scan_grads_f64(lam, V, gy, init_state=init, gfin=gfin, t_offset=t_offset)
    assert torch.allclose(dv, V64.grad, rtol=1e-12, atol=1e-13)
    assert torch.allclose(dl, lam64.grad, rtol=1e-11, atol=0)
    if init is not None:
        assert torch.allclose(di, init64.grad, rtol=1e-12, atol=1e-13)


def test_e2e_model_runs_on_cpu_with_oracle_decay():
    """Host-side check of the end-to-end restatement (shapes, tied head, finite loss)."""
    from tests.e2e_model import E2EConfig, KilatE2E

    torch.manual_seed(42)
    cfg = E2EConfig(vocab_size=128, n_embd=32, n_layer=2, n_head=4, num_experts=4, active_experts=2)
    model = KilatE2E(cfg, O.global_decay).eval()
    assert model.lm_head.weight is model.wte.weight
    assert model.layers[0].attn.n_global == 2 and model.layers[0].attn.latent == 8
    assert len(model.layers[0].mlp.shared_experts) == 2
    ids = torch.randint(0, 128, (2, 9))
    with torch.no_grad():
        logits, loss = model(ids, labels=ids)
    assert logits.shape == (2, 9, 128) and torch.isfinite(loss)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rounding_check_catches_truncation_and_double_rounding(dtype):
    """The check the GPU tests apply to 2-byte outputs (assert_rounded_once):
    the oracle's 2-byte output is its fp32 output rounded once to nearest-even
    (what out = zeros_like(V) does, triton_ops.py:240,246); the check accepts
    it, and values one ulp off on a few elements; it rejects a truncating
    store (about half the elements off) and a double rounding through a
    narrower mantissa."""
    lam, V = c2_inputs(seed=7, B=2, N=600, H=4)
    V = V.float().to(dtype)
    y2, _ = O.scan(lam, V)
    y32, _ = O.scan(lam, V, out_dtype=torch.float32)
    assert torch.equal(y2, y32.to(dtype))  # one rounding, nearest-even
    assert_rounded_once(y2, y32, "oracle")
    # one ulp off on 1 element in 2000: still accepted
    flat = ordered_bits(y2).reshape(-1).clone()
    flat[::2000] += 1
    near = torch.where(flat < 0, (-flat) | 0x8000, flat).to(torch.int16).view(dtype).reshape(y2.shape)
    assert_rounded_once(near, y32, "one ulp off on a few elements")
    # a truncating store: the fp32 value cut towards zero to the type's significand
    sig = 8 if dtype == torch.bfloat16 else 11
    m, e = torch.frexp(y32.double())
    trunc = (torch.trunc(m * 2 ** sig) / 2 ** sig * torch.pow(2.0, e.double())).to(dtype)
    d = (ordered_bits(trunc) - ordered_bits(y2)).abs()
    assert 0.3 <= float((d != 0).double().mean()) <= 0.7
    with pytest.raises(AssertionError):
        assert_rounded_once(trunc, y32, "truncated")
    # rounding twice: first to a significand 3 bits shorter, then to the type
    coarse = (torch.round(m * 2 ** (sig - 3)) / 2 ** (sig - 3) * torch.pow(2.0, e.double())).float()
    with pytest.raises(AssertionError):
        assert_rounded_once(coarse.to(dtype), y32, "rounded twice")

