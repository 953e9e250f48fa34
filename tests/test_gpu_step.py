"""GPU parity of the fused decode step (kdecay_step via kilat_amd.decay_step)
against the oracle restatement of /root/reference/src/kilat/arc/attention.py:344-360.

The state must match bit for bit after every step (fp32, same layout
[B,H,D]); the normalised output too, except where the double-precision power
inside z may round one ulp apart (checked as <= 1 ulp).
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import kilat_amd
from oracle import c_oracle as C
from oracle import decay_oracle as O
from tests.decay_cases import c3_inputs, lam_uniform

pytestmark = pytest.mark.gpu


def ulps(a: torch.Tensor, b: torch.Tensor) -> np.ndarray:
    x = a.detach().cpu().float().numpy().view(np.int32).astype(np.int64)
    y = b.detach().cpu().float().numpy().view(np.int32).astype(np.int64)
    return np.abs(x - y)


def test_step_scalar_tpos_bitwise(hip_device, kdecay_lib):
    g = torch.Generator().manual_seed(20)
    lam = lam_uniform(6, 0.5, 0.9999, g)
    state = torch.randn(8, 6, 64, generator=g) * 4
    # 65534 and 65535 straddle the kernel's switch from its unrolled power
    # (exponent t_pos + 1 below 2^16) to the general loop.
    for tp in (0, 1, 2, 3, 4, 17, 1000, 65534, 65535, 100000, 1 << 20, (1 << 31) + 5):
        v = torch.randn(8, 6, 64, generator=g).to(torch.bfloat16)
        print(f"  step t_pos={tp}", flush=True)
        out, ns = kilat_amd.decay_step(lam.to(hip_device), state.to(hip_device), v.to(hip_device), tp)
        ro, rs = O.step(lam, state, v, tp)
        torch.cuda.synchronize()
        assert torch.equal(ns.cpu(), rs), tp
        assert out.dtype == torch.float32 and ulps(out, ro).max() <= 1, tp
        state = rs


def test_step_mixed_positions_in_one_wavefront(hip_device, kdecay_lib):
    """Per-sequence positions on both sides of the unrolled-power limit in the
    same wavefronts (4 sequences of 16 threads each share one)."""
    g = torch.Generator().manual_seed(21)
    lam = lam_uniform(3, 0.5, 0.9999, g)
    tps = [0, 1, 2, 3, 4, 65534, 65535, 70000, 5, 1 << 18, 123, 65533, 9, 65536, 2, 40000]
    B = len(tps)
    state = torch.randn(B, 3, 64, generator=g) * 4
    v = torch.randn(B, 3, 64, generator=g).to(torch.bfloat16)
    tpos = torch.tensor(tps, dtype=torch.int32)
    out, ns = kilat_amd.decay_step(lam.to(hip_device), state.to(hip_device), v.to(hip_device), tpos.to(hip_device))
    ro, rs = O.step(lam, state, v, tps)
    torch.cuda.synchronize()
    assert torch.equal(ns.cpu(), rs)
    assert ulps(out, ro).max() <= 1


def test_step_randomized(hip_device, kdecay_lib):
    """A seeded sweep of 40 random decode steps against the C restatement:
    v and out dtypes, batch and head counts, head dims including odd ones
    (the per-element kernel), scalar or per-sequence positions up to 2^20,
    in place or not.  The state is bit-identical; the output is within one
    ulp in fp32 (z's power may round one ulp apart) and one rounding of the
    output dtype otherwise."""
    rng = np.random.default_rng(77)
    dts = [torch.float32, torch.bfloat16, torch.float16]
    for case in range(40):
        vdt, odt = dts[rng.integers(3)], dts[rng.integers(3)]
        B, H = int(rng.integers(1, 65)), int(rng.integers(1, 17))
        D = int(rng.choice([1, 3, 16, 24, 33, 64, 100, 128, 256]))
        per_seq = bool(rng.integers(2))
        tps = [int(rng.choice([0, 1, 2, 3, int(rng.integers(4, 70000)), int(rng.integers(0, 1 << 20))])) for _ in range(B)]
        in_place = bool(rng.integers(2))
        print(f"  step case {case}: v={vdt} out={odt} B={B} H={H} D={D} per_seq={per_seq} in_place={in_place}", flush=True)
        g = torch.Generator().manual_seed(900 + case)
        lam = (0.3 + (0.9999 - 0.3) * torch.rand(H, generator=g)).float()
        state = torch.randn(B, H, D, generator=g) * 3
        v = torch.randn(B, H, D, generator=g).to(vdt)
        t_pos = torch.tensor(tps, dtype=torch.int32) if per_seq else tps[0]
        st_d = state.to(hip_device)
        out, ns = kilat_amd.decay_step(lam.to(hip_device), st_d, v.to(hip_device),
                                       t_pos.to(hip_device) if per_seq else t_pos,
                                       out_dtype=odt, new_state=st_d if in_place else None)
        torch.cuda.synchronize()
        ro, rs = C.step_f32(lam.numpy(), state.numpy(), v.float().numpy(), tps if per_seq else tps[0])
        assert torch.equal(ns.cpu(), torch.from_numpy(rs)), f"case {case}: state"
        if odt == torch.float32:
            assert ulps(out, torch.from_numpy(ro)).max() <= 1, f"case {case}: out"
        else:
            # Both sides round an fp32 value once to the output type; the fp32
            # values are at most 1 ulp apart, so the rounded ones are at most
            # one step of the output type apart (compared as bit patterns,
            # which also covers fp16's subnormal outputs).
            r = torch.from_numpy(ro).to(odt)
            a16 = out.cpu().view(torch.int16).to(torch.int32)
            b16 = r.view(torch.int16).to(torch.int32)
            assert int((a16 - b16).abs().max()) <= 1, f"case {case}: out"


def test_c3_decode_128_steps_bitwise_state(hip_device, kdecay_lib):
    lam, lengths, prefixes, v_steps = c3_inputs()
    S, H, D = len(prefixes), lam.numel(), v_steps.shape[-1]
    # prefixes pre-scanned on the CPU (C oracle: bit-equal to the torch restatement)
    state = np.concatenate([C.scan_f32(lam.numpy(), p.float().numpy())[1] for p in prefixes], 0)
    state = torch.from_numpy(state)
    assert state.shape == (S, H, D)
    dev_state = state.to(hip_device)
    dev_lam = lam.to(hip_device)
    worst = 0
    for k in range(v_steps.shape[0]):
        tpos = lengths + k
        v = v_steps[k]
        out, dev_state = kilat_amd.decay_step(dev_lam, dev_state, v.to(hip_device), tpos.to(hip_device))
        ro, rs = C.step_f32(lam.numpy(), state.numpy(), v.float().numpy(), tpos.tolist())
        if k == 0:  # the torch restatement gives the same bits (per-sequence positions)
            ro_t, rs_t = O.step(lam, state, v, tpos.tolist())
            assert torch.equal(rs_t, torch.from_numpy(rs)) and torch.equal(ro_t, torch.from_numpy(ro))
        torch.cuda.synchronize()
        rs = torch.from_numpy(rs)
        assert torch.equal(dev_state.cpu(), rs), f"state differs at step {k}"
        worst = max(worst, int(ulps(out, torch.from_numpy(ro)).max()))
        state = rs
    assert worst <= 1


def test_step_in_place_and_out_dtypes(hip_device, kdecay_lib):
    g = torch.Generator().manual_seed(21)
    lam = lam_uniform(4, 0.5, 0.999, g).to(hip_device)
    s0 = torch.randn(3, 4, 32, generator=g).to(hip_device)
    v = torch.randn(3, 4, 32, generator=g).to(hip_device)
    out_ref, ns_ref = kilat_amd.decay_step(lam, s0, v, 9)
    s = s0.clone()
    out, ns = kilat_amd.decay_step(lam, s, v, 9, new_state=s)
    torch.cuda.synchronize()
    assert ns.data_ptr() == s.data_ptr() and torch.equal(s, ns_ref) and torch.equal(out, out_ref)
    ob, _ = kilat_amd.decay_step(lam, s0, v, 9, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(ob, out_ref.to(torch.bfloat16))


def test_step_golden_fixture(hip_device, kdecay_lib):
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "decay_golden.npz"))
    lam = torch.from_numpy(d["step_lam"].copy())
    state = torch.from_numpy(d["step_state"].copy())
    v = torch.from_numpy(d["step_v"].view(np.int16).copy()).view(torch.bfloat16)
    out, ns = kilat_amd.decay_step(lam.to(hip_device), state.to(hip_device), v.to(hip_device),
                                   int(d["step_tpos_scalar"]))
    torch.cuda.synchronize()
    assert torch.equal(ns.cpu(), torch.from_numpy(d["step_new_state"]))
    assert ulps(out, torch.from_numpy(d["step_out"])).max() <= 1
    tp = torch.from_numpy(d["step_tpos"].astype(np.int32)).to(hip_device)
    out, ns = kilat_amd.decay_step(lam.to(hip_device), state.to(hip_device), v.to(hip_device), tp)
    torch.cuda.synchronize()
    assert torch.equal(ns.cpu(), torch.from_numpy(d["step_new_state_vec"]))
    assert ulps(out, torch.from_numpy(d["step_out_vec"])).max() <= 1


def test_scan_then_steps_continue_the_sequence(hip_device, kdecay_lib):
    """Prefill with the scan's final state, then decode: equals one longer scan."""
    g = torch.Generator().manual_seed(22)
    lam = lam_uniform(3, 0.5, 0.999, g)
    V = torch.randn(2, 3, 520, 64, generator=g)
    dev = hip_device
    _, s = kilat_amd.global_decay_scan(lam.to(dev), V[:, :, :500].to(dev), return_final_state=True)
    outs = []
    for t in range(500, 520):
        o, s = kilat_amd.decay_step(lam.to(dev), s, V[:, :, t].to(dev), t)
        outs.append(o)
    torch.cuda.synchronize()
    ref, sref = O.scan(lam, V)
    y = torch.stack(outs, 2).cpu()
    assert float(((y - ref[:, :, 500:]).abs().amax() / ref[:, :, 500:].abs().amax())) <= 1e-5
    assert float(((s.cpu() - sref).abs().amax() / sref.abs().amax())) <= 1e-5


def test_step_after_beam_reorder(hip_device, kdecay_lib):
    """Beam search reorders each layer's cached state with index_select(0, beam_idx)
    (/root/reference/src/kilat/pipeline/generation/generation_mixin.py:162-198).
    The state stays fp32 [B,H,D] contiguous, so the step after a reorder is the
    reference's step on the reordered state, bit for bit."""
    g = torch.Generator().manual_seed(23)
    lam = lam_uniform(4, 0.5, 0.999, g)
    V = torch.randn(6, 4, 300, 64, generator=g).to(torch.bfloat16)
    dev = hip_device
    _, s = kilat_amd.global_decay_scan(lam.to(dev), V.to(dev), return_final_state=True)
    beam_idx = torch.tensor([2, 2, 0, 5, 1, 1])
    s_re = s.index_select(0, beam_idx.to(dev))
    v = torch.randn(6, 4, 64, generator=g).to(torch.bfloat16)
    out, ns = kilat_amd.decay_step(lam.to(dev), s_re, v.to(dev), 300)
    torch.cuda.synchronize()
    ro, rs = O.step(lam, s.cpu().index_select(0, beam_idx), v, 300)
    assert torch.equal(ns.cpu(), rs)
    assert ulps(out, ro).max() <= 1


def test_step_scalar_fallback_layouts(hip_device, kdecay_lib):
    """Head dims that are not a multiple of 4, and a misaligned state, use the
    one-element-per-thread kernel; results are the same bits."""
    g = torch.Generator().manual_seed(23)
    lam = lam_uniform(3, 0.5, 0.999, g)
    for D in (6, 13, 64):
        state = torch.randn(5, 3, D, generator=g) * 3
        v = torch.randn(5, 3, D, generator=g).to(torch.bfloat16)
        dev_state = state.to(hip_device)
        if D == 64:  # state at a 4-byte offset: not 16-byte aligned
            buf = torch.zeros(state.numel() + 1, device=hip_device)
            buf[1:].copy_(state.reshape(-1).to(hip_device))
            dev_state = buf[1:].view(5, 3, D)
        print(f"  step fallback D={D}", flush=True)
        out, ns = kilat_amd.decay_step(lam.to(hip_device), dev_state, v.to(hip_device), 11)
        torch.cuda.synchronize()
        ro, rs = O.step(lam, state, v, 11)
        assert torch.equal(ns.cpu(), rs), D
        assert ulps(out, ro).max() <= 1, D


def test_graph_capture_scan_and_step_replays(hip_device, kdecay_lib):
    """The scan (its workspace advances its own epoch) and the decode step
    replay correctly from a HIP graph: several replays, eager work between
    them, every replay checked against the eager result."""
    g = torch.Generator().manual_seed(24)
    lam = lam_uniform(4, 0.5, 0.999, g).to(hip_device)
    V = torch.randn(2, 4, 3000, 64, generator=g).to(torch.bfloat16).to(hip_device)
    s0 = torch.randn(2, 4, 64, generator=g).to(hip_device)
    v = torch.randn(2, 4, 64, generator=g).to(torch.bfloat16).to(hip_device)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        # eager warm-up on the capture stream creates the scan's workspace outside the capture
        y_ref, fin_ref = kilat_amd.global_decay_scan(lam, V, return_final_state=True)
        o_ref, ns_ref = kilat_amd.decay_step(lam, fin_ref, v, 3000)
        y = torch.empty_like(y_ref)
        fin = torch.empty_like(fin_ref)
        o = torch.empty_like(o_ref)
        ns = torch.empty_like(ns_ref)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            y2, fin2 = kilat_amd.global_decay_scan(lam, V, return_final_state=True)
            o2, ns2 = kilat_amd.decay_step(lam, fin2, v, 3000)
            y.copy_(y2)
            fin.copy_(fin2)
            o.copy_(o2)
            ns.copy_(ns2)
    torch.cuda.synchronize()
    # The eager results the replays are compared with, against the oracle:
    # the scan to the bf16 tolerance, the step's state bit for bit and its
    # output within one ulp (the double-precision power inside z).
    lam_c = lam.cpu()
    ref, sref = O.scan(lam_c, V.cpu())
    assert float((y_ref.cpu().double() - ref.double()).abs().max()) <= 2e-2
    assert float(((fin_ref.cpu() - sref).abs().max() / sref.abs().max())) <= 1e-5
    ro, rs = O.step(lam_c, fin_ref.cpu(), v.cpu(), 3000)
    assert torch.equal(ns_ref.cpu(), rs)
    assert ulps(o_ref, ro).max() <= 1
    for r in range(4):
        print(f"  graph replay {r}", flush=True)
        y.zero_(); o.zero_(); ns.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref) and torch.equal(fin, fin_ref), r
        assert torch.equal(o, o_ref) and torch.equal(ns, ns_ref), r
        # eager launches between replays share the workspace of the capture stream
        with torch.cuda.stream(stream):
            ye = kilat_amd.global_decay_scan(lam, V)
        torch.cuda.synchronize()
        assert torch.equal(ye, y_ref)
    assert kilat_amd.workspace_error(V) == 0


def fresh_workspace_stream(dev):
    """A side stream with no workspace yet.  torch hands out streams from a
    small pool, so an earlier test may have used this one: its workspace is
    retired (kept alive, as the shim does) rather than reused."""
    from kilat_amd import triton_ops

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    old = triton_ops._workspaces.pop((dev.index, stream.cuda_stream), None)
    if old is not None:
        triton_ops._retired.append(old)
    return stream


def test_graph_survives_workspace_growth(hip_device, kdecay_lib):
    """A graph captured with the stream's workspace keeps writing to that
    buffer: a later eager scan that needs a larger workspace on the same
    stream must not free it.  Capture, grow the workspace with a longer eager
    scan, let the allocator hand out fresh blocks, then replay and check the
    replay against the oracle."""
    from kilat_amd import triton_ops

    g = torch.Generator().manual_seed(25)
    lam = lam_uniform(4, 0.5, 0.999, g)
    V = torch.randn(2, 4, 3000, 64, generator=g).to(torch.bfloat16)
    Vd, lamd = V.to(hip_device), lam.to(hip_device)
    stream = fresh_workspace_stream(hip_device)
    with torch.cuda.stream(stream):
        kilat_amd.global_decay_scan(lamd, Vd)  # workspace sized for N=3000
        y = torch.empty_like(Vd)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            y.copy_(kilat_amd.global_decay_scan(lamd, Vd))
        key = (hip_device.index, stream.cuda_stream)
        captured = triton_ops._workspaces[key].data_ptr()
        # 40000 rows need a larger workspace: the captured one is replaced
        Vl = torch.randn(2, 4, 40000, 64, generator=g).to(torch.bfloat16)
        yl = kilat_amd.global_decay_scan(lamd, Vl.to(hip_device))
        assert triton_ops._workspaces[key].data_ptr() != captured
        assert any(w.data_ptr() == captured for w in triton_ops._retired)
        filler = [torch.full((1 << 20,), 7, dtype=torch.uint8, device=hip_device) for _ in range(8)]
    torch.cuda.synchronize()
    ref = O.global_decay(lam, V)
    assert float((yl.cpu().double() - O.global_decay(lam, Vl).double()).abs().max()) <= 2e-2
    for r in range(3):
        print(f"  replay after growth {r}", flush=True)
        y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert float((y.cpu().double() - ref.double()).abs().max()) <= 2e-2, r
    assert all(int(f[0]) == 7 and int(f[-1]) == 7 for f in filler)


def test_workspace_growth_inside_capture_raises(hip_device, kdecay_lib):
    """A shape first seen inside a stream capture would need a new workspace
    there: the shim raises with advice instead of allocating in the capture;
    after reserve_workspace the same capture succeeds."""
    g = torch.Generator().manual_seed(26)
    lam = lam_uniform(3, 0.5, 0.999, g).to(hip_device)
    V = torch.randn(2, 3, 5000, 64, generator=g).to(torch.bfloat16).to(hip_device)
    stream = fresh_workspace_stream(hip_device)
    with torch.cuda.stream(stream):
        graph = torch.cuda.CUDAGraph()
        with pytest.raises(RuntimeError, match="reserve_workspace"):
            with torch.cuda.graph(graph, stream=stream):
                kilat_amd.global_decay_scan(lam, V)
        assert kilat_amd.reserve_workspace(2, 3, 5000, 64, torch.bfloat16) > 0
        y = torch.empty_like(V)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            y.copy_(kilat_amd.global_decay_scan(lam, V))
    torch.cuda.synchronize()
    ref = O.global_decay(lam.cpu(), V.cpu())
    for r in range(2):
        y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert float((y.cpu().double() - ref.double()).abs().max()) <= 2e-2, r


@pytest.mark.parametrize("B", [8, 256])
def test_decode_token_all_layers_in_one_graph(hip_device, kdecay_lib, B):
    """One token's decay work through every layer of the C5 model (12 layers
    x 6 heads x 64 channels), captured once in a HIP graph and replayed per
    token, as the reference's decode loop runs one model forward per token
    (generation_mixin.py:484-509) with each layer's inline update
    (attention.py:344-360).  The positions live in device memory and advance
    inside the graph.  Every layer's state after every token is checked bit
    for bit against the oracle's step, and its output within one ulp."""
    L, H, D, T = 12, 6, 64, 6
    g = torch.Generator().manual_seed(27 + B)
    lams = [lam_uniform(H, 0.5, 0.9999, g) for _ in range(L)]
    states = [torch.randn(B, H, D, generator=g) for _ in range(L)]
    vs = torch.randn(T, L, B, H, D, generator=g).to(torch.bfloat16)
    tpos0 = torch.randint(1, 2049, (B,), generator=g, dtype=torch.int32)
    lam_d = [l.to(hip_device) for l in lams]
    st_d = [s.to(hip_device) for s in states]
    v_in = torch.empty(L, B, H, D, dtype=torch.bfloat16, device=hip_device)
    outs = torch.empty(L, B, H, D, device=hip_device)
    tpos = tpos0.to(hip_device)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for l in range(L):
                kilat_amd.decay_step(lam_d[l], st_d[l], v_in[l], tpos, out=outs[l], new_state=st_d[l])
            tpos.add_(1)
    torch.cuda.synchronize()
    ref_states = [s.clone() for s in states]
    for t in range(T):
        v_in.copy_(vs[t].to(hip_device))
        graph.replay()
        torch.cuda.synchronize()
        for l in range(L):
            ro, ref_states[l] = O.step(lams[l], ref_states[l], vs[t, l], (tpos0 + t).tolist())
            assert torch.equal(st_d[l].cpu(), ref_states[l]), (t, l)
            assert ulps(outs[l], ro).max() <= 1, (t, l)
    assert torch.equal(tpos.cpu(), tpos0 + T)


def test_step_float64_v_and_out(hip_device, kdecay_lib):
    """float64 v_t is rounded to fp32 once (the state is fp32, as for every
    type) and a float64 out holds the fp32 result widened: equal bits to the
    same step on v_t rounded to fp32; within fp32 rounding of the oracle's
    step in float64."""
    g = torch.Generator().manual_seed(640)
    lam = lam_uniform(6, 0.5, 0.9999, g)
    dev = hip_device
    state = torch.randn(8, 6, 64, generator=g) * 4
    v = torch.randn(8, 6, 64, generator=g, dtype=torch.float64)
    for tp in (0, 5, 4095):
        print(f"  step float64 t_pos={tp}", flush=True)
        out, ns = kilat_amd.decay_step(lam.to(dev), state.to(dev), v.to(dev), tp, out_dtype=torch.float64)
        out32, ns32 = kilat_amd.decay_step(lam.to(dev), state.to(dev), v.float().to(dev), tp)
        torch.cuda.synchronize()
        assert out.dtype == torch.float64 and ns.dtype == torch.float32
        assert torch.equal(ns, ns32) and torch.equal(out, out32.double())
        ro, rs = O.step(lam, state, v, tp)
        assert ro.dtype == torch.float64
        assert float((out.cpu() - ro).abs().max() / ro.abs().max()) <= 1e-6
        assert float((ns.cpu().double() - rs).abs().max() / rs.abs().max()) <= 1e-6
