"""MI355X drop-in for ``kilat.arc.triton_ops`` — the global-decay path.

``triton_global_decay(lam_scores, V)`` keeps the reference's name, argument
order, output allocation and dtype
(/root/reference/src/kilat/arc/triton_ops.py:249-330) and runs the gfx950
chunked scan of libkdecay.so on torch's current stream.  ``decay_step`` is the
reference's inline incremental update (/root/reference/src/kilat/arc/
attention.py:344-360) as one launch for the whole batch.
``global_decay_scan`` exposes the library's extensions: a carry-in state, the
final unnormalised state (the decode-cache seed the reference computes in a
Python loop, attention.py:383-394), a position offset for chunked prefill and
an fp32 output for bf16/fp16 input.

Only HIP tensors are accepted.  There is no CPU path here: a CPU tensor, or a
missing libkdecay.so, raises.  (A Kilat model that runs on the CPU is simply
not patched by kilat_amd.integration and keeps Kilat's own function.)
"""
from __future__ import annotations

import contextlib
from typing import Optional, Tuple, Union

import torch

from . import _lib

_DTYPE_CODE = {
    torch.float32: _lib.KDECAY_F32,
    torch.bfloat16: _lib.KDECAY_BF16,
    torch.float16: _lib.KDECAY_F16,
    torch.float64: _lib.KDECAY_F64,
}


# Channels of one full 128-byte channel group, per element type.
_GROUP = {torch.float32: 32, torch.bfloat16: 64, torch.float16: 64, torch.float64: 16}


def chunked_head_dim(D: int, dtype: torch.dtype) -> bool:
    """Head dims the chunked kernels take as they are: 16, 32, or a multiple of
    one 128-byte channel group (64 bf16/fp16, 32 fp32 or 16 fp64 channels).  Other head
    dims are zero-padded to the next such size on the way in (channels are
    independent, so the padding changes no value) and sliced on the way out."""
    return D == 16 or D == 32 or (D > 0 and D % _GROUP[dtype] == 0)


def _padded_head_dim(D: int, dtype: torch.dtype) -> int:
    if D <= 16:
        return 16
    if D <= 32:
        return 32
    full = _GROUP[dtype]
    return -(-D // full) * full

# One zero-initialised workspace per (device, stream); the kernels keep it
# consistent from launch to launch, so it is never cleared again.
_workspaces: dict = {}
# Workspaces replaced by a larger one.  A HIP graph captured with a workspace
# keeps its raw address, so a workspace that was ever handed to a launch is
# never freed: it stays referenced here for the life of the process.
_retired: list = []


def _require_hip(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"kilat_amd: {name} must be a torch.Tensor")
    if not t.is_cuda:
        raise RuntimeError(
            f"kilat_amd: {name} is on {t.device}; the kilat_amd decay kernels run on HIP devices only "
            "(the reference's _cpu_global_decay serves CPU tensors)"
        )


def _dtype_code(t: torch.Tensor, name: str) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"kilat_amd: {name} dtype {t.dtype} is not float32/bfloat16/float16/float64") from None


def _vector_layout_ok(t: torch.Tensor) -> bool:
    """The chunked kernel's layout rule: d-stride 1, 16-byte base, and every
    other stride a multiple of 16 bytes (size-1 dims excepted).  Called only
    for head dims the chunked kernels take, whose rows are whole 16-byte
    vectors."""
    if t.data_ptr() & 15:
        return False
    vw = 16 // t.element_size()
    sz, st = t.shape, t.stride()
    return ((st[3] == 1 or sz[3] == 1) and (st[2] % vw == 0 or sz[2] == 1) and (st[1] % vw == 0 or sz[1] == 1)
            and (st[0] % vw == 0 or sz[0] == 1))


def _bwd_rows_fit(t: torch.Tensor) -> bool:
    """The backward kernel's addressing rule: it reads one chunk of rows of V
    and of the upstream gradient through 32-bit byte offsets, so a chunk's
    rows must span less than 2^31 bytes (the library rejects other row
    strides).  A chunk holds at most 4 wavefronts x (64 lanes / lanes per
    row) x 16 rows per lane; the bound below uses that largest chunk, so a
    tensor that passes is accepted whatever chunk size the library picks
    (whole 256-byte rows, 16 lanes each, make 256-row chunks: fewer rows)."""
    B, H, N, D = t.shape
    es = t.element_size()
    lanes_per_row = min(D, 128 // es) * es // 16
    if N <= 1 or lanes_per_row < 1:
        return True
    max_rows = 4 * (64 // lanes_per_row) * 16
    return max_rows * t.stride(2) * es <= 0x7FFFFFFF


if hasattr(torch._C, "_cuda_getCurrentRawStream"):
    def _stream_ptr(device: torch.device) -> int:
        """The raw handle of torch's current stream on `device`."""
        return torch._C._cuda_getCurrentRawStream(device.index)
else:  # pragma: no cover - the public route, one Stream object per call
    def _stream_ptr(device: torch.device) -> int:
        return torch.cuda.current_stream(device).cuda_stream


_SAME_DEVICE = contextlib.nullcontext()


def _on_device(device: torch.device):
    """torch.cuda.device(device), or nothing when it is already current."""
    return _SAME_DEVICE if device.index == torch.cuda.current_device() else torch.cuda.device(device)


_ws_bytes_cache: dict = {}


def _fwd_workspace_bytes(lib, B: int, H: int, N: int, D: int, v_code: int) -> int:
    key = (B, H, N, D, v_code)
    n = _ws_bytes_cache.get(key)
    if n is None:
        if len(_ws_bytes_cache) > 1024:
            _ws_bytes_cache.clear()
        n = _ws_bytes_cache[key] = lib.kdecay_scan_workspace_bytes(B, H, N, D, v_code)
    return n


def _workspace(device: torch.device, stream: int, nbytes: int) -> Optional[torch.Tensor]:
    """The look-back workspace of (device, stream), grown to `nbytes` if needed.

    Growing allocates and zeroes a new buffer, which must not happen inside a
    stream capture (the buffer would belong to the graph's memory pool and
    its zeroing would be replayed); that raises instead.  The replaced buffer
    is kept alive (_retired): graphs captured earlier still write to it.
    """
    if nbytes == 0:
        return None
    key = (device.index, stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(
                f"kilat_amd: this launch needs a decay-scan workspace of {nbytes} bytes on the stream being "
                f"captured, which has {0 if ws is None else ws.numel()}; call kilat_amd.reserve_workspace() "
                "(or run the largest shape once eagerly) on that stream before capturing"
            )
        new = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        if ws is not None:
            _retired.append(ws)
        _workspaces[key] = ws = new
    return ws


def reserve_workspace(
    B: int, H: int, N: int, D: int, dtype: torch.dtype = torch.bfloat16,
    device: Optional[torch.device] = None, backward: bool = True,
) -> int:
    """Make the current stream's workspace large enough for scans of this shape
    (and their backward when `backward`), so that they can be captured into a
    HIP graph.  Returns the workspace size in bytes."""
    dev = torch.device("cuda") if device is None else torch.device(device)
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    code = _dtype_code(torch.empty((), dtype=dtype), "dtype")
    lib = _lib.load()
    nbytes = lib.kdecay_scan_workspace_bytes(B, H, N, D, code)
    if backward:
        # float64 is trained through the fp32 kernels (_scan_with_grad)
        tcode = _lib.KDECAY_F32 if code == _lib.KDECAY_F64 else code
        nbytes = max(nbytes, lib.kdecay_scan_workspace_bytes(B, H, N, D, tcode),
                     lib.kdecay_scan_bwd_workspace_bytes(B, H, N, D, tcode))
    with _on_device(dev):
        ws = _workspace(dev, _stream_ptr(dev), nbytes)
    return 0 if ws is None else ws.numel()


def workspace_error(V: torch.Tensor, clear: bool = False) -> int:
    """Sticky error word of the workspace used for V's device and current stream.

    0: no fault.  1: a bounded wait of some earlier launch gave up (a
    look-back, or the backward's wait for a head's dlam partials).  The launch
    that gave up wrote NaN where it could not compute, and while the word is
    set every later launch on this workspace writes NaN to all its outputs
    (y, the final state, dV, dlam, d(init)): the workspace may hold words of
    that launch tagged as a later launch's, so only a cleared workspace
    computes again.  clear=True zeroes the whole workspace after reading it.
    Synchronises the stream.
    """
    ws = _workspaces.get((V.device.index, _stream_ptr(V.device)))
    if ws is None:
        return 0
    err = int(ws[4:8].view(torch.int32).item())
    if err and clear:
        ws.zero_()
    return err


def _lam32(lam: torch.Tensor, H: int, device: torch.device) -> torch.Tensor:
    _require_hip(lam, "lam_scores")
    if lam.numel() != H:
        raise ValueError(f"kilat_amd: lam_scores has {lam.numel()} elements, V has {H} heads")
    if lam.dtype == torch.float32 and lam.dim() == 1 and lam.is_contiguous() and lam.device == device:
        return lam  # only its memory is read
    return lam.detach().reshape(H).to(device=device, dtype=torch.float32).contiguous()


class _ScanFn(torch.autograd.Function):
    """The chunked scan with a backward (kdecay_scan_fwd_train / kdecay_scan_bwd).

    Inputs: lam (fp32 [H], differentiable), V, init (fp32 [B,H,D] or None),
    t_offset, out dtype, sequential.  Outputs: (y, final state).  The
    reference's GPU path has no backward; its CPU path is differentiated by
    torch autograd through triton_ops.py:240-246, which this replaces on HIP
    tensors.  With sequential=True, y and the final state are then rewritten
    by the sequential kernel (its bits), while the backward uses the states
    the chunked training forward saved (equal to tolerance).
    """

    @staticmethod
    def forward(ctx, lam32, V, init32, t_offset, out_dtype, sequential=False):
        B, H, N, D = V.shape
        dev = V.device
        v_code = _DTYPE_CODE[V.dtype]
        o_code = _DTYPE_CODE[out_dtype]
        # The saved V also feeds the backward kernel, whose addressing takes
        # a narrower range of row strides than the forward's.
        Vk = V if _vector_layout_ok(V) and _bwd_rows_fit(V) else V.contiguous()
        out = torch.empty(Vk.shape, dtype=out_dtype, device=dev) if out_dtype != Vk.dtype else torch.empty_like(Vk)
        if not _vector_layout_ok(out):
            out = torch.empty(Vk.shape, dtype=out_dtype, device=dev)
        final = torch.empty((B, H, D), dtype=torch.float32, device=dev)
        lib = _lib.load()
        nst = lib.kdecay_scan_saved_states_floats(B, H, N, D, v_code)
        states = torch.empty(max(nst, 1), dtype=torch.float32, device=dev)
        with _on_device(dev):
            stream = _stream_ptr(dev)
            nbytes = max(lib.kdecay_scan_workspace_bytes(B, H, N, D, v_code),
                         lib.kdecay_scan_bwd_workspace_bytes(B, H, N, D, v_code))
            ws = _workspace(dev, stream, nbytes)
            rc = lib.kdecay_scan_fwd_train(
                Vk.data_ptr(), v_code, _lib.strides4(Vk.stride()),
                out.data_ptr(), o_code, _lib.strides4(out.stride()),
                lam32.data_ptr(), init32.data_ptr() if init32 is not None else None, final.data_ptr(),
                states.data_ptr(), states.numel(), B, H, N, D, int(t_offset),
                ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, stream,
            )
        _lib.check(rc, "kdecay_scan_fwd_train")
        if sequential:
            with _on_device(dev):
                rc = lib.kdecay_scan_fwd_sequential(
                    Vk.data_ptr(), v_code, _lib.strides4(Vk.stride()),
                    out.data_ptr(), o_code, _lib.strides4(out.stride()),
                    lam32.data_ptr(), init32.data_ptr() if init32 is not None else None, final.data_ptr(),
                    B, H, N, D, int(t_offset), _stream_ptr(dev),
                )
            _lib.check(rc, "kdecay_scan_fwd_sequential")
        ctx.t_offset = int(t_offset)
        ctx.has_init = init32 is not None
        ctx.save_for_backward(lam32, Vk, init32 if init32 is not None else final.new_empty(0), states)
        return out, final

    @staticmethod
    def backward(ctx, gy, gfin):
        lam32, Vk, init32, states = ctx.saved_tensors
        B, H, N, D = Vk.shape
        dev = Vk.device
        v_code = _DTYPE_CODE[Vk.dtype]
        if gy is None:
            gy = torch.zeros_like(Vk)
        gy = gy.to(Vk.dtype)
        if not (_vector_layout_ok(gy) and _bwd_rows_fit(gy)):
            gy = gy.contiguous()
        dV = torch.empty_like(Vk)
        if not _vector_layout_ok(dV):
            dV = torch.empty(Vk.shape, dtype=Vk.dtype, device=dev)
        dlam = torch.empty(H, dtype=torch.float32, device=dev)
        dinit = torch.empty((B, H, D), dtype=torch.float32, device=dev) if ctx.has_init else None
        g_fin = gfin.to(torch.float32).contiguous() if gfin is not None else None
        lib = _lib.load()
        with _on_device(dev):
            stream = _stream_ptr(dev)
            nbytes = lib.kdecay_scan_bwd_workspace_bytes(B, H, N, D, v_code)
            ws = _workspace(dev, stream, nbytes)
            rc = lib.kdecay_scan_bwd(
                Vk.data_ptr(), v_code, _lib.strides4(Vk.stride()),
                gy.data_ptr(), _lib.strides4(gy.stride()),
                dV.data_ptr(), _lib.strides4(dV.stride()),
                lam32.data_ptr(), init32.data_ptr() if ctx.has_init else None, states.data_ptr(),
                g_fin.data_ptr() if g_fin is not None else None,
                dlam.data_ptr(), dinit.data_ptr() if dinit is not None else None,
                B, H, N, D, ctx.t_offset,
                ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, stream,
            )
        _lib.check(rc, "kdecay_scan_bwd")
        return dlam, dV, dinit, None, None, None


def _needs_grad(*ts) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


def global_decay_scan(
    lam: torch.Tensor,
    V: torch.Tensor,
    *,
    initial_state: Optional[torch.Tensor] = None,
    return_final_state: bool = False,
    t_offset: int = 0,
    out: Optional[torch.Tensor] = None,
    out_dtype: Optional[torch.dtype] = None,
    algorithm: str = "chunked",
) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """y[b,h,t] = s[b,h,t] / z_t with s_t = lam_h * s_{t-1} + V[b,h,t].

    lam: [H] (any float dtype; used as fp32).  V: [B,H,N,D] fp32/bf16/fp16/fp64,
    any strides (arithmetic in fp32 for every type, as the reference's kernel
    accumulates).  initial_state: [B,H,D] state before position 0 (default zeros).
    t_offset: absolute position of row 0 (z uses t_offset + t).
    Returns y ([B,H,N,D], dtype out_dtype or V.dtype, laid out like V), and
    with return_final_state also s_{N-1} ([B,H,D] fp32).
    algorithm: "chunked" (default) or "sequential" (the cross-check kernel).
    Head dims the chunked kernels do not take (chunked_head_dim) are
    zero-padded to the next one they do.  When lam, V or initial_state
    requires grad, the result carries a backward for every head dim, layout,
    algorithm and out= (the gradients always come from the chunked backward
    kernel).  The backward kernel takes the upstream gradient in V's dtype:
    with out_dtype=float32 for a bf16/fp16 V, that gradient is rounded to V's
    dtype first.  A float64 V takes float64 out only; with a gradient it runs
    the fp32 training kernels on V rounded to fp32.
    """
    _require_hip(V, "V")
    if V.dim() != 4:
        raise ValueError(f"kilat_amd: V must be [B,H,N,D], got shape {tuple(V.shape)}")
    v_code = _dtype_code(V, "V")
    B, H, N, D = V.shape
    dev = V.device
    if _needs_grad(lam, V, initial_state):
        return _scan_with_grad(lam, V, initial_state, return_final_state, t_offset, out, out_dtype, algorithm)
    lam32 = _lam32(lam, H, dev)
    if out is None:
        out = torch.empty_like(V, dtype=out_dtype or V.dtype)
    else:
        _require_hip(out, "out")
        if out.shape != V.shape or out.device != dev:
            raise ValueError("kilat_amd: out must have V's shape and device")
    o_code = _dtype_code(out, "out")
    if o_code != v_code and (o_code != _lib.KDECAY_F32 or v_code == _lib.KDECAY_F64):
        raise TypeError("kilat_amd: out dtype must be V's dtype or float32 (V's dtype for a float64 V)")
    init32 = None
    if initial_state is not None:
        _require_hip(initial_state, "initial_state")
        if tuple(initial_state.shape) != (B, H, D):
            raise ValueError(f"kilat_amd: initial_state must be [B,H,D]={B, H, D}")
        init32 = initial_state.detach().to(device=dev, dtype=torch.float32).contiguous()
    final = torch.empty((B, H, D), dtype=torch.float32, device=dev) if return_final_state else None
    if algorithm not in ("chunked", "sequential"):
        raise ValueError(f"kilat_amd: unknown algorithm {algorithm!r}")

    lib = _lib.load()
    with _on_device(dev):
        stream = _stream_ptr(dev)
        if algorithm == "sequential":
            rc = lib.kdecay_scan_fwd_sequential(
                V.data_ptr(), v_code, _lib.strides4(V.stride()),
                out.data_ptr(), o_code, _lib.strides4(out.stride()),
                lam32.data_ptr(), init32.data_ptr() if init32 is not None else None,
                final.data_ptr() if final is not None else None, B, H, N, D, int(t_offset), stream,
            )
            _lib.check(rc, "kdecay_scan_fwd_sequential")
        elif chunked_head_dim(D, V.dtype):
            _chunked(lib, V, v_code, out, o_code, lam32, init32, final, t_offset, stream, dev)
        else:  # zero channels up to a head dim the chunked kernels take
            Dp = _padded_head_dim(D, V.dtype)
            Vp = V.new_zeros((B, H, N, Dp))
            Vp[..., :D] = V
            initp = None
            if init32 is not None:
                initp = init32.new_zeros((B, H, Dp))
                initp[..., :D] = init32
            outp = torch.empty((B, H, N, Dp), dtype=out.dtype, device=dev)
            finp = torch.empty((B, H, Dp), dtype=torch.float32, device=dev) if final is not None else None
            _chunked(lib, Vp, v_code, outp, o_code, lam32, initp, finp, t_offset, stream, dev)
            out.copy_(outp[..., :D])
            if final is not None:
                final.copy_(finp[..., :D])
    if return_final_state:
        return out, final
    return out


def _chunked(lib, V, v_code, out, o_code, lam32, init32, final, t_offset, stream, dev) -> None:
    """kdecay_scan_fwd on V into out (through contiguous copies where the
    layout is not one the vector kernel takes)."""
    B, H, N, D = V.shape
    Vk = V if _vector_layout_ok(V) else V.contiguous()
    outk = out if _vector_layout_ok(out) else torch.empty(V.shape, dtype=out.dtype, device=dev)
    nbytes = _fwd_workspace_bytes(lib, B, H, N, D, v_code)
    ws = _workspace(dev, stream, nbytes)
    rc = lib.kdecay_scan_fwd(
        Vk.data_ptr(), v_code, _lib.strides4(Vk.stride()),
        outk.data_ptr(), o_code, _lib.strides4(outk.stride()),
        lam32.data_ptr(), init32.data_ptr() if init32 is not None else None,
        final.data_ptr() if final is not None else None, B, H, N, D, int(t_offset),
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
        stream,
    )
    _lib.check(rc, "kdecay_scan_fwd")
    if outk is not out:
        out.copy_(outk)


def _scan_with_grad(lam, V, initial_state, return_final_state, t_offset, out, out_dtype, algorithm):
    """global_decay_scan when a gradient is required: the chunked training
    forward and backward under _ScanFn, with differentiable zero-padding of
    the channels for head dims the kernels do not take, and a differentiable
    copy into `out` when one is given."""
    B, H, N, D = V.shape
    dev = V.device
    if algorithm not in ("chunked", "sequential"):
        raise ValueError(f"kilat_amd: unknown algorithm {algorithm!r}")
    if out is not None:
        _require_hip(out, "out")
        if out.shape != V.shape or out.device != dev:
            raise ValueError("kilat_amd: out must have V's shape and device")
        if out_dtype is not None and out_dtype != out.dtype:
            raise TypeError("kilat_amd: out_dtype and out.dtype differ")
        y, final = _scan_with_grad(lam, V, initial_state, True, t_offset, None, out.dtype, algorithm)
        out.copy_(y)
        return (out, final) if return_final_state else out
    if V.dtype == torch.float64:
        # The training forward and backward kernels take fp32/bf16/fp16 only.  A
        # float64 V runs them on V rounded to fp32 (the rounding the forward
        # kernels apply to each float64 element as they load it) and y comes
        # back as float64; dV reaches V through the rounding's own gradient.
        if (out_dtype or V.dtype) != torch.float64:
            raise TypeError("kilat_amd: out dtype must be V's dtype for a float64 V")
        y, final = _scan_with_grad(lam, V.float(), initial_state, True, t_offset, None, torch.float32, algorithm)
        y = y.to(torch.float64)
        return (y, final) if return_final_state else y
    if not chunked_head_dim(D, V.dtype):
        Dp = _padded_head_dim(D, V.dtype)
        Vp = torch.nn.functional.pad(V, (0, Dp - D))
        initp = None
        if initial_state is not None:
            _require_hip(initial_state, "initial_state")
            if tuple(initial_state.shape) != (B, H, D):
                raise ValueError(f"kilat_amd: initial_state must be [B,H,D]={B, H, D}")
            initp = torch.nn.functional.pad(initial_state, (0, Dp - D))
        yp, finp = _scan_with_grad(lam, Vp, initp, True, t_offset, None, out_dtype, algorithm)
        y = torch.empty_like(V, dtype=yp.dtype)
        y.copy_(yp[..., :D])  # laid out like V, as empty_like(V) is in the reference
        final = finp[..., :D].contiguous()
        return (y, final) if return_final_state else y
    _require_hip(lam, "lam_scores")
    if lam.numel() != H:
        raise ValueError(f"kilat_amd: lam_scores has {lam.numel()} elements, V has {H} heads")
    lam32 = lam.reshape(H).to(device=dev, dtype=torch.float32).contiguous()
    init32 = None
    if initial_state is not None:
        _require_hip(initial_state, "initial_state")
        if tuple(initial_state.shape) != (B, H, D):
            raise ValueError(f"kilat_amd: initial_state must be [B,H,D]={B, H, D}")
        init32 = initial_state.to(device=dev, dtype=torch.float32).contiguous()
    o_dtype = out_dtype or V.dtype
    if o_dtype not in (V.dtype, torch.float32):
        raise TypeError("kilat_amd: out dtype must be V's dtype or float32")
    y, final = _ScanFn.apply(lam32, V, init32, int(t_offset), o_dtype, algorithm == "sequential")
    if return_final_state:
        return y, final
    return y


def triton_global_decay(lam_scores: torch.Tensor, V: torch.Tensor) -> torch.Tensor:
    """Drop-in for kilat.arc.triton_ops.triton_global_decay (triton_ops.py:249-330).

    lam_scores: [H] decay factors (sigmoid already applied, attention.py:319).
    V: [B,H,N,D] on a HIP device.  Returns out = empty_like(V) filled with
    out[:,:,t] = (sum_{j<=t} lam^(t-j) V[:,:,j]) / z_t, z_t as the reference's
    CPU path computes it (triton_ops.py:245).  Enqueued on the current stream,
    no host synchronisation.  When lam_scores or V requires grad, the result
    carries a backward (dV and dlam on the GPU), as the reference's CPU path
    does through torch autograd; its GPU path has none.
    """
    return global_decay_scan(lam_scores, V)


def decay_step(
    lam: torch.Tensor,
    past_state: torch.Tensor,
    v_t: torch.Tensor,
    t_pos: Union[int, torch.Tensor],
    *,
    out: Optional[torch.Tensor] = None,
    new_state: Optional[torch.Tensor] = None,
    out_dtype: torch.dtype = torch.float32,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """One incremental step for the whole batch (attention.py:344-360).

        new_state = lam.view(1,H,1) * past_state + v_t        (two roundings)
        out       = new_state / ((1 - lam**(t_pos+1)) / (1 - lam + 1e-6))

    past_state: [B,H,D] (used as fp32, as the reference's promotion makes it).
    v_t: [B,H,D] fp32/bf16/fp16/fp64 (any view of [B,1,H*D] reshapes to it;
    fp64 is rounded to fp32 first, out_dtype float64 widens the fp32 result).
    t_pos: int shared by the batch (the reference's cache length) or an int
    tensor [B] of per-sequence positions.  new_state may be past_state itself
    (in-place).  Returns (out [B,H,D] out_dtype, new_state [B,H,D] fp32).
    """
    _require_hip(past_state, "past_state")
    if past_state.dim() != 3:
        raise ValueError(f"kilat_amd: past_state must be [B,H,D], got {tuple(past_state.shape)}")
    B, H, D = past_state.shape
    dev = past_state.device
    _require_hip(v_t, "v_t")
    if v_t.numel() != B * H * D:
        raise ValueError(f"kilat_amd: v_t has {v_t.numel()} elements, expected B*H*D={B * H * D}")
    v_code = _dtype_code(v_t, "v_t")
    vk = v_t.detach().reshape(B, H, D).contiguous()
    if v_code == _lib.KDECAY_F64:  # the step kernel takes v_t as fp32 (rounded once), as every type
        vk, v_code = vk.float(), _lib.KDECAY_F32
    lam32 = _lam32(lam, H, dev)
    s_in = past_state.detach()
    if s_in.dtype != torch.float32 or not s_in.is_contiguous():
        s_in = s_in.to(torch.float32).contiguous()
    if new_state is None:
        new_state = torch.empty((B, H, D), dtype=torch.float32, device=dev)
    elif new_state.dtype != torch.float32 or not new_state.is_contiguous() or tuple(new_state.shape) != (B, H, D):
        raise ValueError("kilat_amd: new_state must be a contiguous float32 [B,H,D] tensor")
    if out is None:
        out = torch.empty((B, H, D), dtype=out_dtype, device=dev)
    elif not out.is_contiguous() or out.numel() != B * H * D:
        raise ValueError("kilat_amd: out must be contiguous with B*H*D elements")
    o_code = _dtype_code(out, "out")
    outk = out
    if o_code == _lib.KDECAY_F64:  # computed in fp32, then widened exactly
        outk, o_code = torch.empty((B, H, D), dtype=torch.float32, device=dev), _lib.KDECAY_F32
    tpos_ptr, tpos_scalar, tpos_dev = None, 0, None
    if isinstance(t_pos, torch.Tensor):
        if t_pos.numel() != B:
            raise ValueError(f"kilat_amd: t_pos tensor must have B={B} elements")
        tpos_dev = t_pos.detach().reshape(B).to(device=dev, dtype=torch.int32).contiguous()
        tpos_ptr = tpos_dev.data_ptr()
    else:
        tpos_scalar = int(t_pos)
    lib = _lib.load()
    with _on_device(dev):
        rc = lib.kdecay_step(
            lam32.data_ptr(), s_in.data_ptr(), vk.data_ptr(), v_code,
            new_state.data_ptr(), outk.data_ptr(), o_code,
            tpos_ptr, tpos_scalar, B, H, D, _stream_ptr(dev),
        )
    _lib.check(rc, "kdecay_step")
    if outk is not out:
        out.copy_(outk.reshape(out.shape))
    return out, new_state


__all__ = ["triton_global_decay", "decay_step", "global_decay_scan", "workspace_error", "reserve_workspace",
           "chunked_head_dim"]
