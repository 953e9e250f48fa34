"""C ABI and host-side logic, without a GPU: the library loads into a torch
process, exports every symbol include/kdecay.h declares, and rejects bad
arguments before any HIP call.  No kernel is launched here."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest
import torch

from kilat_amd import _build, _lib
from tests.decay_cases import WORKSPACE_HEADER_BYTES as HDR

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kdecay.h")

FAKE = 0x10000  # a 16-byte aligned non-null address; never dereferenced on the host


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kdecay_\w+)\s*\(", text)))


def test_header_declarations_match_binding():
    assert declared_symbols() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol(kdecay_lib):
    out = subprocess.run(["nm", "-D", "--defined-only", _build.LIBRARY], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\bT (kdecay_\w+)", out.stdout))
    for sym in declared_symbols():
        assert sym in exported, sym
        assert getattr(kdecay_lib, sym) is not None


def test_single_hip_runtime_in_process(kdecay_lib):
    maps = open(f"/proc/{os.getpid()}/maps").read()
    runtimes = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(runtimes) == 1, runtimes


def test_version(kdecay_lib):
    v = kdecay_lib.kdecay_version().decode()
    assert v.startswith("kdecay ") and "gfx950" in v


def test_workspace_bytes(kdecay_lib):
    ws = kdecay_lib.kdecay_scan_workspace_bytes
    # A stream is a (b,h) pair and a 128-byte channel group; a chunk holds 64 KiB of
    # input: 512 rows of a 128-byte group, or half that (8 rows per lane instead of
    # 16) when the 16-row grid has at most 416 chunks (640 with 2 chunks per stream,
    # 160 with 1).  Words: one per channel per chunk.
    assert ws(8, 12, 4096, 64, _lib.KDECAY_BF16) == HDR + 8 * 12 * 8 * 64 * 8  # 768 chunks
    assert ws(1, 16, 65536, 128, _lib.KDECAY_BF16) == HDR + 16 * 128 * 128 * 8  # 4096 chunks
    assert ws(2, 6, 512, 64, _lib.KDECAY_BF16) == HDR + 2 * 6 * 2 * 64 * 8  # small grid: 256-row chunks
    assert ws(2, 6, 256, 64, _lib.KDECAY_BF16) == 0  # one chunk per stream
    # float64: 16-channel groups, 8 lanes per row as fp32's 32-channel groups, so
    # D fp64 channels make the streams and chunks of 2D fp32 channels, with half
    # the channels' words
    for B, H, N, D in ((8, 12, 4096, 64), (2, 6, 512, 16), (1, 16, 65536, 128), (2, 3, 3000, 48)):
        assert ws(B, H, N, D, _lib.KDECAY_F64) - HDR == (ws(B, H, N, 2 * D, _lib.KDECAY_F32) - HDR) // 2 > 0
    assert ws(2, 6, 128, 16, _lib.KDECAY_F64) == 0  # one chunk per stream
    # heads of four or more 128-byte groups, a full round of 512-row chunks or more and at
    # most 32 per stream: 256-row chunks (the six-per-CU kernel)
    assert ws(8, 12, 4096, 256, _lib.KDECAY_BF16) == HDR + 8 * 12 * 16 * 256 * 8  # 3072 chunks at 512 rows
    assert ws(2, 16, 16384, 256, _lib.KDECAY_BF16) == HDR + 2 * 16 * 64 * 256 * 8  # 32 per stream
    assert ws(1, 16, 32768, 256, _lib.KDECAY_BF16) == HDR + 16 * 64 * 256 * 8  # 64 per stream: 512 rows
    assert ws(2, 12, 4096, 256, _lib.KDECAY_BF16) == HDR + 2 * 12 * 8 * 256 * 8  # 768 chunks: 512 rows
    assert ws(8, 12, 4096, 192, _lib.KDECAY_BF16) == HDR + 8 * 12 * 8 * 192 * 8  # three groups: 512 rows
    assert ws(2, 6, 1024, 64, _lib.KDECAY_F32) == HDR + 2 * 6 * 4 * 64 * 8  # 2 groups of 32, 256-row chunks
    assert ws(1, 2, 4096, 32, _lib.KDECAY_BF16) == HDR + 2 * 8 * 32 * 8  # 32-channel rows: 512-row chunks
    assert ws(8, 12, 2048, 64, _lib.KDECAY_BF16) == HDR + 8 * 12 * 8 * 64 * 8  # 384 chunks at 16 rows: 8
    assert ws(4, 13, 4096, 64, _lib.KDECAY_BF16) == HDR + 4 * 13 * 16 * 64 * 8  # 416 chunks at 16 rows: 8
    assert ws(4, 13, 4097, 64, _lib.KDECAY_BF16) == HDR + 4 * 13 * 9 * 64 * 8  # 468: 16 rows
    assert ws(20, 16, 1024, 64, _lib.KDECAY_BF16) == HDR + 20 * 16 * 4 * 64 * 8  # 640, 2 per stream: 8 rows
    assert ws(21, 16, 1024, 64, _lib.KDECAY_BF16) == HDR + 21 * 16 * 2 * 64 * 8  # 672: 16 rows
    assert ws(10, 16, 512, 64, _lib.KDECAY_BF16) == HDR + 10 * 16 * 2 * 64 * 8  # 160, 1 per stream: 8 rows
    assert ws(11, 16, 512, 64, _lib.KDECAY_BF16) == 0  # 176 single-chunk streams: 16 rows, no look-back
    assert ws(2, 6, 1024, 48, _lib.KDECAY_BF16) == 0  # unsupported D
    # Heads of one full 128-byte group, B >= 2, at most 8 chunks of 512 rows per
    # stream and more than 1024 of them: balanced batch slices of at most 1024
    # chunks, one launch each, one after another on the workspace (the largest
    # slice's words); 512-row chunks.
    assert ws(10, 12, 4096, 64, _lib.KDECAY_BF16) == HDR + 10 * 12 * 8 * 64 * 8  # 960: one launch
    assert ws(11, 12, 4096, 64, _lib.KDECAY_BF16) == HDR + 6 * 12 * 8 * 64 * 8  # 1056: slices of 5 and 6
    assert ws(13, 12, 4096, 64, _lib.KDECAY_BF16) == HDR + 7 * 12 * 8 * 64 * 8  # 1248: 6 + 7
    assert ws(16, 12, 4096, 64, _lib.KDECAY_BF16) == HDR + 8 * 12 * 8 * 64 * 8  # 1536: 8 + 8
    assert ws(17, 12, 4096, 64, _lib.KDECAY_BF16) == HDR + 9 * 12 * 8 * 64 * 8  # 1632: 8 + 9
    assert ws(64, 12, 4096, 64, _lib.KDECAY_BF16) == HDR + 8 * 12 * 8 * 64 * 8  # 8 slices of 768 chunks, not 7 of 864-960
    assert ws(20, 12, 4096, 64, _lib.KDECAY_BF16) == HDR + 10 * 12 * 8 * 64 * 8  # 2 of 960 (4 per CU), not 4 of 480
    assert ws(40, 16, 4096, 64, _lib.KDECAY_BF16) == HDR + 8 * 16 * 8 * 64 * 8  # 5 of 1024
    assert ws(16, 12, 4096, 32, _lib.KDECAY_F32) == HDR + 8 * 12 * 8 * 32 * 8  # fp32 D=32: 8 + 8
    assert ws(128, 12, 512, 64, _lib.KDECAY_BF16) == 0  # 2 slices of single-chunk streams
    assert ws(80, 12, 4096, 64, _lib.KDECAY_BF16) == HDR + 10 * 12 * 8 * 64 * 8  # 8 slices at most
    assert ws(72, 12, 4096, 64, _lib.KDECAY_BF16) == HDR + 72 * 12 * 8 * 64 * 8  # 8 slices of 864: one launch
    assert ws(56, 12, 4096, 64, _lib.KDECAY_BF16) == HDR + 8 * 12 * 8 * 64 * 8  # 7 slices of 768
    assert ws(96, 12, 4096, 64, _lib.KDECAY_BF16) == HDR + 96 * 12 * 8 * 64 * 8  # more than 8 needed: one launch
    assert ws(14, 12, 4097, 64, _lib.KDECAY_BF16) == HDR + 14 * 12 * 9 * 64 * 8  # 9 per stream: one launch
    assert ws(3, 12, 8192, 64, _lib.KDECAY_BF16) == HDR + 3 * 12 * 16 * 64 * 8  # 16 per stream: one launch
    # At B=1, just above one resident round of 512-row chunks (8 or fewer per
    # stream, full 128-byte groups): 256-row chunks, six workgroups per compute unit.
    assert ws(1, 156, 4096, 64, _lib.KDECAY_BF16) == HDR + 156 * 8 * 64 * 8  # 1248: 16 rows
    assert ws(1, 168, 4096, 64, _lib.KDECAY_BF16) == HDR + 168 * 16 * 64 * 8  # 1344: 8 rows
    assert ws(1, 192, 4096, 64, _lib.KDECAY_BF16) == HDR + 192 * 16 * 64 * 8  # 1536: 8 rows
    assert ws(1, 204, 4096, 64, _lib.KDECAY_BF16) == HDR + 204 * 8 * 64 * 8  # 1632: 16 rows
    assert ws(5, 12, 4096, 128, _lib.KDECAY_BF16) == HDR + 5 * 12 * 8 * 128 * 8  # 960 in 2 groups: one round, 16 rows
    assert ws(6, 12, 4096, 128, _lib.KDECAY_BF16) == HDR + 6 * 12 * 16 * 128 * 8  # 1152 in 2 groups: 8 rows
    assert ws(8, 12, 4096, 64, _lib.KDECAY_F32) == HDR + 8 * 12 * 16 * 64 * 8  # 1536 in 2 groups: 8 rows
    # Small grids of long streams: from 64 chunks of 256 rows per stream on, 512-row
    # chunks of 8 wavefronts (full 128-byte groups).
    assert ws(1, 6, 16128, 64, _lib.KDECAY_BF16) == HDR + 6 * 63 * 64 * 8  # 63 per stream: 256 rows
    assert ws(1, 6, 16384, 64, _lib.KDECAY_BF16) == HDR + 6 * 32 * 64 * 8  # 64: 512 rows
    assert ws(1, 2, 16384, 64, _lib.KDECAY_F32) == HDR + 2 * 32 * 64 * 8  # two groups of 32 fp32: 512 rows
    assert ws(1, 2, 65536, 32, _lib.KDECAY_BF16) == HDR + 2 * 128 * 32 * 8  # 64-byte rows keep 4 x 8: 512 rows
    assert ws(32, 12, 4096, 32, _lib.KDECAY_BF16) == HDR + 32 * 12 * 4 * 32 * 8  # 1536 of 64-byte rows: 1024-row chunks


def test_backward_workspace_bytes(kdecay_lib):
    wb = kdecay_lib.kdecay_scan_bwd_workspace_bytes
    # 512-row chunks (16 rows x 4 wavefronts x 8 row groups for a 128-byte
    # group); 256-row chunks (8 rows) when the 512-row grid has more than 192
    # and at most 512 chunks; 128-row chunks (4 rows) when it has at most 192;
    # header + look-back words (one per channel per chunk) + one 8-byte tagged
    # dlam partial per chunk of every stream, rounded up to 256 bytes.
    nst, nch = 8 * 12, 4096 // 512
    assert wb(8, 12, 4096, 64, _lib.KDECAY_BF16) == HDR + nst * nch * 64 * 8 + (nst * nch * 8 + 255) // 256 * 256
    nst, nch = 8 * 6, 1024 // 128  # 96 chunks at 512 rows: the small-grid shape
    assert wb(8, 6, 1024, 64, _lib.KDECAY_BF16) == HDR + nst * nch * 64 * 8 + (nst * nch * 8 + 255) // 256 * 256
    nst, nch = 8 * 12, 2048 // 256  # 384 chunks at 512 rows: 256-row chunks
    assert wb(8, 12, 2048, 64, _lib.KDECAY_BF16) == HDR + nst * nch * 64 * 8 + (nst * nch * 8 + 255) // 256 * 256
    nst, nch = 8 * 12, 9  # 480 chunks at 512 rows: 256-row chunks, 9 per stream
    assert wb(8, 12, 2049, 64, _lib.KDECAY_BF16) == HDR + nst * nch * 64 * 8 + (nst * nch * 8 + 255) // 256 * 256
    nst, nch = 4 * 12, 4096 // 256  # 384 chunks at 512 rows: 256-row chunks
    assert wb(4, 12, 4096, 64, _lib.KDECAY_BF16) == HDR + nst * nch * 64 * 8 + (nst * nch * 8 + 255) // 256 * 256
    nst, nch = 8 * 14, 2048 // 256  # 448 chunks at 512 rows: 256-row chunks
    assert wb(8, 14, 2048, 64, _lib.KDECAY_BF16) == HDR + nst * nch * 64 * 8 + (nst * nch * 8 + 255) // 256 * 256
    nst, nch = 8 * 12, 1024 // 128  # 192 chunks at 512 rows: 128-row chunks
    assert wb(8, 12, 1024, 64, _lib.KDECAY_BF16) == HDR + nst * nch * 64 * 8 + (nst * nch * 8 + 255) // 256 * 256
    nst, nch = 4 * 16, 2048 // 256  # 256 chunks at 512 rows: 256-row chunks
    assert wb(4, 16, 2048, 64, _lib.KDECAY_BF16) == HDR + nst * nch * 64 * 8 + (nst * nch * 8 + 255) // 256 * 256
    nst, nch = 5 * 16, 4096 // 512  # 640 chunks: 512-row chunks
    assert wb(5, 16, 4096, 64, _lib.KDECAY_BF16) == HDR + nst * nch * 64 * 8 + (nst * nch * 8 + 255) // 256 * 256
    # one chunk per stream: no look-back words, but the header and the partials
    assert wb(2, 6, 100, 64, _lib.KDECAY_BF16) == HDR + 256
    assert wb(2, 6, 100, 48, _lib.KDECAY_BF16) == 0  # unsupported D
    # 128 bf16 channels on a large grid with short chains: whole 256-byte rows,
    # one stream per head, 256-row chunks (16 per stream, 1536 in all)
    nst, nch = 8 * 12, 4096 // 256
    assert wb(8, 12, 4096, 128, _lib.KDECAY_BF16) == HDR + nst * nch * 128 * 8 + (nst * nch * 8 + 255) // 256 * 256
    # long chains (256 of 256 rows): two 128-byte streams per head, 512-row chunks
    nst, nch = 1 * 16 * 2, 65536 // 512
    assert wb(1, 16, 65536, 128, _lib.KDECAY_BF16) == HDR + nst * nch * 64 * 8 + (nst * nch * 8 + 255) // 256 * 256
    # a grid of 256-row chunks below 512 (4 x 6 x 16 = 384): two 128-byte streams per head,
    # 384 chunks of 512 rows: 256-row chunks
    nst, nch = 4 * 6 * 2, 4096 // 256
    assert wb(4, 6, 4096, 128, _lib.KDECAY_BF16) == HDR + nst * nch * 64 * 8 + (nst * nch * 8 + 255) // 256 * 256

    def words(B, H, N, D, nst, nch):
        return HDR + B * H * nch * D * 8 + (nst * nch * 8 + 255) // 256 * 256

    # heads of two or more 128-byte groups, more than one round of 512-row chunks
    # (768) and at least 48 streams: 256-row chunks (8 rows per lane)
    assert wb(8, 12, 4096, 64, _lib.KDECAY_F32) == words(8, 12, 4096, 64, 192, 16)  # 1536 chunks at 512 rows
    assert wb(5, 12, 4096, 64, _lib.KDECAY_F32) == words(5, 12, 4096, 64, 120, 16)  # 960
    assert wb(4, 12, 4096, 64, _lib.KDECAY_F32) == words(4, 12, 4096, 64, 96, 8)  # 768, one round: 512 rows
    assert wb(12, 12, 4096, 32, _lib.KDECAY_F32) == words(12, 12, 4096, 32, 144, 8)  # one group: 512 rows
    assert wb(2, 16, 32768, 128, _lib.KDECAY_BF16) == words(2, 16, 32768, 128, 64, 128)  # 64 streams of 128 B
    assert wb(1, 16, 65536, 128, _lib.KDECAY_F32) == words(1, 16, 65536, 128, 64, 256)  # four groups of 32 fp32
    # one-group heads on 512-row chunks, at most 8 per stream, in exactly two or three
    # resident rounds (768 chunks each) that the batch divides evenly: one launch per
    # round-sized batch slice, one after another on the workspace (one slice's words),
    # and the earlier slices' dlam sums in double (256-byte aligned)
    sums = lambda n, H: ((n - 1) * H * 8 + 255) // 256 * 256
    assert wb(16, 12, 4096, 64, _lib.KDECAY_BF16) == words(8, 12, 4096, 64, 96, 8) + sums(2, 12)  # 2 x 768
    assert wb(24, 12, 4096, 64, _lib.KDECAY_BF16) == words(8, 12, 4096, 64, 96, 8) + sums(3, 12)  # 3 x 768
    assert wb(12, 16, 4096, 64, _lib.KDECAY_F16) == words(6, 16, 4096, 64, 96, 8) + sums(2, 16)
    assert wb(96, 12, 1024, 64, _lib.KDECAY_BF16) == words(32, 12, 1024, 64, 384, 2) + sums(3, 12)  # chains of 2
    assert wb(16, 12, 4096, 32, _lib.KDECAY_F32) == words(8, 12, 4096, 32, 96, 8) + sums(2, 12)  # fp32 D=32
    assert wb(20, 12, 4096, 64, _lib.KDECAY_BF16) == words(20, 12, 4096, 64, 240, 8)  # 1920: one launch
    assert wb(32, 12, 4096, 64, _lib.KDECAY_BF16) == words(32, 12, 4096, 64, 384, 8)  # four rounds: one launch
    assert wb(16, 12, 4097, 64, _lib.KDECAY_BF16) == words(16, 12, 4097, 64, 192, 9)  # 9 per stream: one launch
    assert wb(2, 6, 65536, 64, _lib.KDECAY_BF16) == words(2, 6, 65536, 64, 12, 128)  # 1536 in chains of 128: one


def test_saved_states_floats(kdecay_lib):
    """The training forward's buffer for the backward: the state at each backward
    chunk boundary (B*H*D per chunk of rows) followed by two row terms (1/z and
    d(1/z)/dlam) per row of every head; nothing when the backward has one chunk."""
    sf = kdecay_lib.kdecay_scan_saved_states_floats
    assert sf(8, 12, 4096, 64, _lib.KDECAY_BF16) == 8 * 12 * 64 * (4096 // 512) + 2 * 12 * 4096
    assert sf(8, 6, 1024, 64, _lib.KDECAY_BF16) == 8 * 6 * 64 * (1024 // 128) + 2 * 6 * 1024  # 128-row chunks
    assert sf(8, 12, 2049, 64, _lib.KDECAY_BF16) == 8 * 12 * 64 * 9 + 2 * 12 * 2049  # 256-row chunks, ragged last
    assert sf(1, 16, 65536, 128, _lib.KDECAY_BF16) == 16 * 128 * (65536 // 512) + 2 * 16 * 65536
    assert sf(8, 12, 4096, 128, _lib.KDECAY_BF16) == 8 * 12 * 128 * (4096 // 256) + 2 * 12 * 4096  # whole rows
    assert sf(2, 6, 100, 64, _lib.KDECAY_BF16) == 0  # one chunk per stream
    assert sf(2, 6, 4096, 48, _lib.KDECAY_BF16) == 0  # unsupported D
    assert sf(8, 12, 4096, 64, _lib.KDECAY_F64) == 0  # no float64 training kernels
    assert sf(8, 12, 4096, 64, _lib.KDECAY_F32) == 8 * 12 * 64 * (4096 // 256) + 2 * 12 * 4096  # 256-row chunks


def _scan(lib, v_dtype=_lib.KDECAY_BF16, out_dtype=None, D=64, N=4096, vstr=None, ostr=None,
          V=FAKE, out=FAKE, ws=None, wsb=0):
    out_dtype = v_dtype if out_dtype is None else out_dtype
    B, H = 2, 3
    vstr = vstr or (H * N * D, N * D, D, 1)
    ostr = ostr or (H * N * D, N * D, D, 1)
    return lib.kdecay_scan_fwd(V, v_dtype, _lib.strides4(vstr), out, out_dtype, _lib.strides4(ostr),
                               FAKE, None, None, B, H, N, D, 0, ws, wsb, None)


def test_scan_rejects_bad_arguments(kdecay_lib):
    lib = kdecay_lib
    assert _scan(lib, v_dtype=7) == _lib.KDECAY_EDTYPE
    assert _scan(lib, v_dtype=_lib.KDECAY_BF16, out_dtype=_lib.KDECAY_F16) == _lib.KDECAY_EDTYPE
    assert _scan(lib, v_dtype=_lib.KDECAY_F64, out_dtype=_lib.KDECAY_F32) == _lib.KDECAY_EDTYPE
    assert _scan(lib, v_dtype=_lib.KDECAY_F32, out_dtype=_lib.KDECAY_F64) == _lib.KDECAY_EDTYPE
    assert _scan(lib, v_dtype=_lib.KDECAY_F64, D=24) == _lib.KDECAY_ESHAPE
    assert _scan(lib, v_dtype=_lib.KDECAY_F64, D=48) == _lib.KDECAY_EWORKSPACE  # a float64 head dim
    assert _scan(lib, D=48) == _lib.KDECAY_ESHAPE
    assert _scan(lib, V=FAKE + 2) == _lib.KDECAY_ELAYOUT
    assert _scan(lib, vstr=(3 * 4096 * 64, 4096 * 64, 64, 2)) == _lib.KDECAY_ELAYOUT
    assert _scan(lib, vstr=(3 * 4096 * 64, 4096 * 64, 68, 1)) == _lib.KDECAY_ELAYOUT
    assert _scan(lib, V=None) == _lib.KDECAY_EINVAL
    assert _scan(lib) == _lib.KDECAY_EWORKSPACE  # 16 chunks per stream need a workspace
    assert _scan(lib, ws=FAKE, wsb=100) == _lib.KDECAY_EWORKSPACE
    assert "workspace" in lib.kdecay_last_error_string().decode()
    rc = lib.kdecay_scan_fwd(FAKE, 0, _lib.strides4((1, 1, 1, 1)), FAKE, 0, _lib.strides4((1, 1, 1, 1)),
                             FAKE, None, None, -1, 1, 1, 16, 0, None, 0, None)
    assert rc == _lib.KDECAY_EINVAL


def _bwd(lib, N=4096, D=64, vstr=None, gstr=None, V=FAKE, states=FAKE, ws=FAKE, wsb=1 << 30):
    B, H = 8, 12  # 768 chunks of 512 rows
    vstr = vstr or (H * N * D, N * D, D, 1)
    gstr = gstr or (H * N * D, N * D, D, 1)
    dstr = (H * N * D, N * D, D, 1)
    return lib.kdecay_scan_bwd(V, _lib.KDECAY_BF16, _lib.strides4(vstr), FAKE, _lib.strides4(gstr), FAKE,
                               _lib.strides4(dstr), FAKE, None, states, None, FAKE, None, B, H, N, D, 0,
                               ws, wsb, None)


def test_backward_rejects_bad_arguments(kdecay_lib):
    """The backward's checks run before any HIP call.  Its rows are read
    through 32-bit buffer offsets from each chunk's first row, so a row stride
    at which one chunk (512 rows here) spans 2^31 bytes or more, and a
    negative row stride, are refused with KDECAY_ELAYOUT."""
    lib = kdecay_lib
    H, N, D = 12, 4096, 64
    assert _bwd(lib, D=48) == _lib.KDECAY_ESHAPE
    assert _bwd(lib, V=FAKE + 2) == _lib.KDECAY_ELAYOUT
    assert _bwd(lib, vstr=(H * N * D, N * D, -D, 1)) == _lib.KDECAY_ELAYOUT
    assert "negative row stride" in lib.kdecay_last_error_string().decode()
    # 512 rows x 2 bytes x stride: 2^21 elements reach 2^31 bytes, 2^21 - 64 stay below
    big = 1 << 21
    assert _bwd(lib, gstr=(H * N * big, N * big, big, 1)) == _lib.KDECAY_ELAYOUT
    assert "2^31" in lib.kdecay_last_error_string().decode()
    assert _bwd(lib, vstr=(H * N * big, N * big, big, 1)) == _lib.KDECAY_ELAYOUT
    ok = big - 64
    assert _bwd(lib, vstr=(H * N * ok, N * ok, ok, 1), ws=None, wsb=0) == _lib.KDECAY_EWORKSPACE
    assert _bwd(lib, states=None) == _lib.KDECAY_EINVAL  # several chunks need the saved states
    assert _bwd(lib, ws=None, wsb=0) == _lib.KDECAY_EWORKSPACE
    assert _bwd(lib, ws=FAKE + 16) == _lib.KDECAY_EWORKSPACE  # not 256-byte aligned


def test_backward_row_stride_predicate_of_the_shim(kdecay_lib):
    """The shim's _bwd_rows_fit (which sends V and the upstream gradient to
    the backward kernel as they lie, or as contiguous copies) never passes a
    row stride the library's backward refuses: for bf16 D=64 (512-row chunks
    at most), bf16 D=32 (1024) and bf16 D=16 (2048), every stride it accepts
    gets past the library's layout check (the call then stops at the missing
    workspace, before any HIP call), and strides just above its bound are
    refused by the library with KDECAY_ELAYOUT where the library uses that
    largest chunk."""
    from kilat_amd.triton_ops import _bwd_rows_fit

    class Strided:  # shape, strides and element size of a [B,H,N,D] bf16 view, no memory
        def __init__(self, shape, row_stride):
            self.shape = shape
            self._st = (shape[1] * shape[2] * row_stride, shape[2] * row_stride, row_stride, 1)

        def stride(self, k):
            return self._st[k]

        def element_size(self):
            return 2

    lib = kdecay_lib
    B, H, N = 8, 12, 16384  # 8 or more chunks per stream: the library takes its largest chunks
    for D, rows in ((64, 512), (32, 1024), (16, 2048)):
        limit = 0x7FFFFFFF // (rows * 2)
        for S in (D, 4096, limit - 64, limit, limit + 1, limit + 64, 1 << 22):
            S = S // 8 * 8  # keep every row 16-byte aligned
            if S < D:
                continue
            t = Strided((B, H, N, D), S)
            vstr = (H * N * S, N * S, S, 1)
            rc = lib.kdecay_scan_bwd(FAKE, _lib.KDECAY_BF16, _lib.strides4(vstr), FAKE, _lib.strides4(vstr), FAKE,
                                     _lib.strides4((H * N * D, N * D, D, 1)), FAKE, None, FAKE, None, FAKE, None,
                                     B, H, N, D, 0, None, 0, None)
            if _bwd_rows_fit(t):
                assert rc == _lib.KDECAY_EWORKSPACE, (D, S, rc)
            else:
                assert rc == _lib.KDECAY_ELAYOUT, (D, S, rc)
    # one row per stream: no chunk spans anything
    assert _bwd_rows_fit(Strided((1, 1, 1, 64), 1 << 40))


def test_noalloc_scan_rejects_oversized_and_bad_arguments(kdecay_lib):
    """The allocation-free entry point checks its arguments, and that the
    shape's workspace fits its fixed device array, before it touches the
    device: a shape needing more than KDECAY_NOALLOC_WORKSPACE_BYTES is
    refused with KDECAY_EWORKSPACE and a message naming the limit."""
    lib = kdecay_lib
    cap = _lib.KDECAY_NOALLOC_WORKSPACE_BYTES
    B, H, D = 64, 32, 64
    N = 40 * 512  # 2048 streams x 40 chunks of 512 bf16 rows
    need = lib.kdecay_scan_workspace_bytes(B, H, N, D, _lib.KDECAY_BF16)
    assert need > cap
    st = _lib.strides4((H * N * D, N * D, D, 1))
    rc = lib.kdecay_scan_fwd_noalloc(FAKE, _lib.KDECAY_BF16, st, FAKE, _lib.KDECAY_BF16, st, FAKE, None, None,
                                     B, H, N, D, 0, None)
    assert rc == _lib.KDECAY_EWORKSPACE
    msg = lib.kdecay_last_error_string().decode()
    assert str(need) in msg and str(cap) in msg
    assert lib.kdecay_scan_fwd_noalloc(FAKE, 7, st, FAKE, 7, st, FAKE, None, None, 1, 1, 1, 64, 0,
                                       None) == _lib.KDECAY_EDTYPE
    assert lib.kdecay_scan_fwd_noalloc(None, 0, st, FAKE, 0, st, FAKE, None, None, 1, 1, 1, 64, 0,
                                       None) == _lib.KDECAY_EINVAL
    # the largest C4-like shape fits: 1 x 16 x 65536 x 128 bf16 needs 2 MiB
    assert lib.kdecay_scan_workspace_bytes(1, 16, 65536, 128, _lib.KDECAY_BF16) <= cap


def test_sequential_and_step_reject_bad_arguments(kdecay_lib):
    lib = kdecay_lib
    s4 = _lib.strides4((1, 1, 1, 1))
    assert lib.kdecay_scan_fwd_sequential(FAKE, 9, s4, FAKE, 0, s4, FAKE, None, None, 1, 1, 1, 16, 0,
                                          None) == _lib.KDECAY_EDTYPE
    assert lib.kdecay_scan_fwd_sequential(FAKE, 0, s4, FAKE, 0, s4, FAKE, None, None, 1, 1, 1, 2048, 0,
                                          None) == _lib.KDECAY_ESHAPE
    assert lib.kdecay_step(FAKE, FAKE, FAKE, 5, FAKE, FAKE, 0, None, 0, 1, 1, 1, None) == _lib.KDECAY_EDTYPE
    # float64 is taken by the three forward scans only
    f64 = _lib.KDECAY_F64
    assert lib.kdecay_step(FAKE, FAKE, FAKE, f64, FAKE, FAKE, 0, None, 0, 1, 1, 4, None) == _lib.KDECAY_EDTYPE
    assert lib.kdecay_step(FAKE, FAKE, FAKE, 0, FAKE, FAKE, f64, None, 0, 1, 1, 4, None) == _lib.KDECAY_EDTYPE
    st = _lib.strides4((3 * 4096 * 64, 4096 * 64, 64, 1))
    assert lib.kdecay_scan_fwd_train(FAKE, f64, st, FAKE, f64, st, FAKE, None, None, FAKE, 1 << 30, 2, 3, 4096, 64,
                                     0, FAKE, 1 << 30, None) == _lib.KDECAY_EDTYPE
    assert lib.kdecay_scan_bwd_workspace_bytes(8, 12, 4096, 64, f64) == 0
    assert lib.kdecay_scan_fwd_sequential(FAKE, f64, s4, FAKE, 0, s4, FAKE, None, None, 1, 1, 1, 16, 0,
                                          None) == _lib.KDECAY_EDTYPE  # out must be float64 too
    assert lib.kdecay_step(None, FAKE, FAKE, 0, FAKE, FAKE, 0, None, 0, 1, 1, 1, None) == _lib.KDECAY_EINVAL
    assert lib.kdecay_step(FAKE, FAKE, FAKE, 0, FAKE, FAKE, 0, None, 0, -1, 1, 1, None) == _lib.KDECAY_EINVAL
    # empty problems are valid no-ops
    assert lib.kdecay_step(None, None, None, 0, None, None, 0, None, 0, 0, 12, 64, None) == 0


def test_python_check_raises_with_library_message(kdecay_lib):
    rc = _scan(kdecay_lib, D=48)
    with pytest.raises(RuntimeError, match="head dim"):
        _lib.check(rc, "kdecay_scan_fwd")


def test_shim_refuses_cpu_tensors():
    import kilat_amd

    lam = torch.full((2,), 0.9)
    V = torch.randn(1, 2, 8, 16)
    with pytest.raises(RuntimeError, match="HIP"):
        kilat_amd.triton_global_decay(lam, V)
    with pytest.raises(RuntimeError, match="HIP"):
        kilat_amd.decay_step(lam, torch.zeros(1, 2, 16), torch.zeros(1, 2, 16), 3)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIBRARY", str(tmp_path / "libkdecay.so"))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.load()


def test_ctypes_signatures_cover_header(kdecay_lib):
    # every declared function has an explicit restype (a missing one would
    # silently truncate size_t / pointer returns to int)
    for sym in declared_symbols():
        assert getattr(kdecay_lib, sym).restype in (ctypes.c_int, ctypes.c_uint32, ctypes.c_size_t, ctypes.c_char_p), sym


def test_integration_patches_every_module_by_name():
    import types

    import kilat_amd
    from kilat_amd import integration

    def ref_op(lam, V):
        return "reference"

    mods = [types.ModuleType(n) for n in integration.KILAT_MODULES]
    for m in mods:
        m.triton_global_decay = ref_op
    prev = integration.install(mods)
    assert all(m.triton_global_decay is kilat_amd.triton_global_decay for m in mods)
    integration.uninstall(prev)
    assert all(m.triton_global_decay is ref_op for m in mods)
    with pytest.raises(AttributeError):
        integration.install([types.ModuleType("kilat.arc.blocks")])


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N>1 exits with a message before touching a GPU."""
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_bench_buffer_sets_are_disjoint_and_back_to_back():
    """bench.py's rotated (V, y) sets: each tensor a contiguous view of one
    allocation, pairs back to back with no overlap, V seeded and y of the
    output type (checked on the CPU; the bench carves them on the GPU)."""
    import bench

    shape, n = (2, 3, 5, 8), 2 * 3 * 5 * 8
    for ti, to in ((torch.bfloat16, torch.float32), (torch.float16, torch.float16), (torch.float32, torch.float32)):
        sets = bench.carved_pairs(torch, torch.device("cpu"), shape, ti, to, 3, seed=4)
        base = sets[0][0].data_ptr()
        ei, eo = torch.empty(0, dtype=ti).element_size(), torch.empty(0, dtype=to).element_size()
        for k, (V, y) in enumerate(sets):
            assert V.dtype == ti and y.dtype == to and V.shape == shape == y.shape
            assert V.is_contiguous() and y.is_contiguous()
            assert V.data_ptr() - base == k * n * (ei + eo)
            assert y.data_ptr() - base == k * n * (ei + eo) + n * ei
        again = bench.carved_pairs(torch, torch.device("cpu"), shape, ti, to, 3, seed=4)
        assert all(torch.equal(a[0], b[0]) for a, b in zip(sets, again))
        assert not torch.equal(sets[0][0], sets[1][0])
    sets = bench.rotated_sets(torch, torch.device("cpu"), shape, 4)
    base = sets[0][0].data_ptr()
    for k, (V, y) in enumerate(sets):
        assert V.dtype == y.dtype == torch.bfloat16
        assert V.data_ptr() - base == 2 * k * n * 2 and y.data_ptr() - base == (2 * k + 1) * n * 2


def test_integration_doc_holds_the_tested_ctypes_stub():
    """The integration guide's ctypes stub is the text tests/ctypes_stub.py runs on the GPU."""
    from tests.ctypes_stub import STUB_SOURCE

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    doc = os.path.join(root, "INTEGRATION.md")
    if not os.path.exists(doc):
        pytest.skip("the integration guide is not in this copy of the tree")
    assert STUB_SOURCE in open(doc).read()


def test_chunked_head_dims_and_padding():
    """The chunked kernels take D = 16, 32 or a multiple of one 128-byte channel
    group; the shim pads any other D to the next such size."""
    import torch

    from kilat_amd.triton_ops import _padded_head_dim, chunked_head_dim

    for dt, full in ((torch.bfloat16, 64), (torch.float16, 64), (torch.float32, 32), (torch.float64, 16)):
        for D in (16, 32, full, 2 * full, 3 * full, 8 * full):
            assert chunked_head_dim(D, dt), (dt, D)
            assert _padded_head_dim(D, dt) == D
        for D in (1, 8, 15, 17, 31, 33, full + 1, 3 * full - 1):
            assert not chunked_head_dim(D, dt), (dt, D)
            p = _padded_head_dim(D, dt)
            assert p >= D and chunked_head_dim(p, dt) and p - D < full, (dt, D, p)


def test_library_takes_the_same_head_dims(kdecay_lib):
    """kdecay_scan_workspace_bytes is non-zero exactly for the head dims the
    shim sends to the chunked kernels (several chunks per stream here)."""
    import torch

    from kilat_amd.triton_ops import chunked_head_dim

    for dt, code in ((torch.bfloat16, _lib.KDECAY_BF16), (torch.float32, _lib.KDECAY_F32),
                     (torch.float64, _lib.KDECAY_F64)):
        for D in range(1, 400):
            ok = kdecay_lib.kdecay_scan_workspace_bytes(2, 3, 100000, D, code) > 0
            assert ok == chunked_head_dim(D, dt), (dt, D)


def test_fast_division_matches_exact_division(kdecay_lib):
    """The kernels divide by launch-invariant integers (streams, channel
    groups, heads, head dims, chunks) with a multiply and a shift derived on
    the host; the same host code answers kdecay_debug_fastdiv.  Checked
    against exact division for every divisor up to 4096 at edge and random
    dividends, and for large and power-of-two divisors up to 2^31 - 1."""
    import numpy as np

    fd = kdecay_lib.kdecay_debug_fastdiv
    rng = np.random.default_rng(7)
    top = (1 << 31) - 1
    divisors = list(range(1, 4097)) + [int(x) for x in rng.integers(4097, top, 400)]
    divisors += [1 << k for k in range(31)] + [(1 << k) + 1 for k in range(1, 31)] + [(1 << k) - 1 for k in range(2, 32)]
    for d in divisors:
        ns = {0, 1, d - 1, d, d + 1, 2 * d - 1, top, top - 1, top - d, (top // d) * d, (top // d) * d - 1}
        ns.update(int(x) for x in rng.integers(0, top, 8))
        for n in ns:
            if 0 <= n <= top:
                assert fd(n, d, 0) == n // d, (n, d)
                assert fd(n, d, 1) == n % d, (n, d)
