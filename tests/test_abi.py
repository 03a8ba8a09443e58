"""The C-ABI library: loads, exports every entry point declared in
include/*.h, reports the 64-bit index ABI, and rejects bad arguments on the
host before any device work (no GPU needed)."""
from __future__ import annotations

import ctypes
import glob
import importlib
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = []
    for hdr in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(hdr).read()
        names += re.findall(r"NSH_API\s+[\w\s\*]+?\b(nsh_\w+)\s*\(", text)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    from neural_shift_cuda_amd import _C
    return ctypes.CDLL(_C.LIBRARY_PATH)


def test_header_declares_entry_points():
    names = _declared()
    assert "nsh_accumulate_uz_forward" in names and "nsh_metropolis_aggregate" in names
    assert len(names) >= 15


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_index_width_and_version(lib):
    lib.nsh_index_width_bits.restype = ctypes.c_int
    assert lib.nsh_index_width_bits() == 64
    ext = importlib.import_module("neural_shift_cuda._C")
    assert ext.index_width_bits() == 64
    assert "gfx950" in ext.version()


def _err(lib) -> str:
    lib.nsh_last_error.restype = ctypes.c_char_p
    return lib.nsh_last_error().decode()


def test_host_side_argument_errors(lib):
    i64 = ctypes.c_int64
    f = lib.nsh_accumulate_uz_forward
    f.restype = ctypes.c_int
    dummy = ctypes.c_void_p(16)
    nows = (None, i64(0), None)  # workspace, workspace_bytes, stream
    rc = f(dummy, dummy, dummy, i64(0), i64(1), i64(1), i64(4), i64(4), 3, dummy, dummy, *nows)
    assert rc == 1 and "1 <= S <= 1024" in _err(lib)
    rc = f(dummy, dummy, dummy, i64(1025), i64(1), i64(1), i64(4), i64(4), 3, dummy, dummy, *nows)
    assert rc == 1 and "1 <= S <= 1024" in _err(lib)
    rc = f(dummy, dummy, dummy, i64(5), i64(1), i64(1), i64(4), i64(4), 9, dummy, dummy, *nows)
    assert rc == 1 and "dtype" in _err(lib)
    rc = f(dummy, dummy, dummy, i64(5), i64(1), i64(1), i64(1 << 16), i64(1 << 16), 3, dummy,
           dummy, *nows)
    assert rc == 1 and "2^31" in _err(lib)
    g = lib.nsh_shift_gather_forward
    g.restype = ctypes.c_int
    rc = g(dummy, dummy, i64(3), i64(4), i64(1), i64(1), i64(4), i64(4), 3, dummy, dummy, None)
    assert rc == 1 and "columns" in _err(lib)
    m = lib.nsh_metropolis_aggregate
    m.restype = ctypes.c_int
    rc = m(dummy, dummy, dummy, i64(1), i64(5), i64(1), i64(4), i64(4), 3, 1, ctypes.c_double(1e-6),
           None, dummy, dummy, None, i64(0), None)
    assert rc == 1 and "null" in _err(lib)


def test_module_rejects_host_tensors():
    from neural_shift_cuda_amd import _C
    x = torch.ones(1, 1, 4, 4)
    sh = torch.zeros(1, 3, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        _C.accumulate_uz_forward(x, x, sh)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        _C.shift_gather_forward(x, sh)


def test_gpu_op_without_library_fails_loudly(monkeypatch):
    from neural_shift_cuda_amd import ops
    monkeypatch.setattr(ops, "_HAS_CUDA_EXT", False)
    monkeypatch.setattr(ops, "_EXT_IMPORT_ERROR", OSError("libneural_shift_hip.so: missing"))
    with pytest.raises(RuntimeError, match="failed to load"):
        ops._require_cuda_ext("accumulate_uz")


def test_accumulate_workspace_size(lib):
    """Workspace of the once-per-element weight stream: a 256-byte header,
    then spill blocks of the tiles' window borders (radius up to 8): for the
    fp32 forward two arrays (U, Z) of 2*8*(128+16) + 16*32 = 2816 entries per
    128x32 tile, for the backward one array of 2816 entries per 128x32 tile;
    none when a direction has fewer than 2 tiles."""
    f = lib.nsh_accumulate_uz_workspace_bytes
    f.restype = ctypes.c_int64
    f.argtypes = [ctypes.c_int64] * 5 + [ctypes.c_int, ctypes.c_int]
    t_fwd = (8192 // 128) * (8192 // 32)
    t_bwd = (8192 // 128) * (8192 // 32)
    assert f(85, 1, 1, 8192, 8192, 3, 0) == 256 + 2 * t_fwd * 2816 * 4
    assert f(85, 1, 1, 8192, 8192, 3, 1) == 256 + t_bwd * 2816 * 4
    # fp16 backward: fp32 gx partial sums ride along (one rounding at the end)
    assert f(85, 1, 1, 8192, 8192, 1, 1) == 256 + t_bwd * 2816 * 4 + 8192 * 8192 * 4
    assert f(25, 1, 1, 20, 24, 3, 0) == 0
    assert f(0, 1, 1, 8192, 8192, 3, 0) == -1


def test_metropolis_workspace_size(lib):
    """Metropolis workspace: a 256-byte header, spill blocks (pass 1: one
    array, pass 2: two arrays, of 2*8*(128+16) + 16*32 = 2816 entries per
    128x32 tile; the larger of the two), then two ring arrays of
    2*8*(128+32) = 2560 entries per pass-2 tile; none when a direction has
    fewer than 3 tiles or an edge tile is narrower than 8 pixels."""
    f = lib.nsh_metropolis_workspace_bytes
    f.restype = ctypes.c_int64
    f.argtypes = [ctypes.c_int64] * 5 + [ctypes.c_int]
    t = (8192 // 128) * (8192 // 32)

    def a256(b):
        return (b + 255) // 256 * 256

    spill = a256(max(t * 2816, 2 * t * 2816) * 4)
    part = a256(2 * t * 2560 * 4)
    assert f(1, 85, 1, 8192, 8192, 3) == 256 + spill + part
    assert f(1, 85, 1, 64, 8192, 3) == 0      # two tile rows of 32
    assert f(1, 85, 1, 8192, 8198, 3) == 0    # last tile column 6 pixels wide
    assert f(1, 85, 1, 8192, 8200, 3) > 0     # ... 8 pixels wide
    assert f(1, 0, 1, 64, 64, 3) == -1
def test_metropolis_backward_workspace_size(lib):
    """Fused Metropolis backward workspace: a 256-byte header, two spill
    arrays (gd, gx) of 2*8*(64+16) + 16*16 = 1536 entries per 64x16 edge-pass
    tile (fp32), then fp32 gd and gx planes of B*C*H*W entries each; 0 when
    a direction has fewer than 3 tiles or an edge tile is narrower than 8
    pixels.  fp64 tiles are 32x32: 2*8*(32+16) + 16*32 = 1280 entries."""
    f = lib.nsh_metropolis_backward_workspace_bytes
    f.restype = ctypes.c_int64
    f.argtypes = [ctypes.c_int64] * 5 + [ctypes.c_int]

    def a256(b):
        return (b + 255) // 256 * 256

    t = (8192 // 64) * (8192 // 16)
    plane = a256(2 * 8192 * 8192 * 4)
    assert f(2, 85, 1, 8192, 8192, 3) == 256 + a256(2 * 2 * t * 1536 * 4) + 2 * plane
    t64 = (1024 // 32) * (1024 // 32)
    assert f(1, 85, 1, 1024, 1024, 4) == 256 + a256(2 * t64 * 1280 * 8) + 2 * a256(1024 * 1024 * 8)
    assert f(1, 85, 1, 40, 8192, 3) > 0       # tile rows of 16, 16 and 8
    assert f(1, 85, 1, 32, 8192, 3) == 0      # two tile rows
    assert f(1, 85, 1, 38, 8192, 3) == 0      # last tile row 6 pixels tall
    assert f(1, 85, 1, 8192, 136, 3) > 0      # 64 + 64 + 8
    assert f(1, 85, 1, 8192, 134, 3) == 0     # 64 + 64 + 6
    assert f(1, 0, 1, 64, 64, 3) == -1
    # the 6-pixel border hint (NSH_NARROW_HALO) does not change the workspace
    for shape in [(2, 85, 1, 8192, 8192), (1, 85, 1, 40, 8192), (1, 85, 1, 1024, 1024)]:
        for code in (1, 2, 3, 4):
            assert f(*shape, code | 0x1000) == f(*shape, code)


def test_normalized_narrow_hint_workspace(lib):
    """With the hint the fp64 backward's workspace query returns the larger
    of the two plans (32 x 16 tiles on the 6-pixel border, 32 x 32 on the
    8-pixel one); the forward's and the other types' do not change."""
    f = lib.nsh_normalized_workspace_bytes
    f.restype = ctypes.c_int64
    f.argtypes = [ctypes.c_int64] * 5 + [ctypes.c_int, ctypes.c_int]
    for shape in [(121, 2, 3, 256, 256), (25, 1, 2, 72, 76)]:
        for code in (1, 3, 4):
            for bwd in (0, 1):
                plain, hinted = f(*shape, code, bwd), f(*shape, code | 0x1000, bwd)
                if code == 4 and bwd:
                    assert hinted >= plain > 0
                else:
                    assert hinted == plain


def test_metropolis_backward_argument_errors(lib):
    i64 = ctypes.c_int64
    f = lib.nsh_metropolis_aggregate_backward
    f.restype = ctypes.c_int
    d = ctypes.c_void_p(256)
    args = [d, d, d, i64(1), i64(5), i64(1), i64(256), i64(256), 3, 1, ctypes.c_double(1e-6),
            d, d, d, d, d, d]
    rc = f(*args[:11], None, *args[12:], d, i64(1 << 30), None)
    assert rc == 1 and "null" in _err(lib)
    rc = f(*args, d, i64(64), None)
    assert rc == 1 and "workspace" in _err(lib)
    small = args[:6] + [i64(32), i64(64)] + args[8:]
    rc = f(*small, d, i64(1 << 30), None)
    assert rc == 1 and "3 tiles" in _err(lib)


# A (b, c) plane of 2^31 bytes or more (in the accumulator type) is refused
# by every entry point before any device work: in-plane offsets are 32-bit.
# 23171^2 fp32 elements = 2,147,580,964 bytes; 16384^2 fp64 = 2^31 bytes.
_BIG = [(3, 23171, 23171), (1, 23171, 23171), (4, 16384, 16384)]


@pytest.mark.parametrize("dtype,H,W", _BIG)
def test_plane_size_limit_every_entry_point(lib, dtype, H, W):
    i64, dbl = ctypes.c_int64, ctypes.c_double
    p = ctypes.c_void_p(256)
    S, B, C = 5, 1, 1
    calls = {
        "nsh_accumulate_uz_forward": (p, p, p, i64(S), i64(B), i64(C), i64(H), i64(W), dtype, p,
                                      p, None, i64(0), None),
        "nsh_accumulate_uz_backward": (p, p, p, p, p, i64(S), i64(B), i64(C), i64(H), i64(W),
                                       dtype, p, p, None, i64(0), None),
        "nsh_normalized_accumulate_uz_forward": (p, p, p, i64(S), i64(B), i64(C), i64(H), i64(W),
                                                 dtype, 1, p, p, None, i64(0), None),
        "nsh_normalized_accumulate_uz_backward": (p, p, p, p, p, p, p, i64(S), i64(B), i64(C),
                                                  i64(H), i64(W), dtype, 1, p, p, None, i64(0),
                                                  None),
        "nsh_accumulate_uz_scalar_forward": (p, p, p, i64(S), i64(3), i64(B), i64(C), i64(H),
                                             i64(W), dtype, p, p, None),
        "nsh_shift_gather_forward": (p, p, i64(S), i64(3), i64(B), i64(C), i64(H), i64(W), dtype,
                                     p, p, None),
        "nsh_pair_gather_backward": (p, p, i64(S), i64(3), i64(B), i64(C), i64(H), i64(W), dtype,
                                     p, None),
        "nsh_metropolis_aggregate": (p, p, p, i64(B), i64(S), i64(C), i64(H), i64(W), dtype, 1,
                                     dbl(1e-6), p, p, p, None, i64(0), None),
    }
    for name, args in calls.items():
        f = getattr(lib, name)
        f.restype = ctypes.c_int
        rc = f(*args)
        assert rc == 1 and "2^31" in _err(lib), (name, rc, _err(lib))
    for q in ("nsh_accumulate_uz_workspace_bytes", "nsh_normalized_workspace_bytes"):
        f = getattr(lib, q)
        f.restype = ctypes.c_int64
        assert f(i64(S), i64(B), i64(C), i64(H), i64(W), dtype, 0) == -1, q


def test_stream_probe_host_checks(monkeypatch):
    """The probe wrapper rejects, before any native call, buffers the
    grid-stride kernels would run past: a copy into a smaller dst, a read
    sink under the 4 KiB the read kernels may write, non-contiguous views,
    a non-tensor src and an unknown kind.  (The CUDA-residency check is
    bypassed so that host tensors reach the later checks; the native call
    is replaced so nothing runs.)"""
    from neural_shift_cuda_amd import _C
    calls = []
    monkeypatch.setattr(_C, "_cuda", lambda t, name: None)
    monkeypatch.setattr(_C, "_call", lambda *a: calls.append(a))
    monkeypatch.setattr(_C, "_stream", lambda t: 0)
    monkeypatch.setattr(torch.cuda, "device", lambda d: __import__("contextlib").nullcontext())
    src = torch.zeros(4096, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="copy needs 4096"):
        _C.stream_probe("copy", src, torch.zeros(1024, dtype=torch.uint8), workgroups=1)
    with pytest.raises(RuntimeError, match="4096 bytes"):
        _C.stream_probe("read", src, torch.zeros(1024, dtype=torch.uint8), workgroups=1)
    with pytest.raises(RuntimeError, match="contiguous"):
        _C.stream_probe("read_nt", torch.zeros(64, 128)[:, ::2], torch.zeros(4096,
                                                                            dtype=torch.uint8),
                        workgroups=1)
    with pytest.raises(RuntimeError, match="contiguous"):
        _C.stream_probe("fill", None, torch.zeros(64, 128)[:, ::2], workgroups=1)
    with pytest.raises(RuntimeError, match="must be a tensor"):
        _C.stream_probe("copy", None, torch.zeros(4096, dtype=torch.uint8), workgroups=1)
    with pytest.raises(RuntimeError, match="unknown kind"):
        _C.stream_probe("scan", src, torch.zeros(4096, dtype=torch.uint8), workgroups=1)
    assert not calls
    _C.stream_probe("copy", src, torch.zeros(4096, dtype=torch.uint8), workgroups=1)
    _C.stream_probe("read", src, torch.zeros(4096, dtype=torch.uint8), workgroups=1)
    assert len(calls) == 2 and calls[0][4] == 4096


def test_metropolis_table_records_its_radius():
    """metropolis.py builds its device table from the Python shift list and
    records the radius it already knows (the 6-pixel border hint of the
    fused backward, NSH_NARROW_HALO, is set from it without a device read):
    the recorded value is what table_radius would compute."""
    from neural_shift_cuda_amd import _C
    from neural_shift_cuda_amd import metropolis as metro
    for rows, r in [([(1, 2, True), (-6, 0, False)], 6), ([(0, 7, True)], 7),
                    ([(2 ** 40, 0, True)], 2 ** 30)]:
        t = metro._shifts_to_tensor(rows, "cpu")
        ent = _C._RADII.get(id(t))
        assert ent is not None and ent[2] == r
        _C._RADII.pop(id(t))
        assert _C.table_radius(t) == r


def test_table_radius_hint():
    """The Python layer's radius of a shift table (what selects the
    16-pixel scatter border, NSH_WIDE_HALO): clamped like the kernels'
    decode, cached per tensor object and version, carried from a host table
    to the device copy ops makes of it."""
    from neural_shift_cuda_amd import _C, ops
    t = torch.tensor([[3, -10, 1], [0, 2, 0]])
    assert _C.table_radius(t) == 10 and _C._halo_flag(t) == _C.NSH_WIDE_HALO
    t[1, 0] = -17  # in place: a new version, read again
    assert _C.table_radius(t) == 17 and _C._halo_flag(t) == _C.NSH_WIDER_HALO
    t[1, 0] = 25
    assert _C._halo_flag(t) == 0
    assert _C._halo_flag(torch.tensor([[8, -8, 1]])) == 0
    assert _C.table_radius(torch.tensor([[2 ** 40, 0]])) == 2 ** 30
    big = torch.tensor([[0, 0, 0]] * 300)
    _C.remember_table_radius(big, 12)
    assert _C.table_radius(big) == 12
    # the copy ops makes of an int32 host table carries the radius
    t32 = torch.tensor([[1, 16, 1], [0, 1, 0]], dtype=torch.int32)
    out = ops._prep_shifts_for_cuda(t32, torch.device("cpu"))
    assert out is not t32 and _C._RADII[id(out)][2] == 16
    # and so does a row-code rewrite of a table
    codes, rows = ops._mirror_table(torch.tensor([[9, 1, 1], [0, 1, 0]]), True)
    assert rows and _C._RADII[id(codes)][2] == 9
