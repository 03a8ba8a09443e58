"""nsh_accumulate_uz_forward_noalloc: the allocation-free accumulate_uz
forward (static per-GPU scratch instead of a caller workspace), called
through the C ABI and compared bit for bit with nsh_accumulate_uz_forward
given a caller workspace: the same scatter kernels in the same order.

Two calls in a row, the second on a smaller input, check that nothing of
the first call's scratch contents leaks into the second; a shape whose
workspace exceeds the scratch is rejected on the host before any launch.
"""
from __future__ import annotations

import ctypes
import sys

import pytest
import torch

from neural_shift_cuda_amd import _C
from neural_shift_cuda_amd.workloads import halfplane_shifts, softplus_weights, synthetic_image

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]
DEV = torch.device("cuda:0")
_CODE = {torch.float16: 1, torch.bfloat16: 2, torch.float32: 3, torch.float64: 4}


def _case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _lib():
    lib = ctypes.CDLL(_C.LIBRARY_PATH)
    P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.nsh_accumulate_uz_forward_noalloc.argtypes = [P, P, P, I64, I64, I64, I64, I64, I, P, P, P]
    lib.nsh_accumulate_uz_forward_noalloc.restype = I
    lib.nsh_accumulate_uz_forward.argtypes = [P, P, P, I64, I64, I64, I64, I64, I, P, P, P, I64, P]
    lib.nsh_accumulate_uz_forward.restype = I
    lib.nsh_accumulate_uz_workspace_bytes.argtypes = [I64, I64, I64, I64, I64, I, I]
    lib.nsh_accumulate_uz_workspace_bytes.restype = I64
    lib.nsh_last_error.restype = ctypes.c_char_p
    return lib


def _inputs(B, C, H, W, R, dtype, seed):
    sh = halfplane_shifts(R)
    x = synthetic_image(B, C, H, W, seed=seed).to(dtype)
    w = softplus_weights((sh.size(0) * B, C, H, W), seed=seed + 1).to(dtype)
    return x.to(DEV), w.to(DEV), sh.to(DEV)


def _outputs(x):
    acc = torch.float64 if x.dtype == torch.float64 else torch.float32
    return torch.empty(x.shape, dtype=acc, device=DEV), torch.empty(x.shape, dtype=acc, device=DEV)


def _noalloc(lib, x, w, sh):
    B, C, H, W = x.shape
    U, Z = _outputs(x)
    st = torch.cuda.current_stream().cuda_stream
    rc = lib.nsh_accumulate_uz_forward_noalloc(x.data_ptr(), w.data_ptr(), sh.data_ptr(),
                                               sh.size(0), B, C, H, W, _CODE[x.dtype],
                                               U.data_ptr(), Z.data_ptr(), st)
    assert rc == 0, lib.nsh_last_error().decode()
    return U, Z


def _with_workspace(lib, x, w, sh, use_ws=True):
    B, C, H, W = x.shape
    U, Z = _outputs(x)
    n = lib.nsh_accumulate_uz_workspace_bytes(sh.size(0), B, C, H, W, _CODE[x.dtype], 0)
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=DEV) if (use_ws and n > 0) else None
    st = torch.cuda.current_stream().cuda_stream
    rc = lib.nsh_accumulate_uz_forward(x.data_ptr(), w.data_ptr(), sh.data_ptr(), sh.size(0), B,
                                       C, H, W, _CODE[x.dtype], U.data_ptr(), Z.data_ptr(),
                                       None if ws is None else ws.data_ptr(),
                                       n if ws is not None else 0, st)
    assert rc == 0, lib.nsh_last_error().decode()
    return U, Z, n


# (shape B, C, H, W, radius, dtype): the first is the c2 shape (10 MiB of
# workspace), then smaller scatter shapes, then one that takes the gather
# kernels (no workspace)
CASES = [
    ((4, 1, 512, 512), 7, torch.float16),
    ((1, 2, 72, 200), 3, torch.float32),
    ((1, 1, 104, 104), 2, torch.float64),
    ((1, 1, 30, 44), 2, torch.float32),
]


def test_noalloc_matches_workspace_entry_point():
    lib = _lib()
    for i, ((B, C, H, W), R, dtype) in enumerate(CASES):
        _case(f"noalloc forward call {i}: {(B, C, H, W)} R={R} {dtype}")
        x, w, sh = _inputs(B, C, H, W, R, dtype, 100 + i)
        U, Z = _noalloc(lib, x, w, sh)
        Ur, Zr, need = _with_workspace(lib, x, w, sh)
        assert need <= (32 << 20)
        torch.cuda.synchronize()
        assert torch.equal(U, Ur) and torch.equal(Z, Zr), f"call {i} differs"
        if need > 0:
            # the scatter path really ran: the gather kernels sum in another order
            Ug, _, _ = _with_workspace(lib, x, w, sh, use_ws=False)
            assert torch.allclose(U, Ug, rtol=1e-4, atol=1e-4)


def test_noalloc_repeated_calls_and_shrinking_input():
    """Two calls in a row, the second smaller, each equal to the workspace
    entry point; the first result is not disturbed by the second call."""
    lib = _lib()
    _case("noalloc forward: large then small")
    xa, wa, sha = _inputs(2, 1, 512, 384, 6, torch.float32, 7)
    xb, wb, shb = _inputs(1, 1, 136, 200, 4, torch.float32, 9)
    Ua, Za = _noalloc(lib, xa, wa, sha)
    Ub, Zb = _noalloc(lib, xb, wb, shb)
    Ura, Zra, na = _with_workspace(lib, xa, wa, sha)
    Urb, Zrb, nb = _with_workspace(lib, xb, wb, shb)
    torch.cuda.synchronize()
    assert na > nb > 0
    assert torch.equal(Ua, Ura) and torch.equal(Za, Zra)
    assert torch.equal(Ub, Urb) and torch.equal(Zb, Zrb)


def test_noalloc_rejects_shapes_beyond_the_scratch():
    """The c4 shape needs 352 MiB of workspace: refused on the host."""
    lib = _lib()
    _case("noalloc forward: oversized shape")
    x = torch.empty(16, device=DEV)
    p = x.data_ptr()
    need = lib.nsh_accumulate_uz_workspace_bytes(85, 1, 1, 8192, 8192, 3, 0)
    assert need > (32 << 20)
    rc = lib.nsh_accumulate_uz_forward_noalloc(p, p, p, 85, 1, 1, 8192, 8192, 3, p, p, None)
    assert rc == 1
    msg = lib.nsh_last_error().decode()
    assert "static scratch" in msg and str(need) in msg
