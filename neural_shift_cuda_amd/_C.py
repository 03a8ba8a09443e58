"""``_C``: the native module of the package, over the C ABI of
``libneural_shift_hip.so`` (declared in ``include/neural_shift_hip.h``).

It exposes the same attribute names, argument lists and return conventions
as the reference's pybind11 module ``neural_shift_cuda._C``
(csrc/shift_ops.cpp:347-368 and csrc/metropolis.cpp:42-48 in
trishitmg/neural_shift_cuda), so the guards in ``ops.py`` and
``metropolis.py`` probe it the same way.  Differences from the reference:

* outputs are allocated here with ``torch.empty`` and the library only
  launches kernels on the current stream of the tensors' device;
* fp16 and bf16 tensors are accepted everywhere; accumulation happens in
  fp32 (fp64 for fp64 inputs), so U/Z/D/log_C come back in that
  accumulator dtype while gradients come back in the input dtype;
* argument errors raise ``RuntimeError`` with the reference's messages;
* the accumulate and normalized functions take a keyword ``row_codes``
  (default False: the reference's has_inverse flag, nonzero = mirror): True
  marks a table whose third column holds the library's row codes
  (``NSH_SHIFT_CODES``: circular mirrors, in-kernel forward box);
* and a keyword ``shared_weights`` (default False): True takes weights of
  shape (S*B, 1, H, W) used for every channel (``NSH_SHARED_WEIGHTS``); the
  weight gradient then still comes back per channel, (S*B, C, H, W).

Importing this module raises ``OSError`` when the library has not been built
(``python -m neural_shift_cuda_amd.build``); ``ops.py`` keeps that error and
reports it when a GPU tensor reaches an op, instead of falling back.
"""
from __future__ import annotations

import ctypes
import os
import weakref
from typing import List, Optional, Sequence

import torch  # must precede the CDLL: the library binds to torch's HIP runtime

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libneural_shift_hip.so")
_lib = ctypes.CDLL(_LIB_PATH)

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int

# include/neural_shift_hip.h: the table's third column holds row codes
NSH_SHIFT_CODES = 0x100
NSH_SHARED_WEIGHTS = 0x200
NSH_WIDE_HALO = 0x400
NSH_WIDER_HALO = 0x800
NSH_NARROW_HALO = 0x1000  # Metropolis backward: every shift within 6 pixels
NSH_ERR_UNSUPPORTED = 3

_SIGS = {
    "nsh_last_error": ([], ctypes.c_char_p),
    "nsh_index_width_bits": ([], _I),
    "nsh_version": ([], ctypes.c_char_p),
    "nsh_shift_gather_forward": ([_P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P, _P, _P], _I),
    "nsh_pair_gather_forward": ([_P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P, _P, _P], _I),
    "nsh_shift_gather_backward": ([_P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P, _P], _I),
    "nsh_pair_gather_backward": ([_P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P, _P], _I),
    "nsh_accumulate_uz_forward": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _I64,
                                   _P], _I),
    "nsh_accumulate_uz_backward": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _P, _P,
                                    _P, _I64, _P], _I),
    "nsh_accumulate_uz_workspace_bytes": ([_I64, _I64, _I64, _I64, _I64, _I, _I], _I64),
    "nsh_accumulate_uz_forward_band": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I,
                                        _P, _P, _P, _I64, _P], _I),
    "nsh_accumulate_uz_backward_band": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                                         _I64, _I, _P, _P, _P, _I64, _P], _I),
    "nsh_normalized_accumulate_uz_forward": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _I,
                                              _P, _P, _P, _I64, _P], _I),
    "nsh_normalized_accumulate_uz_forward_mixed": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                                    _I64, _I64, _I, _P, _P, _P, _I64, _P], _I),
    "nsh_head_mix_forward": ([_P, _P, _I64, _I64, _I64, _I64, _I, _P, _P], _I),
    "nsh_head_mix_workspace_bytes": ([_I64, _I64, _I64, _I64, _I], _I64),
    "nsh_head_mix_backward": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _I64, _P],
                              _I),
    "nsh_normalized_accumulate_uz_backward": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64,
                                               _I64, _I64, _I, _I, _P, _P, _P, _I64, _P], _I),
    "nsh_normalized_workspace_bytes": ([_I64, _I64, _I64, _I64, _I64, _I, _I], _I64),
    "nsh_scalar_backward_splits": ([_I64, _I64], _I),
    "nsh_accumulate_uz_scalar_forward": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P,
                                          _P, _P], _I),
    "nsh_accumulate_uz_scalar_backward": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                                           _I, _P, _P, _P, _P], _I),
    "nsh_metropolis_aggregate": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _I,
                                  ctypes.c_double, _P, _P, _P, _P, _I64, _P], _I),
    "nsh_metropolis_workspace_bytes": ([_I64, _I64, _I64, _I64, _I64, _I], _I64),
    "nsh_metropolis_aggregate_backward": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _I,
                                           ctypes.c_double, _P, _P, _P, _P, _P, _P, _P, _I64,
                                           _P], _I),
    "nsh_metropolis_backward_workspace_bytes": ([_I64, _I64, _I64, _I64, _I64, _I], _I64),
    "nsh_stream_probe": ([_I, _P, _P, _I64, _I, _P], _I),
}
for _name, (_args, _res) in _SIGS.items():
    _fn = getattr(_lib, _name)
    _fn.argtypes = _args
    _fn.restype = _res

LIBRARY_PATH = _LIB_PATH

_DTYPE_CODE = {
    torch.float16: 1,
    torch.bfloat16: 2,
    torch.float32: 3,
    torch.float64: 4,
}


def _acc_dtype(dtype: torch.dtype) -> torch.dtype:
    return torch.float64 if dtype == torch.float64 else torch.float32


def _code(t: torch.Tensor, op: str) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise RuntimeError(f"\"{op}\" not implemented for '{t.dtype}'") from None


def _check(ok: bool, msg: str) -> None:
    if not ok:
        raise RuntimeError(msg)


def _cuda(t: torch.Tensor, name: str) -> None:
    _check(t.is_cuda, f"{name} must be a CUDA tensor")


def _contig(t: torch.Tensor, name: str) -> None:
    _check(t.is_contiguous(), f"{name} must be contiguous")


def _nchw(t: torch.Tensor, name: str) -> None:
    _check(t.dim() == 4, f"{name} must have 4 dims (N,C,H,W)")


def _prep_shifts(shifts: torch.Tensor, device: torch.device) -> torch.Tensor:
    """(S, 2|3) int64 contiguous table on `device` (shift_ops.cpp:65-75)."""
    _check(shifts.dim() == 2, "shifts must be 2-D (S, 2 or 3)")
    _check(shifts.size(1) in (2, 3), "shifts must have 2 or 3 columns")
    return shifts.to(device=device, dtype=torch.int64).contiguous()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _call(name: str, *args) -> None:
    rc = getattr(_lib, name)(*args)
    if rc != 0:
        msg = _lib.nsh_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"{name} failed with code {rc}")


def _ptr(t) -> int:
    return t.data_ptr() if t is not None else None


# ---------------------------------------------------------------------------
# Module API (names as in the reference's _C)
# ---------------------------------------------------------------------------

def index_width_bits() -> int:
    """Width of device tensor indices and shift offsets (always 64)."""
    return int(_lib.nsh_index_width_bits())


def version() -> str:
    return _lib.nsh_version().decode()


def _gather_forward(op: str, fn: str, guide: torch.Tensor, shifts: torch.Tensor, pair: bool):
    _cuda(guide, "guide")
    _contig(guide, "guide")
    _nchw(guide, "guide")
    sh = _prep_shifts(shifts, guide.device)
    B, C, H, W = guide.shape
    S = sh.size(0)
    out = torch.empty((S * B, 2 * C if pair else C, H, W), dtype=guide.dtype, device=guide.device)
    mask = torch.empty((S * B, 1, H, W), dtype=guide.dtype, device=guide.device)
    if out.numel() == 0:
        return [out, mask]
    with torch.cuda.device(guide.device):
        _call(fn, guide.data_ptr(), sh.data_ptr(), S, sh.size(1), B, C, H, W, _code(guide, op),
              out.data_ptr(), mask.data_ptr(), _stream(guide))
    return [out, mask]


def _gather_backward(op: str, fn: str, grad_out: torch.Tensor, shifts: torch.Tensor, B: int,
                     C: int, H: int, W: int) -> torch.Tensor:
    _cuda(grad_out, "grad_out")
    _contig(grad_out, "grad_out")
    _nchw(grad_out, "grad_out")
    sh = _prep_shifts(shifts, grad_out.device)
    grad = torch.empty((B, C, H, W), dtype=grad_out.dtype, device=grad_out.device)
    if grad.numel() == 0:
        return grad
    with torch.cuda.device(grad_out.device):
        _call(fn, grad_out.data_ptr(), sh.data_ptr(), sh.size(0), sh.size(1), B, C, H, W,
              _code(grad_out, op), grad.data_ptr(), _stream(grad_out))
    return grad


def shift_gather_forward(guide: torch.Tensor, shifts: torch.Tensor) -> List[torch.Tensor]:
    """[out (S*B,C,H,W), mask (S*B,1,H,W)] (shift_ops.cpp:81-100)."""
    return _gather_forward("shift_gather_fwd", "nsh_shift_gather_forward", guide, shifts, False)


def shift_gather_backward(grad_out: torch.Tensor, shifts: torch.Tensor, B: int, C: int, H: int,
                          W: int) -> torch.Tensor:
    """Gather-form adjoint (shift_ops.cpp:102-115)."""
    return _gather_backward("shift_gather_bwd", "nsh_shift_gather_backward", grad_out, shifts,
                            B, C, H, W)


def pair_gather_forward(guide: torch.Tensor, shifts: torch.Tensor) -> List[torch.Tensor]:
    """[pair (S*B,2C,H,W), mask (S*B,1,H,W)] (shift_ops.cpp:121-140)."""
    return _gather_forward("pair_gather_fwd", "nsh_pair_gather_forward", guide, shifts, True)


def pair_gather_backward(grad_out: torch.Tensor, shifts: torch.Tensor, B: int, C: int, H: int,
                         W: int) -> torch.Tensor:
    """Deterministic gather-form adjoint (shift_ops.cpp:142-154)."""
    return _gather_backward("pair_gather_bwd", "nsh_pair_gather_backward", grad_out, shifts,
                            B, C, H, W)


def _check_pair(op: str, x: torch.Tensor, weights: torch.Tensor, shifts: torch.Tensor,
                weight_shape_msg: str, shared: bool = False):
    _cuda(x, "x")
    _contig(x, "x")
    _nchw(x, "x")
    _cuda(weights, "weights")
    _contig(weights, "weights")
    _nchw(weights, "weights")
    _check(shifts.dim() == 2 and shifts.size(1) == 3, f"{op}: shifts must be (S, 3)")
    sh = _prep_shifts(shifts, x.device)
    B, C, H, W = x.shape
    S = sh.size(0)
    _check(0 < S <= 1024, f"{op}: tree reduction requires 1 <= S <= 1024")
    _check(weights.device == x.device, f"{op}: x and weights must be on the same device")
    _check(weights.dtype == x.dtype, f"{op}: x and weights must have the same dtype")
    if shared:
        _check(tuple(weights.shape) == (S * B, 1, H, W),
               f"{op}: shared weights must be (S*B, 1, H, W)")
    else:
        _check(tuple(weights.shape) == (S * B, C, H, W), weight_shape_msg)
    return sh, B, C, H, W, S


def _flags(row_codes: bool, shared: bool) -> int:
    return (NSH_SHIFT_CODES if row_codes else 0) | (NSH_SHARED_WEIGHTS if shared else 0)


# Radius of a shift table, per tensor object and version: id -> (weakref,
# version, radius).  A device table is read (one host sync) the first time
# it is seen; ops._prep_shifts_for_cuda records the radius of the device
# copies it makes from host tables, so those are never read back.
_RADII: dict = {}
_KERNEL_CLAMP = 1 << 30  # the kernels clamp dx, dy to +-2^30 when they decode a table


def remember_table_radius(shifts: torch.Tensor, radius: int) -> None:
    """Record the radius of `shifts` (as table_radius would compute it)."""
    key = id(shifts)
    try:
        ref = weakref.ref(shifts, lambda _, k=key: _RADII.pop(k, None))
    except TypeError:
        return
    _RADII[key] = (ref, shifts._version, int(radius))


def table_radius(shifts: torch.Tensor) -> Optional[int]:
    """max(|dx|, |dy|) over the rows of a (S, 2|3) shift table, with each
    value clamped to +-2^30 as the kernels decode it; None when a device
    table is seen for the first time during stream capture (reading it
    would wait on the stream)."""
    ent = _RADII.get(id(shifts))
    if ent is not None and ent[0]() is shifts and ent[1] == shifts._version:
        return ent[2]
    if shifts.numel() == 0:
        return 0
    if shifts.is_cuda and torch.cuda.is_current_stream_capturing():
        return None
    r = int(shifts[:, :2].clamp(-_KERNEL_CLAMP, _KERNEL_CLAMP).abs().amax().item())
    remember_table_radius(shifts, r)
    return r


def _narrow_halo_flag(shifts: torch.Tensor) -> int:
    """NSH_NARROW_HALO when every row of the table lies within 6 pixels: the
    fused Metropolis backward's edge pass and the fp64 normalized backward then
    run on a 6-pixel border with three workgroups per CU
    (include/neural_shift_hip.h).  Only a hint."""
    r = table_radius(shifts)
    return NSH_NARROW_HALO if r is not None and r <= 6 else 0


# Tables with more rows than the (2 * 8 + 1)^2 distinct shifts of radius 8
# reach beyond it (unless they repeat rows): the hint when the radius is
# unknown.
_HALO8_ROWS = (2 * 8 + 1) ** 2


def _halo_flag(shifts: torch.Tensor) -> int:
    """NSH_WIDE_HALO when the table's radius is 9..16, NSH_WIDER_HALO for
    17..24: accumulate_uz's scatter tiles then carry a 16- or 24-pixel border
    (include/neural_shift_hip.h).  Only a hint; the kernels check the radius
    themselves."""
    r = table_radius(shifts)
    if r is None:
        return NSH_WIDE_HALO if shifts.size(0) > _HALO8_ROWS else 0
    if 8 < r <= 16:
        return NSH_WIDE_HALO
    return NSH_WIDER_HALO if 16 < r <= 24 else 0


def _band_args(band) -> tuple:
    """(row_origin, image_height) of a band call, checked."""
    org, hg = (int(v) for v in band)
    _check(hg >= 1, "band: image_height must be >= 1")
    return org, hg


def accumulate_uz_forward(x: torch.Tensor, weights: torch.Tensor,
                          shifts: torch.Tensor, *, row_codes: bool = False,
                          shared_weights: bool = False, band=None) -> List[torch.Tensor]:
    """[U, Z] in the accumulator dtype (shift_ops.cpp:160-192).  `band`
    (row_origin, image_height): x holds one horizontal band of a larger
    image, local row h being image row (row_origin + h) mod image_height
    for every box test (nsh_accumulate_uz_forward_band)."""
    sh, B, C, H, W, S = _check_pair("accumulate_uz", x, weights, shifts,
                                    "weights shape must be (S*B, C, H, W)", shared_weights)
    acc = _acc_dtype(x.dtype)
    code = _code(x, "accumulate_uz_fwd") | _flags(row_codes, shared_weights) | _halo_flag(shifts)
    U = torch.empty(x.shape, dtype=acc, device=x.device)
    Z = torch.empty(x.shape, dtype=acc, device=x.device)
    ws, nws = _workspace(S, B, C, H, W, code, False, x.device)
    with torch.cuda.device(x.device):
        if band is None:
            _call("nsh_accumulate_uz_forward", x.data_ptr(), weights.data_ptr(), sh.data_ptr(),
                  S, B, C, H, W, code, U.data_ptr(), Z.data_ptr(), _ptr(ws), nws, _stream(x))
        else:
            org, hg = _band_args(band)
            _call("nsh_accumulate_uz_forward_band", x.data_ptr(), weights.data_ptr(),
                  sh.data_ptr(), S, B, C, H, W, org, hg, code, U.data_ptr(), Z.data_ptr(),
                  _ptr(ws), nws, _stream(x))
    return [U, Z]


def _workspace(S, B, C, H, W, code, backward, device):
    """Scratch buffer of accumulate_uz (spilled window borders of the
    once-per-element weight stream); (None, 0) when the shape needs none."""
    n = int(_lib.nsh_accumulate_uz_workspace_bytes(S, B, C, H, W, code, int(backward)))
    if n <= 0:
        return None, 0
    return torch.empty(n, dtype=torch.uint8, device=device), n


def _grad_in(g: torch.Tensor, like: torch.Tensor, acc: torch.dtype, name: str) -> torch.Tensor:
    _cuda(g, name)
    _check(tuple(g.shape) == tuple(like.shape), f"{name} must match the shape of x")
    return g.to(acc).contiguous()


def accumulate_uz_backward(x: torch.Tensor, weights: torch.Tensor, grad_U: torch.Tensor,
                           grad_Z: torch.Tensor, shifts: torch.Tensor, *,
                           row_codes: bool = False, shared_weights: bool = False,
                           band=None) -> List[torch.Tensor]:
    """[grad_x, grad_w] in the input dtype (shift_ops.cpp:194-212); grad_w
    is per channel, (S*B, C, H, W), also for shared weights.  `band` as in
    accumulate_uz_forward."""
    sh, B, C, H, W, S = _check_pair("accumulate_uz", x, weights, shifts,
                                    "weights shape must be (S*B, C, H, W)", shared_weights)
    acc = _acc_dtype(x.dtype)
    gU = _grad_in(grad_U, x, acc, "grad_U")
    gZ = _grad_in(grad_Z, x, acc, "grad_Z")
    code = _code(x, "accumulate_uz_bwd") | _flags(row_codes, shared_weights) | _halo_flag(shifts)
    gx = torch.empty_like(x)
    gw = torch.empty((S * B, C, H, W), dtype=weights.dtype, device=weights.device)
    ws, nws = _workspace(S, B, C, H, W, code, True, x.device)
    with torch.cuda.device(x.device):
        if band is None:
            _call("nsh_accumulate_uz_backward", x.data_ptr(), weights.data_ptr(), gU.data_ptr(),
                  gZ.data_ptr(), sh.data_ptr(), S, B, C, H, W, code, gx.data_ptr(),
                  gw.data_ptr(), _ptr(ws), nws, _stream(x))
        else:
            org, hg = _band_args(band)
            _call("nsh_accumulate_uz_backward_band", x.data_ptr(), weights.data_ptr(),
                  gU.data_ptr(), gZ.data_ptr(), sh.data_ptr(), S, B, C, H, W, org, hg, code,
                  gx.data_ptr(), gw.data_ptr(), _ptr(ws), nws, _stream(x))
    return [gx, gw]


def normalized_accumulate_uz_forward(x: torch.Tensor, weights: torch.Tensor, shifts: torch.Tensor,
                                     log_weights: bool, *, row_codes: bool = False,
                                     shared_weights: bool = False) -> List[torch.Tensor]:
    """[D, log_C] in the accumulator dtype (shift_ops.cpp:218-252)."""
    sh, B, C, H, W, S = _check_pair("normalized_accumulate_uz", x, weights, shifts,
                                    "normalized_accumulate_uz: weights must be (S*B, C, H, W)",
                                    shared_weights)
    acc = _acc_dtype(x.dtype)
    code = _code(x, "normalized_accumulate_uz_fwd") | _flags(row_codes, shared_weights)
    D = torch.empty(x.shape, dtype=acc, device=x.device)
    L = torch.empty(x.shape, dtype=acc, device=x.device)
    ws, nws = _norm_workspace(S, B, C, H, W, code, False, x.device)
    with torch.cuda.device(x.device):
        _call("nsh_normalized_accumulate_uz_forward", x.data_ptr(), weights.data_ptr(),
              sh.data_ptr(), S, B, C, H, W, code, int(bool(log_weights)), D.data_ptr(),
              L.data_ptr(), _ptr(ws), nws, _stream(x))
    return [D, L]


def normalized_accumulate_uz_forward_mixed(x: torch.Tensor, head_weights: torch.Tensor,
                                           head_mix: torch.Tensor, shifts: torch.Tensor, *,
                                           row_codes: bool = False
                                           ) -> Optional[List[torch.Tensor]]:
    """[D, log_C] of the positive-weight forward whose channel-c weights are
    sum_j head_mix[c, j] * head_weights[:, j], formed in the kernels' weight
    load (nsh_normalized_accumulate_uz_forward_mixed).  head_weights is
    (S*B, heads, H, W) in x's dtype, head_mix (C, heads).  None when the
    entry point does not serve the shape or head count (the caller mixes
    the heads and runs the plain forward)."""
    op = "normalized_accumulate_uz_forward_mixed"
    for t, name in ((x, "x"), (head_weights, "head_weights")):
        _cuda(t, name)
        _contig(t, name)
        _nchw(t, name)
    _check(shifts.dim() == 2 and shifts.size(1) == 3, f"{op}: shifts must be (S, 3)")
    sh = _prep_shifts(shifts, x.device)
    B, C, H, W = x.shape
    S = sh.size(0)
    heads = head_weights.size(1)
    _check(0 < S <= 1024, f"{op}: tree reduction requires 1 <= S <= 1024")
    _check(head_weights.device == x.device, f"{op}: x and head_weights must be on the same device")
    _check(head_weights.dtype == x.dtype, f"{op}: x and head_weights must have the same dtype")
    _check(tuple(head_weights.shape) == (S * B, heads, H, W),
           f"{op}: head_weights must be (S*B, heads, H, W)")
    _check(head_mix.dim() == 2 and tuple(head_mix.shape) == (C, heads),
           f"{op}: head_mix must be (C, heads)")
    acc = _acc_dtype(x.dtype)
    mix = head_mix.detach().to(device=x.device, dtype=acc).contiguous()
    code = _code(x, op) | _flags(row_codes, False)
    D = torch.empty(x.shape, dtype=acc, device=x.device)
    L = torch.empty(x.shape, dtype=acc, device=x.device)
    ws, nws = _norm_workspace(S, B, C, H, W, code, False, x.device)
    with torch.cuda.device(x.device):
        rc = _lib.nsh_normalized_accumulate_uz_forward_mixed(
            x.data_ptr(), head_weights.data_ptr(), mix.data_ptr(), sh.data_ptr(), S, B, C, H, W,
            heads, code, D.data_ptr(), L.data_ptr(), _ptr(ws), nws, _stream(x))
    if rc == NSH_ERR_UNSUPPORTED:
        return None
    if rc != 0:
        msg = _lib.nsh_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"{op} failed with code {rc}")
    return [D, L]


def _mix_check(w: torch.Tensor, mix: torch.Tensor, op: str):
    _cuda(w, "w")
    _contig(w, "w")
    _check(w.dim() == 3, f"{op}: w must be (N, heads, P)")
    _check(mix.dim() == 2 and mix.size(1) == w.size(1), f"{op}: mix must be (C, heads)")
    return _acc_dtype(w.dtype)


def head_mix_forward(w: torch.Tensor, mix: torch.Tensor) -> Optional[torch.Tensor]:
    """(N, C, P) = sum_j mix[c, j] * w[:, j] for w (N, heads, P) and mix
    (C, heads) (nsh_head_mix_forward); None for head or channel counts the
    kernels do not serve."""
    op = "head_mix_forward"
    acc = _mix_check(w, mix, op)
    N, h, P = w.shape
    C = mix.size(0)
    m = mix.detach().to(device=w.device, dtype=acc).contiguous()
    out = torch.empty(N, C, P, dtype=w.dtype, device=w.device)
    with torch.cuda.device(w.device):
        rc = _lib.nsh_head_mix_forward(w.data_ptr(), m.data_ptr(), N, h, C, P,
                                       _code(w, op), out.data_ptr(), _stream(w))
    if rc == NSH_ERR_UNSUPPORTED:
        return None
    if rc != 0:
        raise RuntimeError(_lib.nsh_last_error().decode(errors="replace") or f"{op}: code {rc}")
    return out


def head_mix_backward(w: torch.Tensor, mix: torch.Tensor, grad_out: torch.Tensor
                      ) -> List[torch.Tensor]:
    """[grad_w (N, heads, P) in w's dtype, grad_mix (C, heads) in the
    accumulator type] of head_mix_forward (nsh_head_mix_backward)."""
    op = "head_mix_backward"
    acc = _mix_check(w, mix, op)
    N, h, P = w.shape
    C = mix.size(0)
    _cuda(grad_out, "grad_out")
    _check(tuple(grad_out.shape) == (N, C, P), f"{op}: grad_out must be (N, C, P)")
    g = grad_out.to(w.dtype).contiguous()
    m = mix.detach().to(device=w.device, dtype=acc).contiguous()
    gw = torch.empty_like(w)
    gm = torch.empty(C, h, dtype=acc, device=w.device)
    code = _code(w, op)
    n = int(_lib.nsh_head_mix_workspace_bytes(N, h, C, P, code))
    _check(n > 0, f"{op}: {_lib.nsh_last_error().decode(errors='replace')}")
    ws = torch.empty(n, dtype=torch.uint8, device=w.device)
    with torch.cuda.device(w.device):
        _call("nsh_head_mix_backward", w.data_ptr(), m.data_ptr(), g.data_ptr(), N, h, C, P,
              code, gw.data_ptr(), gm.data_ptr(), ws.data_ptr(), n, _stream(w))
    return [gw, gm]


def _norm_workspace(S, B, C, H, W, code, backward, device):
    """Scratch buffer of normalized_accumulate_uz (spilled window borders and
    the partial states of tile-edge pixels); (None, 0) when the shape needs
    none."""
    n = int(_lib.nsh_normalized_workspace_bytes(S, B, C, H, W, code, int(backward)))
    if n <= 0:
        return None, 0
    return torch.empty(n, dtype=torch.uint8, device=device), n


def normalized_accumulate_uz_backward(x: torch.Tensor, weights: torch.Tensor, D: torch.Tensor,
                                      log_C: torch.Tensor, grad_D: torch.Tensor,
                                      grad_log_C: torch.Tensor, shifts: torch.Tensor,
                                      log_weights: bool, *, row_codes: bool = False,
                                      shared_weights: bool = False) -> List[torch.Tensor]:
    """[grad_x, grad_w] (shift_ops.cpp:254-280); grad_w is per channel,
    (S*B, C, H, W), also for shared weights."""
    sh, B, C, H, W, S = _check_pair("normalized_accumulate_uz", x, weights, shifts,
                                    "normalized_accumulate_uz: weights must be (S*B, C, H, W)",
                                    shared_weights)
    acc = _acc_dtype(x.dtype)
    Dc = _grad_in(D, x, acc, "D")
    Lc = _grad_in(log_C, x, acc, "log_C")
    gD = _grad_in(grad_D, x, acc, "grad_D")
    gL = _grad_in(grad_log_C, x, acc, "grad_log_C")
    gx = torch.empty_like(x)
    gw = torch.empty((S * B, C, H, W), dtype=weights.dtype, device=weights.device)
    code = _code(x, "normalized_accumulate_uz_bwd") | _flags(row_codes, shared_weights)
    if x.dtype == torch.float64:
        code |= _narrow_halo_flag(sh)
    ws, nws = _norm_workspace(S, B, C, H, W, code, True, x.device)
    with torch.cuda.device(x.device):
        _call("nsh_normalized_accumulate_uz_backward", x.data_ptr(), weights.data_ptr(),
              Dc.data_ptr(), Lc.data_ptr(), gD.data_ptr(), gL.data_ptr(), sh.data_ptr(), S, B, C,
              H, W, code, int(bool(log_weights)), gx.data_ptr(), gw.data_ptr(), _ptr(ws), nws,
              _stream(x))
    return [gx, gw]


def _check_scalar(x: torch.Tensor, weights: torch.Tensor, shifts: torch.Tensor):
    _cuda(x, "x")
    _contig(x, "x")
    _nchw(x, "x")
    _cuda(weights, "weights")
    _contig(weights, "weights")
    _check(weights.dim() == 3, "accumulate_uz_scalar: weights must be (S, B, C)")
    sh = _prep_shifts(shifts, x.device)
    B, C, H, W = x.shape
    S = sh.size(0)
    _check(0 < S <= 1024, "accumulate_uz_scalar: tree reduction requires 1 <= S <= 1024")
    _check(weights.device == x.device,
           "accumulate_uz_scalar: x and weights must be on the same device")
    _check(weights.dtype == x.dtype,
           "accumulate_uz_scalar: x and weights must have the same dtype")
    _check(tuple(weights.shape) == (S, B, C), "weights shape must be (S, B, C)")
    return sh, B, C, H, W, S


def accumulate_uz_scalar_forward(x: torch.Tensor, weights: torch.Tensor,
                                 shifts: torch.Tensor) -> List[torch.Tensor]:
    """[U, Z] for (S, B, C) scalar weights (shift_ops.cpp:289-316)."""
    sh, B, C, H, W, S = _check_scalar(x, weights, shifts)
    acc = _acc_dtype(x.dtype)
    U = torch.empty(x.shape, dtype=acc, device=x.device)
    Z = torch.empty(x.shape, dtype=acc, device=x.device)
    with torch.cuda.device(x.device):
        _call("nsh_accumulate_uz_scalar_forward", x.data_ptr(), weights.data_ptr(),
              sh.data_ptr(), S, sh.size(1), B, C, H, W, _code(x, "accumulate_uz_scalar_fwd"),
              U.data_ptr(), Z.data_ptr(), _stream(x))
    return [U, Z]


def accumulate_uz_scalar_backward(x: torch.Tensor, weights: torch.Tensor, grad_U: torch.Tensor,
                                  grad_Z: torch.Tensor, shifts: torch.Tensor) -> List[torch.Tensor]:
    """[grad_x, grad_w] (shift_ops.cpp:318-337)."""
    sh, B, C, H, W, S = _check_scalar(x, weights, shifts)
    acc = _acc_dtype(x.dtype)
    gU = _grad_in(grad_U, x, acc, "grad_U")
    gZ = _grad_in(grad_Z, x, acc, "grad_Z")
    gx = torch.empty_like(x)
    gw = torch.empty_like(weights)
    nsplit = int(_lib.nsh_scalar_backward_splits(H, W))
    part = torch.empty(S * B * C * nsplit, dtype=acc, device=x.device)
    with torch.cuda.device(x.device):
        _call("nsh_accumulate_uz_scalar_backward", x.data_ptr(), weights.data_ptr(),
              gU.data_ptr(), gZ.data_ptr(), sh.data_ptr(), S, sh.size(1), B, C, H, W,
              _code(x, "accumulate_uz_scalar_bwd"), gx.data_ptr(), gw.data_ptr(),
              part.data_ptr(), _stream(x))
    return [gx, gw]




def metropolis_aggregate(w_half: torch.Tensor, img: torch.Tensor, shifts: torch.Tensor,
                         use_box: int, eps: float = 1e-6) -> List[torch.Tensor]:
    """[Wx, d_hat] in the input dtype (metropolis_cuda.cu:195-240)."""
    return metropolis_aggregate_with_degree(w_half, img, shifts, use_box, eps)[:2]


def metropolis_backward_supported(w_half: torch.Tensor) -> bool:
    """Whether the fused backward serves this shape (else the caller keeps
    the differentiable edge path)."""
    B, S, C, H, W = w_half.shape
    code = _DTYPE_CODE.get(w_half.dtype)
    return code is not None and int(_lib.nsh_metropolis_backward_workspace_bytes(
        B, S, C, H, W, code)) > 0


def metropolis_aggregate_backward(w_half: torch.Tensor, img: torch.Tensor, shifts: torch.Tensor,
                                  use_box: int, eps: float, degree: torch.Tensor,
                                  d_hat: torch.Tensor, grad_Wx: torch.Tensor,
                                  grad_d_hat: torch.Tensor) -> List[torch.Tensor]:
    """[grad_w_half, grad_img] of (Wx, d_hat) = metropolis_aggregate(...),
    from the forward's degree and d_hat (no counterpart in the reference's
    native module; the reference differentiates metropolis.py:117-192)."""
    w_half = w_half.contiguous()
    img = img.contiguous()
    sh = shifts.contiguous()
    B, S, C, H, W = w_half.shape
    code = _code(img, "metropolis_aggregate_backward")
    gWx = grad_Wx.to(img.dtype).contiguous()
    gdh = grad_d_hat.to(img.dtype).contiguous()
    n = int(_lib.nsh_metropolis_backward_workspace_bytes(B, S, C, H, W, code))
    _check(n > 0, "metropolis_aggregate_backward: shape not supported by the fused backward")
    flag = _narrow_halo_flag(sh)
    ws = torch.empty(n, dtype=torch.uint8, device=img.device)
    gw = torch.empty_like(w_half)
    gx = torch.empty_like(img)
    with torch.cuda.device(img.device):
        _call("nsh_metropolis_aggregate_backward", w_half.data_ptr(), img.data_ptr(),
              sh.data_ptr(), B, S, C, H, W, code | flag, int(bool(use_box)), float(eps),
              degree.data_ptr(), d_hat.contiguous().data_ptr(), gWx.data_ptr(), gdh.data_ptr(),
              gw.data_ptr(), gx.data_ptr(), ws.data_ptr(), n, _stream(img))
    return [gw, gx]


def metropolis_aggregate_with_degree(w_half: torch.Tensor, img: torch.Tensor,
                                     shifts: torch.Tensor, use_box: int,
                                     eps: float = 1e-6) -> List[torch.Tensor]:
    """[Wx, d_hat, degree]: the forward plus the raw degree d = K e that the
    fused backward needs (accumulator dtype)."""
    _check(w_half.is_cuda, "w_half must be CUDA")
    _check(img.is_cuda, "img must be CUDA")
    _check(shifts.is_cuda and shifts.dtype == torch.int64, "shifts must be int64 CUDA (S,3)")
    _check(w_half.dim() == 5, "w_half must be (B, S, C, H, W)")
    _check(img.dim() == 4, "img must be (B, C, H, W)")
    _check(shifts.dim() == 2 and shifts.size(1) == 3, "shifts must be int64 CUDA (S,3)")
    w_half = w_half.contiguous()
    img = img.contiguous()
    sh = shifts.contiguous()
    B, S, C, H, W = w_half.shape
    _check(tuple(img.shape) == (B, C, H, W), "img must be (B, C, H, W) matching w_half")
    _check(sh.size(0) == S, "shifts must have one row per w_half shift plane")
    _check(img.dtype == w_half.dtype, "w_half and img must have the same dtype")
    Wx = torch.empty_like(img)
    d_hat = torch.empty_like(img)
    degree = torch.empty(img.shape, dtype=_acc_dtype(img.dtype), device=img.device)
    code = _code(img, "metropolis_aggregate_cuda")
    n = int(_lib.nsh_metropolis_workspace_bytes(B, S, C, H, W, code))
    ws = torch.empty(n, dtype=torch.uint8, device=img.device) if n > 0 else None
    with torch.cuda.device(img.device):
        _call("nsh_metropolis_aggregate", w_half.data_ptr(), img.data_ptr(), sh.data_ptr(), B, S,
              C, H, W, code, int(bool(use_box)), float(eps), Wx.data_ptr(), d_hat.data_ptr(),
              degree.data_ptr(), _ptr(ws), max(n, 0), _stream(img))
    return [Wx, d_hat, degree]


__all__ = [
    "index_width_bits",
    "shift_gather_forward",
    "shift_gather_backward",
    "pair_gather_forward",
    "pair_gather_backward",
    "accumulate_uz_forward",
    "accumulate_uz_backward",
    "normalized_accumulate_uz_forward",
    "normalized_accumulate_uz_backward",
    "accumulate_uz_scalar_forward",
    "accumulate_uz_scalar_backward",
    "metropolis_aggregate",
]


# ---------------------------------------------------------------------------
# Measurement: streaming bandwidth probe (no counterpart in the reference)
# ---------------------------------------------------------------------------

PROBE_KINDS = {"read": 0, "read_nt": 1, "copy": 2, "fill": 3}
PROBE_UNROLL = {4: 2 << 8, 8: 3 << 8, 16: 4 << 8}
PROBE_PLAIN_LOADS, PROBE_PLAIN_STORES, PROBE_1024_LANES = 0x1000, 0x2000, 0x4000
PROBE_RING = 0x8000


def stream_probe(kind: str, src, dst: torch.Tensor, workgroups: int = 0, *, unroll: int = 8,
                 plain_loads: bool = False, plain_stores: bool = False,
                 lanes: int = 256, ring: bool = False) -> None:
    """One launch of the streaming probe over `dst` (fill) or `src` (read,
    read_nt, copy; `dst` a sink of >= 4 KiB for the reads).  workgroups
    defaults to 16 per CU.  Variants: `unroll` loads in flight per lane (4,
    8, 16), temporal instead of streaming loads (copy) or stores (copy,
    fill), `lanes` per workgroup (256, 1024), `ring` (copy: a per-lane
    prefetch ring instead of bursts)."""
    _check(unroll in PROBE_UNROLL, f"stream_probe: unroll must be 4, 8 or 16, not {unroll}")
    _check(lanes in (256, 1024), f"stream_probe: lanes must be 256 or 1024, not {lanes}")
    _check(kind in PROBE_KINDS, f"stream_probe: unknown kind {kind!r}")
    _cuda(dst, "dst")
    _contig(dst, "dst")
    dst_bytes = dst.numel() * dst.element_size()
    if kind in ("read", "read_nt", "copy"):
        _check(isinstance(src, torch.Tensor), "stream_probe: src must be a tensor")
        _cuda(src, "src")
        _contig(src, "src")
        _check(src.device == dst.device, "stream_probe: src and dst must be on the same device")
        nbytes = src.numel() * src.element_size()
        if kind == "copy":
            _check(dst_bytes >= nbytes, f"stream_probe: dst holds {dst_bytes} bytes, copy "
                                        f"needs {nbytes}")
        else:
            # the read kernels' sink: one 16-byte vector per lane of a workgroup
            _check(dst_bytes >= 4096, "stream_probe: the read sink needs at least 4096 bytes")
    else:
        nbytes = dst_bytes
    if workgroups <= 0:
        workgroups = 16 * torch.cuda.get_device_properties(dst.device).multi_processor_count
    with torch.cuda.device(dst.device):
        code = (PROBE_KINDS[kind] | PROBE_UNROLL[unroll]
                | (PROBE_PLAIN_LOADS if plain_loads else 0)
                | (PROBE_PLAIN_STORES if plain_stores else 0)
                | (PROBE_1024_LANES if lanes == 1024 else 0)
                | (PROBE_RING if ring else 0))
        _call("nsh_stream_probe", code, _ptr(src), dst.data_ptr(), nbytes, int(workgroups),
              _stream(dst))
