"""Write the golden input/output vectors in ``tests/golden/`` from the
reference's own CPU fallbacks (trishitmg/neural_shift_cuda,
neural_shift_cuda/ops.py and neural_shift_cuda/metropolis.py).

Run in the build container only, where the reference checkout is mounted::

    python tests/golden/make_golden.py [/root/reference]

The reference code never leaves this script: only the seeded inputs and the
outputs it computes are written (``golden.npz`` + ``golden.json``).  The
script imports the reference for exactly the behaviour that no closed form,
known-answer test or invariant pins:

* the fp32/fp64 bit patterns of the fallbacks' term order and pairwise tree
  (``accumulate_uz_reference``, ``normalized_accumulate_uz_reference``,
  ``accumulate_uz_scalar_reference``, ops.py:77-92, 157-390);
* the fallbacks' edge semantics: NaN weight gradients at zero positive
  weights (ops.py:227-231), empty rows (D = 0, log_C = -inf, ops.py:309-318),
  out-of-contract weights with ``validate=False``, the R = 0 gather branch and
  its mask dtype (ops.py:112-116), bf16 gathers;
* autograd through the reference graphs, including the checkpointed
  Metropolis training path (metropolis.py:117-238), at shapes small enough
  for the explicit-edge path and large enough for the fused backward;
* BASELINE configuration c0 at full size (outputs only; the inputs are
  regenerated from seeds and tied to the outputs by a digest);
* the NECTR installer (integration/nectr_patch.py) on the vendored official
  model (models/NECTR_models1.py): the models' parameters, the unpatched
  forward and the reference installer's patched forward;
* the NeKDe, GASD and Metropolis installers (integration/
  nekde_drunet_attn_patch.py, gasd_drunet_attn_patch.py,
  nkd_metropolis_attn_patch.py) on the stand-in model classes of
  tests/installer_models.py: forward, transpose and cached forms and the
  parameter gradients of the reference installers' patched paths.

Storage: ``golden.npz`` (no pickles) holds one array per
``<case>/<role>/<name>``; bf16 tensors are stored as their int16 bit
patterns.  ``golden.json`` lists every case with its op, parameters and the
torch dtype of each array.
"""
from __future__ import annotations

import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))


def _import_reference(path: str):
    # The repository ships its own package named ``neural_shift_cuda``; make
    # sure the reference checkout is the one that imports.
    sys.path[:] = [p for p in sys.path
                   if os.path.abspath(p or os.getcwd()) not in (REPO, HERE)]
    sys.path.insert(0, path)
    import neural_shift_cuda as ref  # noqa: E402
    from neural_shift_cuda import metropolis as ref_metro  # noqa: E402
    from neural_shift_cuda import ops as ref_ops  # noqa: E402
    if not os.path.abspath(ref.__file__).startswith(os.path.abspath(path)):
        raise RuntimeError(f"imported the wrong neural_shift_cuda: {ref.__file__}")
    if ref_ops._HAS_CUDA_EXT:
        raise RuntimeError("reference CUDA extension unexpectedly importable")
    return ref, ref_ops, ref_metro


def halfplane(R):
    rows = [(dx, dy, 1) for dx in range(-R, R + 1) for dy in range(1, R + 1)]
    rows += [(dx, 0, 0 if dx == 0 else 1) for dx in range(0, R + 1)]
    return rows


def window(R, flag=True):
    return [((dx, dy, 0) if flag else (dx, dy))
            for dx in range(-R, R + 1) for dy in range(-R, R + 1)]


def main() -> int:
    ref_path = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    if not os.path.isdir(os.path.join(ref_path, "neural_shift_cuda")):
        print(f"make_golden: no reference checkout at {ref_path}", file=sys.stderr)
        return 2
    import numpy as np
    import torch
    import torch.nn.functional as F

    ref, ref_ops, ref_metro = _import_reference(ref_path)
    torch.set_num_threads(1)

    arrays = {}
    manifest = {"source": "trishitmg/neural_shift_cuda CPU fallbacks (ops.py, metropolis.py)",
                "torch": torch.__version__, "cases": []}

    def put(case, role, name, t):
        t = t.detach().contiguous().cpu()
        key = f"{case['name']}/{role}/{name}"
        if t.dtype == torch.bfloat16:
            arrays[key] = t.view(torch.int16).numpy()
        elif t.dtype == torch.bool:
            arrays[key] = t.numpy()
        else:
            arrays[key] = t.numpy()
        case.setdefault(role, {})[name] = str(t.dtype).replace("torch.", "")

    def gen(seed):
        return torch.Generator().manual_seed(seed)

    def box_weights(sh, B, C, H, W, g, dtype, positive=True):
        S = len(sh)
        w = torch.randn(S * B, C, H, W, generator=g, dtype=torch.float64)
        if positive:
            w = F.softplus(w)
        R = max(max(abs(a), abs(b)) for a, b, *_ in sh)
        box = F.pad(torch.ones(1, 1, H, W, dtype=torch.float64), (R, R, R, R), value=0.0)
        m = torch.cat([box[:, :, R + dx:R + dx + H, R + dy:R + dy + W]
                       for dx, dy, *_ in sh], 0)
        m = m.unsqueeze(1).expand(S, B, 1, H, W).reshape(S * B, 1, H, W)
        return (w * m).to(dtype)

    # ------------------------------------------------------------------
    # accumulate_uz_reference: forward + autograd backward
    # ------------------------------------------------------------------
    acc_cases = [
        ("acc_f32_half_r2", torch.float32, (2, 2, 9, 11), halfplane(2), True),
        ("acc_f64_half_r3", torch.float64, (1, 3, 8, 10), halfplane(3), True),
        ("acc_f32_window_r1", torch.float32, (2, 1, 6, 7), window(1), False),
        ("acc_f16_half_r1", torch.float16, (1, 2, 8, 8), halfplane(1), True),
        ("acc_f32_half_r4_big", torch.float32, (1, 1, 16, 13), halfplane(4), True),
    ]
    for i, (name, dt, (B, C, H, W), sh, comp_box) in enumerate(acc_cases):
        g = gen(100 + i)
        x = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(dt)
        w = box_weights(sh, B, C, H, W, g, dt) if comp_box else \
            F.softplus(torch.randn(len(sh) * B, C, H, W, generator=g,
                                   dtype=torch.float64)).to(dt)
        acc = torch.float64 if dt == torch.float64 else torch.float32
        gU = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(acc)
        gZ = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(acc)
        shifts = torch.tensor(sh, dtype=torch.int32)
        xr = x.clone().requires_grad_(True)
        wr = w.clone().requires_grad_(True)
        U, Z = ref.accumulate_uz_reference(xr, wr, shifts)
        torch.autograd.backward([U, Z], [gU, gZ])
        case = {"name": name, "op": "accumulate_uz", "comp_box": comp_box}
        for n, t in (("x", x), ("w", w), ("shifts", shifts), ("gU", gU), ("gZ", gZ)):
            put(case, "inputs", n, t)
        for n, t in (("U", U), ("Z", Z), ("gx", xr.grad), ("gw", wr.grad)):
            put(case, "outputs", n, t)
        manifest["cases"].append(case)

    # ------------------------------------------------------------------
    # normalized_accumulate_uz_reference
    # ------------------------------------------------------------------
    def normalized_case(name, dt, shape, sh, *, log_weights, weights, validate=True,
                        grads=True, return_log_degree=True, seed=0):
        B, C, H, W = shape
        g = gen(seed)
        x = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(dt)
        acc = torch.float64 if dt == torch.float64 else torch.float32
        gD = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(acc)
        gL = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(acc)
        shifts = torch.tensor(sh, dtype=torch.int64)
        xr = x.clone().requires_grad_(grads)
        wr = weights.clone().requires_grad_(grads)
        out = ref.normalized_accumulate_uz_reference(
            xr, wr, shifts, log_weights=log_weights, return_log_degree=return_log_degree,
            validate=validate)
        case = {"name": name, "op": "normalized_accumulate_uz", "log_weights": log_weights,
                "validate": validate, "return_log_degree": return_log_degree}
        for n, t in (("x", x), ("w", weights), ("shifts", shifts)):
            put(case, "inputs", n, t)
        if return_log_degree:
            D, L = out
            put(case, "outputs", "D", D)
            put(case, "outputs", "log_C", L)
        else:
            D, L = out, None
            put(case, "outputs", "D", D)
        if grads:
            if L is not None:
                torch.autograd.backward([D, L], [gD, gL])
                put(case, "inputs", "gL", gL)
            else:
                torch.autograd.backward([D], [gD])
            put(case, "inputs", "gD", gD)
            put(case, "outputs", "gx", xr.grad)
            put(case, "outputs", "gw", wr.grad)
        manifest["cases"].append(case)

    # positive mode, fp64, comp_box weights (exact zeros: NaN gradient quirk)
    sh = halfplane(2)
    g = gen(200)
    normalized_case("nrm_pos_f64_half_r2", torch.float64, (2, 2, 7, 6), sh,
                    log_weights=False, weights=box_weights(sh, 2, 2, 7, 6, g, torch.float64),
                    seed=201)
    # positive mode, fp32, D only
    g = gen(210)
    normalized_case("nrm_pos_f32_window_r1_donly", torch.float32, (1, 3, 6, 8), window(1),
                    log_weights=False,
                    weights=F.softplus(torch.randn(9, 3, 6, 8, generator=g)),
                    return_log_degree=False, seed=211)
    # log mode, fp32, N(0, var 4) logits with 1% at +-80 and some -inf masks
    sh = halfplane(2)
    g = gen(220)
    B, C, H, W = 2, 1, 9, 8
    lw = 2.0 * torch.randn(len(sh) * B, C, H, W, generator=g)
    sel = torch.rand(lw.shape, generator=g) < 0.04
    sgn = torch.where(torch.rand(lw.shape, generator=g) < 0.5, -80.0, 80.0)
    lw = torch.where(sel, sgn, lw)
    lw = torch.where(torch.rand(lw.shape, generator=g) < 0.05, float("-inf"), lw)
    normalized_case("nrm_log_f32_half_r2_pm80", torch.float32, (B, C, H, W), sh,
                    log_weights=True, weights=lw, seed=221)
    # log mode, fp64, empty rows: every weight of batch 1 masked, and a few
    # fully masked pixels in batch 0
    sh = halfplane(1)
    g = gen(230)
    B, C, H, W = 2, 2, 5, 6
    S = len(sh)
    lw = torch.randn(S * B, C, H, W, generator=g, dtype=torch.float64)
    lw5 = lw.view(S, B, C, H, W)
    lw5[:, 1] = float("-inf")
    normalized_case("nrm_log_f64_empty_rows", torch.float64, (B, C, H, W), sh,
                    log_weights=True, weights=lw, seed=231)
    # positive mode, window table (no mirror), uniform huge weights: exact mean
    g = gen(240)
    normalized_case("nrm_pos_f64_window_huge", torch.float64, (1, 1, 5, 5), window(1),
                    log_weights=False, weights=torch.full((9, 1, 5, 5), 1e300,
                                                          dtype=torch.float64),
                    seed=241)
    # validate=False with out-of-contract positive weights (negative, +inf, NaN)
    g = gen(250)
    wbad = F.softplus(torch.randn(9, 1, 4, 5, generator=g))
    wbad[0, 0, 0, 0] = -1.0
    wbad[1, 0, 1, 1] = float("inf")
    wbad[2, 0, 2, 2] = float("nan")
    normalized_case("nrm_pos_f32_invalid_novalidate", torch.float32, (1, 1, 4, 5), window(1),
                    log_weights=False, weights=wbad, validate=False, grads=False, seed=251)

    # ------------------------------------------------------------------
    # gathers
    # ------------------------------------------------------------------
    def gather_case(name, fn, dt, shape, sh, seed):
        B, C, H, W = shape
        g = gen(seed)
        guide = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(dt)
        shifts = torch.tensor(sh, dtype=torch.int64)
        gr = guide.clone().requires_grad_(True)
        out, mask = fn(gr, shifts)
        gout = torch.randn(out.shape, generator=g, dtype=torch.float64).to(dt)
        out.backward(gout)
        case = {"name": name, "op": fn.__name__.replace("_reference", "")}
        for n, t in (("guide", guide), ("shifts", shifts), ("gout", gout)):
            put(case, "inputs", n, t)
        for n, t in (("out", out), ("mask", mask), ("gguide", gr.grad)):
            put(case, "outputs", n, t)
        manifest["cases"].append(case)

    gather_case("sg_f32_half_r2", ref.shift_gather_reference, torch.float32, (2, 3, 7, 9),
                halfplane(2), 300)
    gather_case("sg_bf16_window_r2_xy", ref.shift_gather_reference, torch.bfloat16,
                (2, 2, 6, 5), window(2, flag=False), 301)
    gather_case("sg_f64_r0", ref.shift_gather_reference, torch.float64, (2, 1, 4, 3),
                [(0, 0), (0, 0)], 302)
    gather_case("pg_f32_half_r1", ref.pair_gather_reference, torch.float32, (2, 2, 5, 6),
                halfplane(1), 303)
    gather_case("pg_bf16_window_r1", ref.pair_gather_reference, torch.bfloat16, (1, 3, 4, 4),
                window(1), 304)
    gather_case("pg_f16_r0", ref.pair_gather_reference, torch.float16, (1, 2, 3, 3),
                [(0, 0, 0)], 305)

    # ------------------------------------------------------------------
    # accumulate_uz_scalar_reference
    # ------------------------------------------------------------------
    for i, (name, dt, (B, C, H, W), sh, per_channel) in enumerate([
            ("sc_f32_sbc_r1", torch.float32, (2, 3, 6, 7), window(1, flag=False), True),
            ("sc_f64_sb_r2", torch.float64, (2, 2, 5, 5), window(2, flag=False), False),
    ]):
        g = gen(400 + i)
        S = len(sh)
        x = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(dt)
        w = torch.randn(*((S, B, C) if per_channel else (S, B)), generator=g,
                        dtype=torch.float64).to(dt)
        acc = torch.float64 if dt == torch.float64 else torch.float32
        gU = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(acc)
        gZ = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(acc)
        shifts = torch.tensor(sh, dtype=torch.int64)
        xr = x.clone().requires_grad_(True)
        wr = w.clone().requires_grad_(True)
        U, Z = ref.accumulate_uz_scalar_reference(xr, wr, shifts)
        torch.autograd.backward([U, Z], [gU, gZ])
        case = {"name": name, "op": "accumulate_uz_scalar"}
        for n, t in (("x", x), ("w", w), ("shifts", shifts), ("gU", gU), ("gZ", gZ)):
            put(case, "inputs", n, t)
        for n, t in (("U", U), ("Z", Z), ("gx", xr.grad), ("gw", wr.grad)):
            put(case, "outputs", n, t)
        manifest["cases"].append(case)

    # ------------------------------------------------------------------
    # Metropolis: dispatcher without grad (fused path on CPU), the torch
    # reference, and the checkpointed training path's gradients.  The
    # "_fused" cases are large enough (>= 3 backward tiles per direction:
    # 16 x 64 pixels for fp32, 32 x 32 for fp64) that a GPU run of the same
    # inputs differentiates through the fused two-pass HIP backward.
    # ------------------------------------------------------------------
    for i, (name, dt, (B, C, H, W), R, use_box) in enumerate([
            ("metro_f64_box_r2", torch.float64, (1, 2, 8, 9), 2, True),
            ("metro_f32_circ_r1", torch.float32, (2, 1, 6, 7), 1, False),
            ("metro_f64_circ_r2", torch.float64, (1, 1, 7, 7), 2, False),
            ("metro_f64_box_r2_fused", torch.float64, (1, 1, 72, 80), 2, True),
            ("metro_f32_circ_r2_fused", torch.float32, (1, 1, 40, 136), 2, False),
    ]):
        g = gen(500 + i)
        rows = [(dx, dy, bool(inv)) for dx, dy, inv in halfplane(R)]
        S = len(rows)
        w_half = F.softplus(torch.randn(B, S, C, H, W, generator=g,
                                        dtype=torch.float64)).to(dt)
        img = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(dt)
        gWx = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(dt)
        gDh = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(dt)
        with torch.no_grad():
            Wx, d_hat = ref_metro.metropolis_aggregate(w_half, img, rows, use_box)
            Wx_t, d_hat_t = ref_metro.metropolis_aggregate_torch(w_half, img, rows, use_box)
        wr = w_half.clone().requires_grad_(True)
        ir = img.clone().requires_grad_(True)
        Wx_g, d_hat_g = ref_metro.metropolis_aggregate(wr, ir, rows, use_box,
                                                       checkpoint_train=True)
        torch.autograd.backward([Wx_g, d_hat_g], [gWx, gDh])
        case = {"name": name, "op": "metropolis_aggregate", "use_box": use_box,
                "eps": 1e-6}
        for n, t in (("w_half", w_half), ("img", img),
                     ("shifts", torch.tensor(halfplane(R), dtype=torch.int64)),
                     ("gWx", gWx), ("gDh", gDh)):
            put(case, "inputs", n, t)
        for n, t in (("Wx", Wx), ("d_hat", d_hat), ("Wx_torch", Wx_t),
                     ("d_hat_torch", d_hat_t), ("Wx_train", Wx_g), ("d_hat_train", d_hat_g),
                     ("g_w_half", wr.grad), ("g_img", ir.grad)):
            put(case, "outputs", n, t)
        manifest["cases"].append(case)

    # ------------------------------------------------------------------
    # BASELINE configs[0] at full size: the reference dispatcher's CPU
    # forward (accumulate_uz -> accumulate_uz_reference, ops.py:612-631).
    # Only the outputs are stored: the inputs are regenerated by
    # neural_shift_cuda_amd/workloads.py:config0_inputs, and their sha256
    # digest ties the outputs to them.
    # ------------------------------------------------------------------
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "_nsh_workloads", os.path.join(REPO, "neural_shift_cuda_amd", "workloads.py"))
    workloads = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(workloads)
    x0, w0, sh0 = workloads.config0_inputs()
    with torch.no_grad():
        U0, Z0 = ref.accumulate_uz(x0, w0, sh0)
    case = {"name": "c0_full", "op": "accumulate_uz_config", "config": "c0",
            "inputs_sha256": workloads.tensor_digest(x0, w0, sh0)}
    put(case, "inputs", "shifts", sh0)
    for n, t in (("U", U0), ("Z", Z0)):
        put(case, "outputs", n, t)
    manifest["cases"].append(case)

    # ------------------------------------------------------------------
    # The NECTR installer on the vendored official model
    # (models/NECTR_models1.py:12-244): tiny seeded fp64 models, their
    # parameters, the unpatched forward, and the reference installer's
    # patched forward (integration/nectr_patch.py:248-299) from the
    # guide and from the unpatched forward's cache, all on the CPU paths.
    # ------------------------------------------------------------------
    import contextlib
    import io
    import types
    from neural_shift_cuda.integration import nectr_patch as ref_nectr
    spec = importlib.util.spec_from_file_location(
        "_ref_nectr_models1", os.path.join(ref_path, "models", "NECTR_models1.py"))
    models1 = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(models1)
    nectr_cases = [
        ("nectr_exp_blind", "exp", True, 1, 2, (2, 1, 12, 12)),
        ("nectr_csig_sigma", "control_sigmoid", False, 2, 2, (1, 2, 10, 14)),
    ]
    built = []
    for i, (name, act, blind, cin, R, shape) in enumerate(nectr_cases):
        args = types.SimpleNamespace(model_type="concat", residual_depth=2, proj_depth=1,
                                     latent_dim=4, blind=blind, patch_rad=1,
                                     output_activation=act, window_rad=R, in_channel=cin)
        torch.manual_seed(700 + i)
        with contextlib.redirect_stdout(io.StringIO()):
            model = models1.NECTR_denoiser(args, "cpu").double()
        g = gen(710 + i)
        x = torch.rand(*shape, generator=g, dtype=torch.float64)
        sig = None if blind else torch.full((shape[0],), 0.1, dtype=torch.float64)
        with torch.no_grad():
            D0, Z0, cache0 = model(x, sig=sig, store_cache=True)
        built.append((name, act, blind, cin, R, model, x, sig, D0, Z0, cache0))
    ref_nectr.install_cuda_shift(models1.NECTR_denoiser)
    for name, act, blind, cin, R, model, x, sig, D0, Z0, cache0 in built:
        with torch.no_grad():
            D1, Z1, cache1 = model(x, sig=sig, store_cache=True)
            D2, Z2 = model(x, sig=sig, cache=cache0)
        case = {"name": name, "op": "nectr_installer", "output_activation": act,
                "blind": blind, "in_channel": cin, "window_rad": R, "latent_dim": 4,
                "residual_depth": 2, "proj_depth": 1, "patch_rad": 1,
                "cache_weight_kind": cache1.weight_kind,
                "params": sorted(model.state_dict().keys())}
        put(case, "inputs", "x", x)
        if sig is not None:
            put(case, "inputs", "sig", sig)
        for pname, t in model.state_dict().items():
            put(case, "inputs", "param." + pname, t)
        for n, t in (("D_model", D0), ("Z_model", Z0), ("D_patched", D1), ("Z_patched", Z1),
                     ("D_plain_cache", D2), ("Z_plain_cache", Z2)):
            put(case, "outputs", n, t)
        manifest["cases"].append(case)

    # ------------------------------------------------------------------
    # The NeKDe, GASD and Metropolis installers on the stand-in model
    # classes of tests/installer_models.py: the reference installers' own
    # patched paths (nekde_drunet_attn_patch.py:245-560,
    # gasd_drunet_attn_patch.py:156-620, nkd_metropolis_attn_patch.py:52-190)
    # called on CPU fp64 tensors (the reference ops then run their CPU
    # fallbacks; the installed methods route CPU inputs to the class's own
    # method, so the paths are called directly).  Stored: the parameters,
    # the inputs, the forward (train and eval), K^T / NLM_transpose /
    # laplacian_grw, the cached forms on the stand-in's own weights, and
    # the gradients of a fixed loss with respect to the input and every
    # parameter.
    # ------------------------------------------------------------------
    from neural_shift_cuda.integration import gasd_drunet_attn_patch as ref_gasd
    from neural_shift_cuda.integration import nekde_drunet_attn_patch as ref_nekde
    from neural_shift_cuda.integration import nkd_metropolis_attn_patch as ref_mp
    spec = importlib.util.spec_from_file_location(
        "_nsh_installer_models", os.path.join(os.path.dirname(HERE), "installer_models.py"))
    im = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(im)
    shape = dict(B=2, C=3, H=12, W=14)

    def store_model(case, m):
        for pname, t in m.state_dict().items():
            put(case, "inputs", "param." + pname, t)
        case["params"] = sorted(m.state_dict().keys())

    def param_grads(case, m, x, loss_of):
        """Gradients of the loss; not stored where the reference CPU
        fallback's zero-positive-weight quirk (ops.py:227-231: log(0) in the
        graph) makes them NaN -- the box-masked weights of comp_box=True."""
        m.zero_grad()
        xg = x.clone().requires_grad_(True)
        loss_of(xg).backward()
        grads = [("grad.x", xg.grad)] + [("grad.param." + n, p.grad)
                                         for n, p in m.named_parameters() if p.grad is not None]
        if any(bool(torch.isnan(t).any()) for _, t in grads):
            case["grads"] = "nan: zero positive weights in the reference CPU fallback"
        else:
            for n, t in grads:
                put(case, "outputs", n, t)
        m.zero_grad()

    def loss_weights(seed, n):
        g = gen(seed)
        return [torch.randn(shape["B"], shape["C"], shape["H"], shape["W"], generator=g,
                            dtype=torch.float64) for _ in range(n)]

    # comp_box=True cases pin values only (their reference CPU gradients are
    # NaN, see param_grads); the comp_box=False twins pin the gradients too
    nekde_kws = [dict(comp_box=True), dict(comp_box=False), dict(activation="control_sigmoid"),
                 dict(legacy=True), dict(legacy=True, comp_box=False, activation="control_sigmoid"),
                 dict(heads=1, pos_act="none"), dict(heads=1, pos_act="none", comp_box=False),
                 dict(heads=3, pos_act="none"), dict(pos_act="softplus"),
                 dict(activation="control_sigmoid", comp_box=False),
                 dict(legacy=True, comp_box=False), dict(heads=3, pos_act="none", comp_box=False),
                 dict(pos_act="softplus", comp_box=False)]
    for i, kw in enumerate(nekde_kws):
        sub, m = im._fresh(im.FakeNeKDe, seed=800 + i, **kw)
        ref_nekde.install_cuda_shift(sub)  # attaches the shift-table helper
        x, guide = im._inputs(seed=810 + i, **shape)
        case = {"name": f"nekde_installer_{i}", "op": "nekde_installer", "kwargs": kw,
                "seed": 800 + i}
        store_model(case, m)
        put(case, "inputs", "x", x)
        put(case, "inputs", "guide", guide)
        m.train()
        with torch.no_grad():
            D, Z = ref_nekde._forward_cuda(m, x, guide=guide, sig=0.1)
            put(case, "outputs", "D_train", D)
            put(case, "outputs", "Z_train", Z)
            m.eval()
            D2, _ = ref_nekde._forward_cuda(m, x, return_D=False)
            put(case, "outputs", "D_eval", D2)
            for apply in (False, True):
                U, Zk = ref_nekde._kt_action_cuda(m, x, guide=guide, return_D=True,
                                                  apply_Dinv=apply)
                put(case, "outputs", f"KT_U_{int(apply)}", U)
                put(case, "outputs", f"KT_Z_{int(apply)}", Zk)
            ws, shifts = m._weights(x, guide, torch.tensor(0.1, dtype=torch.float64))
            cache = types.SimpleNamespace(C=shape["C"], shifts=shifts, w_fwd_list=ws,
                                          comp_box=m.comp_box, D=None)
            Dc, degc = ref_nekde._forward_cached_cuda(types.SimpleNamespace(), x, cache, True)
            put(case, "outputs", "cached_D", Dc)
            put(case, "outputs", "cached_degree", degc)
        m.train()
        gD, gZ = loss_weights(820 + i, 2)
        param_grads(case, m, x, lambda xg: sum(
            (t * gt).sum() for t, gt in zip(ref_nekde._forward_cuda(m, xg, sig=0.1), (gD, gZ))))
        manifest["cases"].append(case)

    gasd_kws = [dict(comp_box=True), dict(comp_box=False), dict(legacy=True),
                dict(activation="control_sigmoid", heads=1, pos_act="none"),
                dict(legacy=True, comp_box=False),
                dict(activation="control_sigmoid", heads=1, pos_act="none", comp_box=False)]
    for i, kw in enumerate(gasd_kws):
        sub, m = im._fresh(im.FakeGASD, seed=840 + i, **kw)
        ref_gasd.install_cuda_shift(sub)
        x, guide = im._inputs(seed=850 + i, **shape)
        case = {"name": f"gasd_installer_{i}", "op": "gasd_installer", "kwargs": kw,
                "seed": 840 + i}
        store_model(case, m)
        put(case, "inputs", "x", x)
        put(case, "inputs", "guide", guide)
        m.train()
        with torch.no_grad():
            D, Z = ref_gasd._forward_cuda(m, x, guide=guide)
            put(case, "outputs", "D_train", D)
            put(case, "outputs", "Z_train", Z)
            m.eval()
            put(case, "outputs", "D_eval", ref_gasd._forward_cuda(m, x, return_D=False)[0])
            put(case, "outputs", "KT", ref_gasd._kt_action_cuda(m, x, guide=guide))
            WT, Dt = ref_gasd._nlm_transpose_cuda(m, x, guide=guide, return_D=True)
            put(case, "outputs", "NLM_T", WT)
            put(case, "outputs", "NLM_T_D", Dt)
            put(case, "outputs", "laplacian_grw", ref_gasd._laplacian_grw_cuda(m, x, guide))
            ws, shifts = m._weights(x, guide, None)
            cache = types.SimpleNamespace(C=shape["C"], shifts=shifts, w_list=ws, Z=None)
            mc = types.SimpleNamespace()
            Dc, degc = ref_gasd._forward_cached_cuda(mc, x, cache, True)
            put(case, "outputs", "cached_D", Dc)
            put(case, "outputs", "cached_degree", degc)
            put(case, "outputs", "cached_KT", ref_gasd._kt_action_cached_cuda(mc, guide, cache))
            put(case, "outputs", "cached_laplacian_grw",
                ref_gasd._laplacian_grw_cached_cuda(mc, x, cache))
        m.train()
        gD, gZ = loss_weights(860 + i, 2)
        param_grads(case, m, x, lambda xg: sum(
            (t * gt).sum() for t, gt in zip(ref_gasd._forward_cuda(m, xg), (gD, gZ))))
        manifest["cases"].append(case)

    for i, comp_box in enumerate((True, False)):
        sub, m = im._fresh(im.FakeMetropolis, seed=880 + i, comp_box=comp_box)
        ref_mp.install_cuda_shift(sub)
        x, guide = im._inputs(seed=890 + i, **shape)
        case = {"name": f"metropolis_installer_{i}", "op": "metropolis_installer",
                "kwargs": {"comp_box": comp_box}, "seed": 880 + i}
        store_model(case, m)
        put(case, "inputs", "x", x)
        put(case, "inputs", "guide", guide)
        with torch.no_grad():
            Wx, dh = ref_mp._forward_cuda(m, x, guide=guide, return_D=True)
            put(case, "outputs", "Wx", Wx)
            put(case, "outputs", "d_hat", dh)
            shifts = m._collect_shifts()
            g = gen(895 + i)
            w_hat = [0.08 * (torch.rand(x.shape, generator=g, dtype=torch.float64) + 0.1)
                     for _ in shifts]
            for k, t in enumerate(w_hat):
                put(case, "inputs", f"w_hat.{k}", t)
            cache = types.SimpleNamespace(C=shape["C"], shifts=shifts, w_hat_fwd_list=w_hat,
                                          comp_box=comp_box, degree_hat=None)
            Wc, dc = ref_mp._forward_cached_cuda(types.SimpleNamespace(), x, cache, True)
            put(case, "outputs", "cached_Wx", Wc)
            put(case, "outputs", "cached_d_hat", dc)
        gW, gd = loss_weights(898 + i, 2)
        param_grads(case, m, x, lambda xg: sum(
            (t * gt).sum() for t, gt in zip(ref_mp._forward_cuda(m, xg, return_D=True),
                                           (gW, gd))))
        manifest["cases"].append(case)

    np.savez_compressed(os.path.join(HERE, "golden.npz"), **arrays)
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    size = os.path.getsize(os.path.join(HERE, "golden.npz"))
    print(f"make_golden: {len(manifest['cases'])} cases, {len(arrays)} arrays, "
          f"{size / 1024:.0f} KiB")
    return 0


if __name__ == "__main__":
    sys.exit(main())
