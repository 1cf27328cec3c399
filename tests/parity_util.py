"""Helpers shared by the GPU parity tests: seeded inputs and error statistics.

Pass bar, per tensor, against the unrounded fp64 oracle:
  * every element: |got - ref| <= max(MAX_ABS, ulp(ref)), where ulp is one unit
    in the last place of the output dtype at |ref| -- 2e-2 everywhere bf16 can
    represent it (|ref| < 4), one bf16 ulp above that (0.03125 on [4, 8));
  * allclose(atol=2e-2, rtol=5e-2) against the oracle rounded to the output
    dtype, the reference harness's own criterion
    (training/train/train_ssa_triton/check_ssa_triton_parity.py:124-149,206,
    219-237, tolerances :1060-1069);
  * dn / db: |got - ref| <= 2e-3 + 2e-2 |ref| (the reference's scalar bar).
fp32 tensors take the reference's fp32 bars instead: allclose(atol=5e-4,
rtol=1e-3) against the unrounded oracle for every element, and
|got - ref| <= 5e-5 + 1e-4 |ref| for dn / db (the same lines).
The reported "max_abs" is the plain maximum |got - ref|.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle import ssa_oracle as so

# max abs error <= 2e-2 in bf16 against the fp32/fp64 oracle.
MAX_ABS = 2e-2
# Reference harness allclose tolerances for bf16/fp16 tensors and scalars
# (check_ssa_triton_parity.py:1060-1069).
ATOL, RTOL = 2e-2, 5e-2
SCALAR_ATOL, SCALAR_RTOL = 2e-3, 2e-2
# fp32 operands (check_ssa_triton_parity.py:1064-1065, 1068-1069)
ATOL_F32, RTOL_F32 = 5e-4, 1e-3
SCALAR_ATOL_F32, SCALAR_RTOL_F32 = 5e-5, 1e-4


def make_inputs(B, Hq, Hkv, N, D, dtype, device, layout="contig", seed=1234, qkv_scale=1.0):
    """Seeded q, k, v, dout on `device` (drawn on the CPU so every device sees the same values)."""
    g = torch.Generator().manual_seed(seed)

    def draw(h, scale):
        if layout == "contig":
            x = torch.randn(B, h, N, D, generator=g) * scale
            return x.to(dtype).to(device)
        if layout == "strided":  # Megatron [S, B, H, D] viewed as [B, H, S, D]
            x = torch.randn(N, B, h, D, generator=g) * scale
            return x.to(dtype).to(device).permute(1, 2, 0, 3)
        raise ValueError(layout)

    q = draw(Hq, qkv_scale)
    k = draw(Hkv, qkv_scale)
    v = draw(Hkv, qkv_scale)
    do = draw(Hq, 1.0)
    return q, k, v, do


def _np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def oracle_fwd_bwd(q, k, v, do, scale, n, b, causal, out_for_delta=None):
    """fp64 oracle on the CPU copies of (already rounded) kernel inputs.

    ``out_for_delta``: the kernel's forward output, when the backward is to be
    checked as the kernel-level function of (q, k, v, out, dout, m).
    """
    ofd = None if out_for_delta is None else _np64(out_for_delta)
    return so.ssa_forward_backward(_np64(q), _np64(k), _np64(v), _np64(do), scale, n, b, causal, ofd)


def ulp(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """One unit in the last place of `dtype` at |x| (normal range)."""
    mant = {torch.bfloat16: 7, torch.float16: 10}.get(dtype, 23)
    e = torch.floor(torch.log2(x.abs().clamp_min(1e-30)))
    return torch.pow(2.0, e - mant)


def tensor_err(got: torch.Tensor, ref: np.ndarray) -> dict:
    g = got.detach().float().cpu()
    r = torch.from_numpy(np.ascontiguousarray(ref)).float()
    r_round = r.to(got.dtype).float() if got.dtype in (torch.bfloat16, torch.float16) else r
    d_raw = (g - r).abs()
    if got.dtype == torch.float32:
        bound = ATOL_F32 + RTOL_F32 * r.abs()
        atol, rtol = ATOL_F32, RTOL_F32
    else:
        bound = torch.maximum(torch.full_like(r, MAX_ABS), ulp(r, got.dtype))
        atol, rtol = ATOL, RTOL
    return {
        "max_abs": float(d_raw.max()) if d_raw.numel() else 0.0,
        "max_abs_vs_rounded": float((g - r_round).abs().max()) if d_raw.numel() else 0.0,
        "within_bound": bool((d_raw <= bound).all()),
        "rel_rmse": float(torch.sqrt(((g - r) ** 2).mean()) / (torch.sqrt((r ** 2).mean()) + 1e-12)),
        "allclose": bool(torch.allclose(g, r_round, atol=atol, rtol=rtol)),
        "finite": bool(torch.isfinite(g).all()),
    }


def scalar_err(got, ref: float, fp32: bool = False) -> dict:
    gv = float(got)
    diff = abs(gv - ref)
    atol, rtol = (SCALAR_ATOL_F32, SCALAR_RTOL_F32) if fp32 else (SCALAR_ATOL, SCALAR_RTOL)
    return {
        "got": gv,
        "ref": ref,
        "abs_diff": diff,
        "rel": diff / max(abs(ref), 1e-12),
        "allclose": diff <= atol + rtol * abs(ref),
    }


def compare(outs: dict, ref: dict, names=("out", "dq", "dk", "dv"), scalars=("dn", "db")) -> dict:
    res = {name: tensor_err(outs[name], ref[name]) for name in names if name in outs}
    fp32 = any(outs[name].dtype == torch.float32 for name in res)
    for name in scalars:
        if name in outs:
            res[name] = scalar_err(outs[name], ref[name], fp32)
    return res


def assert_parity(res: dict, label: str) -> None:
    for name, st in res.items():
        if name in ("dn", "db"):
            assert st["allclose"], f"{label}: {name} {st}"
            continue
        assert st["finite"], f"{label}: {name} has non-finite values"
        assert st["within_bound"], f"{label}: {name} exceeds its per-element bound ({st})"
        assert st["allclose"], f"{label}: {name} not allclose ({st})"


def scale_for(D: int) -> float:
    return 1.0 / math.sqrt(D)
