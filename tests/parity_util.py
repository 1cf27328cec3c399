"""Helpers shared by the GPU parity tests: seeded inputs and error statistics.

Error metric (same as the reference harness,
training/train/train_ssa_triton/check_ssa_triton_parity.py:124-149,206,219-237):
kernel tensors are compared with the fp64 oracle rounded to the kernel's
dtype (the reference's oracle returns out.to(q.dtype) and grads in the dtype
of the leaves).  Pass bar: max |err| <= MAX_ABS and allclose(atol=ATOL,
rtol=RTOL) per tensor; dn / db by relative error.
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


def oracle_fwd_bwd(q, k, v, do, scale, n, b, causal):
    """fp64 oracle on the CPU copies of (already rounded) kernel inputs."""
    c = lambda t: t.detach().float().cpu().numpy().astype(np.float64)  # noqa: E731
    return so.ssa_forward_backward(c(q), c(k), c(v), c(do), scale, n, b, causal)


def tensor_err(got: torch.Tensor, ref: np.ndarray) -> dict:
    g = got.detach().float().cpu()
    r = torch.from_numpy(np.ascontiguousarray(ref)).float()
    r_round = r.to(got.dtype).float() if got.dtype in (torch.bfloat16, torch.float16) else r
    d = (g - r_round).abs()
    d_raw = (g - r).abs()
    return {
        "max_abs": float(d.max()) if d.numel() else 0.0,
        "max_abs_vs_unrounded": float(d_raw.max()) if d.numel() else 0.0,
        "rel_rmse": float(torch.sqrt(((g - r) ** 2).mean()) / (torch.sqrt((r ** 2).mean()) + 1e-12)),
        "allclose": bool(torch.allclose(g, r_round, atol=ATOL, rtol=RTOL)),
        "finite": bool(torch.isfinite(g).all()),
    }


def scalar_err(got, ref: float) -> dict:
    gv = float(got)
    diff = abs(gv - ref)
    return {
        "got": gv,
        "ref": ref,
        "abs_diff": diff,
        "rel": diff / max(abs(ref), 1e-12),
        "allclose": diff <= SCALAR_ATOL + SCALAR_RTOL * abs(ref),
    }


def compare(outs: dict, ref: dict, names=("out", "dq", "dk", "dv")) -> dict:
    res = {name: tensor_err(outs[name], ref[name]) for name in names if name in outs}
    for name in ("dn", "db"):
        if name in outs:
            res[name] = scalar_err(outs[name], ref[name])
    return res


def assert_parity(res: dict, label: str, check_db: bool = True) -> None:
    for name, st in res.items():
        if name in ("dn", "db"):
            if name == "db" and not check_db:
                continue
            assert st["allclose"], f"{label}: {name} {st}"
            continue
        assert st["finite"], f"{label}: {name} has non-finite values"
        assert st["max_abs"] <= MAX_ABS, f"{label}: {name} max_abs {st['max_abs']:.3e} > {MAX_ABS} ({st})"
        assert st["allclose"], f"{label}: {name} not allclose ({st})"


def scale_for(D: int) -> float:
    return 1.0 / math.sqrt(D)
