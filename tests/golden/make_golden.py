#!/usr/bin/env python3
"""Generate the golden SSA vectors in this directory with the fp64 oracle.

Inputs are drawn from torch's CPU generator seeded with 1234 (the reference
harness's default seed, training/train/train_ssa_triton/check_ssa_triton_parity.py:1008)
and rounded to bf16 (stored as their 16-bit patterns), so a GPU kernel sees
exactly the stored values.  Outputs
are the oracle's float64 results stored as float32.  Shapes follow the tiny
matrix of the reference suite (D in 32/64/128, MHA and GQA, causal and not,
trained values of n) plus one varlen batch.

    python tests/golden/make_golden.py      # rewrites tests/golden/ssa_golden.npz
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import ssa_oracle as so  # noqa: E402

CASES = [
    # name, B, Hq, Hkv, N, D, causal, n
    ("mha_d32_causal", 1, 2, 2, 32, 32, True, 1.5),
    ("gqa_d64_causal", 1, 4, 2, 24, 64, True, 1.5),
    ("gqa_d128_noncausal", 1, 4, 1, 16, 128, False, 1.5),
    ("mha_d128_n_neg", 1, 2, 2, 17, 128, True, -3.484375),
    ("mha_d64_n4", 2, 2, 2, 8, 64, True, 4.0),
    ("mha_d64_n_m302", 1, 2, 2, 16, 64, True, -302.0),
]
VARLEN = ("varlen_d64", [0, 5, 6, 19, 32], 4, 2, 64, True, 1.5)


def _bf16(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).float().numpy()


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    """Exact bf16 values stored as their 16-bit patterns (half the bytes of float32)."""
    return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def main() -> None:
    g = torch.Generator().manual_seed(1234)
    out = {}
    for name, B, Hq, Hkv, N, D, causal, n in CASES:
        q = _bf16(torch.randn(B, Hq, N, D, generator=g) * 0.5)
        k = _bf16(torch.randn(B, Hkv, N, D, generator=g) * 0.5)
        v = _bf16(torch.randn(B, Hkv, N, D, generator=g) * 0.5)
        do = _bf16(torch.randn(B, Hq, N, D, generator=g))
        scale = 1.0 / math.sqrt(D)
        r = so.ssa_forward_backward(q, k, v, do, scale, n, 0.8, causal)
        meta = np.array([B, Hq, Hkv, N, D, int(causal)], dtype=np.int64)
        out[f"{name}/meta"] = meta
        out[f"{name}/params"] = np.array([n, 0.8, scale], dtype=np.float64)
        for key, val in (("q", q), ("k", k), ("v", v), ("do", do)):
            out[f"{name}/{key}"] = _bf16_bits(val)
        for key in ("out", "m", "dq", "dk", "dv", "delta"):
            out[f"{name}/{key}"] = r[key].astype(np.float32)
        out[f"{name}/dndb"] = np.array([r["dn"], r["db"]], dtype=np.float64)
    name, cu, Hq, Hkv, D, causal, n = VARLEN
    T = cu[-1]
    q = _bf16(torch.randn(T, Hq, D, generator=g) * 0.5)
    k = _bf16(torch.randn(T, Hkv, D, generator=g) * 0.5)
    v = _bf16(torch.randn(T, Hkv, D, generator=g) * 0.5)
    do = _bf16(torch.randn(T, Hq, D, generator=g))
    scale = 1.0 / math.sqrt(D)
    r = so.ssa_varlen_forward_backward(q, k, v, do, np.array(cu), scale, n, 0.8, causal)
    out[f"{name}/cu_seqlens"] = np.array(cu, dtype=np.int32)
    out[f"{name}/meta"] = np.array([T, Hq, Hkv, D, int(causal)], dtype=np.int64)
    out[f"{name}/params"] = np.array([n, 0.8, scale], dtype=np.float64)
    for key, val in (("q", q), ("k", k), ("v", v), ("do", do)):
        out[f"{name}/{key}"] = _bf16_bits(val)
    for key in ("out", "m", "dq", "dk", "dv", "delta"):
        out[f"{name}/{key}"] = r[key].astype(np.float32)
    out[f"{name}/dndb"] = np.array([r["dn"], r["db"]], dtype=np.float64)
    np.savez_compressed(HERE / "ssa_golden.npz", **out)
    print(f"wrote {HERE / 'ssa_golden.npz'} ({len(out)} arrays)")


if __name__ == "__main__":
    main()
