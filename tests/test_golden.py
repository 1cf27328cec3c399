"""Golden fixtures (tests/golden/ssa_golden.npz): bf16 inputs and fp64-oracle outputs.

CPU: the oracle reproduces every stored case (regression lock), and for the
smallest cases an independent pure-Python brute force of the forward agrees
with the stored outputs.  GPU: the HIP kernels, called through the reference
API on exactly the stored bf16 inputs, meet the parity bar of parity_util
(the divergent n = -302 case to its normwise bar).  The varlen case has no
dense kernel entry; it pins the oracle only.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import ssa_oracle as so
from parity_util import assert_parity, compare, oracle_fwd_bwd

GOLDEN = Path(__file__).resolve().parent / "golden" / "ssa_golden.npz"
DENSE = ["mha_d32_causal", "gqa_d64_causal", "gqa_d128_noncausal", "mha_d128_n_neg", "mha_d64_n4", "mha_d64_n_m302"]


def _bits_to_f32(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def _load(name):
    z = np.load(GOLDEN)
    case = {key.split("/", 1)[1]: z[key] for key in z.files if key.startswith(name + "/")}
    for key in ("q", "k", "v", "do"):
        case[key] = _bits_to_f32(case[key]).astype(np.float64)
    return case


@pytest.mark.parametrize("name", DENSE)
def test_oracle_reproduces_golden(name):
    c = _load(name)
    n, b, scale = c["params"]
    causal = bool(c["meta"][5])
    r = so.ssa_forward_backward(c["q"], c["k"], c["v"], c["do"], scale, n, b, causal)
    for key in ("out", "m", "dq", "dk", "dv", "delta"):
        np.testing.assert_allclose(r[key], c[key], rtol=1e-5, atol=1e-6, err_msg=f"{name}/{key}")
    np.testing.assert_allclose([r["dn"], r["db"]], c["dndb"], rtol=1e-10)


def test_oracle_reproduces_golden_varlen():
    c = _load("varlen_d64")
    n, b, scale = c["params"]
    r = so.ssa_varlen_forward_backward(c["q"], c["k"], c["v"], c["do"], c["cu_seqlens"].astype(np.int64),
                                       scale, n, b, bool(c["meta"][4]))
    for key in ("out", "m", "dq", "dk", "dv", "delta"):
        np.testing.assert_allclose(r[key], c[key], rtol=1e-5, atol=1e-6, err_msg=f"varlen/{key}")


@pytest.mark.parametrize("name", ["mha_d64_n4", "mha_d128_n_neg"])
def test_golden_forward_matches_bruteforce(name):
    # Independent of the oracle: pure-Python loops over (b, h, i, j).
    c = _load(name)
    n, b, scale = c["params"]
    B, Hq, Hkv, N, D, causal = (int(x) for x in c["meta"])
    G = Hq // Hkv
    out = np.zeros((B, Hq, N, D))
    for bi in range(B):
        for h in range(Hq):
            for i in range(N):
                ts = []
                for j in range(N if not causal else i + 1):
                    s = scale * sum(c["q"][bi, h, i, d] * c["k"][bi, h // G, j, d] for d in range(D))
                    ts.append(n * math.copysign(1.0, s) * math.log1p(b * abs(s)) if s != 0 else 0.0)
                mx = max(ts)
                w = [math.exp(t - mx) for t in ts]
                tot = sum(w)
                for d in range(D):
                    out[bi, h, i, d] = sum(w[j] * c["v"][bi, h // G, j, d] for j in range(len(w))) / tot
    np.testing.assert_allclose(c["out"], out, rtol=1e-5, atol=1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("name", DENSE)
def test_kernel_matches_golden(gpu, name):
    from SSA.ssa_triton_kernel import ssa_flash_attn_backward, ssa_flash_attn_forward

    c = _load(name)
    n_val, b_val, scale = (float(x) for x in c["params"])
    causal = bool(c["meta"][5])
    print(f"[gpu case] golden {name}", flush=True)
    t = {key: torch.from_numpy(c[key].astype(np.float32)).to(torch.bfloat16).to(gpu) for key in ("q", "k", "v", "do")}
    n = torch.tensor(n_val, device=gpu)
    b = torch.tensor(b_val, device=gpu)
    out, m = ssa_flash_attn_forward(t["q"], t["k"], t["v"], scale, n, b, causal=causal)
    dq, dk, dv, dn, db = ssa_flash_attn_backward(t["q"], t["k"], t["v"], out, t["do"], m, scale, n, b, causal=causal)
    torch.cuda.synchronize()
    got = {"out": out, "dq": dq, "dk": dk, "dv": dv}
    ref = {key: c[key].astype(np.float64) for key in ("out", "dq", "dk", "dv")}
    res = compare(got, ref, scalars=())
    assert (m.float().cpu().numpy() - c["m"]).__abs__().max() < 1e-2
    if n_val < -100:
        # Near one-hot rows with dS amplified by n b = -241: the gradients are
        # checked normwise as kernel-level functions of the out the backward is
        # handed (Delta = rowsum(dO * out)), as in test_gpu_parity; out elementwise.
        assert_parity({"out": res["out"]}, name)
        ref_k = oracle_fwd_bwd(t["q"], t["k"], t["v"], t["do"], scale, n_val, b_val, causal, out_for_delta=out)
        res_k = compare({"dq": dq, "dk": dk, "dv": dv}, ref_k, scalars=(), names=("dq", "dk", "dv"))
        for key in ("dq", "dk", "dv"):
            assert res_k[key]["finite"] and res_k[key]["rel_rmse"] <= 1e-2, f"{name}: {key} {res_k[key]}"
        return
    assert_parity(res, name)
    # dn / db gated as kernel-level functions of the out the backward is handed
    # (Delta = rowsum(dO * out)), as in test_gpu_parity.
    ref_k = oracle_fwd_bwd(t["q"], t["k"], t["v"], t["do"], scale, n_val, b_val, causal, out_for_delta=out)
    res_k = compare({"dq": dq, "dk": dk, "dv": dv, "dn": dn.item(), "db": db.item()}, ref_k, names=("dq", "dk", "dv"))
    assert_parity(res_k, name + " [kernel-level]")
