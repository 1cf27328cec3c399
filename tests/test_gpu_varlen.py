"""GPU parity of the packed-sequence (varlen) entry points.

Token streams [T, H, D] split into documents by cu_seqlens (Megatron
PackedSeqParams layout); attention stays inside each document.  The reference
has no varlen path (training/train/train_ssa_triton/SSA/ssa_triton_attention.py:154-156
rejects packed sequences), so the oracle defines it as independent dense runs
per document (oracle/ssa_oracle.py, pinned in tests/test_oracle.py against
per-document dense results); checked here to the bar of parity_util, with
dn / db gated as kernel-level functions of the forward output, as in
test_gpu_parity.  Also: a one-document stream equals the dense path bitwise,
the committed golden varlen case, and a malformed table (clamped on the
device, never read out of bounds) against the oracle on the clamped table.
Every case runs both backward paths: dQ recomputed from the scores and dQ as
a product with the dS' workspace written by dK/dV (ds=True).
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import ssa_oracle as so
from parity_util import assert_parity, compare

pytestmark = pytest.mark.gpu


def _np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _inputs(lens, Hq, Hkv, D, dtype, dev, seed=1234, scale=0.5):
    g = torch.Generator().manual_seed(seed)
    T = int(sum(lens))
    q = (torch.randn(T, Hq, D, generator=g) * scale).to(dtype).to(dev)
    k = (torch.randn(T, Hkv, D, generator=g) * scale).to(dtype).to(dev)
    v = (torch.randn(T, Hkv, D, generator=g) * scale).to(dtype).to(dev)
    do = torch.randn(T, Hq, D, generator=g).to(dtype).to(dev)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    return q, k, v, do, cu


def _run(dev, q, k, v, do, cu_host, max_seqlen, causal, n_val=1.5, b_val=0.8, oracle_cu=None, ds=False):
    from SSA.ssa_hip_kernel import ssa_flash_attn_varlen_backward, ssa_flash_attn_varlen_forward

    D = q.shape[-1]
    scale = 1.0 / math.sqrt(D)
    n = torch.tensor(n_val, device=dev)
    b = torch.tensor(b_val, device=dev)
    cu = cu_host.to(dev)
    out, m = ssa_flash_attn_varlen_forward(q, k, v, cu, max_seqlen, scale, n, b, causal)
    dq, dk, dv, dn, db = ssa_flash_attn_varlen_backward(q, k, v, out, do, m, cu, max_seqlen, scale, n, b, causal,
                                                        ds=ds)
    torch.cuda.synchronize()
    ocu = cu_host.numpy() if oracle_cu is None else np.asarray(oracle_cu)
    ref = so.ssa_varlen_forward_backward(_np64(q), _np64(k), _np64(v), _np64(do), ocu, scale, n_val, b_val, causal)
    ref_k = so.ssa_varlen_forward_backward(_np64(q), _np64(k), _np64(v), _np64(do), ocu, scale, n_val, b_val,
                                           causal, out_for_delta=_np64(out))
    res = compare({"out": out, "dq": dq, "dk": dk, "dv": dv}, ref, scalars=())
    res_k = compare({"dq": dq, "dk": dk, "dv": dv, "dn": dn.item(), "db": db.item()}, ref_k, names=("dq", "dk", "dv"))
    mref = ref["m"].T  # [Hq, T]
    valid = np.isfinite(mref)
    merr = float(np.abs(m.cpu().numpy()[valid] - mref[valid]).max()) if valid.any() else 0.0
    return out, m, (dq, dk, dv, dn, db), res, res_k, merr


CASES = [
    # lens, Hq, Hkv, D, causal
    ((1,), 2, 2, 64, True),
    ((7, 1, 33), 4, 2, 64, True),
    ((64, 64), 4, 4, 128, True),
    ((5, 100, 33, 260, 1), 4, 2, 128, True),
    ((300, 513), 2, 1, 128, True),
    ((129, 31, 200), 4, 2, 128, False),
    ((40, 90, 257), 2, 2, 32, True),
    ((40, 90, 257), 4, 2, 16, True),  # head dim 16: zero-padded onto the D = 32 kernels
    ((70, 3, 200), 4, 2, 256, True),  # head dim 256: the vector-ALU kernels (the dS' workspace unused)
]


@pytest.mark.parametrize("ds", [False, True], ids=["recompute", "ds"])
@pytest.mark.parametrize("lens,Hq,Hkv,D,causal", CASES)
def test_varlen_parity(gpu, lens, Hq, Hkv, D, causal, ds):
    label = f"lens={lens} Hq={Hq} Hkv={Hkv} D={D} causal={int(causal)} ds={int(ds)}"
    print(f"[gpu case] varlen {label}", file=sys.stderr, flush=True)
    q, k, v, do, cu = _inputs(lens, Hq, Hkv, D, torch.bfloat16, gpu)
    _, _, _, res, res_k, merr = _run(gpu, q, k, v, do, cu, max(lens), causal, ds=ds)
    assert merr < 1e-2, f"{label}: m {merr}"
    assert_parity(res, label)
    assert_parity(res_k, label + " [kernel-level]")


@pytest.mark.parametrize("ds", [False, True], ids=["recompute", "ds"])
def test_varlen_fp16(gpu, ds):
    print(f"[gpu case] varlen fp16 ds={int(ds)}", file=sys.stderr, flush=True)
    q, k, v, do, cu = _inputs((50, 200, 77), 4, 2, 64, torch.float16, gpu)
    _, _, _, res, res_k, merr = _run(gpu, q, k, v, do, cu, 200, True, ds=ds)
    assert merr < 1e-2
    assert_parity(res, "varlen fp16")
    assert_parity(res_k, "varlen fp16 [kernel-level]")


@pytest.mark.parametrize("ds", [False, True], ids=["recompute", "ds"])
def test_varlen_one_document_equals_dense_bitwise(gpu, ds):
    from SSA.ssa_hip_kernel import (ssa_flash_attn_backward, ssa_flash_attn_forward,
                                    ssa_flash_attn_varlen_backward, ssa_flash_attn_varlen_forward)

    print(f"[gpu case] varlen one document ds={int(ds)}", file=sys.stderr, flush=True)
    q, k, v, do, cu = _inputs((333,), 4, 2, 128, torch.bfloat16, gpu)
    n = torch.tensor(1.5, device=gpu)
    b = torch.tensor(0.8, device=gpu)
    s = 1.0 / math.sqrt(128)
    out_v, m_v = ssa_flash_attn_varlen_forward(q, k, v, cu.to(gpu), 333, s, n, b, True)
    g_v = ssa_flash_attn_varlen_backward(q, k, v, out_v, do, m_v, cu.to(gpu), 333, s, n, b, True, ds=ds)
    dense = lambda t: t.permute(1, 0, 2).unsqueeze(0)  # [T, H, D] -> [1, H, T, D] view
    out_d, m_d = ssa_flash_attn_forward(dense(q), dense(k), dense(v), s, n, b, True)
    # the same backward path on the dense batch (the workspace layouts differ,
    # the tiles in them and every product do not)
    g_d = ssa_flash_attn_backward(dense(q), dense(k), dense(v), out_d, dense(do), m_d, s, n, b, True, ds=ds)
    torch.cuda.synchronize()
    assert torch.equal(out_v, out_d[0].permute(1, 0, 2))
    assert torch.equal(m_v, m_d[0])
    for a, c in zip(g_v[:3], g_d[:3]):
        assert torch.equal(a, c[0].permute(1, 0, 2))
    assert torch.equal(g_v[3], g_d[3]) and torch.equal(g_v[4], g_d[4])


@pytest.mark.parametrize("ds", [False, True], ids=["recompute", "ds"])
def test_varlen_golden(gpu, ds):
    print(f"[gpu case] varlen golden ds={int(ds)}", file=sys.stderr, flush=True)
    z = np.load(Path(__file__).resolve().parent / "golden" / "ssa_golden.npz")
    name = "varlen_d64"

    def bits(key):
        return torch.from_numpy(((z[f"{name}/{key}"].astype(np.uint32) << 16).view(np.float32)).copy())

    q, k, v, do = (bits(t).to(torch.bfloat16).to(gpu) for t in ("q", "k", "v", "do"))
    cu = torch.from_numpy(z[f"{name}/cu_seqlens"].astype(np.int32))
    n_val, b_val, _ = (float(x) for x in z[f"{name}/params"])
    causal = bool(z[f"{name}/meta"][4])
    out, m, (dq, dk, dv, dn, db), res, res_k, merr = _run(gpu, q, k, v, do, cu, int(np.diff(cu.numpy()).max()),
                                                          causal, n_val, b_val, ds=ds)
    assert merr < 1e-2
    assert_parity(res, "golden varlen (live oracle)")
    assert_parity(res_k, "golden varlen [kernel-level]")
    stored = {key: z[f"{name}/{key}"].astype(np.float64) for key in ("out", "dq", "dk", "dv")}
    assert_parity(compare({"out": out, "dq": dq, "dk": dk, "dv": dv}, stored, scalars=()), "golden varlen (fixture)")


@pytest.mark.parametrize("ds", [False, True], ids=["recompute", "ds"])
def test_varlen_malformed_table_is_clamped(gpu, ds):
    # cu = [-5, 40, 250] over T = 100 tokens: clamped on the device to the
    # documents [0, 40) and [40, 100) (a negative start, an end past T).
    print(f"[gpu case] varlen clamped table ds={int(ds)}", file=sys.stderr, flush=True)
    q, k, v, do, _ = _inputs((100,), 2, 2, 64, torch.bfloat16, gpu)
    cu = torch.tensor([-5, 40, 250], dtype=torch.int32)
    _, _, _, res, res_k, merr = _run(gpu, q, k, v, do, cu, 100, True, oracle_cu=[0, 40, 100], ds=ds)
    assert merr < 1e-2
    assert_parity(res, "clamped table")


@pytest.mark.parametrize("lens,D,causal", [((5, 100, 33, 260, 1), 128, True), ((40, 90, 257), 16, False),
                                           ((7, 1, 33), 64, True), ((70, 3, 200), 256, True)])
def test_varlen_fp32(gpu, lens, D, causal):
    """fp32 token streams on the fp32 kernels, at the reference's fp32 tolerances."""
    label = f"varlen fp32 lens={lens} D={D} causal={int(causal)}"
    print(f"[gpu case] {label}", file=sys.stderr, flush=True)
    q, k, v, do, cu = _inputs(lens, 4, 2, D, torch.float32, gpu)
    _, _, _, res, res_k, merr = _run(gpu, q, k, v, do, cu, max(lens), causal)
    assert merr < 1e-4, f"{label}: m {merr}"
    assert_parity(res, label)
    assert_parity(res_k, label + " [kernel-level]")


@pytest.mark.parametrize("ds,dtype", [(False, torch.bfloat16), (True, torch.bfloat16), (False, torch.float32)],
                         ids=["recompute", "ds", "fp32"])
def test_varlen_uncovered_rows_are_written(gpu, ds, dtype):
    """Tokens in no document -- after cu[-1] < T, and the tail of a document
    longer than max_seqlen (cut to its first max_seqlen tokens) -- come back as
    out = 0, m = -inf and dq = dk = dv = 0, never as stale memory: the caching
    allocator is first filled with NaN blocks of the output sizes, which the
    outputs then reuse."""
    lens_cover, T, max_seqlen = (37, 83), 200, 60   # covered: [0, 37), [37, 97); tokens 97..199 are not
    label = f"varlen uncovered rows ds={int(ds)} {str(dtype)[6:]}"
    print(f"[gpu case] {label}", file=sys.stderr, flush=True)
    Hq, Hkv, D = 4, 2, 64
    q, k, v, do, _ = _inputs((T,), Hq, Hkv, D, dtype, gpu)
    poison = [torch.full((T, h, D), float("nan"), device=gpu, dtype=dtype) for h in (Hq, Hq, Hkv, Hkv)]
    poison.append(torch.full((Hq, T), float("nan"), device=gpu))
    del poison
    cu = torch.tensor([0, 37, 37 + 83], dtype=torch.int32)
    out, m, (dq, dk, dv, dn, db), res, res_k, merr = _run(gpu, q, k, v, do, cu, max_seqlen, True,
                                                          oracle_cu=[0, 37, 37 + max_seqlen], ds=ds)
    for name, t in (("out", out), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert not torch.isnan(t).any(), f"{label}: {name} has NaN (stale rows)"
        assert (t[97:] == 0).all(), f"{label}: {name} rows 97.. not zero"
    assert torch.isneginf(m[:, 97:]).all(), f"{label}: m of uncovered rows"
    assert merr < 1e-2
    assert_parity(res, label)
    assert_parity(res_k, label + " [kernel-level]")
