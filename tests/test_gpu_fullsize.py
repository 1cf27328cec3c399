"""GPU parity at the benchmark's full sizes.

The kernels run on the whole problem (every head, every key block, the real
dispatch order and workspace sizes), and one (batch, kv-head group) slice of
the result -- a complete set of heads, independent of every other slice --
goes through the fp64 oracle (oracle/ssa_oracle.py): out and m against the
exact forward, dq / dk / dv against the kernel-level backward (delta from the
kernel's own out, as ssa_triton_kernel.py:291-294 defines it), to the bar of
parity_util.  dn / db, sums over every pair of every head, are checked for the
whole problem: the chunked fp64 oracle (ssa_forward_backward_chunked, the
kernel-level backward of the kernel's own out) runs on every (batch, kv-head)
slice in a thread pool and the slices' sums are added in a fixed order, to the
scalar bar of parity_util (2e-3 + 2e-2 |ref|, the reference's
check_ssa_triton_parity.py:1060-1069).  The packed case checks one head of the
16,384-token stream.
"""

from __future__ import annotations

import concurrent.futures as cf
import math
import os
import sys

import numpy as np
import pytest
import torch

from oracle import ssa_oracle as so
from parity_util import assert_parity, compare, make_inputs, scalar_err

pytestmark = pytest.mark.gpu


def _np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def whole_dn_db(q, k, v, do, out, scale, n_val, b_val, causal=True):
    """dn, db of the whole problem from the chunked fp64 oracle: one task per
    (batch, kv-head) slice (a complete set of heads), run in threads (NumPy
    releases the GIL in its array loops; BLAS is held to one thread per call so
    the threads do not oversubscribe the cores), summed in slice order."""
    from threadpoolctl import threadpool_limits

    B, Hq, Hkv = q.shape[0], q.shape[1], k.shape[1]
    G = Hq // Hkv
    qn, kn, vn, don, on = (_np64(t) for t in (q, k, v, do, out))

    def one(bh):
        bi, hk = bh
        hs = slice(hk * G, (hk + 1) * G)
        r = so.ssa_forward_backward_chunked(qn[bi:bi + 1, hs], kn[bi:bi + 1, hk:hk + 1], vn[bi:bi + 1, hk:hk + 1],
                                            don[bi:bi + 1, hs], scale, n_val, b_val, causal,
                                            out_for_delta=on[bi:bi + 1, hs])
        return r["dn"], r["db"]

    slices = [(bi, hk) for bi in range(B) for hk in range(Hkv)]
    with threadpool_limits(limits=1), cf.ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
        parts = list(ex.map(one, slices))
    return sum(p[0] for p in parts), sum(p[1] for p in parts)


DENSE = [
    # name, B, Hq, Hkv, N, D, (batch, kv-head) checked
    ("s4096", 4, 16, 16, 4096, 128, (3, 11)),
    ("s2048", 4, 16, 16, 2048, 128, (1, 6)),
    ("gqa_d64", 4, 32, 8, 4096, 64, (2, 5)),
]


@pytest.mark.parametrize("name,B,Hq,Hkv,N,D,sl", DENSE, ids=[c[0] for c in DENSE])
def test_fullsize_slice_matches_oracle(gpu, name, B, Hq, Hkv, N, D, sl):
    from SSA.ssa_triton_kernel import ssa_flash_attn_backward, ssa_flash_attn_forward

    label = f"full size {name}: B={B} Hq={Hq} Hkv={Hkv} N={N} D={D}, slice (b, hk)={sl}"
    print(f"[gpu case] {label}", file=sys.stderr, flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, gpu, "contig", 1234, 0.5)
    scale, n_val, b_val = 1.0 / math.sqrt(D), 1.5, 0.8
    n = torch.tensor(n_val, device=gpu)
    b = torch.tensor(b_val, device=gpu)
    out, m = ssa_flash_attn_forward(q, k, v, scale, n, b, causal=True)
    dq, dk, dv, dn, db = ssa_flash_attn_backward(q, k, v, out, do, m, scale, n, b, causal=True)
    torch.cuda.synchronize()
    assert torch.isfinite(dn) and torch.isfinite(db)
    ref_dn, ref_db = whole_dn_db(q, k, v, do, out, scale, n_val, b_val)
    sres = {"dn": scalar_err(dn.item(), ref_dn), "db": scalar_err(db.item(), ref_db)}
    print(f"[gpu result] {label}: whole-problem dn {dn.item():.6e} vs {ref_dn:.6e} (rel {sres['dn']['rel']:.1e}), "
          f"db {db.item():.6e} vs {ref_db:.6e} (rel {sres['db']['rel']:.1e})", file=sys.stderr, flush=True)
    assert_parity(sres, label + " [whole-problem dn / db]")

    bi, hk = sl
    G = Hq // Hkv
    hs = slice(hk * G, (hk + 1) * G)
    qs, dos = _np64(q[bi:bi + 1, hs]), _np64(do[bi:bi + 1, hs])
    ks, vs = _np64(k[bi:bi + 1, hk:hk + 1]), _np64(v[bi:bi + 1, hk:hk + 1])
    out_s = out[bi:bi + 1, hs]
    ref_out, ref_m = so.ssa_forward(qs, ks, vs, scale, n_val, b_val, True)
    rdq, rdk, rdv, _, _, _ = so.ssa_backward(qs, ks, vs, dos, scale, n_val, b_val, True, out_for_delta=_np64(out_s))
    res = compare({"out": out_s}, {"out": ref_out}, names=("out",), scalars=())
    res_k = compare({"dq": dq[bi:bi + 1, hs], "dk": dk[bi:bi + 1, hk:hk + 1], "dv": dv[bi:bi + 1, hk:hk + 1]},
                    {"dq": rdq, "dk": rdk, "dv": rdv}, names=("dq", "dk", "dv"), scalars=())
    merr = float(np.abs(m[bi:bi + 1, hs].cpu().numpy() - ref_m).max())
    print(f"[gpu result] {label}: " + ", ".join(f"{k_} max_abs={v_['max_abs']:.2e}"
                                                 for k_, v_ in {**res, **res_k}.items()) + f", m={merr:.1e}",
          file=sys.stderr, flush=True)
    assert merr < 1e-2, f"{label}: m {merr}"
    assert_parity(res, label)
    assert_parity(res_k, label + " [kernel-level]")


# Document lengths of the packed benchmark (16,384 tokens; lengths uniform in
# [64, 4096] from random.Random(1234), the last one truncated to fill).
VARLEN_LENS = (4022, 3251, 1869, 542, 94, 435, 3795, 2376)


def test_fullsize_varlen_head_matches_oracle(gpu):
    from SSA.ssa_hip_kernel import ssa_flash_attn_varlen_backward, ssa_flash_attn_varlen_forward

    T, H, D, h = sum(VARLEN_LENS), 16, 128, 9
    label = f"full size varlen16k: T={T} H={H} D={D}, head {h}"
    print(f"[gpu case] {label}", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(1234)
    q, k, v = ((torch.randn(T, H, D, generator=g) * 0.5).to(torch.bfloat16).to(gpu) for _ in range(3))
    do = torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(gpu)
    cu_host = torch.tensor([0] + list(np.cumsum(VARLEN_LENS)), dtype=torch.int32)
    scale, n_val, b_val = 1.0 / math.sqrt(D), 1.5, 0.8
    n = torch.tensor(n_val, device=gpu)
    b = torch.tensor(b_val, device=gpu)
    cu = cu_host.to(gpu)
    out, m = ssa_flash_attn_varlen_forward(q, k, v, cu, max(VARLEN_LENS), scale, n, b, True)
    dq, dk, dv, dn, db = ssa_flash_attn_varlen_backward(q, k, v, out, do, m, cu, max(VARLEN_LENS), scale, n, b, True)
    torch.cuda.synchronize()
    one = lambda t: _np64(t[:, h:h + 1])
    ref = so.ssa_varlen_forward_backward(one(q), one(k), one(v), one(do), cu_host.numpy(), scale, n_val, b_val, True,
                                         out_for_delta=one(out))
    res = compare({"out": out[:, h:h + 1]}, ref, names=("out",), scalars=())
    res_k = compare({"dq": dq[:, h:h + 1], "dk": dk[:, h:h + 1], "dv": dv[:, h:h + 1]}, ref,
                    names=("dq", "dk", "dv"), scalars=())
    merr = float(np.abs(m[h].cpu().numpy() - ref["m"][:, 0]).max())
    assert merr < 1e-2, f"{label}: m {merr}"
    assert_parity(res, label)
    assert_parity(res_k, label + " [kernel-level]")

    # dn / db of the whole stream: every head through the oracle (threads), summed in head order
    from threadpoolctl import threadpool_limits

    qn, kn, vn, don, on = (_np64(t) for t in (q, k, v, do, out))
    cun = cu_host.numpy()

    def head(hh):
        r = so.ssa_varlen_forward_backward(qn[:, hh:hh + 1], kn[:, hh:hh + 1], vn[:, hh:hh + 1], don[:, hh:hh + 1],
                                           cun, scale, n_val, b_val, True, out_for_delta=on[:, hh:hh + 1])
        return r["dn"], r["db"]

    with threadpool_limits(limits=1), cf.ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
        parts = list(ex.map(head, range(H)))
    ref_dn, ref_db = sum(p_[0] for p_ in parts), sum(p_[1] for p_ in parts)
    sres = {"dn": scalar_err(dn.item(), ref_dn), "db": scalar_err(db.item(), ref_db)}
    print(f"[gpu result] {label}: whole-stream dn rel {sres['dn']['rel']:.1e}, db rel {sres['db']['rel']:.1e}",
          file=sys.stderr, flush=True)
    assert_parity(sres, label + " [whole-stream dn / db]")
