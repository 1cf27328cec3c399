"""ssa_bwd_noalloc: the backward that allocates nothing (Delta and the dn/db
partials in the library's static device scratch, dQ recomputed).

Called through the C ABI on three problems in a row -- each smaller, so each
runs on the scratch the previous one left behind, the last on the fp32
kernels -- and compared with ssa_bwd on
the same arguments (recompute path, caller workspaces): bitwise equal, and
within the parity bar of the fp64 oracle (tests/parity_util.py).  The
caller's delta / partials fields are NULL, so nothing of the caller's is used
for them.
"""

from __future__ import annotations

import ctypes
import sys

import pytest
import torch

from parity_util import assert_parity, compare, make_inputs, oracle_fwd_bwd, scale_for

pytestmark = pytest.mark.gpu

CALLS = [
    # B, Hq, Hkv, N, D, causal, dtype: larger first, then smaller (the last on
    # the fp32 kernels, to the fp32 bars)
    (2, 8, 4, 700, 128, True, torch.bfloat16),
    (1, 4, 2, 200, 64, False, torch.bfloat16),
    (1, 4, 4, 150, 16, True, torch.float32),
]


def test_noalloc_equals_ssa_bwd_on_two_calls(gpu):
    from SSA import _lib
    from SSA.ssa_hip_kernel import BackwardLaunch, ssa_flash_attn_forward

    lib = _lib.lib()
    for i, (B, Hq, Hkv, N, D, causal, dtype) in enumerate(CALLS):
        label = f"noalloc call {i}: B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={int(causal)} {dtype}"
        print(f"[gpu case] {label}", file=sys.stderr, flush=True)
        q, k, v, do = make_inputs(B, Hq, Hkv, N, D, dtype, gpu, "contig", 1234 + i, 0.5)
        n = torch.tensor(1.5, device=gpu)
        b = torch.tensor(0.8, device=gpu)
        scale = scale_for(D)
        out, m = ssa_flash_attn_forward(q, k, v, scale, n, b, causal)
        ref = BackwardLaunch(q, k, v, out, do, m, scale, n, b, causal, ds=False)
        ref.run()
        na = BackwardLaunch(q, k, v, out, do, m, scale, n, b, causal, ds=False)
        for t in (na.dq, na.dk, na.dv, na.dn, na.db):
            t.fill_(float("nan"))
        na.args.delta = None
        na.args.partials = None
        na.args.ds_workspace = None
        stream = torch.cuda.current_stream(gpu).cuda_stream
        st = lib.ssa_bwd_noalloc(ctypes.byref(na.args), ctypes.c_void_p(stream))
        assert st == _lib.SSA_OK, f"{label}: status {st} ({_lib.status_text(st)})"
        torch.cuda.synchronize()
        for name, a, r in zip(("dq", "dk", "dv", "dn", "db"), na.results(), ref.results()):
            assert torch.equal(a, r), f"{label}: {name} differs from ssa_bwd"
        oracle = oracle_fwd_bwd(q, k, v, do, scale, 1.5, 0.8, causal, out_for_delta=out)
        res = compare({"dq": na.dq, "dk": na.dk, "dv": na.dv, "dn": na.dn.item(), "db": na.db.item()}, oracle,
                      names=("dq", "dk", "dv"))
        assert_parity(res, label)
