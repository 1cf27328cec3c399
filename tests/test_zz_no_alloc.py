"""ssa_bwd_noalloc: the backward that allocates nothing (Delta and the dn/db
partials in the library's static device scratch, dQ recomputed).

Called through the C ABI on four problems in a row -- each smaller, so each
runs on the scratch the previous one left behind, the last two on the
vector-ALU kernels (fp32 at head dim 16, bf16 at head dim 256) -- and
compared with ssa_bwd on
the same arguments (recompute path, caller workspaces): bitwise equal, and
within the parity bar of the fp64 oracle (tests/parity_util.py).  The
caller's delta / partials fields are NULL, so nothing of the caller's is used
for them.  Also captured into a HIP graph (after one call outside capture, which
looks up the scratch address): every replay equals ssa_bwd bit for bit.
"""

from __future__ import annotations

import ctypes
import sys

import pytest
import torch

from parity_util import assert_parity, compare, make_inputs, oracle_fwd_bwd, scale_for

pytestmark = pytest.mark.gpu

CALLS = [
    # B, Hq, Hkv, N, D, causal, dtype: larger first, then smaller (the last two
    # on the vector-ALU kernels: fp32 to the fp32 bars, bf16 at head dim 256)
    (2, 8, 4, 700, 128, True, torch.bfloat16),
    (1, 4, 2, 200, 64, False, torch.bfloat16),
    (1, 4, 4, 150, 16, True, torch.float32),
    (1, 2, 2, 130, 256, True, torch.bfloat16),
]


def test_noalloc_equals_ssa_bwd_on_four_calls(gpu):
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


def test_noalloc_under_graph_capture(gpu):
    """One call outside capture (the first call on a device looks up the
    scratch address), then ssa_bwd_noalloc captured into a graph on a side
    stream; three replays, each after eager work that overwrites the outputs
    with NaN, must each equal ssa_bwd bit for bit."""
    from SSA import _lib
    from SSA.ssa_hip_kernel import BackwardLaunch, ssa_flash_attn_forward

    print("[gpu case] noalloc under graph capture", file=sys.stderr, flush=True)
    lib = _lib.lib()
    B, Hq, Hkv, N, D, causal = 1, 4, 2, 384, 128, True
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, gpu, "contig", 77, 0.5)
    n = torch.tensor(1.5, device=gpu)
    b = torch.tensor(0.8, device=gpu)
    scale = scale_for(D)
    out, m = ssa_flash_attn_forward(q, k, v, scale, n, b, causal)
    ref = BackwardLaunch(q, k, v, out, do, m, scale, n, b, causal, ds=False)
    ref.run()
    na = BackwardLaunch(q, k, v, out, do, m, scale, n, b, causal, ds=False)
    na.args.delta = None
    na.args.partials = None
    na.args.ds_workspace = None
    cur = torch.cuda.current_stream(gpu)
    assert lib.ssa_bwd_noalloc(ctypes.byref(na.args), ctypes.c_void_p(cur.cuda_stream)) == _lib.SSA_OK
    torch.cuda.synchronize()

    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(cur)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        st = lib.ssa_bwd_noalloc(ctypes.byref(na.args), ctypes.c_void_p(side.cuda_stream))
    assert st == _lib.SSA_OK, _lib.status_text(st)
    torch.cuda.synchronize()
    for rep in range(3):
        for t in na.results():
            t.fill_(float("nan"))
        (q.float() @ q.float().transpose(-1, -2).contiguous()).sum().item()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, r in zip(("dq", "dk", "dv", "dn", "db"), na.results(), ref.results()):
            assert torch.equal(a, r), f"replay {rep}: {name} differs from ssa_bwd"
