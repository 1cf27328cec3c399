"""Bitwise run-to-run determinism, at the breadth of the reference's suite and beyond.

The reference runs forward + backward twice on the same inputs and requires
every output to match with atol 0 (determinism_atol=0.0), for each kernel
dtype, N in {128, 1024}, causal and not, contiguous and strided inputs
(training/train/train_ssa_triton/check_ssa_triton_parity.py:505-624, defaults
:1021-1034).  Here: bf16, fp16 and fp32 inputs, head dims 32 (the reference's
default) and 128 (the benchmark's), 256 (the largest), both backward paths of the 16-bit kernels
(dQ from the dS' workspace and dQ recomputed), GQA, and a packed stream.
Every reduction in these kernels has a fixed order (no float atomics), so two
runs agree bit for bit, dn and db included.
"""

from __future__ import annotations

import math
import sys

import pytest
import torch

from parity_util import make_inputs

pytestmark = pytest.mark.gpu

DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def _twice(fn):
    runs = []
    for _ in range(2):
        res = fn()
        torch.cuda.synchronize()
        runs.append(res)
    return runs


def _assert_same(label, names, a, c):
    for name, x, y in zip(names, a, c):
        assert torch.equal(x, y), f"{label}: {name} differs between two runs"


@pytest.mark.parametrize("dtype,dq_path", [("bf16", "ds"), ("bf16", "recompute"), ("fp16", "ds"),
                                           ("fp16", "recompute"), ("fp32", "recompute")])
@pytest.mark.parametrize("N", [128, 1024])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("layout", ["contig", "strided"])
@pytest.mark.parametrize("D", [32, 128])
def test_two_runs_bitwise_equal(gpu, dtype, dq_path, N, causal, layout, D):
    from SSA.ssa_triton_kernel import ssa_flash_attn_backward, ssa_flash_attn_forward

    label = f"determinism {dtype} N={N} D={D} causal={int(causal)} {layout} dq={dq_path}"
    print(f"[gpu case] {label}", file=sys.stderr, flush=True)
    q, k, v, do = make_inputs(2, 8, 4, N, D, DTYPES[dtype], gpu, layout, seed=4321)
    scale = 1.0 / math.sqrt(D)
    n = torch.tensor(1.5, device=gpu)
    b = torch.tensor(0.8, device=gpu)
    ds = None if dtype == "fp32" else dq_path == "ds"

    def run():
        out, m = ssa_flash_attn_forward(q, k, v, scale, n, b, causal=causal)
        return (out, m) + tuple(ssa_flash_attn_backward(q, k, v, out, do, m, scale, n, b, causal=causal, ds=ds))

    a, c = _twice(run)
    _assert_same(label, ("out", "m", "dq", "dk", "dv", "dn", "db"), a, c)


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
@pytest.mark.parametrize("causal", [True, False])
def test_head_dim_256_bitwise_equal(gpu, dtype, causal):
    """Head dim 256 runs on the vector-ALU kernels: the same fixed-order reductions."""
    from SSA.ssa_triton_kernel import ssa_flash_attn_backward, ssa_flash_attn_forward

    label = f"determinism {dtype} N=300 D=256 causal={int(causal)}"
    print(f"[gpu case] {label}", file=sys.stderr, flush=True)
    q, k, v, do = make_inputs(2, 4, 2, 300, 256, DTYPES[dtype], gpu, "contig", seed=4321)
    n = torch.tensor(1.5, device=gpu)
    b = torch.tensor(0.8, device=gpu)

    def run():
        out, m = ssa_flash_attn_forward(q, k, v, 1.0 / 16, n, b, causal=causal)
        return (out, m) + tuple(ssa_flash_attn_backward(q, k, v, out, do, m, 1.0 / 16, n, b, causal=causal))

    a, c = _twice(run)
    _assert_same(label, ("out", "m", "dq", "dk", "dv", "dn", "db"), a, c)


@pytest.mark.parametrize("dq_path", ["ds", "recompute"])
def test_packed_stream_bitwise_equal(gpu, dq_path):
    from SSA.ssa_hip_kernel import ssa_flash_attn_varlen_backward, ssa_flash_attn_varlen_forward

    lens = (300, 7, 1024, 65, 129)
    T, Hq, Hkv, D = sum(lens), 8, 4, 128
    g = torch.Generator().manual_seed(99)
    q = (torch.randn(T, Hq, D, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    k = (torch.randn(T, Hkv, D, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    v = (torch.randn(T, Hkv, D, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    do = torch.randn(T, Hq, D, generator=g).to(torch.bfloat16).to(gpu)
    cu = torch.tensor([0, *torch.tensor(lens).cumsum(0).tolist()], dtype=torch.int32, device=gpu)
    scale = 1.0 / math.sqrt(D)
    n = torch.tensor(1.5, device=gpu)
    b = torch.tensor(0.8, device=gpu)

    def run():
        out, m = ssa_flash_attn_varlen_forward(q, k, v, cu, max(lens), scale, n, b, True)
        return (out, m) + tuple(ssa_flash_attn_varlen_backward(q, k, v, out, do, m, cu, max(lens), scale, n, b, True,
                                                               ds=dq_path == "ds"))

    a, c = _twice(run)
    _assert_same(f"packed stream dq={dq_path}", ("out", "m", "dq", "dk", "dv", "dn", "db"), a, c)
