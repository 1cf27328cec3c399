"""GPU parity of both dK/dV kernels at every head dim: the two-waves-per-SIMD
kernel (csrc/ssa_bwd_dkdv2w.hip, the default at head dim 128) and the
single-wave kernel (csrc/ssa_bwd.hip, the default at 32 and 64), each forced
with SSA_DKDV2W=1 / =0 at launch time, so that the kernel the library does
not pick for a head dim stays tested too.

Same oracle and bars as test_gpu_parity: head dims 32-128, bf16 / fp16,
causal / non-causal, MHA / GQA, both backward paths (their dS' tiles feed
the same dQ pass), sequence lengths that are not multiples of the kernels'
query steps or 128-key blocks, the divergent-layer n = -302,
Megatron-strided inputs, bitwise determinism, and packed sequences.
"""

from __future__ import annotations

import os

import pytest
import torch

import test_gpu_parity as tp
import test_gpu_varlen as tv
from parity_util import assert_parity

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["1", "0"], ids=["2w", "1w"])
def dkdv2w(request):
    old = os.environ.get("SSA_DKDV2W")
    os.environ["SSA_DKDV2W"] = request.param
    yield
    if old is None:
        del os.environ["SSA_DKDV2W"]
    else:
        os.environ["SSA_DKDV2W"] = old


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("heads", [(4, 4), (8, 2)])
@pytest.mark.parametrize("ds", [True, False], ids=["ds", "recompute"])
def test_dkdv2w_matrix(gpu, dkdv2w, D, dtype, causal, heads, ds):
    tp._check(*tp._run(gpu, 1, heads[0], heads[1], 320, D, dtype, causal, ds=ds))


@pytest.mark.parametrize("N", [1, 17, 64, 129, 200, 511])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("ds", [True, False], ids=["ds", "recompute"])
def test_dkdv2w_ragged(gpu, dkdv2w, N, D, ds):
    tp._check(*tp._run(gpu, 2, 4, 2, N, D, torch.bfloat16, True, ds=ds))


@pytest.mark.parametrize("layout", ["strided", "contig"])
def test_dkdv2w_strided_and_trained_n(gpu, dkdv2w, layout):
    tp._check(*tp._run(gpu, 2, 4, 4, 384, 128, torch.bfloat16, True, layout=layout, n_val=-3.484375))


def test_dkdv2w_divergent_n(gpu, dkdv2w):
    label, res_exact, res_kernel, mres = tp._run(gpu, 1, 4, 4, 256, 64, torch.bfloat16, True, n_val=-302.0)
    assert mres < 1e-2
    for name in ("dq", "dk", "dv"):
        st = res_kernel[name]
        assert st["finite"] and st["rel_rmse"] <= 1e-2, f"{label}: {name} {st}"


def test_dkdv2w_deterministic(gpu, dkdv2w):
    from SSA.ssa_triton_kernel import ssa_flash_attn_backward, ssa_flash_attn_forward
    from parity_util import make_inputs

    q, k, v, do = make_inputs(2, 8, 4, 640, 128, torch.bfloat16, gpu, "contig")
    n = torch.tensor(1.5, device=gpu)
    b = torch.tensor(0.8, device=gpu)
    runs = []
    for _ in range(2):
        out, m = ssa_flash_attn_forward(q, k, v, 0.088, n, b, causal=True)
        runs.append(ssa_flash_attn_backward(q, k, v, out, do, m, 0.088, n, b, causal=True))
        torch.cuda.synchronize()
    for a, c in zip(runs[0], runs[1]):
        assert torch.equal(a, c)


@pytest.mark.parametrize("ds", [False, True], ids=["recompute", "ds"])
def test_dkdv2w_varlen(gpu, dkdv2w, ds):
    lens, Hq, Hkv, D, causal = (300, 7, 128, 65, 512), 8, 4, 128, True
    q, k, v, do, cu = tv._inputs(lens, Hq, Hkv, D, torch.bfloat16, gpu)
    _, _, _, res, res_k, merr = tv._run(gpu, q, k, v, do, cu, max(lens), causal, ds=ds)
    assert merr < 1e-2
    assert_parity(res, f"dkdv2w varlen ds={int(ds)}")
    assert_parity(res_k, f"dkdv2w varlen ds={int(ds)} [kernel-level]")
