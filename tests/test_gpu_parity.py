"""GPU parity: HIP kernels vs the fp64 CPU oracle, through the reference API.

Mirrors the reference kernel suite (training/train/train_ssa_triton/
check_ssa_triton_parity.py:295-504): kernel-level ssa_flash_attn_forward /
ssa_flash_attn_backward on seeded inputs, contiguous and Megatron-strided
layouts, MHA and GQA, causal and non-causal, bf16, fp16 and fp32 (the last
at the reference's fp32 tolerances) -- extended to D in {16, 32, 64, 128},
ragged N, and trained values of n.
"""

from __future__ import annotations

import math
import sys

import pytest
import torch

from parity_util import assert_parity, compare, make_inputs, oracle_fwd_bwd, scale_for

pytestmark = pytest.mark.gpu


def _run(gpu, B, Hq, Hkv, N, D, dtype, causal, layout="contig", n_val=1.5, b_val=0.8, seed=1234, qkv_scale=1.0,
         ds=None):
    """Forward + backward through the reference-named API, checked two ways.

    res_exact -- out, dq, dk, dv against the exact fp64 function of (q, k, v, dO)
                 (dn / db relative errors reported);
    res_kernel -- dq, dk, dv, dn, db against the fp64 kernel-level backward as
                 the reference defines it: a function of the `out` it is handed
                 (delta = rowsum(dO * out), ssa_triton_kernel.py:291-294).
    """
    from SSA.ssa_triton_kernel import ssa_flash_attn_backward, ssa_flash_attn_forward

    label = (f"B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} {str(dtype)[6:]} causal={int(causal)} "
             f"{layout} n={n_val} b={b_val} dq={'default' if ds is None else ('ds' if ds else 'recompute')}")
    print(f"[gpu case] {label}", file=sys.stderr, flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, dtype, gpu, layout, seed, qkv_scale)
    scale = scale_for(D)
    n = torch.tensor(n_val, dtype=torch.float32, device=gpu)
    b = torch.tensor(b_val, dtype=torch.float32, device=gpu)
    out, m = ssa_flash_attn_forward(q, k, v, scale, n, b, causal=causal)
    dq, dk, dv, dn, db = ssa_flash_attn_backward(q, k, v, out, do, m, scale, n, b, causal=causal, ds=ds)
    torch.cuda.synchronize()
    got = {"out": out, "dq": dq, "dk": dk, "dv": dv, "dn": dn.item(), "db": db.item()}
    ref = oracle_fwd_bwd(q, k, v, do, scale, n_val, b_val, causal)
    res_exact = compare(got, ref, names=("out", "dq", "dk", "dv"), scalars=())
    ref_k = oracle_fwd_bwd(q, k, v, do, scale, n_val, b_val, causal, out_for_delta=out)
    res_kernel = compare(got, ref_k, names=("dq", "dk", "dv"))
    mres = (m.float().cpu() - torch.from_numpy(ref["m"]).float()).abs().max().item()
    print(f"[gpu result] {label}: " + ", ".join(
        f"{k_} max_abs={v_['max_abs']:.2e}" if "max_abs" in v_ else f"{k_} rel={v_['rel']:.2e}"
        for k_, v_ in res_exact.items()) + f", m={mres:.1e}, dn/db rel vs exact: "
        f"{abs(dn.item() - ref['dn']) / max(abs(ref['dn']), 1e-12):.2e}/"
        f"{abs(db.item() - ref['db']) / max(abs(ref['db']), 1e-12):.2e}", file=sys.stderr, flush=True)
    return label, res_exact, res_kernel, mres


def _check(label, res_exact, res_kernel, mres):
    assert mres < (1e-4 if "float32" in label else 1e-2), f"{label}: m max abs {mres}"
    assert_parity(res_exact, label + " [exact]")
    assert_parity(res_kernel, label + " [kernel-level]")


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("heads", [(4, 4), (8, 2)])
@pytest.mark.parametrize("dq_path", ["ds", "recompute"])
def test_parity_matrix(gpu, D, dtype, causal, heads, dq_path):
    _check(*_run(gpu, 1, heads[0], heads[1], 256, D, dtype, causal, ds=dq_path == "ds"))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("heads", [(4, 4), (8, 2)])
@pytest.mark.parametrize("N", [7, 256])
def test_parity_head_dim_16(gpu, dtype, causal, heads, N):
    """Head dim 16 (the reference kernel's smallest): zero-padded onto the D = 32 kernels."""
    _check(*_run(gpu, 1, heads[0], heads[1], N, 16, dtype, causal))


@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("heads", [(4, 4), (8, 2)])
@pytest.mark.parametrize("N", [7, 256])
def test_parity_fp32(gpu, D, causal, heads, N):
    """fp32 operands (the reference's fp32 path) on the fp32 vector-ALU kernels,
    at the reference's fp32 tolerances (atol 5e-4, rtol 1e-3; dn / db 5e-5 + 1e-4 |ref|)."""
    _check(*_run(gpu, 1, heads[0], heads[1], N, D, torch.float32, causal))


@pytest.mark.parametrize("N", [1, 129, 511])
@pytest.mark.parametrize("layout", ["contig", "strided"])
def test_parity_fp32_ragged_strided(gpu, N, layout):
    _check(*_run(gpu, 2, 4, 2, N, 64, torch.float32, True, layout=layout))


def test_parity_fp32_trained_n(gpu):
    _check(*_run(gpu, 1, 4, 4, 300, 128, torch.float32, False, n_val=4.0, qkv_scale=0.5))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("heads", [(4, 4), (8, 2)])
@pytest.mark.parametrize("N", [7, 200])
def test_parity_head_dim_256(gpu, dtype, causal, heads, N):
    """Head dim 256 (the largest power of two the reference's Triton tiles take) on the
    fp32-arithmetic vector-ALU kernels: bf16 / fp16 elements widened on load.  N = 200
    fills the first 64-key pass of a 128-key block and part of the second."""
    _check(*_run(gpu, 1, heads[0], heads[1], N, 256, dtype, causal))


@pytest.mark.parametrize("layout", ["contig", "strided"])
@pytest.mark.parametrize("N", [1, 129, 300])
def test_parity_head_dim_256_ragged_strided(gpu, layout, N):
    """Batch 2, GQA, Megatron-strided inputs; a dS' workspace asked for is ignored there."""
    _check(*_run(gpu, 2, 4, 2, N, 256, torch.bfloat16, True, layout=layout, ds=True))


def test_parity_head_dim_256_trained_n(gpu):
    _check(*_run(gpu, 1, 4, 4, 300, 256, torch.float16, False, n_val=-3.484375, qkv_scale=0.5))


@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("layout", ["contig", "strided"])
def test_delta_direct(gpu, D, dtype, layout):
    """Delta = rowsum(dO * O) (ssa_triton_kernel.py:267-298) from ssa_bwd_preprocess against
    the fp64 row sums of the same (rounded) values: fp32 accumulation over D terms, so
    |err| <= 1e-5 * sum_d |o_d dO_d| + 1e-7."""
    from SSA.ssa_hip_kernel import ssa_bwd_preprocess

    print(f"[gpu case] delta D={D} {dtype} {layout}", file=sys.stderr, flush=True)
    o, _, _, do = make_inputs(2, 3, 3, 300, D, dtype, gpu, layout, seed=99)
    delta = ssa_bwd_preprocess(o, do)
    torch.cuda.synchronize()
    od = o.double().cpu() * do.double().cpu()
    ref, mag = od.sum(-1), od.abs().sum(-1)
    err = (delta.double().cpu() - ref).abs()
    assert delta.shape == (2, 3, 300) and bool((err <= 1e-5 * mag + 1e-7).all()), float((err / (mag + 1e-12)).max())


@pytest.mark.parametrize("D", [8, 512])
def test_unsupported_head_dims_raise(gpu, D):
    from SSA.ssa_triton_kernel import ssa_flash_attn_forward

    q = torch.randn(1, 2, 64, D, dtype=torch.bfloat16, device=gpu)
    n = torch.tensor(1.5, device=gpu)
    with pytest.raises(ValueError):
        ssa_flash_attn_forward(q, q, q, 1.0 / math.sqrt(D), n, n, causal=True)


@pytest.mark.parametrize("N", [1, 7, 64, 129, 200, 511])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dq_path", ["ds", "recompute"])
def test_parity_ragged_lengths(gpu, N, D, causal, dq_path):
    _check(*_run(gpu, 2, 4, 2, N, D, torch.bfloat16, causal, ds=dq_path == "ds"))


@pytest.mark.parametrize("layout", ["contig", "strided"])
@pytest.mark.parametrize("causal", [True, False])
def test_parity_layouts(gpu, layout, causal):
    _check(*_run(gpu, 2, 8, 4, 384, 128, torch.bfloat16, causal, layout=layout))


@pytest.mark.parametrize("n_val", [4.0, -3.484375, 0.0])
def test_parity_trained_n(gpu, n_val):
    # trained values of n from the production run (layers 0..23)
    _check(*_run(gpu, 1, 4, 4, 256, 128, torch.bfloat16, True, n_val=n_val, qkv_scale=0.5))


def test_parity_divergent_layer_n_m302(gpu):
    # n = -302 (the divergent layer 23): rows of P are near one-hot, dS is
    # amplified by n b = -241 and the sums dS K cancel, so elementwise bounds
    # on dq / dk do not apply to any bf16 kernel; the bar here is normwise:
    # rel-RMSE <= 1e-2 for every gradient, elementwise for out, finite dn / db.
    label, res_exact, res_kernel, mres = _run(gpu, 1, 4, 4, 256, 128, torch.bfloat16, True,
                                              n_val=-302.0, qkv_scale=0.5)
    assert mres < 1e-2
    assert_parity({"out": res_exact["out"]}, label)
    for name in ("dq", "dk", "dv"):
        st = res_kernel[name]
        assert st["finite"] and st["rel_rmse"] <= 1e-2, f"{label}: {name} {st}"
    assert math.isfinite(res_kernel["dn"]["got"]) and math.isfinite(res_kernel["db"]["got"])


def test_parity_baseline_distribution(gpu):
    # BASELINE.json config distribution: Q/K/V = 0.5 N(0,1), dO ~ N(0,1)
    _check(*_run(gpu, 1, 4, 4, 1024, 128, torch.bfloat16, True, qkv_scale=0.5))


def test_determinism_bitwise(gpu):
    from SSA.ssa_triton_kernel import ssa_flash_attn_backward, ssa_flash_attn_forward

    for layout in ("contig", "strided"):
        q, k, v, do = make_inputs(2, 8, 4, 640, 128, torch.bfloat16, gpu, layout)
        n = torch.tensor(1.5, device=gpu)
        b = torch.tensor(0.8, device=gpu)
        runs = []
        for _ in range(2):
            out, m = ssa_flash_attn_forward(q, k, v, 0.088, n, b, causal=True)
            grads = ssa_flash_attn_backward(q, k, v, out, do, m, 0.088, n, b, causal=True)
            torch.cuda.synchronize()
            runs.append((out, m) + tuple(grads))
        for a, c in zip(runs[0], runs[1]):
            assert torch.equal(a, c), f"non-deterministic result ({layout})"


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("ds", [True, False], ids=["ds", "recompute"])
def test_whole_backward_equals_its_stages_bitwise(gpu, D, ds):
    """ssa_bwd (on the workspace path the dQ pass also sums dn / db) against the
    four staged entry points, ssa_bwd_preprocess / _dkdv / _dq / _reduce, on the
    same arguments: every output bit for bit."""
    from SSA.ssa_hip_kernel import BackwardLaunch, ssa_flash_attn_forward

    print(f"[gpu case] whole vs staged backward D={D} ds={ds}", file=sys.stderr, flush=True)
    q, k, v, do = make_inputs(2, 8, 2, 700, D, torch.bfloat16, gpu, "contig", 77, 0.5)
    n = torch.tensor(1.5, device=gpu)
    b = torch.tensor(0.8, device=gpu)
    out, m = ssa_flash_attn_forward(q, k, v, scale_for(D), n, b, True)
    whole = BackwardLaunch(q, k, v, out, do, m, scale_for(D), n, b, True, ds=ds)
    staged = BackwardLaunch(q, k, v, out, do, m, scale_for(D), n, b, True, ds=ds)
    for t in whole.results() + staged.results():
        t.fill_(float("nan"))
    whole.run()
    for stage in BackwardLaunch.STAGES:
        staged.run_stage(stage)
    torch.cuda.synchronize()
    for name, a, c in zip(("dq", "dk", "dv", "dn", "db"), whole.results(), staged.results()):
        assert torch.equal(a, c), f"D={D} ds={ds}: {name} of ssa_bwd differs from the staged backward"
    assert torch.isfinite(whole.dn) and torch.isfinite(whole.db)


@pytest.mark.parametrize("ds", [True, False], ids=["ds", "recompute"])
def test_dkdv_wide_row_range_bitwise(gpu, ds):
    """dK/dV addresses a workgroup's Q / dO rows with 32-bit offsets when they
    lie within 2 GiB of the workgroup's first q-head, and with 64-bit
    arithmetic otherwise.  A q view whose two heads (one kv-head, G = 2) lie
    2 GiB apart takes the second path; its gradients must equal, bit for bit,
    those of the same values in a contiguous q (the first path): only the
    addressing differs."""
    from SSA.ssa_triton_kernel import ssa_flash_attn_backward, ssa_flash_attn_forward

    print(f"[gpu case] dK/dV 64-bit row range ds={int(ds)}", file=sys.stderr, flush=True)
    N, D, step = 256, 128, 1 << 15  # head stride 2**30 elements = 2 GiB of bf16
    g = torch.Generator().manual_seed(5)
    vals = (torch.randn(1, 2, N, D, generator=g) * 0.5).to(torch.bfloat16)
    k = (torch.randn(1, 1, N, D, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    v = (torch.randn(1, 1, N, D, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    do = torch.randn(1, 2, N, D, generator=g).to(torch.bfloat16).to(gpu)
    big = torch.empty(1, step + 1, N, D, device=gpu, dtype=torch.bfloat16)  # 2.1 GB
    q_wide = big[:, ::step]
    q_wide.copy_(vals.to(gpu))
    assert q_wide.stride(1) == 1 << 30
    q = q_wide.contiguous()
    n = torch.tensor(1.5, device=gpu)
    b = torch.tensor(0.8, device=gpu)
    s = 1.0 / math.sqrt(D)
    out, m = ssa_flash_attn_forward(q, k, v, s, n, b, causal=True)
    wide = ssa_flash_attn_backward(q_wide, k, v, out, do, m, s, n, b, causal=True, ds=ds)
    dense = ssa_flash_attn_backward(q, k, v, out, do, m, s, n, b, causal=True, ds=ds)
    torch.cuda.synchronize()
    for a, c in zip(wide, dense):
        assert torch.equal(a, c)
    del big, q_wide
    torch.cuda.empty_cache()
