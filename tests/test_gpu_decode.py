"""GPU parity of the decode step (one new token per sequence against a KV cache).

The reference has no decode kernel: its generation loop re-runs the whole
prefix through the forward for every token
(training/train/train_ssa_triton/generate_triton.py:315-331), so the result a
decode step must reproduce is the last row of the causal forward over the
cached prefix.  The oracle states exactly that (oracle/ssa_oracle.py
``ssa_decode``, pinned in tests/test_oracle.py against the causal forward).
Checked here to the bar of parity_util (max(2e-2, 1 ulp) absolute plus
allclose at 2e-2 / 5e-2) for the output, and |dm| <= 1e-3 (1 + |m|) for the
base-2 normaliser; cases cover ragged and empty caches, GQA groups wider than
the 32-column MFMA tile, every head dim, forced and automatic key splits,
strided caches and negative n.  Also: decode equals this library's own causal
forward on the prefix, results are bitwise reproducible, and the module's
cached generation equals re-running the prefix (what the reference does).
"""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
import torch

from oracle import ssa_oracle as so
from parity_util import assert_parity, compare

pytestmark = pytest.mark.gpu


def _np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _case(dev, B, Hq, Hkv, cap, D, dtype, seed=1234, layout="bhsd"):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, Hq, D, generator=g) * 0.5).to(dtype).to(dev)
    if layout == "bhsd":
        kc = (torch.randn(B, Hkv, cap, D, generator=g) * 0.5).to(dtype).to(dev)
        vc = (torch.randn(B, Hkv, cap, D, generator=g) * 0.5).to(dtype).to(dev)
    else:  # [B, cap, Hkv, D] memory viewed as [B, Hkv, cap, D]
        kc = (torch.randn(B, cap, Hkv, D, generator=g) * 0.5).to(dtype).to(dev).transpose(1, 2)
        vc = (torch.randn(B, cap, Hkv, D, generator=g) * 0.5).to(dtype).to(dev).transpose(1, 2)
    return q, kc, vc


def _check(dev, q, kc, vc, lens, n_val=1.5, b_val=0.8, num_splits=0, label=""):
    from SSA.ssa_hip_kernel import ssa_decode_attention

    D = q.shape[-1]
    scale = 1.0 / math.sqrt(D)
    n = torch.tensor(n_val, device=dev)
    b = torch.tensor(b_val, device=dev)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=dev)
    out, m = ssa_decode_attention(q, kc, vc, lens_t, scale, n, b, num_splits=num_splits, return_m=True)
    torch.cuda.synchronize()
    ref_out, ref_m = so.ssa_decode(_np64(q), _np64(kc), _np64(vc), lens, scale, n_val, b_val)
    res = compare({"out": out}, {"out": ref_out}, scalars=())
    assert_parity(res, label)
    got_m = m.cpu().double().numpy()
    empty = np.isneginf(ref_m)
    assert np.array_equal(np.isneginf(got_m), empty), f"{label}: m -inf pattern"
    dm = np.abs(got_m[~empty] - ref_m[~empty])
    assert np.all(dm <= 1e-3 * (1 + np.abs(ref_m[~empty]))), f"{label}: m err {dm.max() if dm.size else 0}"
    return out, m


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize(
    "B,Hq,Hkv,cap,lens,splits",
    [
        (3, 8, 8, 300, [300, 1, 157], 0),
        (2, 8, 2, 1024, [1000, 33], 0),
        (2, 8, 2, 1024, [1000, 33], 1),
        (2, 8, 2, 1024, [1024, 640], 5),
        (4, 16, 1, 96, [0, 96, 95, 64], 0),      # empty cache, exact fits, one split
        (1, 64, 1, 200, [190], 3),               # GQA 64: two 32-wide q-head groups
        (2, 6, 3, 37, [37, 20], 0),              # ragged group (G = 2) and short cache
    ],
)
def test_decode_matches_oracle(gpu, D, B, Hq, Hkv, cap, lens, splits):
    label = f"decode D={D} B={B} Hq={Hq} Hkv={Hkv} cap={cap} lens={lens} splits={splits}"
    print(f"[gpu case] {label}", file=sys.stderr, flush=True)
    q, kc, vc = _case(gpu, B, Hq, Hkv, cap, D, torch.bfloat16)
    _check(gpu, q, kc, vc, lens, num_splits=splits, label=label)


@pytest.mark.parametrize("B,Hq,Hkv,cap,D", [(16, 16, 16, 4096, 128), (16, 32, 8, 4096, 64)],
                         ids=["decode_s4096", "decode_gqa_d64"])
def test_decode_full_size(gpu, B, Hq, Hkv, cap, D):
    """The benchmark's decode steps at full size (every cache full at 4096
    keys, the default splits) against the oracle on every head."""
    label = f"decode full size B={B} Hq={Hq} Hkv={Hkv} cap={cap} D={D}"
    print(f"[gpu case] {label}", file=sys.stderr, flush=True)
    q, kc, vc = _case(gpu, B, Hq, Hkv, cap, D, torch.bfloat16)
    _check(gpu, q, kc, vc, [cap] * B, label=label)


@pytest.mark.parametrize("n_val", [0.0, -3.484375, -302.0, 5.0])
def test_decode_scalars(gpu, n_val):
    label = f"decode n={n_val}"
    print(f"[gpu case] {label}", file=sys.stderr, flush=True)
    q, kc, vc = _case(gpu, 2, 8, 4, 700, 128, torch.bfloat16, seed=5)
    _check(gpu, q, kc, vc, [700, 411], n_val=n_val, label=label)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_fp16_and_strided_cache(gpu, dtype):
    label = f"decode {dtype} strided"
    print(f"[gpu case] {label}", file=sys.stderr, flush=True)
    q, kc, vc = _case(gpu, 3, 16, 4, 513, 64, dtype, seed=11, layout="bshd")
    assert not kc.is_contiguous()
    _check(gpu, q, kc, vc, [513, 2, 300], label=label)


def test_decode_clamps_lengths_past_capacity(gpu):
    q, kc, vc = _case(gpu, 2, 4, 4, 64, 64, torch.bfloat16, seed=3)
    out_big, m_big = _check(gpu, q, kc, vc, [1000, 64], label="len > cap")
    # the oracle clamps the same way; equal to an explicit full-cache length
    out_cap, m_cap = _check(gpu, q, kc, vc, [64, 64], label="len = cap")
    assert torch.equal(out_big, out_cap) and torch.equal(m_big, m_cap)


def test_decode_equals_own_forward_last_row(gpu):
    """Decode over a prefix of length L equals the last row of this library's
    causal forward over the same L rows (same math, different summation order,
    so checked to the parity bar, not bitwise)."""
    from SSA.ssa_hip_kernel import ssa_decode_attention, ssa_flash_attn_forward

    B, Hq, Hkv, L, D = 2, 16, 4, 777, 128
    print(f"[gpu case] decode vs forward L={L}", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(21)
    q = (torch.randn(B, Hq, L, D, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    k = (torch.randn(B, Hkv, L, D, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    v = (torch.randn(B, Hkv, L, D, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    n = torch.tensor(1.5, device=gpu)
    b = torch.tensor(0.8, device=gpu)
    scale = 1.0 / math.sqrt(D)
    fo, fm = ssa_flash_attn_forward(q, k, v, scale, n, b, causal=True)
    lens = torch.full((B,), L, dtype=torch.int32, device=gpu)
    do, dm = ssa_decode_attention(q[:, :, L - 1], k, v, lens, scale, n, b, return_m=True)
    torch.cuda.synchronize()
    assert (do.float() - fo[:, :, L - 1].float()).abs().max().item() <= 2e-2
    assert (dm - fm[:, :, L - 1]).abs().max().item() <= 1e-3


def test_decode_bitwise_reproducible(gpu):
    from SSA.ssa_hip_kernel import ssa_decode_attention

    q, kc, vc = _case(gpu, 4, 16, 16, 2048, 128, torch.bfloat16, seed=8)
    lens = torch.tensor([2048, 1500, 7, 999], dtype=torch.int32, device=gpu)
    n = torch.tensor(1.5, device=gpu)
    b = torch.tensor(0.8, device=gpu)
    r1 = ssa_decode_attention(q, kc, vc, lens, 0.088, n, b, return_m=True)
    r2 = ssa_decode_attention(q, kc, vc, lens, 0.088, n, b, return_m=True)
    torch.cuda.synchronize()
    assert torch.equal(r1[0], r2[0]) and torch.equal(r1[1], r2[1])


def test_decode_rejects_cache_layouts_it_cannot_read(gpu):
    from SSA.ssa_hip_kernel import ssa_decode_attention

    q, kc, vc = _case(gpu, 1, 4, 4, 64, 64, torch.bfloat16)
    lens = torch.tensor([10], dtype=torch.int32, device=gpu)
    padded = torch.zeros(1, 4, 64, 68, dtype=torch.bfloat16, device=gpu)[..., :64]  # row stride 68
    with pytest.raises(ValueError, match="k_cache"):
        ssa_decode_attention(q, padded, vc, lens, 0.1, 1.5, 0.8)
    with pytest.raises(ValueError, match="v_cache"):  # head dim not contiguous
        ssa_decode_attention(q, kc, vc.transpose(2, 3).contiguous().transpose(2, 3), lens, 0.1, 1.5, 0.8)


def test_module_cached_generation_equals_prefix_recompute(gpu):
    """SSAKVCache + forward_decode for a prompt and a few generated tokens
    equals running the module's full causal forward over the whole prefix at
    every step (the reference's generation loop), token by token."""
    from SSA.ssa_attention import SSAAttention, SSAKVCache

    B, Hq, Hkv, D, P, steps = 2, 8, 2, 128, 45, 6
    print(f"[gpu case] module generation P={P} steps={steps}", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(31)
    T = P + steps
    mk = lambda h: (torch.randn(T, B, h, D, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    q, k, v = mk(Hq), mk(Hkv), mk(Hkv)
    mod = SSAAttention(Hq, Hkv, D).to(gpu).eval()
    cache = SSAKVCache(B, Hkv, 128, D, torch.bfloat16, gpu)
    with torch.no_grad():
        ctx_p = mod(q[:P], k[:P], v[:P])  # prompt: dense causal forward
        cache.append(k[:P].permute(1, 2, 0, 3), v[:P].permute(1, 2, 0, 3))
        full = mod(q, k, v)
        assert (ctx_p.float() - full[:P].float()).abs().max().item() <= 2e-2
        for t in range(P, T):
            ctx_t = mod.forward_decode(q[t : t + 1], k[t : t + 1], v[t : t + 1], cache)
            assert ctx_t.shape == (1, B, Hq * D)
            err = (ctx_t.float() - full[t : t + 1].float()).abs().max().item()
            assert err <= 2e-2, f"step {t}: {err}"
    torch.cuda.synchronize()
    assert cache.seqlens.tolist() == [T] * B
