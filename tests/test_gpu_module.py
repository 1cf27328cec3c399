"""SSAAttention (the Megatron-free module) on MI355X.

Mirrors SSATritonAttention.forward (training/train/train_ssa_triton/SSA/
ssa_triton_attention.py:132-202): [S, B, H, D] in, [S, B, Hq * D] out, grads for
q, k, v and the learnable n (and b).  Checked against the fp64 oracle; the
boundary is checked to be copy-free (inputs read through permuted views,
output written in [S, B, H, D] memory order).
"""

from __future__ import annotations

import math
import sys
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import ssa_oracle as so
from parity_util import assert_parity, compare

pytestmark = pytest.mark.gpu


def _np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("learnable_b,dtype", [(False, torch.bfloat16), (True, torch.bfloat16),
                                                (True, torch.float32)])
def test_module_sbhd_matches_oracle(gpu, learnable_b, dtype):
    from SSA.ssa_attention import SSAAttention

    S, B, Hq, Hkv, D = 200, 2, 8, 2, 128
    print(f"[gpu case] module S={S} B={B} Hq={Hq} Hkv={Hkv} learnable_b={learnable_b} {dtype}", file=sys.stderr,
          flush=True)
    g = torch.Generator().manual_seed(7)
    mk = lambda h: (torch.randn(S, B, h, D, generator=g) * 0.5).to(dtype).to(gpu).requires_grad_()
    q, k, v = mk(Hq), mk(Hkv), mk(Hkv)
    mod = SSAAttention(Hq, Hkv, D, learnable_b=learnable_b).to(gpu)
    ctx = mod(q, k, v)
    assert ctx.shape == (S, B, Hq * D) and ctx.is_contiguous()
    dctx = torch.randn(S, B, Hq * D, generator=g).to(dtype).to(gpu)
    ctx.backward(dctx)
    torch.cuda.synchronize()
    perm = lambda t: _np64(t).transpose(1, 2, 0, 3)  # [S,B,H,D] -> [B,H,S,D]
    do = _np64(dctx.view(S, B, Hq, D)).transpose(1, 2, 0, 3)
    ref = so.ssa_forward_backward(perm(q), perm(k), perm(v), do, 1.0 / math.sqrt(D), 1.5, 0.8, True)
    got_out = ctx.view(S, B, Hq, D).permute(1, 2, 0, 3)
    res = compare({"out": got_out, "dq": q.grad.permute(1, 2, 0, 3), "dk": k.grad.permute(1, 2, 0, 3),
                   "dv": v.grad.permute(1, 2, 0, 3)}, ref, scalars=())
    assert_parity(res, "module")
    # n (and b) gradients against the kernel-level oracle of the module's own output
    ref_k = so.ssa_forward_backward(perm(q), perm(k), perm(v), do, 1.0 / math.sqrt(D), 1.5, 0.8, True,
                                    out_for_delta=_np64(got_out))
    atol, rtol = (5e-5, 1e-4) if dtype == torch.float32 else (2e-3, 2e-2)  # check_ssa_triton_parity.py:1066-1069
    assert abs(mod.ssa_n_raw.grad.item() - ref_k["dn"]) <= atol + rtol * abs(ref_k["dn"])
    if learnable_b:
        assert abs(mod.ssa_b_raw.grad.item() - ref_k["db"]) <= atol + rtol * abs(ref_k["db"])


def test_module_boundary_is_copy_free(gpu):
    from SSA import ssa_hip_kernel as hk

    S, B, H, D = 64, 2, 4, 64
    x = torch.randn(S, B, H, D, device=gpu).to(torch.bfloat16)
    view = x.permute(1, 2, 0, 3)
    assert hk._kernel_layout(view) is view  # read in place
    out, _ = hk.ssa_flash_attn_forward(view, view, view, 0.125, torch.tensor(1.5, device=gpu),
                                       torch.tensor(0.8, device=gpu), True)
    assert out.stride() == view.stride()  # written in [S, B, H, D] order
    assert out.permute(2, 0, 1, 3).is_contiguous()


def test_module_packed_sequences(gpu):
    from SSA.ssa_attention import SSAAttention

    lens = [37, 120, 3]
    T, Hq, Hkv, D = sum(lens), 4, 2, 64
    g = torch.Generator().manual_seed(11)
    mk = lambda h: (torch.randn(T, 1, h, D, generator=g) * 0.5).to(torch.bfloat16).to(gpu).requires_grad_()
    q, k, v = mk(Hq), mk(Hkv), mk(Hkv)
    cu = torch.tensor([0, 37, 157, 160], dtype=torch.int32, device=gpu)
    psp = SimpleNamespace(cu_seqlens_q=cu, max_seqlen_q=120)
    mod = SSAAttention(Hq, Hkv, D).to(gpu)
    ctx = mod(q, k, v, packed_seq_params=psp)
    assert ctx.shape == (T, 1, Hq * D)
    ctx.float().sum().backward()
    torch.cuda.synchronize()
    ref = so.ssa_varlen_forward_backward(_np64(q[:, 0]), _np64(k[:, 0]), _np64(v[:, 0]),
                                         np.ones((T, Hq, D)), cu.cpu().numpy(), 1.0 / math.sqrt(D), 1.5, 0.8, True)
    res = compare({"out": ctx.view(T, Hq, D), "dv": v.grad[:, 0]}, ref, names=("out", "dv"), scalars=())
    assert_parity(res, "module packed")


@pytest.mark.parametrize("layer", [1, 6, 12])
def test_module_query_key_layer_scaling(gpu, layer):
    """apply_query_key_layer_scaling divides the softmax scale by the layer
    number (ssa_triton_attention.py:91-97); the reference's module suite runs
    layers 1, 6 and 12 (check_ssa_triton_parity.py:648-759, :1038)."""
    from SSA.ssa_attention import SSAAttention

    S, B, Hq, Hkv, D = 160, 2, 4, 2, 64
    print(f"[gpu case] module layer scaling, layer {layer}", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(100 + layer)
    mk = lambda h: (torch.randn(S, B, h, D, generator=g) * 2.0).to(torch.bfloat16).to(gpu).requires_grad_()
    q, k, v = mk(Hq), mk(Hkv), mk(Hkv)
    mod = SSAAttention(Hq, Hkv, D, layer_number=layer, apply_query_key_layer_scaling=True).to(gpu)
    scale = 1.0 / math.sqrt(D) / layer
    assert mod.softmax_scale == pytest.approx(scale, rel=1e-12)
    ctx = mod(q, k, v)
    dctx = torch.randn(S, B, Hq * D, generator=g).to(torch.bfloat16).to(gpu)
    ctx.backward(dctx)
    torch.cuda.synchronize()
    perm = lambda t: _np64(t).transpose(1, 2, 0, 3)
    do = _np64(dctx.view(S, B, Hq, D)).transpose(1, 2, 0, 3)
    got_out = ctx.view(S, B, Hq, D).permute(1, 2, 0, 3)
    ref = so.ssa_forward_backward(perm(q), perm(k), perm(v), do, scale, 1.5, 0.8, True, out_for_delta=_np64(got_out))
    res = compare({"out": got_out, "dq": q.grad.permute(1, 2, 0, 3), "dk": k.grad.permute(1, 2, 0, 3),
                   "dv": v.grad.permute(1, 2, 0, 3)}, ref, scalars=())
    assert_parity(res, f"module layer {layer}")
    assert abs(mod.ssa_n_raw.grad.item() - ref["dn"]) <= 2e-3 + 2e-2 * abs(ref["dn"])
    if layer > 1:  # the scale really changed the result
        ref1 = so.ssa_forward(perm(q), perm(k), perm(v), 1.0 / math.sqrt(D), 1.5, 0.8, True)[0]
        assert np.abs(ref1 - ref["out"]).max() > 0.1


def test_module_output_dropout(gpu):
    """Dropout is applied to the attention output after the op, never inside
    it (ssa_triton_attention.py:187-193; SSAFlashAttnFunc ignores dropout_p):
    in training every output element is either 0 or the undropped value /
    (1 - p), about a fraction p are 0, and the gradient passes through the same
    mask; in eval mode the output is the undropped one."""
    from SSA.ssa_attention import SSAAttention

    S, B, H, D, p = 128, 2, 4, 64, 0.25
    print("[gpu case] module output dropout", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(5)
    mk = lambda: (torch.randn(S, B, H, D, generator=g) * 0.5).to(torch.bfloat16).to(gpu).requires_grad_()
    q, k, v = mk(), mk(), mk()
    ref_mod = SSAAttention(H, H, D, attention_dropout=0.0).to(gpu)
    mod = SSAAttention(H, H, D, attention_dropout=p).to(gpu)
    base = ref_mod(q, k, v).detach().float()
    torch.manual_seed(0)
    ctx = mod(q, k, v)
    out = ctx.detach().float()
    kept = out != 0
    frac_dropped = 1.0 - kept.float().mean().item()
    assert abs(frac_dropped - p) < 0.02, frac_dropped
    scaled = (base / (1.0 - p)).to(torch.bfloat16).float()
    assert torch.allclose(out[kept], scaled[kept], rtol=1e-2, atol=1e-3)
    ctx.float().sum().backward()
    gv = v.grad.detach().float()
    assert torch.isfinite(gv).all() and gv.abs().sum() > 0
    mod.eval()
    with torch.no_grad():
        ev = mod(q, k, v).float()
    assert torch.equal(ev, base)
