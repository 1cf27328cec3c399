"""PyTorch-eager fp32 SSA oracle on the CPU (autograd backward).

TEST INFRASTRUCTURE ONLY.  Used by ``tests/`` as an independent restatement
(autograd instead of the closed form in ``ssa_oracle.py``) and by ``bench.py``'s
``cpu_baseline`` leg, which times it on the host cores.  The product path never
imports it.

Restates ``training/train/train_ssa_triton/check_ssa_triton_parity.py:169-237``
(``_ssa_reference_forward`` + ``_run_reference_grads``: GQA by
``repeat_interleave``, causal ``triu`` mask, ``t = n sign(s) log1p(b|s|)``,
softmax over t, loss ``sum(out * dout)`` differentiated by autograd with
respect to q, k, v, n and b).  One deliberate difference: the softmax is
max-subtracted, because the reference's ``w / sum(w)`` overflows in fp32 for
trained values of n such as -302 (layer 23 of the production run).
"""

from __future__ import annotations

import torch


def ssa_reference_forward(q, k, v, softmax_scale, ssa_n, ssa_b, causal=True):
    """q [B,Hq,N,D], k/v [B,Hkv,N,D] (any float dtype) -> (out fp32, M fp32 [B,Hq,N], base 2)."""
    bsz, hq, n_ctx, _ = q.shape
    hkv = k.shape[1]
    if hq % hkv != 0:
        raise ValueError(f"HQ={hq} must be divisible by HKV={hkv}")
    g = hq // hkv
    dt = torch.float64 if q.dtype == torch.float64 else torch.float32
    k_exp = k.repeat_interleave(g, dim=1)
    v_exp = v.repeat_interleave(g, dim=1)
    s = torch.matmul(q.to(dt), k_exp.to(dt).transpose(-1, -2)) * float(softmax_scale)
    if causal:
        cm = torch.triu(torch.ones((n_ctx, n_ctx), dtype=torch.bool, device=s.device), diagonal=1)
        s = s.masked_fill(cm.view(1, 1, n_ctx, n_ctx), float("-inf"))
    valid = torch.isfinite(s)
    s_safe = torch.where(valid, s, torch.zeros_like(s))
    t = ssa_n.to(dt) * torch.sign(s_safe) * torch.log1p(ssa_b.to(dt) * s_safe.abs())
    t = torch.where(valid, t, torch.full_like(t, float("-inf")))
    tmax = t.amax(dim=-1, keepdim=True).detach()
    tmax = torch.where(torch.isfinite(tmax), tmax, torch.zeros_like(tmax))
    w = torch.where(valid, torch.exp(t - tmax), torch.zeros_like(t))
    l = w.sum(dim=-1, keepdim=True)
    p = w / l.clamp_min(1e-30)
    out = torch.matmul(p, v_exp.to(dt))
    m = (tmax + torch.log(l)).squeeze(-1) / torch.log(torch.tensor(2.0, dtype=dt))
    return out, m


def run_reference_grads(q, k, v, softmax_scale, ssa_n, ssa_b, dout, causal=True):
    """Forward + autograd backward of loss = sum(out * dout).  Returns a dict of CPU tensors."""
    q_r = q.detach().clone().requires_grad_(True)
    k_r = k.detach().clone().requires_grad_(True)
    v_r = v.detach().clone().requires_grad_(True)
    n_r = ssa_n.detach().clone().requires_grad_(True)
    b_r = ssa_b.detach().clone().requires_grad_(True)
    out_r, m_r = ssa_reference_forward(q_r, k_r, v_r, softmax_scale, n_r, b_r, causal)
    loss = torch.sum(out_r * dout.to(out_r.dtype))
    loss.backward()
    return {
        "out": out_r.detach(),
        "m": m_r.detach(),
        "dq": q_r.grad.detach(),
        "dk": k_r.grad.detach(),
        "dv": v_r.grad.detach(),
        "dn": float(n_r.grad.item()),
        "db": float(b_r.grad.item()),
    }
