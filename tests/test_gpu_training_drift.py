"""Training drift: 80 AdamW steps through the HIP kernels against the same
steps through the fp32 oracle.

Mirrors the reference's training-drift suite
(training/train/train_ssa_triton/check_ssa_triton_parity.py:786-960): free
fp32 leaves q, k, v ~ 0.05 N(0,1) and a learnable n (init 1.5, b = 0.8 fixed),
cast to bf16 for the attention op, loss = MSE(out, target) with target ~
N(0,1), AdamW(lr 1e-3, betas (0.9, 0.99), no weight decay), causal.  The
oracle engine is the fp32 torch restatement (oracle/ssa_oracle_torch.py)
computed from the same bf16-cast inputs, its output rounded to bf16 as the
reference's ``_ssa_reference_forward`` returns it (:169-206, :761-782).
Pass bar, the reference's own (:1054-1057): at every step
|loss_kernel - loss_oracle| <= 6e-3 and max |param_kernel - param_oracle|
<= 3e-2 over q, k, v and n.  A systematic bias in dn (or in any gradient)
accumulates over the steps, which single-step parity cannot see.
"""

from __future__ import annotations

import math
import sys

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

LOSS_TOL, PARAM_TOL = 6e-3, 3e-2
STEPS = 80

CASES = [
    # B, Hq, Hkv, N, D: the reference's defaults (:1035-1040), then head dim 128
    (2, 24, 8, 128, 32),
    (2, 8, 4, 256, 128),
]


@pytest.mark.parametrize("B,Hq,Hkv,N,D", CASES, ids=[f"b{c[0]}_h{c[1]}x{c[2]}_n{c[3]}_d{c[4]}" for c in CASES])
def test_training_drift_matches_oracle(gpu, B, Hq, Hkv, N, D):
    from oracle.ssa_oracle_torch import ssa_reference_forward
    from SSA.ssa_flash_attention import ssa_flash_attention

    label = f"drift B={B} Hq={Hq} Hkv={Hkv} N={N} D={D}"
    print(f"[gpu case] {label}", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(1234)
    init = {
        "q": torch.randn(B, Hq, N, D, generator=g) * 0.05,
        "k": torch.randn(B, Hkv, N, D, generator=g) * 0.05,
        "v": torch.randn(B, Hkv, N, D, generator=g) * 0.05,
        "n": torch.tensor(1.5),
    }
    target = torch.randn(B, Hq, N, D, generator=g).to(gpu)
    b = torch.tensor(0.8, device=gpu)
    scale = 1.0 / math.sqrt(D)
    params = {eng: {k_: torch.nn.Parameter(v_.clone().to(gpu)) for k_, v_ in init.items()}
              for eng in ("kernel", "oracle")}
    opts = {eng: torch.optim.AdamW(list(p.values()), lr=1e-3, betas=(0.9, 0.99), weight_decay=0.0)
            for eng, p in params.items()}

    def forward(eng):
        p = params[eng]
        qd, kd, vd = (p[x].to(torch.bfloat16) for x in ("q", "k", "v"))
        if eng == "kernel":
            return ssa_flash_attention(qd, kd, vd, scale, p["n"], b, causal=True)
        out, _ = ssa_reference_forward(qd, kd, vd, scale, p["n"], b, causal=True)
        return out.to(torch.bfloat16)

    worst_loss = worst_param = 0.0
    for step in range(1, STEPS + 1):
        losses = {}
        for eng in ("kernel", "oracle"):
            opts[eng].zero_grad(set_to_none=True)
            loss = F.mse_loss(forward(eng).float(), target)
            assert torch.isfinite(loss), f"{label}: non-finite {eng} loss at step {step}"
            loss.backward()
            opts[eng].step()
            losses[eng] = loss.item()
        worst_loss = max(worst_loss, abs(losses["kernel"] - losses["oracle"]))
        pdiff = max(float((params["kernel"][x].detach() - params["oracle"][x].detach()).abs().max())
                    for x in ("q", "k", "v", "n"))
        worst_param = max(worst_param, pdiff)
        if step == 1 or step % 20 == 0:
            print(f"[gpu result] {label} step {step}: loss {losses['kernel']:.6f} vs {losses['oracle']:.6f}, "
                  f"param diff {pdiff:.2e}, n {params['kernel']['n'].item():.5f} vs "
                  f"{params['oracle']['n'].item():.5f}", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    # n must actually move under training (its gradient is exercised)
    assert abs(params["kernel"]["n"].item() - 1.5) > 1e-3, label
    assert worst_loss <= LOSS_TOL, f"{label}: worst loss diff {worst_loss:.3e} > {LOSS_TOL}"
    assert worst_param <= PARAM_TOL, f"{label}: worst param diff {worst_param:.3e} > {PARAM_TOL}"
