"""The Llama-style SSA decoder (SSA/ssa_decoder.py) on MI355X.

The decoder wires SSAAttention into the reference's SSA GPT layer
(training/train/train_ssa_triton/SSA/ssa_triton_layer_specs.py:96-127).  Its
attention is checked by swapping the core op for the fp32 torch oracle
(oracle/ssa_oracle_torch.py, computed from the same bf16 q / k / v) in an
otherwise identical model: logits, loss and gradients must agree to
bf16-level relative error (||a - b|| / ||b|| <= 2e-2 for logits, <= 5e-2 for
gradients, |d loss| <= 1e-2), which catches a wrong head grouping, RoPE
placement, causal direction or layout at the op boundary.  Also: training
steps lower the loss on a fixed batch and move n, and cached generation
(decode kernel) gives the logits of re-running the full prefix at every step,
as the reference's generation loop does.
"""

from __future__ import annotations

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def _tiny(gqa: bool):
    from SSA.ssa_decoder import SSADecoderConfig

    return SSADecoderConfig(num_layers=2, hidden_size=256, num_attention_heads=4,
                            num_query_groups=2 if gqa else 4, kv_channels=64, ffn_hidden_size=512,
                            vocab_size=512, seq_length=256, init_std=0.05)


def _rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-12)).item()


@pytest.mark.parametrize("gqa", [False, True])
def test_decoder_attention_matches_oracle(gpu, gqa, monkeypatch):
    import SSA.ssa_attention as sa
    from SSA.ssa_decoder import SSADecoder
    from oracle.ssa_oracle_torch import ssa_reference_forward

    print(f"[gpu case] decoder vs oracle attention gqa={gqa}", file=sys.stderr, flush=True)
    torch.manual_seed(0)
    cfg = _tiny(gqa)
    model = SSADecoder(cfg).to(gpu)
    ids = torch.randint(0, cfg.vocab_size, (2, 200), device=gpu)
    labels = torch.randint(0, cfg.vocab_size, (2, 200), device=gpu)

    def run():
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = model(ids)
            loss = torch.nn.functional.cross_entropy(logits.float().view(-1, cfg.vocab_size), labels.t().reshape(-1))
        loss.backward()
        grads = {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}
        return logits.detach(), loss.detach(), grads

    logits, loss, grads = run()

    def oracle_op(q, k, v, scale, n, b, causal=True, dropout_p=0.0, training=True):
        with torch.autocast("cuda", enabled=False):  # fp32 products, no bf16 batched matmuls
            out, _ = ssa_reference_forward(q.float(), k.float(), v.float(), scale, n.float(), b.float(), causal)
        return out.to(q.dtype)

    monkeypatch.setattr(sa, "ssa_flash_attention", oracle_op)
    r_logits, r_loss, r_grads = run()
    torch.cuda.synchronize()
    assert torch.isfinite(logits).all()
    assert _rel(logits, r_logits) <= 2e-2, _rel(logits, r_logits)
    assert abs(loss.item() - r_loss.item()) <= 1e-2
    assert set(grads) == set(r_grads)
    for name in grads:
        if name.endswith("ssa_n_raw"):
            g, r = grads[name].item(), r_grads[name].item()
            assert abs(g - r) <= 5e-2 * abs(r) + 1e-4, (name, g, r)
        else:
            assert _rel(grads[name], r_grads[name]) <= 5e-2, (name, _rel(grads[name], r_grads[name]))


def test_decoder_train_steps_lower_the_loss(gpu):
    from SSA.ssa_decoder import SSADecoder, train_step

    print("[gpu case] decoder train steps", file=sys.stderr, flush=True)
    torch.manual_seed(1)
    cfg = _tiny(True)
    model = SSADecoder(cfg).to(gpu)
    opt = torch.optim.AdamW(model.parameters(), lr=3e-3)
    ids = torch.randint(0, cfg.vocab_size, (2, 128), device=gpu)
    labels = torch.roll(ids, -1, dims=1)
    n0 = [l.self_attention.core_attention.ssa_n_raw.item() for l in model.layers]
    losses = [train_step(model, opt, ids, labels).item() for _ in range(60)]
    torch.cuda.synchronize()
    assert all(torch.isfinite(torch.tensor(losses)))
    assert losses[-1] < 0.5 * losses[0], losses
    n1 = [l.self_attention.core_attention.ssa_n_raw.item() for l in model.layers]
    assert all(a != b for a, b in zip(n0, n1))  # n is learned


def test_decoder_cached_generation_equals_prefix_recompute(gpu):
    from SSA.ssa_decoder import SSADecoder

    print("[gpu case] decoder generation", file=sys.stderr, flush=True)
    torch.manual_seed(2)
    cfg = _tiny(True)
    model = SSADecoder(cfg).to(gpu).eval()
    prompt = torch.randint(0, cfg.vocab_size, (2, 37), device=gpu)
    steps = 8
    tokens, step_logits = model.generate(prompt, steps)
    assert tokens.shape == (2, 37 + steps)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        for t in range(steps):
            full = model(tokens[:, : 37 + t])[-1].float()  # the whole prefix, as the reference re-runs it
            assert _rel(step_logits[t], full) <= 2e-2, (t, _rel(step_logits[t], full))
    torch.cuda.synchronize()


def test_decoder_full_size_train_steps(gpu):
    """BASELINE.json configs[4] at its real size: ``SSADecoderConfig()`` (24
    layers, hidden 2048, 16 x 128 heads, SwiGLU 5632, vocab 65536), micro-batch
    4 x 4096 tokens, three ``train_step`` calls with fused AdamW (the layer
    order of ssa_triton_layer_specs.py:96-127).  The first loss is
    ln 65536 + init_std^2 * hidden / 2 (Gaussian logits at init), losses and every gradient are
    finite, every layer's n moves, and one head of one layer's attention output
    (captured at the op boundary during the first step) equals the fp64 oracle
    of that head's own q / k / v, as the kernels' full-size tests check it."""
    import math as _math

    import numpy as np

    from oracle import ssa_oracle as so
    from parity_util import assert_parity, compare
    from SSA.ssa_decoder import SSADecoder, SSADecoderConfig, train_step

    cfg = SSADecoderConfig()
    B, S = 4, cfg.seq_length
    print(f"[gpu case] decoder full size: {cfg.num_layers} layers, hidden {cfg.hidden_size}, vocab "
          f"{cfg.vocab_size}, {B} x {S} tokens", file=sys.stderr, flush=True)
    torch.manual_seed(3)
    model = SSADecoder(cfg).to(gpu)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, fused=True)
    ids = torch.randint(0, cfg.vocab_size, (B, S), device=gpu)
    labels = torch.randint(0, cfg.vocab_size, (B, S), device=gpu)
    layer_i, bi, h = 11, 2, 7
    core = model.layers[layer_i].self_attention.core_attention
    seen = {}

    def hook(mod, args, out):
        if "q" not in seen:
            seen.update(q=args[0].detach().clone(), k=args[1].detach().clone(), v=args[2].detach().clone(),
                        out=out.detach().clone())

    handle = core.register_forward_hook(hook)
    n0 = [l.self_attention.core_attention.ssa_n_raw.item() for l in model.layers]
    losses = []
    for step in range(3):
        losses.append(train_step(model, opt, ids, labels).item())
        bad = [n_ for n_, p_ in model.named_parameters() if p_.grad is not None and not torch.isfinite(p_.grad).all()]
        assert not bad, f"step {step}: non-finite gradients in {bad[:5]}"
        print(f"[gpu result] decoder full size step {step}: loss {losses[-1]:.4f}", file=sys.stderr, flush=True)
    handle.remove()
    torch.cuda.synchronize()
    assert all(_math.isfinite(x) for x in losses), losses
    # Gaussian logits at init (variance init_std^2 * hidden after the final
    # RMSNorm): the expected cross-entropy is ln V + var / 2
    expect0 = _math.log(cfg.vocab_size) + cfg.init_std ** 2 * cfg.hidden_size / 2
    assert abs(losses[0] - expect0) < 0.1, (losses[0], expect0)
    n1 = [l.self_attention.core_attention.ssa_n_raw.item() for l in model.layers]
    assert all(a != b for a, b in zip(n0, n1)), "n did not move in every layer"

    # one head of the captured attention call against the oracle
    D = cfg.kv_channels
    G = cfg.num_attention_heads // cfg.num_query_groups
    q = seen["q"][:, bi, h].float().cpu().numpy().astype(np.float64)[None, None]          # [1, 1, S, D]
    k = seen["k"][:, bi, h // G].float().cpu().numpy().astype(np.float64)[None, None]
    v = seen["v"][:, bi, h // G].float().cpu().numpy().astype(np.float64)[None, None]
    out = seen["out"].view(S, B, cfg.num_attention_heads, D)[:, bi, h][None, None]      # [1, 1, S, D]
    ref = so.ssa_forward_backward_chunked(q, k, v, np.zeros_like(q), core.softmax_scale, n0[layer_i],
                                          cfg.ssa_b, True)
    res = compare({"out": out}, ref, names=("out",), scalars=())
    print(f"[gpu result] decoder full size layer {layer_i + 1} head {h}: out max_abs "
          f"{res['out']['max_abs']:.2e}", file=sys.stderr, flush=True)
    assert_parity(res, "decoder full size attention head")


@pytest.mark.parametrize("D,dtype", [(128, torch.bfloat16), (64, torch.bfloat16), (128, torch.float16)])
def test_fused_rope_matches_torch(gpu, D, dtype):
    """ssa_rope (FusedRoPE) against the PyTorch rotate-half form in fp32, on a
    strided view like the k slice of the fused QKV output, forward and
    backward: within one unit in the last place of the dtype."""
    from SSA.ssa_decoder import FusedRoPE, apply_rope, rope_tables

    print(f"[gpu case] fused RoPE D={D} {dtype}", file=sys.stderr, flush=True)
    torch.manual_seed(3)
    S, B, H = 300, 2, 3
    base = torch.randn(S, B, H, 3 * D, device=gpu).to(dtype)
    x = base[..., D:2 * D]  # strided [S, B, H, D] view
    cos, sin = rope_tables(torch.arange(7, 7 + S, device=gpu), D, 10000.0)
    cos_h, sin_h = cos[:, 0, 0, :D // 2].contiguous(), sin[:, 0, 0, :D // 2].contiguous()
    xa = x.detach().clone().requires_grad_(True)
    xb = x.detach().clone().requires_grad_(True)
    ya = FusedRoPE.apply(xa, cos_h, sin_h)
    yb = apply_rope(xb.float(), cos, sin)  # fp32 reference
    w = torch.randn_like(yb)
    (ya.float() * w).sum().backward()
    (yb * w).sum().backward()
    torch.cuda.synchronize()
    # error bound per rotated pair (i, i + D/2): a rotation keeps the pair's
    # norm, and both sides round inputs or outputs to the dtype once
    tol = 2.0 ** (-8 if dtype == torch.bfloat16 else -11)

    def pair_norm(t):
        t1, t2 = t.chunk(2, dim=-1)
        r = torch.sqrt(t1 * t1 + t2 * t2)
        return torch.cat([r, r], dim=-1)

    assert ((ya.float() - yb).abs() <= tol * pair_norm(yb) + 1e-6).all()
    ga, gb = xa.grad.float(), xb.grad.float()
    assert ((ga - gb).abs() <= 2 * tol * pair_norm(gb) + 1e-6).all()


def test_decoder_fused_ops_equal_torch_ops(gpu):
    """The same decoder with the fused RoPE, RMSNorm and SwiGLU kernels and with
    the PyTorch forms: logits and gradients agree to bf16-level relative error."""
    import dataclasses

    from SSA.ssa_decoder import SSADecoder

    print("[gpu case] decoder fused vs torch RoPE / RMSNorm", file=sys.stderr, flush=True)
    torch.manual_seed(4)
    cfg = _tiny(True)
    model = SSADecoder(cfg).to(gpu)
    ids = torch.randint(0, cfg.vocab_size, (2, 160), device=gpu)
    labels = torch.randint(0, cfg.vocab_size, (2, 160), device=gpu)

    def run(fused):
        model.cfg = dataclasses.replace(cfg, fused_rope=fused)
        for mod in model.modules():
            if hasattr(mod, "fused"):
                mod.fused = fused  # RMSNorm, MLP (SwiGLU)
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = model(ids)
            loss = torch.nn.functional.cross_entropy(logits.float().view(-1, cfg.vocab_size), labels.t().reshape(-1))
        loss.backward()
        return logits.detach(), {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}

    la, ga = run(True)
    lb, gb = run(False)
    torch.cuda.synchronize()
    assert _rel(la, lb) <= 1e-2, _rel(la, lb)
    for name in ga:
        assert _rel(ga[name], gb[name]) <= 3e-2, (name, _rel(ga[name], gb[name]))


@pytest.mark.parametrize("H", [2048, 1000, 4096])
@pytest.mark.parametrize("autocast", [True, False])
def test_fused_rmsnorm_matches_torch(gpu, autocast, H):
    """ssa_rmsnorm_fwd / _bwd against the PyTorch form in fp32: the output in
    the autocast dtype (bf16) or fp32, dx and the weight gradient (a sum over
    all rows, reduced in a fixed order)."""
    from SSA.ssa_decoder import RMSNorm

    print(f"[gpu case] fused RMSNorm autocast={autocast} H={H}", file=sys.stderr, flush=True)
    torch.manual_seed(5)
    S, B = 513, 3
    norm = RMSNorm(H, 1e-5).to(gpu)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * torch.randn(H, device=gpu))
    x = torch.randn(S, B, H, device=gpu) * 3
    up = torch.randn(S, B, H, device=gpu)
    xa = x.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        ya = norm(xa)
    (ya.float() * up).sum().backward()
    ga_x, ga_w = xa.grad.clone(), norm.weight.grad.clone()
    norm.weight.grad = None
    xb = x.clone().requires_grad_(True)
    yb = norm.reference(xb)
    dy = up.to(ya.dtype).float()  # the upstream gradient as the fused backward sees it
    (yb * dy).sum().backward()
    torch.cuda.synchronize()
    assert ya.dtype == (torch.bfloat16 if autocast else torch.float32)
    tol = 2.0 ** -8 if autocast else 1e-5
    assert ((ya.float() - yb).abs() <= tol * yb.abs() + 1e-5).all()
    assert _rel(ga_x, xb.grad) <= 1e-4, _rel(ga_x, xb.grad)
    assert _rel(ga_w, norm.weight.grad) <= 1e-4, _rel(ga_w, norm.weight.grad)


@pytest.mark.parametrize("F", [5632, 100])
def test_fused_swiglu_matches_torch(gpu, F):
    """ssa_swiglu against silu(gate) * up in fp32, forward and backward (both
    halves of the fc1 gradient): within bf16 rounding."""
    from SSA.ssa_decoder import FusedSwiGLU

    print(f"[gpu case] fused SwiGLU F={F}", file=sys.stderr, flush=True)
    torch.manual_seed(6)
    z = (torch.randn(700, 3, 2 * F, device=gpu) * 2).to(torch.bfloat16)
    za = z.clone().requires_grad_(True)
    zb = z.float().requires_grad_(True)
    ha = FusedSwiGLU.apply(za)
    g, u = zb.chunk(2, dim=-1)
    hb = torch.nn.functional.silu(g) * u
    w = torch.randn_like(hb)
    (ha.float() * w).sum().backward()
    (hb * w.to(torch.bfloat16).float()).sum().backward()
    torch.cuda.synchronize()
    tol = 2.0 ** -8
    assert ((ha.float() - hb).abs() <= tol * hb.abs() + 1e-4).all()
    ga, gb = za.grad.float(), zb.grad
    assert ((ga - gb).abs() <= 2 * tol * gb.abs() + 1e-3).all()


@pytest.mark.parametrize("V", [65536, 1000])
def test_fused_cross_entropy_matches_torch(gpu, V):
    """ssa_cross_entropy against F.cross_entropy on the fp32 logits, with
    ignored labels (-100): the mean loss and the logits gradient."""
    from SSA.ssa_decoder import FusedCrossEntropy

    print(f"[gpu case] fused cross-entropy V={V}", file=sys.stderr, flush=True)
    torch.manual_seed(7)
    R = 1000
    logits = (torch.randn(R, V, device=gpu) * 4).to(torch.bfloat16)
    labels = torch.randint(0, V, (R,), device=gpu)
    labels[::7] = -100
    la = logits.clone().requires_grad_(True)
    lb = logits.float().requires_grad_(True)
    loss_a = FusedCrossEntropy.apply(la, labels)
    loss_b = torch.nn.functional.cross_entropy(lb, labels)
    (loss_a * 3).backward()
    (loss_b * 3).backward()
    torch.cuda.synchronize()
    assert abs(loss_a.item() - loss_b.item()) <= 1e-5 * abs(loss_b.item()), (loss_a.item(), loss_b.item())
    ga, gb = la.grad.float(), lb.grad
    assert ((ga - gb).abs() <= 2.0 ** -8 * gb.abs() + 1e-3 * gb.abs().max()).all()
    assert (ga[::7] == 0).all()
