"""A Llama-style decoder with SSA attention, without Megatron or NeMo.

The layer mirrors the reference's SSA GPT layer spec
(training/train/train_ssa_triton/SSA/ssa_triton_layer_specs.py:96-127):
input RMSNorm -> fused QKV projection -> RoPE -> SSA core attention
(``SSAAttention``, the module of ssa_triton_attention.py) -> output
projection -> residual; pre-MLP RMSNorm -> SwiGLU MLP -> residual.  Tensors
flow in Megatron's [S, B, hidden] order, the fused QKV weight uses Megatron's
grouped layout (per query group: G query heads, one key head, one value
head) and the parameter names follow Megatron's
(``self_attention.linear_qkv``, ``core_attention.ssa_n_raw``, ``mlp.linear_fc1``
...), so a state dict maps one to one.

``SSADecoderConfig()`` defaults to the end-to-end configuration of the
benchmark: 24 layers, hidden 2048, 16 heads x 128, SwiGLU FFN 5632, RMSNorm,
RoPE, vocab 65536, sequence 4096 (about 1.5 B parameters with an untied output
layer).  ``train_step`` is one optimizer step under bf16 autocast;
``generate`` runs the prompt through the dense forward once and then one
decode step per token against per-layer KV caches (the reference's loop
re-runs the whole prefix per token, training/train/train_ssa_triton/generate_triton.py:315-331).
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import List, Optional

import torch
import torch.nn.functional as F
from torch import nn

from .ssa_attention import SSAAttention, SSAKVCache


@dataclass
class SSADecoderConfig:
    num_layers: int = 24
    hidden_size: int = 2048
    num_attention_heads: int = 16
    num_query_groups: int = 16
    kv_channels: int = 128
    ffn_hidden_size: int = 5632
    vocab_size: int = 65536
    seq_length: int = 4096
    rotary_base: float = 10000.0
    norm_eps: float = 1e-5
    ssa_n: float = 1.5
    ssa_b: float = 0.8
    learnable_ssa: bool = True
    learnable_b: bool = False
    init_std: float = 0.02
    fused_rope: bool = True  # ssa_rope on the GPU (False: the PyTorch form)
    fused_norm: bool = True  # ssa_rmsnorm_* on the GPU (False: the PyTorch form)
    fused_swiglu: bool = True  # ssa_swiglu on the GPU (False: the PyTorch form)
    fused_loss: bool = True  # ssa_cross_entropy on the GPU (False: F.cross_entropy on fp32 logits)

    def num_parameters(self) -> int:
        h, f, v = self.hidden_size, self.ffn_hidden_size, self.vocab_size
        qkv = h * (self.num_attention_heads + 2 * self.num_query_groups) * self.kv_channels
        proj = self.num_attention_heads * self.kv_channels * h
        per_layer = qkv + proj + 3 * h * f + 2 * h + (2 if self.learnable_b else 1) * int(self.learnable_ssa)
        return self.num_layers * per_layer + 2 * v * h + h


_OPS_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


class FusedRMSNormFn(torch.autograd.Function):
    """RMSNorm of fp32 rows as one HIP pass each way (``ssa_rmsnorm_fwd`` /
    ``ssa_rmsnorm_bwd``), the output written in ``out_dtype`` (the next GEMM's
    input dtype under autocast)."""

    @staticmethod
    def forward(ctx, x, weight, eps, out_dtype):
        from . import _lib

        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).contiguous()
        T, H = x2.shape
        y = torch.empty((T, H), device=x.device, dtype=out_dtype)
        rstd = torch.empty(T, device=x.device, dtype=torch.float32)
        w = weight.contiguous()
        args = _lib.RmsNormFwdArgs(x2.data_ptr(), w.data_ptr(), y.data_ptr(), rstd.data_ptr(), T, H,
                                   _OPS_DTYPES[out_dtype], float(eps))
        with torch.cuda.device(x.device):
            stream = torch.cuda.current_stream(x.device).cuda_stream
            _lib.check(_lib.lib().ssa_rmsnorm_fwd(ctypes.byref(args), ctypes.c_void_p(stream)), "ssa_rmsnorm_fwd")
        ctx.save_for_backward(x2, w, rstd)
        ctx.shape = shape
        return y.view(shape)

    @staticmethod
    def backward(ctx, dy):
        from . import _lib

        x2, w, rstd = ctx.saved_tensors
        T, H = x2.shape
        dy2 = dy.reshape(T, H).contiguous()
        dx = torch.empty_like(x2)
        dw = torch.empty(H, device=x2.device, dtype=torch.float32)
        lib = _lib.lib()
        ws = torch.empty(int(lib.ssa_rmsnorm_workspace_floats(T, H)), device=x2.device, dtype=torch.float32)
        args = _lib.RmsNormBwdArgs(x2.data_ptr(), w.data_ptr(), dy2.data_ptr(), rstd.data_ptr(), dx.data_ptr(),
                                   dw.data_ptr(), ws.data_ptr(), T, H, _OPS_DTYPES[dy2.dtype])
        with torch.cuda.device(x2.device):
            stream = torch.cuda.current_stream(x2.device).cuda_stream
            _lib.check(lib.ssa_rmsnorm_bwd(ctypes.byref(args), ctypes.c_void_p(stream)), "ssa_rmsnorm_bwd")
        return dx.view(ctx.shape), dw.to(w.dtype), None, None


class RMSNorm(nn.Module):
    def __init__(self, hidden: int, eps: float, fused: bool = True):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden))
        self.eps = eps
        self.fused = fused

    def forward(self, x):
        H = x.shape[-1]
        if (self.fused and x.is_cuda and x.dtype == torch.float32 and self.weight.dtype == torch.float32
                and H % 4 == 0 and H <= 4096):
            out = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else torch.float32
            return FusedRMSNormFn.apply(x, self.weight, self.eps, out)
        return self.reference(x)

    def reference(self, x):
        """The PyTorch form (fp32 math), against which the fused kernel is tested."""
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


def rope_tables(positions: torch.Tensor, dim: int, base: float):
    """cos / sin [S, 1, 1, dim] (fp32) for the rotate-half RoPE of Megatron's
    default (non-interleaved) rotary embedding."""
    inv = 1.0 / (base ** (torch.arange(0, dim, 2, device=positions.device, dtype=torch.float32) / dim))
    ang = positions.float()[:, None] * inv[None, :]
    emb = torch.cat([ang, ang], dim=-1)[:, None, None, :]
    return emb.cos(), emb.sin()


def apply_rope(x, cos, sin):
    """Rotate-half RoPE in PyTorch (fp32 math): the reference form the fused
    kernel is tested against."""
    xf = x.float()
    x1, x2 = xf.chunk(2, dim=-1)
    rot = torch.cat([-x2, x1], dim=-1)
    return (xf * cos + rot * sin).to(x.dtype)


def _rope_launch(x, cos_h, sin_h, inverse: bool):
    from . import _lib

    if x.dim() != 4 or x.stride(-1) != 1:
        x = x.contiguous()
    S, B, H, D = x.shape
    y = torch.empty((S, B, H, D), device=x.device, dtype=x.dtype)
    args = _lib.RopeArgs(x.data_ptr(), x.stride(0), x.stride(1), x.stride(2), y.data_ptr(), cos_h.data_ptr(),
                         sin_h.data_ptr(), S, B, H, D, 0 if x.dtype == torch.bfloat16 else 1, int(inverse))
    with torch.cuda.device(x.device):
        stream = torch.cuda.current_stream(x.device).cuda_stream
        _lib.check(_lib.lib().ssa_rope(ctypes.byref(args), ctypes.c_void_p(stream)), "ssa_rope")
    return y


class FusedRoPE(torch.autograd.Function):
    """apply_rope as one HIP pass each way (``ssa_rope``; the backward rotates
    by the negative angle).  x: [S, B, H, D] bf16/fp16, D in {64, 128}."""

    @staticmethod
    def forward(ctx, x, cos_h, sin_h):
        ctx.save_for_backward(cos_h, sin_h)
        return _rope_launch(x, cos_h, sin_h, False)

    @staticmethod
    def backward(ctx, dy):
        cos_h, sin_h = ctx.saved_tensors
        return _rope_launch(dy, cos_h, sin_h, True), None, None


def rope(x, cos, sin, cos_h=None, sin_h=None):
    """RoPE for the layer: the fused kernel for bf16/fp16 inputs with head dim
    64 or 128 on the GPU (``cos_h`` / ``sin_h`` its tables), PyTorch otherwise."""
    if (cos_h is not None and x.is_cuda and x.dtype in (torch.bfloat16, torch.float16)
            and x.shape[-1] in (64, 128)):
        return FusedRoPE.apply(x, cos_h, sin_h)
    return apply_rope(x, cos, sin)


class SelfAttention(nn.Module):
    def __init__(self, cfg: SSADecoderConfig, layer_number: int):
        super().__init__()
        self.cfg = cfg
        self.np, self.ng, self.hn = cfg.num_attention_heads, cfg.num_query_groups, cfg.kv_channels
        self.linear_qkv = nn.Linear(cfg.hidden_size, (self.np + 2 * self.ng) * self.hn, bias=False)
        self.core_attention = SSAAttention(self.np, self.ng, self.hn, layer_number=layer_number, ssa_n=cfg.ssa_n,
                                           ssa_b=cfg.ssa_b, learnable_ssa=cfg.learnable_ssa,
                                           learnable_b=cfg.learnable_b)
        self.linear_proj = nn.Linear(self.np * self.hn, cfg.hidden_size, bias=False)

    def _qkv(self, x, rot):
        S, B = x.shape[0], x.shape[1]
        g = self.np // self.ng
        mixed = self.linear_qkv(x).view(S, B, self.ng, (g + 2) * self.hn)
        q, k, v = torch.split(mixed, [g * self.hn, self.hn, self.hn], dim=-1)
        q = q.reshape(S, B, self.np, self.hn)
        return rope(q, *rot), rope(k, *rot), v

    def forward(self, x, rot, cache: Optional[SSAKVCache] = None):
        """rot = (cos, sin, cos_h, sin_h) from ``SSADecoder.rotary``."""
        q, k, v = self._qkv(x, rot)
        if cache is None:
            ctx = self.core_attention(q, k, v)
        elif x.shape[0] == 1:
            ctx = self.core_attention.forward_decode(q, k, v, cache)
        else:  # prompt: dense causal forward, then the keys and values go to the cache
            ctx = self.core_attention(q, k, v)
            cache.append(k.permute(1, 2, 0, 3), v.permute(1, 2, 0, 3))
        return self.linear_proj(ctx)


def _swiglu_launch(z, dh, backward: bool):
    from . import _lib

    F2 = z.shape[-1]
    rows = z.numel() // F2
    shape = z.shape[:-1] + ((F2,) if backward else (F2 // 2,))
    out = torch.empty(shape, device=z.device, dtype=z.dtype)
    args = _lib.SwigluArgs(z.data_ptr(), dh.data_ptr() if dh is not None else None, out.data_ptr(), rows, F2 // 2,
                           0 if z.dtype == torch.bfloat16 else 1, int(backward))
    with torch.cuda.device(z.device):
        stream = torch.cuda.current_stream(z.device).cuda_stream
        _lib.check(_lib.lib().ssa_swiglu(ctypes.byref(args), ctypes.c_void_p(stream)), "ssa_swiglu")
    return out


class FusedSwiGLU(torch.autograd.Function):
    """silu(gate) * up of z = [gate | up] (the fc1 output) as one HIP pass each
    way (``ssa_swiglu``); the backward writes both halves of dz directly."""

    @staticmethod
    def forward(ctx, z):
        z = z.contiguous()
        ctx.save_for_backward(z)
        return _swiglu_launch(z, None, False)

    @staticmethod
    def backward(ctx, dh):
        (z,) = ctx.saved_tensors
        return _swiglu_launch(z, dh.contiguous(), True)


class FusedCrossEntropy(torch.autograd.Function):
    """Mean cross-entropy of bf16/fp16 logits [rows, vocab] against int64 labels
    (``ssa_cross_entropy``): one pass over the logits each way, no fp32 copy;
    labels outside [0, vocab) (e.g. -100) are ignored, as by
    ``F.cross_entropy``."""

    @staticmethod
    def _launch(args):
        from . import _lib

        with torch.cuda.device(torch.cuda.current_device()):
            stream = torch.cuda.current_stream().cuda_stream
            _lib.check(_lib.lib().ssa_cross_entropy(ctypes.byref(args), ctypes.c_void_p(stream)), "ssa_cross_entropy")

    @staticmethod
    def forward(ctx, logits, labels):
        from . import _lib

        logits = logits.contiguous()
        labels = labels.to(torch.int64).contiguous()
        R, V = logits.shape
        loss = torch.empty(R, device=logits.device, dtype=torch.float32)
        lse = torch.empty(R, device=logits.device, dtype=torch.float32)
        dt = 0 if logits.dtype == torch.bfloat16 else 1
        with torch.cuda.device(logits.device):
            FusedCrossEntropy._launch(_lib.CrossEntropyArgs(logits.data_ptr(), labels.data_ptr(), loss.data_ptr(),
                                                            lse.data_ptr(), None, None, R, V, dt, 0))
        n = ((labels >= 0) & (labels < V)).sum().clamp_min(1).to(torch.float32)
        ctx.save_for_backward(logits, labels, lse, n)
        return loss.sum() / n

    @staticmethod
    def backward(ctx, g):
        from . import _lib

        logits, labels, lse, n = ctx.saved_tensors
        R, V = logits.shape
        scale = (g.to(torch.float32) / n).reshape(()).contiguous()
        dlogits = torch.empty_like(logits)
        dt = 0 if logits.dtype == torch.bfloat16 else 1
        with torch.cuda.device(logits.device):
            FusedCrossEntropy._launch(_lib.CrossEntropyArgs(logits.data_ptr(), labels.data_ptr(), None, lse.data_ptr(),
                                                            scale.data_ptr(), dlogits.data_ptr(), R, V, dt, 1))
        return dlogits, None


class MLP(nn.Module):
    def __init__(self, cfg: SSADecoderConfig):
        super().__init__()
        self.linear_fc1 = nn.Linear(cfg.hidden_size, 2 * cfg.ffn_hidden_size, bias=False)  # [gate; up]
        self.linear_fc2 = nn.Linear(cfg.ffn_hidden_size, cfg.hidden_size, bias=False)
        self.fused = cfg.fused_swiglu

    def forward(self, x):
        z = self.linear_fc1(x)
        if self.fused and z.is_cuda and z.dtype in (torch.bfloat16, torch.float16) and z.shape[-1] % 8 == 0:
            return self.linear_fc2(FusedSwiGLU.apply(z))
        gate, up = z.chunk(2, dim=-1)
        return self.linear_fc2(F.silu(gate) * up)


class TransformerLayer(nn.Module):
    def __init__(self, cfg: SSADecoderConfig, layer_number: int):
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.norm_eps, cfg.fused_norm)
        self.self_attention = SelfAttention(cfg, layer_number)
        self.pre_mlp_layernorm = RMSNorm(cfg.hidden_size, cfg.norm_eps, cfg.fused_norm)
        self.mlp = MLP(cfg)

    def forward(self, x, rot, cache=None):
        x = x + self.self_attention(self.input_layernorm(x), rot, cache)
        return x + self.mlp(self.pre_mlp_layernorm(x))


class SSADecoder(nn.Module):
    def __init__(self, cfg: SSADecoderConfig):
        super().__init__()
        self.cfg = cfg
        self.embedding = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(TransformerLayer(cfg, i + 1) for i in range(cfg.num_layers))
        self.final_layernorm = RMSNorm(cfg.hidden_size, cfg.norm_eps, cfg.fused_norm)
        self.output_layer = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        self.reset_parameters()

    @torch.no_grad()
    def reset_parameters(self):
        std = self.cfg.init_std
        out_std = std / math.sqrt(2.0 * self.cfg.num_layers)  # scaled init of the residual outputs
        for name, p in self.named_parameters():
            if p.dim() < 2:
                continue
            p.normal_(0.0, out_std if name.endswith(("linear_proj.weight", "linear_fc2.weight")) else std)

    def forward(self, input_ids, caches: Optional[List[SSAKVCache]] = None, start_pos: int = 0):
        """input_ids [B, S] -> logits [S, B, vocab] (Megatron order).  With
        ``caches`` (one per layer) the tokens are positions start_pos .. and
        their keys / values are appended to the caches."""
        S = input_ids.shape[1]
        x = self.embedding(input_ids.t())  # [S, B, h]
        pos = torch.arange(start_pos, start_pos + S, device=input_ids.device)
        rot = self.rotary(pos)
        for i, layer in enumerate(self.layers):
            x = layer(x, rot, None if caches is None else caches[i])
        return self.output_layer(self.final_layernorm(x))

    def rotary(self, positions):
        """(cos, sin) [S, 1, 1, D] for the PyTorch form and, with
        ``fused_rope``, the fp32 [S, D / 2] tables of the fused kernel."""
        cos, sin = rope_tables(positions, self.cfg.kv_channels, self.cfg.rotary_base)
        if not self.cfg.fused_rope:
            return cos, sin, None, None
        half = self.cfg.kv_channels // 2
        return cos, sin, cos[:, 0, 0, :half].contiguous(), sin[:, 0, 0, :half].contiguous()

    def loss(self, input_ids, labels):
        logits = self(input_ids)  # [S, B, V]
        V = logits.shape[-1]
        if self.cfg.fused_loss and logits.is_cuda and logits.dtype in (torch.bfloat16, torch.float16) and V % 4 == 0:
            return FusedCrossEntropy.apply(logits.view(-1, V), labels.t().reshape(-1))
        return F.cross_entropy(logits.float().view(-1, V), labels.t().reshape(-1))

    def new_caches(self, batch: int, capacity: int, dtype=torch.bfloat16) -> List[SSAKVCache]:
        dev = self.embedding.weight.device
        return [SSAKVCache(batch, self.cfg.num_query_groups, capacity, self.cfg.kv_channels, dtype, dev)
                for _ in range(self.cfg.num_layers)]

    @torch.no_grad()
    def generate(self, input_ids, max_new_tokens: int, dtype=torch.bfloat16):
        """Greedy decoding: the prompt through the dense forward, then one decode
        step per new token.  Returns (tokens [B, P + max_new_tokens], the
        logits of every generated position [max_new_tokens, B, vocab])."""
        B, P = input_ids.shape
        caches = self.new_caches(B, P + max_new_tokens, dtype)
        out, steps = input_ids, []
        with torch.autocast("cuda", dtype=dtype):
            logits = self(input_ids, caches, 0)[-1]
            for t in range(max_new_tokens):
                steps.append(logits.float())
                nxt = logits.argmax(-1, keepdim=True)
                out = torch.cat([out, nxt], dim=1)
                if t + 1 < max_new_tokens:
                    logits = self(nxt, caches, P + t)[-1]
        return out, torch.stack(steps)


def train_step(model: SSADecoder, optimizer: torch.optim.Optimizer, input_ids, labels, dtype=torch.bfloat16):
    """One optimizer step: forward and loss under autocast (bf16 GEMMs and SSA
    attention, fp32 norms, RoPE and loss), backward, AdamW update."""
    optimizer.zero_grad(set_to_none=True)
    with torch.autocast("cuda", dtype=dtype):
        loss = model.loss(input_ids, labels)
    loss.backward()
    optimizer.step()
    return loss.detach()
