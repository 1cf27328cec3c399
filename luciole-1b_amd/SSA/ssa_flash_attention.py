"""Autograd boundary for SSA attention on MI355X.

Same contract as ``training/train/train_ssa_triton/SSA/ssa_flash_attention.py:11-97``:
``SSAFlashAttnFunc.apply(q, k, v, softmax_scale, ssa_n, ssa_b, causal, dropout_p, training)``
and ``ssa_flash_attention(...)``.  The forward casts n and b to fp32 device
scalars and saves (q, k, v, out, m, n32, b32); the backward makes dout
contiguous and returns gradients in the forward's argument order
``(dq, dk, dv, None, dn, db, None, None, None)``.  Dropout is never applied
inside the op (the calling module applies it to the output).
"""

from __future__ import annotations

import torch
from torch.autograd import Function

from .ssa_hip_kernel import (
    ssa_flash_attn_backward,
    ssa_flash_attn_forward,
    ssa_flash_attn_varlen_backward,
    ssa_flash_attn_varlen_forward,
)


class SSAFlashAttnFunc(Function):
    """out = softmax_rows(n sign(s) ln(1 + b|s|)) v with s = scale q k^T; grads for q, k, v, n, b."""

    @staticmethod
    def forward(ctx, q, k, v, softmax_scale, ssa_n, ssa_b, causal, dropout_p, training):
        ssa_n_f32 = ssa_n.float().contiguous()
        ssa_b_f32 = ssa_b.float().contiguous()
        out, m = ssa_flash_attn_forward(q, k, v, softmax_scale, ssa_n_f32, ssa_b_f32, causal)
        ctx.save_for_backward(q, k, v, out, m, ssa_n_f32, ssa_b_f32)
        ctx.softmax_scale = softmax_scale
        ctx.causal = causal
        ctx.dropout_p = dropout_p
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, m, ssa_n_f32, ssa_b_f32 = ctx.saved_tensors
        dq, dk, dv, dn, db = ssa_flash_attn_backward(
            q, k, v, out, dout.contiguous(), m, ctx.softmax_scale, ssa_n_f32, ssa_b_f32, ctx.causal
        )
        return dq, dk, dv, None, dn, db, None, None, None


def ssa_flash_attention(q, k, v, softmax_scale, ssa_n, ssa_b, causal=True, dropout_p=0.0, training=True):
    """SSA attention with native GQA: q [B,Hq,N,D], k/v [B,Hkv,N,D] -> out [B,Hq,N,D]."""
    return SSAFlashAttnFunc.apply(q, k, v, softmax_scale, ssa_n, ssa_b, causal, dropout_p, training)


class SSAFlashAttnVarlenFunc(Function):
    """Packed-sequence SSA attention: q [T,Hq,D], k/v [T,Hkv,D] split into
    documents by cu_seqlens; attention stays inside each document.  No
    reference counterpart (the reference rejects packed sequences,
    ``training/train/train_ssa_triton/SSA/ssa_triton_attention.py:154-156``); the
    arguments follow Megatron's PackedSeqParams (cu_seqlens_q, max_seqlen_q)."""

    @staticmethod
    def forward(ctx, q, k, v, cu_seqlens, max_seqlen, softmax_scale, ssa_n, ssa_b, causal):
        ssa_n_f32 = ssa_n.float().contiguous()
        ssa_b_f32 = ssa_b.float().contiguous()
        out, m = ssa_flash_attn_varlen_forward(q, k, v, cu_seqlens, max_seqlen, softmax_scale, ssa_n_f32,
                                               ssa_b_f32, causal)
        ctx.save_for_backward(q, k, v, out, m, cu_seqlens, ssa_n_f32, ssa_b_f32)
        ctx.max_seqlen = int(max_seqlen)
        ctx.softmax_scale = softmax_scale
        ctx.causal = causal
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, m, cu_seqlens, ssa_n_f32, ssa_b_f32 = ctx.saved_tensors
        dq, dk, dv, dn, db = ssa_flash_attn_varlen_backward(
            q, k, v, out, dout.contiguous(), m, cu_seqlens, ctx.max_seqlen, ctx.softmax_scale, ssa_n_f32,
            ssa_b_f32, ctx.causal
        )
        return dq, dk, dv, None, None, None, dn, db, None


def ssa_flash_attention_varlen(q, k, v, cu_seqlens, max_seqlen, softmax_scale, ssa_n, ssa_b, causal=True):
    """Packed-sequence SSA attention: q [T,Hq,D], k/v [T,Hkv,D] -> out [T,Hq,D]."""
    return SSAFlashAttnVarlenFunc.apply(q, k, v, cu_seqlens, max_seqlen, softmax_scale, ssa_n, ssa_b, causal)
