"""SSA self-attention module on the MI355X kernels, without Megatron.

Mirrors ``SSATritonAttention`` (training/train/train_ssa_triton/SSA/ssa_triton_attention.py):

* constructor arguments and parameter names (``ssa_n_raw``, ``ssa_b_raw`` or the
  ``ssa_b`` buffer, ``ssa_n`` buffer when not learnable; :99-113), so reference
  checkpoints load unchanged;
* softmax scale 1/sqrt(head_dim), divided by the layer number under query-key
  layer scaling (:91-97);
* forward(query, key, value [S, B, H, D]) -> context [S, B, Hq * D] (:132-202),
  dropout applied to the attention output, never inside the op (:115-130).

Differences, both at the boundary: the [S, B, H, D] inputs are handed to the
kernels as permuted views (no copies; the reference forces contiguous copies
in production, ``force_contiguous_qkv``), and the kernel writes its output in
[S, B, H, D] memory order, so the final [S, B, Hq * D] reshape is a view;
packed sequences (``packed_seq_params`` with ``cu_seqlens_q`` and
``max_seqlen_q``, tensors [T, H, D] or [T, 1, H, D]) run on the varlen path,
which the reference rejects (:154-156).

Generation: ``SSAKVCache`` + ``SSAAttention.forward_decode`` run one token
per step against the cached keys and values (the decode kernel), where the
reference's generation loop re-runs the whole prefix through the forward for
every token (training/train/train_ssa_triton/generate_triton.py:315-331); the
result is the same causal attention row.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
from torch import nn

from .ssa_flash_attention import ssa_flash_attention, ssa_flash_attention_varlen
from .ssa_hip_kernel import ssa_decode_attention


class SSAKVCache:
    """Keys and values of one attention layer for generation.

    ``k`` / ``v`` are ``[B, Hkv, capacity, D]`` (the decode kernel's layout);
    ``seqlens`` (int32 ``[B]``, on the device) counts the cached tokens of each
    sequence.  Appends write at each sequence's own length without a host
    synchronisation; positions past ``capacity`` are clamped to its last row,
    so the caller sizes the cache for the longest generation.
    """

    def __init__(self, batch: int, heads_kv: int, capacity: int, head_dim: int, dtype=torch.bfloat16,
                 device="cuda"):
        self.k = torch.zeros(batch, heads_kv, capacity, head_dim, dtype=dtype, device=device)
        self.v = torch.zeros_like(self.k)
        self.seqlens = torch.zeros(batch, dtype=torch.int32, device=device)
        self.capacity = capacity

    def append(self, key: torch.Tensor, value: torch.Tensor) -> None:
        """Append ``T`` new tokens per sequence: key / value ``[B, Hkv, T, D]``."""
        B, _, T, _ = key.shape
        pos = self.seqlens.long().unsqueeze(1) + torch.arange(T, device=key.device).unsqueeze(0)
        pos = pos.clamp_(max=self.capacity - 1)
        bidx = torch.arange(B, device=key.device).unsqueeze(1).expand(B, T)
        # advanced indices on dims 0 and 2 -> the indexed view is [B, T, Hkv, D]
        self.k[bidx, :, pos] = key.transpose(1, 2).to(self.k.dtype)
        self.v[bidx, :, pos] = value.transpose(1, 2).to(self.v.dtype)
        self.seqlens += T


class SSAAttention(nn.Module):
    def __init__(
        self,
        num_attention_heads: int,
        num_query_groups: Optional[int] = None,
        kv_channels: int = 128,
        layer_number: int = 1,
        softmax_scale: Optional[float] = None,
        apply_query_key_layer_scaling: bool = False,
        attention_dropout: float = 0.0,
        ssa_n: float = 1.5,
        ssa_b: float = 0.8,
        learnable_ssa: bool = True,
        learnable_b: bool = False,
        causal: bool = True,
    ):
        super().__init__()
        self.num_heads = num_attention_heads
        self.num_query_groups = num_query_groups or num_attention_heads
        if self.num_heads % self.num_query_groups != 0:
            raise ValueError("num_attention_heads must be a multiple of num_query_groups")
        self.head_dim = kv_channels
        self.hidden_size = kv_channels * num_attention_heads
        self.layer_number = max(1, layer_number)
        self.causal = causal
        self.learnable_ssa = learnable_ssa
        self.learnable_b = learnable_b
        self.softmax_scale = 1.0 / math.sqrt(kv_channels) if softmax_scale is None else softmax_scale
        if apply_query_key_layer_scaling:
            self.softmax_scale /= self.layer_number
        if learnable_ssa:
            self.ssa_n_raw = nn.Parameter(torch.tensor(float(ssa_n)))
            if learnable_b:
                self.ssa_b_raw = nn.Parameter(torch.tensor(float(ssa_b)))
            else:
                self.register_buffer("ssa_b", torch.tensor(float(ssa_b)))
        else:
            self.register_buffer("ssa_n", torch.tensor(float(ssa_n)))
            self.register_buffer("ssa_b", torch.tensor(float(ssa_b)))
        self.dropout_p = attention_dropout
        self.attention_dropout = nn.Dropout(attention_dropout)

    def get_ssa_params(self):
        if self.learnable_ssa:
            return self.ssa_n_raw, (self.ssa_b_raw if self.learnable_b else self.ssa_b)
        return self.ssa_n, self.ssa_b

    def forward(self, query, key, value, attention_mask=None, packed_seq_params=None):
        """query [S, B, Hq, D], key/value [S, B, Hkv, D] -> context [S, B, Hq * D].

        With ``packed_seq_params`` (``cu_seqlens_q``, ``max_seqlen_q``): tensors
        [T, H, D] or [T, 1, H, D] -> context [T, Hq * D] (or [T, 1, Hq * D]).
        ``attention_mask`` is ignored (the causal mask is applied in the kernel).
        """
        n, b = self.get_ssa_params()
        if packed_seq_params is not None:
            squeeze = query.dim() == 4
            q, k, v = (t.squeeze(1) if squeeze else t for t in (query, key, value))
            ctx = ssa_flash_attention_varlen(q, k, v, packed_seq_params.cu_seqlens_q,
                                             packed_seq_params.max_seqlen_q, self.softmax_scale, n, b, self.causal)
            if self.training and self.dropout_p > 0:
                ctx = self.attention_dropout(ctx)
            ctx = ctx.reshape(ctx.shape[0], -1)
            return ctx.unsqueeze(1) if squeeze else ctx
        S, B = query.shape[0], query.shape[1]
        # [S, B, H, D] -> [B, H, S, D] views: the kernels read the strides in place
        q, k, v = (t.permute(1, 2, 0, 3) for t in (query, key, value))
        ctx = ssa_flash_attention(q, k, v, self.softmax_scale, n, b, self.causal, self.dropout_p, self.training)
        if self.training and self.dropout_p > 0:
            ctx = self.attention_dropout(ctx)
        # the output has the strides of q, i.e. [S, B, H, D] memory order: views only
        return ctx.permute(2, 0, 1, 3).reshape(S, B, -1)

    def forward_decode(self, query, key, value, cache: SSAKVCache):
        """One generation step.  query [1, B, Hq, D], key/value [1, B, Hkv, D]
        (the new token) -> context [1, B, Hq * D]; the key and value are
        appended to ``cache`` first, so the token attends itself and the
        cached prefix (causal)."""
        if query.shape[0] != 1:
            raise ValueError("forward_decode takes one new token per sequence ([1, B, H, D])")
        n, b = self.get_ssa_params()
        cache.append(key.permute(1, 2, 0, 3), value.permute(1, 2, 0, 3))
        ctx = ssa_decode_attention(query[0], cache.k, cache.v, cache.seqlens, self.softmax_scale, n, b)
        return ctx.reshape(1, query.shape[1], -1)
