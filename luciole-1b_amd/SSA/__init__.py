"""SSA (softmax-substituted attention) for MI355X: hand-written gfx950 HIP
kernels behind the reference's Python operator interface.

Modules mirror the reference package ``training/train/train_ssa_triton/SSA``:
``ssa_flash_attention`` (autograd boundary), ``ssa_triton_kernel`` (launch
layer names, re-exported from ``ssa_hip_kernel``), ``ssa_attention`` (the
attention module of ``ssa_triton_attention``, without Megatron, plus the KV
cache for decoding); ``ssa_decoder`` is the Llama-style decoder of the
reference's SSA GPT layer spec (``ssa_triton_layer_specs.py``) for end-to-end
train steps and cached generation.
"""

from .ssa_attention import SSAAttention, SSAKVCache  # noqa: F401
from .ssa_flash_attention import (  # noqa: F401
    SSAFlashAttnFunc,
    SSAFlashAttnVarlenFunc,
    ssa_flash_attention,
    ssa_flash_attention_varlen,
)
from .ssa_hip_kernel import (  # noqa: F401
    ssa_bwd_preprocess,
    ssa_decode_attention,
    ssa_decode_num_splits,
    ssa_flash_attn_backward,
    ssa_flash_attn_forward,
    ssa_flash_attn_varlen_backward,
    ssa_flash_attn_varlen_forward,
    warmup_ssa_triton_kernels,
)
