"""Import-path compatibility for callers of the reference launch layer.

Code written against ``SSA.ssa_triton_kernel`` (the reference's
``training/train/train_ssa_triton/SSA/ssa_triton_kernel.py``, imported e.g. by
``TS/check_ssa_triton_parity.py:32-35`` and ``TS/train_ssa_triton.py:38``)
resolves to the MI355X HIP implementation unchanged.  No Triton is involved.
"""

from .ssa_hip_kernel import (  # noqa: F401
    ssa_bwd_preprocess,
    ssa_flash_attn_backward,
    ssa_flash_attn_forward,
    warmup_ssa_triton_kernels,
)
