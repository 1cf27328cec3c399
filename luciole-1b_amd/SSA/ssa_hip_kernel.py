"""Kernel-level SSA attention API on MI355X (gfx950 HIP kernels via a C ABI).

Same functions, argument meaning and return values as the reference launch
layer ``training/train/train_ssa_triton/SSA/ssa_triton_kernel.py``:

* ``ssa_flash_attn_forward(q, k, v, softmax_scale, ssa_n, ssa_b, causal=True) -> (out, m)``
  (reference :732-792)
* ``ssa_flash_attn_backward(q, k, v, out, dout, m, softmax_scale, ssa_n, ssa_b, causal=True)
  -> (dq, dk, dv, dn, db)`` (reference :795-897)
* ``warmup_ssa_triton_kernels(B, Hq, Hkv, N, D, dtype, device)`` (reference :904-928)

plus packed-sequence (varlen) versions of the forward and backward, which the
reference does not have (``ssa_flash_attn_varlen_forward`` /
``ssa_flash_attn_varlen_backward``).

Tensors are ``[B, H, N, D]`` with any strides whose last one is 1 (other
layouts are made contiguous first); outputs follow the input strides
(``torch.empty_like``).  ``m`` is the fp32 base-2 row normaliser
``log2(sum_j exp(t_ij))``.  ``ssa_n`` / ``ssa_b`` are scalar tensors read on the
device (no host synchronisation); ``dn`` / ``db`` come back as 0-d fp32 tensors.

Differences from the reference, all widening: any sequence length (the
reference's backward needs N % 128 == 0), and results are bitwise
reproducible.  In bf16 / fp16 the backward by default keeps dS' (the score
gradient, input dtype, causal triangle only: 2 N^2 bytes per (batch, head)) in
a transient workspace so that dQ is one streaming product with K instead of
the reference's recompute of the scores (measured faster at every head dim:
3-6 % of the backward at D = 32 / 64, 7-17 % at D = 128); ``SSA_BWD_DS=0`` /
``1`` forces either path, and a workspace above ``SSA_BWD_DS_MAX_BYTES``
(default 16 GiB) or half of the device's headroom recomputes.  Head dims 32,
64 and 128 run on kernels of their own; in bf16 /
fp16, head dim 16 (the smallest the reference's Triton kernel takes) runs on
the D = 32 kernels with its operands zero-padded to 32 columns, which changes
no score, dP or Delta, and the results are sliced back (the decode step is not
offered at D = 16).  fp32 inputs (the reference's fp32-operand path) run on
fp32 vector-ALU kernels for head dims 16-256 that keep every product in fp32,
without the dS' workspace; bf16 / fp16 at head dim 256 (the largest power of
two the reference takes) run on the same kernels, widened on load (coverage,
not speed); the decode step takes bf16 / fp16 only.  Errors:
``AssertionError`` for ``Hq % Hkv != 0`` and a non-power-of-two head dim, as in
the reference; ``ValueError`` for other head dims and other dtypes.
"""

from __future__ import annotations

import ctypes
import os

import torch

from . import _lib

_DTYPES = {torch.bfloat16: _lib.SSA_DTYPE_BF16, torch.float16: _lib.SSA_DTYPE_FP16,
           torch.float32: _lib.SSA_DTYPE_FP32}


def _is_pow2(x: int) -> bool:
    return x > 0 and (x & (x - 1)) == 0


_MAX_ROW_STRIDE = 1 << 24


def _kernel_layout(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` or a contiguous copy so that stride(-1) == 1, rows are 16-byte
    aligned and the row stride is below 2**24 elements (the kernels' limit)."""
    if t.stride(-1) != 1 or t.data_ptr() % 16 != 0:
        return t.contiguous()
    for dim in range(3):
        if t.shape[dim] > 1 and t.stride(dim) % 8 != 0:
            return t.contiguous()
    if t.shape[2] > 1 and t.stride(2) >= _MAX_ROW_STRIDE:
        return t.contiguous()
    return t


def _t4(t: torch.Tensor) -> _lib.Tensor4:
    st = [t.stride(i) if t.shape[i] > 1 else 0 for i in range(3)]
    return _lib.Tensor4(t.data_ptr(), st[0], st[1], st[2])


def _scalar(x, device) -> torch.Tensor:
    if torch.is_tensor(x):
        if x.numel() != 1:
            raise ValueError("ssa_n / ssa_b must be scalar tensors")
        return x.detach().to(device=device, dtype=torch.float32).reshape(()).contiguous()
    return torch.tensor(float(x), dtype=torch.float32, device=device)


# Head dims that run on the kernels of a wider one, with zero-padded columns.
_PADDED_HEAD_DIM = {16: 32}


def _pad_cols(t: torch.Tensor, width: int) -> torch.Tensor:
    """``t`` with its last dim zero-padded to ``width`` (a new contiguous tensor)."""
    return torch.nn.functional.pad(t, (0, width - t.shape[-1]))


def _check_inputs(q, k, v):
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 4-D [B, H, N, D] tensors")
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    assert Hq % Hkv == 0, f"Hq={Hq} must be divisible by Hkv={Hkv}"
    assert _is_pow2(D), f"Head dim D={D} must be a power of two"
    if tuple(k.shape) != (B, Hkv, N, D) or tuple(v.shape) != (B, Hkv, N, D):
        raise ValueError(f"k/v shapes {tuple(k.shape)}/{tuple(v.shape)} do not match q {tuple(q.shape)}")
    if q.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {q.dtype}: the MI355X SSA kernels take bf16, fp16 or fp32")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, v must share one dtype")
    if not (q.is_cuda and k.device == q.device and v.device == q.device):
        raise ValueError("q, k, v must be on the same GPU device")
    return B, Hq, Hkv, N, D


def _padded_width(D: int, dtype: torch.dtype) -> int:
    """Head dim whose bf16 / fp16 kernels run head dim D zero-padded, or 0 (fp32 has its own D = 16 kernels)."""
    return 0 if dtype == torch.float32 else _PADDED_HEAD_DIM.get(D, 0)


def ssa_flash_attn_forward(q, k, v, softmax_scale, ssa_n, ssa_b, causal=True):
    """SSA attention forward.  Returns ``(out [B,Hq,N,D], m [B,Hq,N] fp32)``."""
    B, Hq, Hkv, N, D = _check_inputs(q, k, v)
    w = _padded_width(D, q.dtype)
    if w:
        out, m = ssa_flash_attn_forward(_pad_cols(q, w), _pad_cols(k, w), _pad_cols(v, w), softmax_scale, ssa_n,
                                        ssa_b, causal)
        return out[..., :D].contiguous(), m
    q, k, v = _kernel_layout(q), _kernel_layout(k), _kernel_layout(v)
    n32 = _scalar(ssa_n, q.device)
    b32 = _scalar(ssa_b, q.device)
    out = _kernel_layout(torch.empty_like(q))
    m = torch.empty((B, Hq, N), device=q.device, dtype=torch.float32)
    args = _lib.FwdArgs(
        _t4(q), _t4(k), _t4(v), _t4(out),
        m.data_ptr(), n32.data_ptr(), b32.data_ptr(),
        B, Hq, Hkv, N, D, _DTYPES[q.dtype], int(bool(causal)), float(softmax_scale),
    )
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        _lib.check(_lib.lib().ssa_fwd(ctypes.byref(args), ctypes.c_void_p(stream)), "ssa_fwd")
    return out, m


def _has_ds_path(dtype: torch.dtype, head_dim: int) -> bool:
    """Whether the backward kernels for ``dtype`` / ``head_dim`` can use a dS'
    workspace: the matrix-core kernels (bf16 / fp16 at head dims up to 128)
    can; the fp32-arithmetic vector-ALU kernels (fp32, and head dim 256) always
    recompute the scores in dq and ignore it."""
    return dtype != torch.float32 and head_dim <= 128


def _device_headroom(device) -> int | None:
    """Bytes a new allocation on ``device`` can take without the caching
    allocator asking the driver for more than it has: the driver's free memory
    plus what the allocator holds reserved but unused.  None if unknown."""
    try:
        free, _ = torch.cuda.mem_get_info(device)
        return int(free) + int(torch.cuda.memory_reserved(device)) - int(torch.cuda.memory_allocated(device))
    except (RuntimeError, AssertionError):
        return None


def _use_ds_workspace(nbytes: int, head_dim: int, ds, device=None) -> bool:
    """Whether the backward keeps dS' in a workspace of ``nbytes`` bytes
    (``ds``: True / False to force, None for the ``SSA_BWD_DS`` policy: on
    within ``SSA_BWD_DS_MAX_BYTES`` and, given ``device``, within half of its
    headroom, so that the transient workspace (a per-layer spike of 2 bytes per
    causal pair and head: 1.1 GB at B = 4, H = 16, S = 4096) never takes the
    memory a training step needs; above either bound dq recomputes the scores
    instead).  ``head_dim`` is kept for callers; every head dim measured faster
    with the workspace."""
    if ds is not None:
        return bool(ds)
    mode = os.environ.get("SSA_BWD_DS", "auto").strip().lower()
    if mode in ("0", "off", "false", "no"):
        return False
    if mode in ("1", "on", "true", "yes"):
        return True
    limit = int(os.environ.get("SSA_BWD_DS_MAX_BYTES", str(16 << 30)))
    if not 0 < nbytes <= limit:
        return False
    room = _device_headroom(device) if device is not None else None
    return room is None or nbytes <= room // 2


class BackwardLaunch:
    """Validated backward arguments plus every buffer they point to.

    ``run()`` enqueues the whole backward (``ssa_bwd``); ``run_stage(name)``
    enqueues one of ``preprocess``, ``dkdv``, ``dq``, ``reduce`` (in that order)
    so callers can time or schedule the kernels separately.  ``ds`` selects the
    dS' workspace (True / False; None: the ``SSA_BWD_DS`` policy).
    """

    STAGES = ("preprocess", "dkdv", "dq", "reduce")

    def __init__(self, q, k, v, out, dout, m, softmax_scale, ssa_n, ssa_b, causal=True, ds=None):
        B, Hq, Hkv, N, D = _check_inputs(q, k, v)
        if tuple(out.shape) != tuple(q.shape) or tuple(dout.shape) != tuple(q.shape):
            raise ValueError("out and dout must have the shape of q")
        if out.dtype != q.dtype:
            raise ValueError("out must have the dtype of q")
        self.q, self.k, self.v = _kernel_layout(q), _kernel_layout(k), _kernel_layout(v)
        self.out = _kernel_layout(out)
        self.dout = _kernel_layout(dout.to(q.dtype))
        self.m = m.to(torch.float32).contiguous()
        if tuple(self.m.shape) != (B, Hq, N):
            raise ValueError(f"m must be [B, Hq, N] = {(B, Hq, N)}, got {tuple(self.m.shape)}")
        dev = q.device
        self.n32 = _scalar(ssa_n, dev)
        self.b32 = _scalar(ssa_b, dev)
        self.dq = _kernel_layout(torch.empty_like(self.q))
        self.dk = _kernel_layout(torch.empty_like(self.k))
        self.dv = _kernel_layout(torch.empty_like(self.v))
        self.delta = torch.empty((B, Hq, N), device=dev, dtype=torch.float32)
        self.lib = _lib.lib()
        count = int(self.lib.ssa_bwd_partials_count(B, Hkv, N))
        self.partials = torch.empty(count, device=dev, dtype=torch.float32)
        self.dn = torch.empty((), device=dev, dtype=torch.float32)
        self.db = torch.empty((), device=dev, dtype=torch.float32)
        ds_bytes = int(self.lib.ssa_bwd_ds_workspace_bytes(B, Hq, N, int(bool(causal))))
        self.ds = (torch.empty(ds_bytes, device=dev, dtype=torch.uint8)
                   if _has_ds_path(q.dtype, D) and _use_ds_workspace(ds_bytes, D, ds, dev) else None)
        self.device = dev
        self.args = _lib.BwdArgs(
            _t4(self.q), _t4(self.k), _t4(self.v), _t4(self.out), _t4(self.dout),
            _t4(self.dq), _t4(self.dk), _t4(self.dv),
            self.m.data_ptr(), self.delta.data_ptr(), self.partials.data_ptr(),
            self.dn.data_ptr(), self.db.data_ptr(), self.n32.data_ptr(), self.b32.data_ptr(),
            B, Hq, Hkv, N, D, _DTYPES[q.dtype], int(bool(causal)), float(softmax_scale),
            self.ds.data_ptr() if self.ds is not None else None,
        )

    def _call(self, fn_name: str) -> None:
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device).cuda_stream
            fn = getattr(self.lib, fn_name)
            _lib.check(fn(ctypes.byref(self.args), ctypes.c_void_p(stream)), fn_name)

    def run(self) -> None:
        self._call("ssa_bwd")

    def run_stage(self, name: str) -> None:
        if name not in self.STAGES:
            raise ValueError(f"unknown backward stage {name!r}")
        self._call({"preprocess": "ssa_bwd_preprocess", "dkdv": "ssa_bwd_dkdv",
                    "dq": "ssa_bwd_dq", "reduce": "ssa_bwd_reduce"}[name])

    def results(self):
        return self.dq, self.dk, self.dv, self.dn, self.db


def ssa_flash_attn_backward(q, k, v, out, dout, m, softmax_scale, ssa_n, ssa_b, causal=True, ds=None):
    """SSA attention backward.  Returns ``(dq, dk, dv, dn, db)``; dn/db are 0-d fp32 tensors.
    ``ds``: keep dS' in a workspace (True / False; None: the ``SSA_BWD_DS`` policy)."""
    D = q.shape[-1] if q.dim() == 4 else 0
    w = _padded_width(D, q.dtype)
    if w and tuple(out.shape) == tuple(q.shape) and tuple(dout.shape) == tuple(q.shape):
        dq, dk, dv, dn, db = ssa_flash_attn_backward(
            _pad_cols(q, w), _pad_cols(k, w), _pad_cols(v, w), _pad_cols(out, w), _pad_cols(dout, w), m,
            softmax_scale, ssa_n, ssa_b, causal, ds)
        return dq[..., :D].contiguous(), dk[..., :D].contiguous(), dv[..., :D].contiguous(), dn, db
    launch = BackwardLaunch(q, k, v, out, dout, m, softmax_scale, ssa_n, ssa_b, causal, ds)
    launch.run()
    return launch.results()


def ssa_bwd_preprocess(out, dout):
    """Delta = rowsum(out * dout) in fp32, ``[B, H, N]`` (the backward's first step)."""
    if out.dim() != 4 or tuple(dout.shape) != tuple(out.shape):
        raise ValueError("out and dout must be matching [B, H, N, D] tensors")
    if out.dtype not in _DTYPES or dout.dtype != out.dtype:
        raise ValueError("out/dout must be bf16, fp16 or fp32 with one dtype")
    B, H, N, D = out.shape
    w = _padded_width(D, out.dtype)
    if w:  # zero columns add nothing to the row sums
        out, dout, D = _pad_cols(out, w), _pad_cols(dout, w), w
    out, dout = _kernel_layout(out), _kernel_layout(dout)
    delta = torch.empty((B, H, N), device=out.device, dtype=torch.float32)
    args = _lib.BwdArgs()
    args.out, args.dout = _t4(out), _t4(dout)
    args.delta = delta.data_ptr()
    args.batch, args.heads_q, args.heads_kv, args.seqlen, args.head_dim = B, H, H, N, D
    args.dtype = _DTYPES[out.dtype]
    with torch.cuda.device(out.device):
        stream = torch.cuda.current_stream(out.device).cuda_stream
        _lib.check(_lib.lib().ssa_bwd_preprocess(ctypes.byref(args), ctypes.c_void_p(stream)),
                   "ssa_bwd_preprocess")
    return delta


# ---------------------------------------------------------------------------
# Packed (varlen) sequences: token streams [T, H, D] split into documents by
# cu_seqlens, the layout of Megatron's PackedSeqParams (cu_seqlens_q,
# max_seqlen_q; training/finetune/nemo_patch/data/packed_sequence.py:116-244).
# The reference rejects packed sequences
# (training/train/train_ssa_triton/SSA/ssa_triton_attention.py:154-156); here
# attention (causal or not) stays inside each document.


def _thd_layout(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` ([T, H, D]) or a contiguous copy that the kernels can address."""
    if t.stride(-1) != 1 or t.data_ptr() % 16 != 0:
        return t.contiguous()
    for dim in range(2):
        if t.shape[dim] > 1 and t.stride(dim) % 8 != 0:
            return t.contiguous()
    if t.shape[0] > 1 and t.stride(0) >= _MAX_ROW_STRIDE:
        return t.contiguous()
    return t


def _t3(t: torch.Tensor) -> _lib.Tensor4:
    return _lib.Tensor4(t.data_ptr(), 0, t.stride(1) if t.shape[1] > 1 else 0, t.stride(0) if t.shape[0] > 1 else 0)


def _check_varlen_inputs(q, k, v, cu_seqlens, max_seqlen):
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("packed q, k, v must be 3-D [total_tokens, H, D] tensors")
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    assert Hq % Hkv == 0, f"Hq={Hq} must be divisible by Hkv={Hkv}"
    assert _is_pow2(D), f"Head dim D={D} must be a power of two"
    if tuple(k.shape) != (T, Hkv, D) or tuple(v.shape) != (T, Hkv, D):
        raise ValueError(f"k/v shapes {tuple(k.shape)}/{tuple(v.shape)} do not match q {tuple(q.shape)}")
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, v must share one dtype, bf16, fp16 or fp32")
    if not (q.is_cuda and k.device == q.device and v.device == q.device):
        raise ValueError("q, k, v must be on the same GPU device")
    if not torch.is_tensor(cu_seqlens) or cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must be a 1-D tensor of documents + 1 offsets")
    cu = cu_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
    max_seqlen = int(max_seqlen)
    return cu, cu.numel() - 1, T, Hq, Hkv, D, max_seqlen


def ssa_flash_attn_varlen_forward(q, k, v, cu_seqlens, max_seqlen, softmax_scale, ssa_n, ssa_b, causal=True):
    """Packed-sequence forward.  q [T,Hq,D], k/v [T,Hkv,D], cu_seqlens [docs+1]
    (int32, on the device), max_seqlen = longest document.  Returns
    ``(out [T,Hq,D], m [Hq,T] fp32)``."""
    cu, docs, T, Hq, Hkv, D, max_seqlen = _check_varlen_inputs(q, k, v, cu_seqlens, max_seqlen)
    w = _padded_width(D, q.dtype)
    if w:
        out, m = ssa_flash_attn_varlen_forward(_pad_cols(q, w), _pad_cols(k, w), _pad_cols(v, w), cu, max_seqlen,
                                               softmax_scale, ssa_n, ssa_b, causal)
        return out[..., :D].contiguous(), m
    q, k, v = _thd_layout(q), _thd_layout(k), _thd_layout(v)
    n32 = _scalar(ssa_n, q.device)
    b32 = _scalar(ssa_b, q.device)
    out = _thd_layout(torch.empty_like(q))
    m = torch.empty((Hq, T), device=q.device, dtype=torch.float32)
    dense = _lib.FwdArgs(
        _t3(q), _t3(k), _t3(v), _t3(out),
        m.data_ptr(), n32.data_ptr(), b32.data_ptr(),
        docs, Hq, Hkv, max_seqlen, D, _DTYPES[q.dtype], int(bool(causal)), float(softmax_scale),
    )
    args = _lib.VarlenFwdArgs(dense, cu.data_ptr(), T)
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        _lib.check(_lib.lib().ssa_varlen_fwd(ctypes.byref(args), ctypes.c_void_p(stream)), "ssa_varlen_fwd")
    return out, m


def ssa_flash_attn_varlen_backward(q, k, v, out, dout, m, cu_seqlens, max_seqlen, softmax_scale, ssa_n, ssa_b,
                                   causal=True, ds=None):
    """Packed-sequence backward.  Returns ``(dq, dk, dv, dn, db)``; dn/db are 0-d fp32 tensors.
    ``ds``: keep dS' in a workspace (True / False; None: the ``SSA_BWD_DS`` policy)."""
    cu, docs, T, Hq, Hkv, D, max_seqlen = _check_varlen_inputs(q, k, v, cu_seqlens, max_seqlen)
    if tuple(out.shape) != tuple(q.shape) or tuple(dout.shape) != tuple(q.shape) or out.dtype != q.dtype:
        raise ValueError("out and dout must have the shape (and out the dtype) of q")
    w = _padded_width(D, q.dtype)
    if w:
        dq, dk, dv, dn, db = ssa_flash_attn_varlen_backward(
            _pad_cols(q, w), _pad_cols(k, w), _pad_cols(v, w), _pad_cols(out, w), _pad_cols(dout, w), m, cu,
            max_seqlen, softmax_scale, ssa_n, ssa_b, causal, ds)
        return dq[..., :D].contiguous(), dk[..., :D].contiguous(), dv[..., :D].contiguous(), dn, db
    q, k, v = _thd_layout(q), _thd_layout(k), _thd_layout(v)
    out, dout = _thd_layout(out), _thd_layout(dout.to(q.dtype))
    m = m.to(torch.float32).contiguous()
    if tuple(m.shape) != (Hq, T):
        raise ValueError(f"m must be [Hq, T] = {(Hq, T)}, got {tuple(m.shape)}")
    dev = q.device
    n32 = _scalar(ssa_n, dev)
    b32 = _scalar(ssa_b, dev)
    dq = _thd_layout(torch.empty_like(q))
    dk = _thd_layout(torch.empty_like(k))
    dv = _thd_layout(torch.empty_like(v))
    delta = torch.empty((Hq, T), device=dev, dtype=torch.float32)
    lib = _lib.lib()
    partials = torch.empty(max(int(lib.ssa_bwd_partials_count(docs, Hkv, max(max_seqlen, 1))), 1),
                           device=dev, dtype=torch.float32)
    dn = torch.empty((), device=dev, dtype=torch.float32)
    db = torch.empty((), device=dev, dtype=torch.float32)
    ds_bytes = int(lib.ssa_varlen_bwd_ds_workspace_bytes(docs, Hq, max_seqlen, T, int(bool(causal))))
    ds_ws = (torch.empty(ds_bytes, device=dev, dtype=torch.uint8)
             if ds_bytes > 0 and _has_ds_path(q.dtype, D) and _use_ds_workspace(ds_bytes, D, ds, dev) else None)
    dense = _lib.BwdArgs(
        _t3(q), _t3(k), _t3(v), _t3(out), _t3(dout), _t3(dq), _t3(dk), _t3(dv),
        m.data_ptr(), delta.data_ptr(), partials.data_ptr(), dn.data_ptr(), db.data_ptr(),
        n32.data_ptr(), b32.data_ptr(),
        docs, Hq, Hkv, max_seqlen, D, _DTYPES[q.dtype], int(bool(causal)), float(softmax_scale),
        ds_ws.data_ptr() if ds_ws is not None else None,
    )
    args = _lib.VarlenBwdArgs(dense, cu.data_ptr(), T)
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        _lib.check(lib.ssa_varlen_bwd(ctypes.byref(args), ctypes.c_void_p(stream)), "ssa_varlen_bwd")
    return dq, dk, dv, dn, db


def warmup_ssa_triton_kernels(
    B: int = 2,
    Hq: int = 24,
    Hkv: int = 8,
    N: int = 128,
    D: int = 32,
    dtype: torch.dtype = torch.bfloat16,
    device: str = "cuda",
):
    """Run one tiny causal forward + backward (loads the library and its code objects)."""
    q = torch.randn(B, Hq, N, D, dtype=dtype, device=device)
    k = torch.randn(B, Hkv, N, D, dtype=dtype, device=device)
    v = torch.randn(B, Hkv, N, D, dtype=dtype, device=device)
    ssa_n = torch.tensor(1.5, dtype=torch.float32, device=device)
    ssa_b = torch.tensor(0.8, dtype=torch.float32, device=device)
    scale = 1.0 / (D ** 0.5)
    out, m = ssa_flash_attn_forward(q, k, v, scale, ssa_n, ssa_b, causal=True)
    dout = torch.randn_like(out)
    ssa_flash_attn_backward(q, k, v, out, dout, m, scale, ssa_n, ssa_b, causal=True)
    torch.cuda.synchronize()


def _check_cache_layout(t: torch.Tensor, name: str) -> None:
    """A KV cache is used in place (a copy per decode step would cost more than
    the step): its layout must already suit the kernels."""
    if t.stride(-1) != 1 or t.data_ptr() % 16 != 0:
        raise ValueError(f"{name}: last dim must be contiguous and the base 16-byte aligned")
    for dim in range(3):
        if t.shape[dim] > 1 and (t.stride(dim) % 8 != 0 or t.stride(dim) < 0):
            raise ValueError(f"{name}: strides must be non-negative multiples of 8 elements")
    if t.shape[2] > 1 and t.stride(2) >= _MAX_ROW_STRIDE:
        raise ValueError(f"{name}: row stride must be below 2**24 elements")


def ssa_decode_num_splits(B: int, Hq: int, Hkv: int, capacity: int, num_splits: int = 0) -> int:
    """Key splits the decode kernel uses (``num_splits`` = 0: its own choice)."""
    return int(_lib.lib().ssa_decode_num_splits(B, Hq, Hkv, capacity, num_splits))


def ssa_decode_attention(q, k_cache, v_cache, cache_seqlens, softmax_scale, ssa_n, ssa_b, num_splits=0,
                         return_m=False):
    """One decode step: the newest token of every sequence attends its KV cache.

    ``q`` is ``[B, Hq, D]`` or ``[B, Hq, 1, D]``; ``k_cache`` / ``v_cache`` are
    ``[B, Hkv, capacity, D]`` (any strides whose last one is 1, used in place);
    ``cache_seqlens`` holds int32 lengths ``[B]``: sequence b attends cache rows
    ``0 .. cache_seqlens[b] - 1`` and the newest token's key / value are already
    at row ``cache_seqlens[b] - 1``.  Returns ``out`` shaped like ``q`` (and
    ``m [B, Hq]`` fp32 with ``return_m``), equal to the last row of
    ``ssa_flash_attn_forward(causal=True)`` over the cached prefix.  Lengths are
    read on the device (clamped to ``[0, capacity]``; an empty cache gives
    ``out = 0``, ``m = -inf``).  No reference counterpart: the reference's
    generation loop re-runs the whole prefix per token
    (training/train/train_ssa_triton/generate_triton.py:315-331).
    """
    squeeze = q.dim() == 3
    q4 = q.unsqueeze(2) if squeeze else q
    if q4.dim() != 4 or q4.shape[2] != 1:
        raise ValueError("q must be [B, Hq, D] or [B, Hq, 1, D]")
    if k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError("k_cache / v_cache must be [B, Hkv, capacity, D]")
    B, Hq, _, D = q4.shape
    Hkv, cap = k_cache.shape[1], k_cache.shape[2]
    assert Hq % Hkv == 0, f"Hq={Hq} must be divisible by Hkv={Hkv}"
    assert _is_pow2(D), f"Head dim D={D} must be a power of two"
    if tuple(k_cache.shape) != (B, Hkv, cap, D) or tuple(v_cache.shape) != (B, Hkv, cap, D):
        raise ValueError(f"cache shapes {tuple(k_cache.shape)}/{tuple(v_cache.shape)} do not match q {tuple(q.shape)}")
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"unsupported dtype {q.dtype}: the decode step takes bf16 or fp16")
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise ValueError("q and the caches must share one dtype")
    if not (q.is_cuda and k_cache.device == q.device and v_cache.device == q.device):
        raise ValueError("q and the caches must be on the same GPU device")
    _check_cache_layout(k_cache, "k_cache")
    _check_cache_layout(v_cache, "v_cache")
    q4 = _kernel_layout(q4)
    lens = torch.as_tensor(cache_seqlens, device=q.device)
    if lens.shape != (B,):
        raise ValueError(f"cache_seqlens must have shape ({B},)")
    lens = lens.to(torch.int32).contiguous()
    n32 = _scalar(ssa_n, q.device)
    b32 = _scalar(ssa_b, q.device)
    out = torch.empty((B, Hq, 1, D), dtype=q.dtype, device=q.device)
    m = torch.empty((B, Hq), dtype=torch.float32, device=q.device) if return_m else None
    ws_bytes = int(_lib.lib().ssa_decode_workspace_bytes(B, Hq, Hkv, cap, D, int(num_splits)))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes > 0 else None
    args = _lib.DecodeArgs(
        _t4(q4), _t4(k_cache), _t4(v_cache), _t4(out),
        m.data_ptr() if m is not None else None, lens.data_ptr(), n32.data_ptr(), b32.data_ptr(),
        B, Hq, Hkv, cap, D, _DTYPES[q.dtype], int(num_splits), float(softmax_scale),
        ws.data_ptr() if ws is not None else None,
    )
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        _lib.check(_lib.lib().ssa_decode(ctypes.byref(args), ctypes.c_void_p(stream)), "ssa_decode")
    out = out.squeeze(2) if squeeze else out
    return (out, m) if return_m else out
