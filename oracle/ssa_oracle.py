"""CPU oracle for SSA (softmax-substituted) attention, float64 numpy.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker.  The product path (``luciole-1b_amd/SSA``) never imports it and fails
loudly when the HIP library is missing.

This is a closed-form restatement of the reference's SSA math:

* forward transform ``t = n * sign(s) * log1p(b * |s|)`` with
  ``s = scale * Q K^T`` -- ``training/train/train_ssa_triton/SSA/ssa_triton_kernel.py:95-107``
  and the fp32 oracle ``training/train/train_ssa_triton/check_ssa_triton_parity.py:169-206``;
* softmax over ``t`` per query row, GQA by ``kv_head = q_head // G``
  (``ssa_triton_kernel.py:192-194``, ``check_ssa_triton_parity.py:183-185``);
  the softmax is max-subtracted here, where the reference oracle's plain
  ``w / sum(w)`` (``check_ssa_triton_parity.py:202-204``) overflows for trained
  values such as n = -302;
* stored normaliser ``M = log2(sum_j exp(t_j))`` (``ssa_triton_kernel.py:247-255``);
* backward chain rule ``dT = P (dP - Delta)``, ``dS = dT * n b / (1 + b|s|)``,
  ``dn = sum dT sign(s) log1p(b|s|)``, ``db = sum dT n sign(s) |s| / (1 + b|s|)``
  (``ssa_triton_kernel.py:371-397,467-477``), with
  ``Delta = rowsum(dO * O)`` (``ssa_triton_kernel.py:267-298``).

Varlen (packed sequences, block-diagonal causal over ``cu_seqlens``) has no
reference implementation (the reference asserts ``packed_seq_params is None``,
``SSA/ssa_triton_attention.py:154-156``); it is defined here as the
concatenation of independent dense runs, one per document.

Decode against a KV cache has no reference kernel either (the reference's
generation loop re-runs the prefix, ``generate_triton.py:315-331``); it is
defined here as the last row of the causal forward over the cached prefix.

Pinning (tests/test_oracle.py): brute-force pure-Python loops plus central
finite differences on tiny inputs, torch float64 autograd of an independent
restatement, n = 0 (cumulative mean), b -> 0 with n b = 1 (softmax attention,
checked against torch's scaled_dot_product_attention), single-key rows,
``M`` against scipy's logsumexp, GQA against repeat_interleave, varlen against
per-document dense runs, causal prefix independence, decode against the
last row of the causal forward.
"""

from __future__ import annotations

import math

import numpy as np

LN2 = math.log(2.0)


def _expand_kv(x: np.ndarray, group: int) -> np.ndarray:
    """[B, Hkv, N, D] -> [B, Hkv*group, N, D], head h reads kv head h // group."""
    return np.repeat(x, group, axis=1)


def _mask(nq: int, nk: int, causal: bool) -> np.ndarray:
    """Valid (q, k) pairs.  Causal is top-left aligned (key j visible to query i iff j <= i)."""
    if not causal:
        return np.ones((nq, nk), dtype=bool)
    return np.arange(nk)[None, :] <= np.arange(nq)[:, None]


def ssa_logits(s: np.ndarray, n: float, b: float) -> np.ndarray:
    """t(s) = n * sign(s) * log1p(b |s|)  (ssa_triton_kernel.py:98-105)."""
    return n * np.sign(s) * np.log1p(b * np.abs(s))


def ssa_forward(q, k, v, scale, n, b, causal=True):
    """Dense SSA attention forward in float64.

    q: [B, Hq, N, D]; k, v: [B, Hkv, N, D].  Returns (out [B,Hq,N,D], M [B,Hq,N])
    where M = log2(sum_j exp(t_ij)) over valid keys (-inf for a row with none).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    bsz, hq, nq, _ = q.shape
    hkv = k.shape[1]
    if hq % hkv != 0:
        raise ValueError(f"Hq={hq} must be divisible by Hkv={hkv}")
    g = hq // hkv
    ke, ve = _expand_kv(k, g), _expand_kv(v, g)
    s = scale * (q @ ke.swapaxes(-1, -2))
    valid = _mask(nq, k.shape[2], causal)[None, None]
    t = np.where(valid, ssa_logits(s, n, b), -np.inf)
    tmax = np.max(t, axis=-1, keepdims=True)
    tmax_safe = np.where(np.isfinite(tmax), tmax, 0.0)
    w = np.where(valid, np.exp(t - tmax_safe), 0.0)
    l = w.sum(axis=-1, keepdims=True)
    p = np.where(l > 0, w / np.where(l > 0, l, 1.0), 0.0)
    out = p @ ve
    with np.errstate(divide="ignore"):
        m = ((tmax_safe + np.log(l)) / LN2)[..., 0]
    return out, m


def ssa_backward(q, k, v, dout, scale, n, b, causal=True, out_for_delta=None):
    """Closed-form SSA backward in float64 (loss = sum(out * dout)).

    Returns (dq, dk, dv, dn, db, delta) with delta = rowsum(dout * out).
    ``out_for_delta``: the forward output the kernel-level backward was given
    (``ssa_flash_attn_backward(q, k, v, out, dout, m, ...)`` takes it as an
    input and its preprocess forms delta from it, ssa_triton_kernel.py:291-294);
    when None, the exact float64 output is used.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    do = np.asarray(dout, dtype=np.float64)
    bsz, hq, nq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    ke, ve = _expand_kv(k, g), _expand_kv(v, g)
    s = scale * (q @ ke.swapaxes(-1, -2))
    valid = _mask(nq, k.shape[2], causal)[None, None]
    s0 = np.where(valid, s, 0.0)
    lg = np.log1p(b * np.abs(s0))
    t = np.where(valid, n * np.sign(s0) * lg, -np.inf)
    tmax = np.max(t, axis=-1, keepdims=True)
    tmax = np.where(np.isfinite(tmax), tmax, 0.0)
    w = np.where(valid, np.exp(t - tmax), 0.0)
    l = w.sum(axis=-1, keepdims=True)
    p = np.where(l > 0, w / np.where(l > 0, l, 1.0), 0.0)
    out = p @ ve if out_for_delta is None else np.asarray(out_for_delta, dtype=np.float64)
    delta = np.sum(do * out, axis=-1)
    dp = do @ ve.swapaxes(-1, -2)
    dt = p * (dp - delta[..., None])
    ds = dt * (n * b / (1.0 + b * np.abs(s0)))
    dq = scale * (ds @ ke)
    dk_e = scale * (ds.swapaxes(-1, -2) @ q)
    dv_e = p.swapaxes(-1, -2) @ do
    dk = dk_e.reshape(bsz, hkv, g, *dk_e.shape[2:]).sum(axis=2)
    dv = dv_e.reshape(bsz, hkv, g, *dv_e.shape[2:]).sum(axis=2)
    sg = np.sign(s0)
    dn = float(np.sum(dt * sg * lg))
    db = float(np.sum(dt * n * sg * np.abs(s0) / (1.0 + b * np.abs(s0))))
    return dq, dk, dv, dn, db, delta


def ssa_forward_backward(q, k, v, dout, scale, n, b, causal=True, out_for_delta=None):
    """Forward and backward in one call: dict with out, m, dq, dk, dv, dn, db, delta."""
    out, m = ssa_forward(q, k, v, scale, n, b, causal)
    dq, dk, dv, dn, db, delta = ssa_backward(q, k, v, dout, scale, n, b, causal, out_for_delta)
    return {"out": out, "m": m, "dq": dq, "dk": dk, "dv": dv, "dn": dn, "db": db, "delta": delta}


def ssa_forward_backward_chunked(q, k, v, dout, scale, n, b, causal=True, out_for_delta=None, chunk=512):
    """``ssa_forward_backward`` evaluated one block of ``chunk`` query rows at a
    time, so that no [N, N] matrix is built whole (a 16k x 16k float64 score
    matrix alone is 2 GiB).  Every row's softmax, and so every quantity of the
    forward and of dq, is a function of that row alone; dk, dv, dn and db are
    sums over rows and are accumulated block by block.  Same arguments and
    result keys as ``ssa_forward_backward`` (pinned against it in
    tests/test_oracle.py).  The math is the dense function's:
    ``check_ssa_triton_parity.py:169-237`` and ``ssa_triton_kernel.py:359-397``.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    do = np.asarray(dout, dtype=np.float64)
    ofd = None if out_for_delta is None else np.asarray(out_for_delta, dtype=np.float64)
    bsz, hq, nq, d = q.shape
    hkv, nk = k.shape[1], k.shape[2]
    if hq % hkv != 0:
        raise ValueError(f"Hq={hq} must be divisible by Hkv={hkv}")
    g = hq // hkv
    res = {
        "out": np.zeros((bsz, hq, nq, d)),
        "m": np.full((bsz, hq, nq), -np.inf),
        "delta": np.zeros((bsz, hq, nq)),
        "dq": np.zeros((bsz, hq, nq, d)),
        "dk": np.zeros((bsz, hkv, nk, d)),
        "dv": np.zeros((bsz, hkv, nk, d)),
        "dn": 0.0,
        "db": 0.0,
    }
    for bi in range(bsz):
        for h in range(hq):
            kh, vh = k[bi, h // g], v[bi, h // g]
            for a in range(0, nq, chunk):
                e = min(a + chunk, nq)
                ke = min(e, nk) if causal else nk  # keys any row of the block can see
                if ke <= 0:
                    continue
                qc, doc = q[bi, h, a:e], do[bi, h, a:e]
                s = scale * (qc @ kh[:ke].T)
                if causal:  # key j visible to query i iff j <= i (top-left aligned)
                    valid = np.arange(ke)[None, :] <= np.arange(a, e)[:, None]
                else:
                    valid = np.ones((e - a, ke), dtype=bool)
                s0 = np.where(valid, s, 0.0)
                lg = np.log1p(b * np.abs(s0))
                sg = np.sign(s0)
                t = np.where(valid, n * sg * lg, -np.inf)
                tmax = np.max(t, axis=-1, keepdims=True)
                tmax = np.where(np.isfinite(tmax), tmax, 0.0)
                w = np.where(valid, np.exp(t - tmax), 0.0)
                l = w.sum(axis=-1, keepdims=True)
                p = np.where(l > 0, w / np.where(l > 0, l, 1.0), 0.0)
                out = p @ vh[:ke]
                res["out"][bi, h, a:e] = out
                with np.errstate(divide="ignore"):
                    res["m"][bi, h, a:e] = ((tmax + np.log(l)) / LN2)[:, 0]
                oc = out if ofd is None else ofd[bi, h, a:e]
                delta = np.sum(doc * oc, axis=-1)
                res["delta"][bi, h, a:e] = delta
                dp = doc @ vh[:ke].T
                dt = p * (dp - delta[:, None])
                ds = dt * (n * b / (1.0 + b * np.abs(s0)))
                res["dq"][bi, h, a:e] = scale * (ds @ kh[:ke])
                res["dk"][bi, h // g, :ke] += scale * (ds.T @ qc)
                res["dv"][bi, h // g, :ke] += p.T @ doc
                res["dn"] += float(np.sum(dt * sg * lg))
                res["db"] += float(np.sum(dt * n * sg * np.abs(s0) / (1.0 + b * np.abs(s0))))
    return res


def ssa_varlen_forward_backward(q, k, v, dout, cu_seqlens, scale, n, b, causal=True, out_for_delta=None):
    """Packed-sequence SSA: q [T, Hq, D], k/v [T, Hkv, D], cu_seqlens int [ndocs+1].

    Each document [cu[i], cu[i+1]) attends only within itself (block-diagonal,
    causal inside each block when ``causal``).  Returns a dict like
    ``ssa_forward_backward`` with token-major tensors ([T, H, D], m/delta [T, H]).
    ``out_for_delta`` ([T, Hq, D]) has the meaning it has in
    ``ssa_forward_backward``, per document.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    do = np.asarray(dout, dtype=np.float64)
    cu = [int(x) for x in np.asarray(cu_seqlens).tolist()]
    tot, hq, d = q.shape
    hkv = k.shape[1]
    res = {
        "out": np.zeros((tot, hq, d)),
        "m": np.full((tot, hq), -np.inf),
        "delta": np.zeros((tot, hq)),
        "dq": np.zeros((tot, hq, d)),
        "dk": np.zeros((tot, hkv, d)),
        "dv": np.zeros((tot, hkv, d)),
        "dn": 0.0,
        "db": 0.0,
    }
    for i in range(len(cu) - 1):
        a, e = cu[i], cu[i + 1]
        if e <= a:
            continue

        def dense(x):
            return x[a:e].transpose(1, 0, 2)[None]

        ofd = None if out_for_delta is None else dense(np.asarray(out_for_delta, dtype=np.float64))
        r = ssa_forward_backward(dense(q), dense(k), dense(v), dense(do), scale, n, b, causal, ofd)
        res["out"][a:e] = r["out"][0].transpose(1, 0, 2)
        res["m"][a:e] = r["m"][0].T
        res["delta"][a:e] = r["delta"][0].T
        res["dq"][a:e] = r["dq"][0].transpose(1, 0, 2)
        res["dk"][a:e] = r["dk"][0].transpose(1, 0, 2)
        res["dv"][a:e] = r["dv"][0].transpose(1, 0, 2)
        res["dn"] += r["dn"]
        res["db"] += r["db"]
    return res


def ssa_decode(q, k_cache, v_cache, seqlens, scale, n, b):
    """One decode step: q [B, Hq, D] (the newest token of each sequence),
    caches [B, Hkv, cap, D], seqlens [B] (clamped to [0, cap]).  Sequence b's
    query attends cache rows 0 .. L_b - 1: the single query of a non-causal
    forward over those rows, which is the last row of the causal forward over
    the prefix.  Returns (out [B, Hq, D], m [B, Hq]); an empty cache gives
    out = 0, m = -inf."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k_cache, dtype=np.float64)
    v = np.asarray(v_cache, dtype=np.float64)
    bsz, hq, d = q.shape
    cap = k.shape[2]
    out = np.zeros((bsz, hq, d))
    m = np.full((bsz, hq), -np.inf)
    for i in range(bsz):
        L = min(max(int(np.asarray(seqlens)[i]), 0), cap)
        if L == 0:
            continue
        o, mm = ssa_forward(q[i : i + 1, :, None], k[i : i + 1, :, :L], v[i : i + 1, :, :L], scale, n, b, causal=False)
        out[i] = o[0, :, 0]
        m[i] = mm[0, :, 0]
    return out, m


def causal_pairs(bsz: int, hq: int, n: int, causal: bool = True) -> int:
    """Number of unmasked (q, k) pairs for a dense launch."""
    return bsz * hq * (n * (n + 1) // 2 if causal else n * n)


def varlen_pairs(cu_seqlens, hq: int, causal: bool = True) -> int:
    cu = [int(x) for x in np.asarray(cu_seqlens).tolist()]
    tot = 0
    for i in range(len(cu) - 1):
        L = cu[i + 1] - cu[i]
        tot += L * (L + 1) // 2 if causal else L * L
    return hq * tot
