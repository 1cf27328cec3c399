"""Pins the CPU oracle (oracle/ssa_oracle.py) before anything is compared to it.

Each check is independent of the closed form being tested: brute-force loops
with central finite differences, torch float64 autograd of a separate
restatement, special cases that reduce to known results (cumulative mean,
softmax attention, a single key), scipy's logsumexp, and structural
invariants (GQA, varlen, causal prefix, key permutation).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import ssa_oracle as so
from oracle import ssa_oracle_torch as sot

N_VALUES = [1.5, 4.0, -3.484375, 0.0, -302.0]


def _rand(rng, *shape, scale=1.0):
    return rng.standard_normal(shape) * scale


# --------------------------------------------------------------------------
# brute force: pure-Python loops + central finite differences


def _bruteforce_out(q, k, v, scale, n, b, causal):
    B, Hq, N, D = q.shape
    G = Hq // k.shape[1]
    out = np.zeros_like(q)
    for bi in range(B):
        for h in range(Hq):
            hk = h // G
            for i in range(N):
                ts = []
                for j in range(N):
                    if causal and j > i:
                        continue
                    s = scale * sum(float(q[bi, h, i, d]) * float(k[bi, hk, j, d]) for d in range(D))
                    sg = (1.0 if s > 0 else 0.0) - (1.0 if s < 0 else 0.0)
                    ts.append((j, n * sg * math.log1p(b * abs(s))))
                mx = max(t for _, t in ts)
                ws = [(j, math.exp(t - mx)) for j, t in ts]
                z = sum(w for _, w in ws)
                for j, w in ws:
                    for d in range(D):
                        out[bi, h, i, d] += w / z * v[bi, hk, j, d]
    return out


def _loss(q, k, v, do, scale, n, b, causal):
    return float(np.sum(_bruteforce_out(q, k, v, scale, n, b, causal) * do))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("n_val", [1.5, -3.484375])
def test_closed_form_matches_bruteforce_finite_differences(causal, n_val):
    rng = np.random.default_rng(7)
    B, Hq, Hkv, N, D = 1, 2, 1, 4, 3
    q, k, v, do = (_rand(rng, B, Hq, N, D), _rand(rng, B, Hkv, N, D),
                   _rand(rng, B, Hkv, N, D), _rand(rng, B, Hq, N, D))
    scale, b = 0.7, 0.8
    r = so.ssa_forward_backward(q, k, v, do, scale, n_val, b, causal)
    np.testing.assert_allclose(r["out"], _bruteforce_out(q, k, v, scale, n_val, b, causal), rtol=1e-12, atol=1e-12)
    eps = 1e-6

    def fd(arr, idx):
        a0 = arr[idx]
        arr[idx] = a0 + eps
        lp = _loss(q, k, v, do, scale, n_val, b, causal)
        arr[idx] = a0 - eps
        lm = _loss(q, k, v, do, scale, n_val, b, causal)
        arr[idx] = a0
        return (lp - lm) / (2 * eps)

    for name, arr in (("dq", q), ("dk", k), ("dv", v)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            num[idx] = fd(arr, idx)
        np.testing.assert_allclose(r[name], num, rtol=1e-5, atol=1e-7, err_msg=name)
    dn_num = (_loss(q, k, v, do, scale, n_val + eps, b, causal) - _loss(q, k, v, do, scale, n_val - eps, b, causal)) / (2 * eps)
    db_num = (_loss(q, k, v, do, scale, n_val, b + eps, causal) - _loss(q, k, v, do, scale, n_val, b - eps, causal)) / (2 * eps)
    assert r["dn"] == pytest.approx(dn_num, rel=1e-5, abs=1e-8)
    assert r["db"] == pytest.approx(db_num, rel=1e-5, abs=1e-8)


# --------------------------------------------------------------------------
# torch float64 autograd of an independent restatement


@pytest.mark.parametrize("n_val", N_VALUES)
@pytest.mark.parametrize("causal", [True, False])
def test_closed_form_matches_torch_autograd(n_val, causal):
    g = torch.Generator().manual_seed(1234)
    B, Hq, Hkv, N, D = 2, 4, 2, 33, 16
    q = torch.randn(B, Hq, N, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, Hkv, N, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, Hkv, N, D, generator=g, dtype=torch.float64)
    do = torch.randn(B, Hq, N, D, generator=g, dtype=torch.float64)
    scale = 1.0 / math.sqrt(D)
    ref = sot.run_reference_grads(q, k, v, scale, torch.tensor(n_val, dtype=torch.float64),
                                  torch.tensor(0.8, dtype=torch.float64), do, causal)
    r = so.ssa_forward_backward(q.numpy(), k.numpy(), v.numpy(), do.numpy(), scale, n_val, 0.8, causal)
    for name in ("out", "m", "dq", "dk", "dv"):
        np.testing.assert_allclose(r[name], ref[name].numpy(), rtol=1e-9, atol=1e-9, err_msg=name)
    assert r["dn"] == pytest.approx(ref["dn"], rel=1e-9, abs=1e-9)
    assert r["db"] == pytest.approx(ref["db"], rel=1e-9, abs=1e-9)


def test_torch_oracle_gradcheck_tiny():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 2, 5, 4, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.randn(1, 1, 5, 4, generator=g, dtype=torch.float64, requires_grad=True)
    v = torch.randn(1, 1, 5, 4, generator=g, dtype=torch.float64, requires_grad=True)
    n = torch.tensor(1.5, dtype=torch.float64, requires_grad=True)
    b = torch.tensor(0.8, dtype=torch.float64, requires_grad=True)
    f = lambda q, k, v, n, b: sot.ssa_reference_forward(q, k, v, 0.5, n, b, True)[0]  # noqa: E731
    assert torch.autograd.gradcheck(f, (q, k, v, n, b), eps=1e-6, atol=1e-6)


# --------------------------------------------------------------------------
# special cases


@pytest.mark.parametrize("causal", [True, False])
def test_n_zero_is_uniform_mean(causal):
    rng = np.random.default_rng(1)
    q, k, v = _rand(rng, 1, 2, 17, 8), _rand(rng, 1, 2, 17, 8), _rand(rng, 1, 2, 17, 8)
    out, m = so.ssa_forward(q, k, v, 0.3, 0.0, 0.8, causal)
    if causal:
        expect = np.cumsum(v, axis=2) / np.arange(1, 18)[None, None, :, None]
        cnt = np.arange(1, 18)
    else:
        expect = np.broadcast_to(v.mean(axis=2, keepdims=True), v.shape)
        cnt = np.full(17, 17)
    np.testing.assert_allclose(out, expect, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(m, np.broadcast_to(np.log2(cnt), m.shape), rtol=1e-12)


def test_small_b_reduces_to_softmax_attention():
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 3, 40, 16, generator=g, dtype=torch.float64)
    k = torch.randn(1, 3, 40, 16, generator=g, dtype=torch.float64)
    v = torch.randn(1, 3, 40, 16, generator=g, dtype=torch.float64)
    b = 1e-7
    out, _ = so.ssa_forward(q.numpy(), k.numpy(), v.numpy(), 0.25, 1.0 / b, b, True)
    sdpa = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True, scale=0.25)
    np.testing.assert_allclose(out, sdpa.numpy(), rtol=0, atol=1e-5)


def test_single_key_row_returns_v0():
    rng = np.random.default_rng(2)
    q, k, v = _rand(rng, 2, 2, 1, 8), _rand(rng, 2, 2, 1, 8), _rand(rng, 2, 2, 1, 8)
    for n_val in N_VALUES:
        out, m = so.ssa_forward(q, k, v, 0.5, n_val, 0.8, True)
        np.testing.assert_array_equal(out, v)
        s = 0.5 * np.sum(q * k, axis=-1)
        np.testing.assert_allclose(m, so.ssa_logits(s, n_val, 0.8) / math.log(2.0), rtol=1e-12, atol=1e-12)


def test_normaliser_is_logsumexp_base2():
    from scipy.special import logsumexp

    rng = np.random.default_rng(4)
    q, k, v = _rand(rng, 1, 1, 23, 8), _rand(rng, 1, 1, 23, 8), _rand(rng, 1, 1, 23, 8)
    for n_val in N_VALUES:
        _, m = so.ssa_forward(q, k, v, 0.4, n_val, 0.8, True)
        s = 0.4 * q[0, 0] @ k[0, 0].T
        t = so.ssa_logits(s, n_val, 0.8)
        expect = [logsumexp(t[i, : i + 1]) / math.log(2.0) for i in range(23)]
        np.testing.assert_allclose(m[0, 0], expect, rtol=1e-12, atol=1e-9)


def test_extreme_n_stays_finite():
    rng = np.random.default_rng(6)
    q, k, v, do = (_rand(rng, 1, 2, 64, 16), _rand(rng, 1, 2, 64, 16), _rand(rng, 1, 2, 64, 16),
                   _rand(rng, 1, 2, 64, 16))
    r = so.ssa_forward_backward(q, k, v, do, 0.25, -302.0, 0.8, True)
    for name in ("out", "m", "dq", "dk", "dv"):
        assert np.all(np.isfinite(r[name])), name
    assert math.isfinite(r["dn"]) and math.isfinite(r["db"])


# --------------------------------------------------------------------------
# structural invariants


def test_gqa_equals_repeat_interleave():
    rng = np.random.default_rng(8)
    B, Hq, Hkv, N, D = 2, 6, 2, 19, 8
    q, k, v, do = (_rand(rng, B, Hq, N, D), _rand(rng, B, Hkv, N, D), _rand(rng, B, Hkv, N, D),
                   _rand(rng, B, Hq, N, D))
    r = so.ssa_forward_backward(q, k, v, do, 0.3, 1.5, 0.8, True)
    ke, ve = np.repeat(k, 3, axis=1), np.repeat(v, 3, axis=1)
    re = so.ssa_forward_backward(q, ke, ve, do, 0.3, 1.5, 0.8, True)
    np.testing.assert_allclose(r["out"], re["out"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(r["dq"], re["dq"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(r["dk"], re["dk"].reshape(B, Hkv, 3, N, D).sum(2), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(r["dv"], re["dv"].reshape(B, Hkv, 3, N, D).sum(2), rtol=1e-12, atol=1e-12)
    assert r["dn"] == pytest.approx(re["dn"], rel=1e-12)


def test_causal_prefix_independence():
    rng = np.random.default_rng(9)
    q, k, v = _rand(rng, 1, 2, 30, 8), _rand(rng, 1, 2, 30, 8), _rand(rng, 1, 2, 30, 8)
    out, m = so.ssa_forward(q, k, v, 0.35, -3.484375, 0.8, True)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 20:] += 5.0
    v2[:, :, 20:] -= 3.0
    out2, m2 = so.ssa_forward(q, k2, v2, 0.35, -3.484375, 0.8, True)
    np.testing.assert_array_equal(out[:, :, :20], out2[:, :, :20])
    np.testing.assert_array_equal(m[:, :, :20], m2[:, :, :20])
    assert not np.allclose(out[:, :, 20:], out2[:, :, 20:])


def test_noncausal_key_permutation_invariance():
    rng = np.random.default_rng(10)
    q, k, v = _rand(rng, 1, 1, 12, 8), _rand(rng, 1, 1, 12, 8), _rand(rng, 1, 1, 12, 8)
    perm = rng.permutation(12)
    out, m = so.ssa_forward(q, k, v, 0.5, 4.0, 0.8, False)
    out2, m2 = so.ssa_forward(q, k[:, :, perm], v[:, :, perm], 0.5, 4.0, 0.8, False)
    np.testing.assert_allclose(out, out2, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(m, m2, rtol=1e-12, atol=1e-12)


def test_varlen_equals_per_document_dense():
    rng = np.random.default_rng(11)
    cu = np.array([0, 5, 6, 19, 32], dtype=np.int32)
    T, Hq, Hkv, D = 32, 4, 2, 8
    q, k, v, do = (_rand(rng, T, Hq, D), _rand(rng, T, Hkv, D), _rand(rng, T, Hkv, D), _rand(rng, T, Hq, D))
    r = so.ssa_varlen_forward_backward(q, k, v, do, cu, 0.3, 1.5, 0.8, True)
    dn = db = 0.0
    for a, e in zip(cu[:-1], cu[1:]):
        dense = lambda x: x[a:e].transpose(1, 0, 2)[None]  # noqa: E731
        rd = so.ssa_forward_backward(dense(q), dense(k), dense(v), dense(do), 0.3, 1.5, 0.8, True)
        np.testing.assert_allclose(r["out"][a:e], rd["out"][0].transpose(1, 0, 2), rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(r["dk"][a:e], rd["dk"][0].transpose(1, 0, 2), rtol=1e-12, atol=1e-12)
        dn += rd["dn"]
        db += rd["db"]
    assert r["dn"] == pytest.approx(dn, rel=1e-12)
    assert r["db"] == pytest.approx(db, rel=1e-12)
    # a packed batch differs from one long causal sequence over the same tokens
    full = so.ssa_forward(q.transpose(1, 0, 2)[None], k.transpose(1, 0, 2)[None], v.transpose(1, 0, 2)[None],
                          0.3, 1.5, 0.8, True)[0]
    assert not np.allclose(full[0].transpose(1, 0, 2)[5:], r["out"][5:])


def test_pair_counts():
    assert so.causal_pairs(4, 16, 4096) == 537_001_984
    assert so.causal_pairs(4, 16, 2048) == 134_283_264
    assert so.causal_pairs(1, 16, 16384) == 2_147_614_720
    assert so.causal_pairs(1, 4, 256) == 131_584
    assert so.varlen_pairs([0, 3, 5], 2) == 2 * (6 + 3)


def test_out_for_delta_only_moves_delta_terms():
    # dV does not depend on Delta; with the exact out the results are identical;
    # Delta = rowsum(P * dP) when out is exact (softmax-backward identity).
    rng = np.random.default_rng(12)
    q, k, v, do = (_rand(rng, 1, 2, 20, 8), _rand(rng, 1, 2, 20, 8), _rand(rng, 1, 2, 20, 8),
                   _rand(rng, 1, 2, 20, 8))
    r = so.ssa_forward_backward(q, k, v, do, 0.3, 1.5, 0.8, True)
    r_same = so.ssa_forward_backward(q, k, v, do, 0.3, 1.5, 0.8, True, out_for_delta=r["out"])
    for name in ("dq", "dk", "dv", "delta"):
        np.testing.assert_array_equal(r[name], r_same[name])
    pert = r["out"] + 1e-3 * rng.standard_normal(r["out"].shape)
    r_p = so.ssa_forward_backward(q, k, v, do, 0.3, 1.5, 0.8, True, out_for_delta=pert)
    np.testing.assert_array_equal(r["dv"], r_p["dv"])
    assert not np.allclose(r["dq"], r_p["dq"], rtol=0, atol=1e-9)
    s = 0.3 * q @ k.swapaxes(-1, -2)
    t = np.where(np.tril(np.ones((20, 20), bool)), so.ssa_logits(s, 1.5, 0.8), -np.inf)
    p = np.exp(t - t.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(r["delta"], np.sum(p * (do @ v.swapaxes(-1, -2)), -1), rtol=1e-12, atol=1e-12)


def test_decode_is_last_row_of_causal_forward():
    """The decode oracle against the (pinned) causal forward: sequence b's
    query, placed as the last row of a random prefix of length L_b, gets the
    causal forward's last-row output and normaliser; cache rows past L_b
    (filled with large garbage) are ignored, lengths clamp to the capacity,
    and an empty cache gives zeros and -inf."""
    rng = np.random.default_rng(12)
    B, Hq, Hkv, cap, D = 4, 6, 3, 23, 8
    kc, vc = _rand(rng, B, Hkv, cap, D), _rand(rng, B, Hkv, cap, D)
    qs = _rand(rng, B, Hq, cap, D)  # full prefixes; the decode query is row L - 1
    lens = [17, 1, 23, 40]
    for n_val in (1.5, -3.484375):
        q_dec = np.stack([qs[i, :, min(lens[i], cap) - 1] for i in range(B)])
        kg, vg = kc.copy(), vc.copy()
        for i in range(B):
            L = min(lens[i], cap)
            kg[i, :, L:] = 1e3
            vg[i, :, L:] = -1e3
        out, m = so.ssa_decode(q_dec, kg, vg, lens, 0.4, n_val, 0.8)
        for i in range(B):
            L = min(lens[i], cap)
            fo, fm = so.ssa_forward(qs[i : i + 1, :, :L], kc[i : i + 1, :, :L], vc[i : i + 1, :, :L], 0.4, n_val, 0.8, True)
            np.testing.assert_allclose(out[i], fo[0, :, L - 1], rtol=1e-12, atol=1e-12)
            np.testing.assert_allclose(m[i], fm[0, :, L - 1], rtol=1e-12, atol=1e-12)
    out, m = so.ssa_decode(q_dec, kc, vc, [0, 0, 5, -3], 0.4, 1.5, 0.8)
    assert np.all(out[[0, 1, 3]] == 0.0) and np.all(np.isneginf(m[[0, 1, 3]]))
    assert np.all(np.isfinite(m[2]))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("chunk", [1, 7, 16, 64])
def test_chunked_equals_dense(causal, chunk):
    """The row-block evaluation (used at S = 16384, where the dense oracle's
    N x N matrices do not fit) against the pinned dense oracle: same outputs
    to rounding, for chunks that divide N, that do not, of one row and of the
    whole sequence; with GQA, ragged N, the kernel-level out_for_delta, and
    n values of both signs."""
    rng = np.random.default_rng(21)
    for (B, Hq, Hkv, N, D), n_val in (((2, 4, 2, 37, 8), 1.5), ((1, 3, 1, 64, 16), -3.484375)):
        q, k, v, do = (_rand(rng, B, Hq, N, D), _rand(rng, B, Hkv, N, D), _rand(rng, B, Hkv, N, D),
                       _rand(rng, B, Hq, N, D))
        ofd = _rand(rng, B, Hq, N, D)
        for out_for_delta in (None, ofd):
            r = so.ssa_forward_backward(q, k, v, do, 0.3, n_val, 0.8, causal, out_for_delta)
            rc = so.ssa_forward_backward_chunked(q, k, v, do, 0.3, n_val, 0.8, causal, out_for_delta, chunk=chunk)
            for name in ("out", "m", "delta", "dq", "dk", "dv"):
                np.testing.assert_allclose(rc[name], r[name], rtol=1e-11, atol=1e-12, err_msg=name)
            for name in ("dn", "db"):
                assert abs(rc[name] - r[name]) <= 1e-11 * max(1.0, abs(r[name])), name
