"""CPU replica of the kernels' global address math: every direct-to-LDS load
and every dS' workspace access stays inside its tensor.

The tile loads issue ``buffer_load ... lds`` / ``global_load_lds`` through raw
buffer descriptors whose range field does not bound anything in practice
(num_records = 0x7fffffff, csrc/ssa_tile.hpp ``raw_rsrc``), so an offset
error would be a wild access, not a clamped one.  This file restates, in
numpy, the offsets that csrc/ssa_tile.hpp computes per lane
(``LoadLane``, ``tile_load_pieces`` with and without row clamping,
``tile_load_pieces_off``, ``rowswz_load``, ``pair32_load_async``) and the
way the dK/dV kernels (both forms), the dS' K pass and the forward call them
(the step walk, the row-0 and clamp decisions, the 32-bit offset paths), and
the dS' workspace tiles (ssa_launch.hpp ``ds_*``; dK/dV stores, dS' K loads),
then checks on dense, GQA, strided, ragged and packed problems:

* every 16-byte load lies inside the rows [0, N) of its sequence and the
  bytes [0, 2 D) of a row, and the byte offset equals row * stride + column;
* the 32-bit offset paths never reach 2^31 (the host's ``dkdv_off32`` test);
* every dS' store lands in its own (head, query tile, key tile) and inside
  the workspace size the library reports, no two stores write the same
  bytes, and the dS' K pass reads only tiles that the stores wrote (or
  clamped copies it multiplies by zero).
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest

from SSA import _lib

LANES = np.arange(64)
BMQ = 32  # dK/dV query sub-tile


# ---------------------------------------------------------------- ssa_tile.hpp
def load_lane(wave, ss):
    """LoadLane: per-lane row within a block, byte offset, half offset."""
    pos, half = LANES & 31, LANES >> 5
    r = pos ^ (4 * (2 * (wave & 1) + half))
    hoff = half * 16
    return r, r * ss * 2 + hoff, hoff


def tile_pieces(D, rows, nw, wave, row0, nrows, ss, clamp):
    """tile_load_pieces: (row, byte column, byte offset from the row-0 base) of every 16-byte lane load."""
    ipb = 32 * D * 2 // 1024
    ninst = rows // 32 * ipb
    per = -(-ninst // nw)
    r, off, hoff = load_lane(wave, ss)
    out = []
    for i in range(per):
        j = wave + nw * i
        if ninst % nw != 0 and j >= ninst:
            break
        blk, cp = j // ipb, j % ipb
        col = cp * 32 + hoff
        if not clamp:
            byte = row0 * ss * 2 + off + (blk * 32 * ss * 2 + cp * 32)
            row = row0 + blk * 32 + r
        else:
            row = np.minimum(row0 + blk * 32 + r, nrows - 1)
            byte = (row * ss + cp * 16) * 2 + hoff
        out.append((row, col, byte))
    return out


def tile_pieces_off(D, rows, nw, wave, soff0, ss2, ss):
    """tile_load_pieces_off: the same loads as 32-bit offsets from a descriptor base."""
    ipb = 32 * D * 2 // 1024
    ninst = rows // 32 * ipb
    per = -(-ninst // nw)
    _, off, _ = load_lane(wave, ss)
    out = []
    for i in range(per):
        j = wave + nw * i
        if ninst % nw != 0 and j >= ninst:
            break
        blk, cp = j // ipb, j % ipb
        out.append(soff0 + blk * 32 * ss2 + cp * 32 + off)
    return out


def rowswz_pieces(rows, nw, wave, row0, nrows, ss):
    """rowswz_load (D = 128): (row, byte column, byte offset from the tensor's sequence base)."""
    rsub = LANES >> 4
    chunk = (LANES & 15) ^ (4 * rsub)
    out = []
    for i in range(rows // 4 // nw):
        j = wave + nw * i
        if row0 + rows <= nrows:
            row = row0 + 4 * j + rsub
            byte = row0 * ss * 2 + rsub * ss * 2 + chunk * 16 + 4 * j * ss * 2
        else:
            row = np.minimum(row0 + 4 * j + rsub, nrows - 1)
            byte = (row * ss + chunk * 8) * 2
        out.append((row, chunk * 16, byte))
    return out


def check_rows(pieces, N, D, ss, label):
    for row, col, byte in pieces:
        assert (row >= 0).all() and (row < N).all(), f"{label}: row outside [0, {N})"
        assert (col >= 0).all() and (col + 16 <= 2 * D).all(), f"{label}: column outside the row"
        np.testing.assert_array_equal(byte, row * ss * 2 + col, err_msg=label)


# ---------------------------------------------------------------- ssa_launch.hpp
def ds_tiles_per_head(N, causal):
    nq = -(-N // 32)
    return nq * (nq + 1) if causal else 2 * nq * nq


def ds_row_offset(qi, N, causal):
    return qi * (qi + 1) if causal else qi * 2 * (-(-N // 32))


def ds_slot_tiles(Nmax, causal):
    nq = -(-Nmax // 32)
    return nq + 1 if causal else 2 * nq


def ds_head_tile(packed, tok0, b, h, Hq, N, Nmax, causal):
    if packed:
        return ((tok0 >> 5) + b) * Hq * ds_slot_tiles(Nmax, causal) + h * ds_tiles_per_head(N, causal)
    return (b * Hq + h) * ds_tiles_per_head(Nmax, causal)


def seq_view(cu, T, Nmax, b):
    """SeqView: (N, tok0) of sequence b (packed tables clamped to [0, T], lengths to Nmax)."""
    if cu is None:
        return Nmax, 0
    s0 = min(max(cu[b], 0), T)
    s1 = min(max(cu[b + 1], s0), T)
    return min(s1 - s0, Nmax), s0


# ---------------------------------------------------------------- dK/dV (both kernels)
def dkdv_steps(N, G, kb, causal):
    """The step walk of the dK/dV kernels: list of (q0, g, masked) in step order."""
    BN = 128
    k0 = kb * BN
    qstart = k0 if causal else 0
    nsub = -(-(N - qstart) // BMQ)
    key_edge = k0 + BN > N
    nlo = nsub if key_edge else (min(BN // BMQ, nsub) if causal else 0)
    ntail = 1 if (not key_edge and N % BMQ != 0 and nsub > nlo) else 0
    per_m, per_u = nlo + ntail, nsub - nlo - ntail
    steps = []
    for g in range(G):
        for j in range(per_m):
            i = j if j < nlo else nsub - 1
            steps.append((qstart + i * BMQ, g, True))
    for g in range(G):
        for j in range(per_u):
            steps.append((qstart + (nlo + j) * BMQ, g, False))
    return steps


def check_dkdv(B, Hq, Hkv, Nmax, D, causal, q_st, cu=None, T=0):
    """Loads of Q / dO sub-tiles, M / Delta rows and the dS' stores of every
    dK/dV workgroup; returns the set of workspace bytes written."""
    G = Hq // Hkv
    sb, sh, ss = q_st
    nkb = -(-Nmax // 128)
    packed = cu is not None
    ws_bytes = (_lib.lib().ssa_varlen_bwd_ds_workspace_bytes(B, Hq, Nmax, T, int(causal)) if packed
                else _lib.lib().ssa_bwd_ds_workspace_bytes(B, Hq, Nmax, int(causal)))
    written = {}
    mrows = Hq * T if packed else B * Hq * Nmax
    # the host's 32-bit test (ssa_bwd.hip dkdv_off32)
    lim = (1 << 31) - 4096
    off32 = ((G - 1) * sh + (Nmax - 1) * ss + D) * 2 < lim and G * ds_tiles_per_head(Nmax, causal) * 1024 < lim
    for b, hk, kb in itertools.product(range(B), range(Hkv), range(nkb)):
        N, tok0 = seq_view(cu, T, Nmax, b)
        if kb * 128 >= N:
            continue
        seq_row0 = tok0 if packed else 0       # first row of the sequence in the token axis
        base_b = 0 if packed else b * sb       # element offset of the sequence (before rows)
        for st, (q0, g, masked) in enumerate(dkdv_steps(N, G, kb, causal)):
            h = hk * G + g
            for wave in range(4):
                label = f"dkdv b={b} hk={hk} kb={kb} step={st} wave={wave}"
                clamp = q0 + BMQ > N
                pieces = tile_pieces(D, BMQ, 4, wave, q0, N, ss, clamp)
                check_rows(pieces, N, D, ss, label)
                if off32 and not clamp:
                    q_hs2, q_ss2 = sh * 2, ss * 2
                    for o in tile_pieces_off(D, BMQ, 4, wave, g * q_hs2 + q0 * q_ss2, q_ss2, ss):
                        assert (o < (1 << 31)).all(), f"{label}: 32-bit offset overflow"
                        # the same bytes as the 64-bit form, measured from the q-head hk G base
                    full = tile_pieces(D, BMQ, 4, wave, q0, N, ss, False)
                    for o, (row, col, _) in zip(tile_pieces_off(D, BMQ, 4, wave, g * q_hs2 + q0 * q_ss2, q_ss2, ss),
                                                full):
                        np.testing.assert_array_equal(o, g * sh * 2 + row * ss * 2 + col, err_msg=label)
                # M / Delta: pair32_load_async, rows clamped to N - 1 (wave 3)
                r = np.minimum(q0 + (LANES & 31), N - 1)
                mrow = (h * T + seq_row0 if packed else (b * Hq + h) * Nmax) + r
                assert (mrow >= 0).all() and (mrow < mrows).all(), f"{label}: M/Delta row"
                _ = base_b
                # dS' stores: this wave's 32 keys, query tile q0 / 32
                k0w = kb * 128 + wave * 32
                skipped = masked and (k0w >= N or (causal and q0 + BMQ - 1 < k0w))
                if skipped:
                    continue
                qi = q0 >> 5
                nkj = 2 * qi + 2 if causal else 2 * (-(-N // 32))
                assert (k0w >> 4) + 1 < nkj, f"{label}: key tile outside the query tile's row"
                tile0 = ds_head_tile(packed, tok0, b, hk * G, Hq, N, Nmax, causal) + (k0w >> 4)
                tile = tile0 + g * ds_tiles_per_head(N, causal) + ds_row_offset(qi, N, causal)
                l32, hh = LANES & 31, LANES >> 5
                ds_lane = (l32 >> 4) * 512 + (l32 & 15) * 8
                voff = (ds_lane + 16 * hh * 8) * 2
                if off32:
                    soff = g * ds_tiles_per_head(N, causal) * 1024 + ds_row_offset(qi, N, causal) * 1024
                    assert soff + voff.max() + 520 + 8 < (1 << 31), f"{label}: dS' 32-bit offset"
                for extra in (0, 8, 512, 520):
                    byte = tile * 1024 + voff + extra
                    assert (byte >= 0).all() and (byte + 8 <= ws_bytes).all(), f"{label}: dS' store outside"
                    # the tile written is (head h, query tile qi, key tile k0w/16 + l32/16)
                    assert ((byte // 1024) - tile0 - g * ds_tiles_per_head(N, causal)
                            - ds_row_offset(qi, N, causal) == (l32 >> 4)).all(), label
                    for x in byte.tolist():
                        key = (x, x + 8)
                        assert key not in written, f"{label}: dS' bytes written twice"
                        written[key] = label
    return written, ws_bytes


def check_dq_ds(B, Hq, Hkv, Nmax, D, causal, k_st, written, cu=None, T=0):
    """The dS' K pass: K tile loads (row-swizzled at D = 128) and the dS' tile
    loads of every wave; every dS' byte read was written by dK/dV unless the
    kernel multiplies it by zero (tiles past the wave's last one)."""
    NW = 8 if D >= 64 else 4
    BM, BN = 32 * NW, 64
    sb, sh, ss = k_st
    packed = cu is not None
    nqb = -(-Nmax // BM)
    wbytes = {k[0] for k in written}
    for b, h, qb in itertools.product(range(B), range(Hq), range(nqb)):
        N, tok0 = seq_view(cu, T, Nmax, b)
        if qb * BM >= N:
            continue
        q0 = qb * BM
        kv_end = min(N, q0 + BM) if causal else N
        ntiles = -(-kv_end // BN)
        for wave in range(NW):
            label = f"dq_ds b={b} h={h} qb={qb} wave={wave}"
            for t in range(ntiles + 1):  # issue_k runs one tile past the last
                if D == 128:
                    check_rows(rowswz_pieces(BN, NW, wave, t * BN, N, ss), N, D, ss, label)
                else:
                    check_rows(tile_pieces(D, BN, NW, wave, t * BN, N, ss, t * BN + BN > N), N, D, ss, label)
            wq0 = q0 + wave * 32
            nk16 = -(-N // 16)
            nkj = 0 if wq0 >= N else (min(2 * (wq0 >> 5) + 2, nk16) if causal else nk16)
            kj_max = max(nkj - 1, 0)
            qi = min(wq0, N - 1) >> 5
            row0 = ds_head_tile(packed, tok0, b, h, Hq, N, Nmax, causal) + ds_row_offset(qi, N, causal)
            ds_src = (16 * (LANES >> 4) + ((LANES & 15) ^ (4 * (LANES >> 4)))) * 16
            for t in range(ntiles + 2):  # issue_ds runs PFD = 2 steps ahead
                for s4 in range(4):
                    kj = min(4 * t + s4, kj_max)
                    byte = (row0 + kj) * 1024 + ds_src
                    if 4 * t + s4 < nkj and t < ntiles:
                        for x in byte.tolist():
                            assert any(y in wbytes for y in (x, x + 8)), f"{label}: reads dS' never written"
                    assert (kj * 1024 + ds_src.max() + 16) < (1 << 31), label


DENSE = [
    # B, Hq, Hkv, N, D, causal, layout
    (1, 4, 4, 256, 128, True, "contig"),
    (2, 4, 2, 200, 128, True, "contig"),
    (1, 2, 1, 129, 64, False, "contig"),
    (2, 8, 2, 511, 64, True, "strided"),
    (1, 3, 1, 33, 32, True, "contig"),
    (2, 2, 2, 7, 128, False, "strided"),
    (1, 2, 2, 1, 64, True, "contig"),
    (1, 6, 2, 300, 32, False, "contig"),
]


def strides(B, H, N, D, layout):
    if layout == "contig":
        return H * N * D, N * D, D
    return H * D, D, B * H * D  # [S, B, H, D] memory viewed as [B, H, S, D]


@pytest.mark.parametrize("B,Hq,Hkv,N,D,causal,layout", DENSE)
def test_dense_addresses_in_bounds(B, Hq, Hkv, N, D, causal, layout):
    written, _ = check_dkdv(B, Hq, Hkv, N, D, causal, strides(B, Hq, N, D, layout))
    check_dq_ds(B, Hq, Hkv, N, D, causal, strides(B, Hkv, N, D, layout), written)
    # forward: K / V tiles of 64 rows, 8 waves (D = 128 / 64) -- the row logic of load_tile
    for NW in (4, 8):
        for t in range(-(-N // 64)):
            for wave in range(NW):
                check_rows(tile_pieces(D, 64, NW, wave, t * 64, N, strides(B, Hkv, N, D, layout)[2],
                                       t * 64 + 64 > N), N, D, strides(B, Hkv, N, D, layout)[2], f"fwd t={t}")


PACKED = [
    # lens (or raw table), T, max_seqlen, Hq, Hkv, D, causal
    ([0, 37, 157, 160], 160, 120, 4, 2, 64, True),
    ([0, 300, 813], 813, 513, 2, 1, 128, True),
    ([0, 129, 160, 360], 360, 200, 4, 2, 128, False),
    ([-5, 40, 250], 100, 100, 2, 2, 64, True),      # malformed: clamped to [0, 40), [40, 100)
    ([0, 37, 120], 200, 60, 4, 2, 64, True),         # uncovered tail and a cut document
    ([0, 5, 105, 138, 398, 399], 399, 260, 4, 2, 128, True),
]


@pytest.mark.parametrize("cu,T,Nmax,Hq,Hkv,D,causal", PACKED)
def test_packed_addresses_in_bounds(cu, T, Nmax, Hq, Hkv, D, causal):
    B = len(cu) - 1
    st = (0, D, Hq * D)  # [T, H, D]
    written, _ = check_dkdv(B, Hq, Hkv, Nmax, D, causal, (0, D, Hq * D), cu=cu, T=T)
    check_dq_ds(B, Hq, Hkv, Nmax, D, causal, (0, D, Hkv * D), written, cu=cu, T=T)
    _ = st


@pytest.mark.parametrize("B,Hq,Hkv,N,D", [(4, 16, 16, 4096, 128), (1, 16, 16, 16384, 128), (4, 32, 8, 4096, 64)])
def test_fullsize_extremes(B, Hq, Hkv, N, D):
    """The benchmark shapes, at the workgroups with the largest offsets (last
    sequence, last heads, last key block, last steps): the 32-bit paths hold
    and every load stays in its rows."""
    sb, sh, ss = strides(B, Hq, N, D, "contig")
    G = Hq // Hkv
    lim = (1 << 31) - 4096
    assert ((G - 1) * sh + (N - 1) * ss + D) * 2 < lim
    assert G * ds_tiles_per_head(N, True) * 1024 < lim
    nkb = -(-N // 128)
    ws = _lib.lib().ssa_bwd_ds_workspace_bytes(B, Hq, N, 1)
    for kb in (0, nkb - 1):
        steps = dkdv_steps(N, G, kb, True)
        for st in (0, len(steps) - 1):
            q0, g, _ = steps[st]
            for wave in range(4):
                check_rows(tile_pieces(D, BMQ, 4, wave, q0, N, ss, q0 + BMQ > N), N, D, ss, "full")
                for o in tile_pieces_off(D, BMQ, 4, wave, g * sh * 2 + q0 * ss * 2, ss * 2, ss):
                    assert o.max() < (1 << 31)
                k0w = kb * 128 + wave * 32
                qi = q0 >> 5
                tile = (ds_head_tile(False, 0, B - 1, (Hkv - 1) * G, Hq, N, N, True) + (k0w >> 4)
                        + g * ds_tiles_per_head(N, True) + ds_row_offset(qi, N, True))
                assert (tile + 2) * 1024 <= ws
