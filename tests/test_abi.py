"""C-ABI checks that need no GPU: exports, status strings, host-side validation.

Validation runs on the host before any launch (include/ssa_mi355x.h), so bad
arguments return their status code here without touching a device.  The
pointers used below are never dereferenced: every call is rejected first.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from SSA import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*([a-z_][a-z0-9_]*)\s*\(", text, re.M):
            names.add(m.group(1))
    return names


def test_header_declares_the_bound_symbols():
    assert HEADERS, "no public header under include/"
    assert _declared_functions() == set(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in _declared_functions():
        assert hasattr(lib, name), f"libssa_mi355x.so does not export {name}"
    assert lib.ssa_abi_version() == _lib.ABI_VERSION


def test_status_strings():
    for code in range(9):
        assert _lib.status_text(code)
    assert _lib.status_text(99) == "unknown status"


def test_partials_count():
    lib = _lib.lib()
    assert lib.ssa_bwd_partials_count(4, 16, 4096) == 2 * 4 * 16 * 32
    assert lib.ssa_bwd_partials_count(1, 1, 129) == 2 * 2
    assert lib.ssa_bwd_partials_count(0, 1, 1) == 0


def _ds_tiles_needed(N, causal):
    """1 KB dS' tiles (32 queries x 16 keys) holding at least one unmasked pair."""
    need = 0
    for qi in range((N + 31) // 32):
        for kj in range((N + 15) // 16):
            qmax = min(32 * qi + 31, N - 1)
            if 16 * kj < N and (not causal or 16 * kj <= qmax):
                need += 1
    return need


@pytest.mark.parametrize("N", [1, 31, 32, 33, 100, 256, 511])
@pytest.mark.parametrize("causal", [0, 1])
def test_ds_workspace_bytes(N, causal):
    lib = _lib.lib()
    nq = (N + 31) // 32
    per_head = nq * (nq + 1) if causal else 2 * nq * nq
    assert lib.ssa_bwd_ds_workspace_bytes(3, 5, N, causal) == 3 * 5 * per_head * 1024
    # every tile the mask needs fits in its query row, and causal rows hold
    # nothing else when N is a multiple of 32
    assert _ds_tiles_needed(N, causal) <= per_head
    if causal and N % 32 == 0:
        assert _ds_tiles_needed(N, causal) == per_head


def test_ds_workspace_bytes_headline_and_empty():
    lib = _lib.lib()
    assert lib.ssa_bwd_ds_workspace_bytes(4, 16, 4096, 1) == 4 * 16 * 128 * 129 * 1024
    # the status text names the size limits a caller may have hit
    text = _lib.status_text(_lib.SSA_ERR_SHAPE)
    for limit in ("2^30", "2^28", "2^31 - 1", "query rows"):
        assert limit in text, (limit, text)
    assert lib.ssa_bwd_ds_workspace_bytes(0, 16, 4096, 1) == 0
    assert lib.ssa_bwd_ds_workspace_bytes(4, 16, 0, 0) == 0


@pytest.mark.parametrize("causal", [0, 1])
def test_varlen_ds_workspace_bytes_holds_every_document(causal):
    # Packed batches: the workspace must hold every document's per-head
    # tiles (as the dense size of that document) for any split of T tokens,
    # including the ones the layout packs worst (many documents just past a
    # multiple of 32 tokens), and 0 for invalid sizes.
    lib = _lib.lib()
    rng = np.random.default_rng(7)
    tables = [[4096], [33] * 31, [1] * 64, [31, 1] * 20, [100, 513, 7, 260]]
    tables += [list(rng.integers(1, 700, size=int(rng.integers(1, 40)))) for _ in range(20)]
    Hq = 6
    for lens in tables:
        T, B, nmax = int(sum(lens)), len(lens), int(max(lens))
        got = lib.ssa_varlen_bwd_ds_workspace_bytes(B, Hq, nmax, T, causal)
        need = sum(lib.ssa_bwd_ds_workspace_bytes(1, Hq, int(L), causal) for L in lens)
        assert got >= need, (lens, got, need)
    assert lib.ssa_varlen_bwd_ds_workspace_bytes(0, Hq, 10, 10, causal) == 0
    assert lib.ssa_varlen_bwd_ds_workspace_bytes(2, Hq, 10, 9, causal) == 0
    assert lib.ssa_varlen_bwd_ds_workspace_bytes(2, 0, 10, 20, causal) == 0


FAKE = 0x10000  # 16-byte aligned, never dereferenced


def _fwd_args(**kw):
    t = _lib.Tensor4(FAKE, 8 * 128 * 64, 8 * 128, 128)
    a = _lib.FwdArgs(t, t, t, t, FAKE, FAKE, FAKE, 1, 8, 8, 64, 128, _lib.SSA_DTYPE_BF16, 1, 0.088)
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def _bwd_args(**kw):
    t = _lib.Tensor4(FAKE, 8 * 128 * 64, 8 * 128, 128)
    a = _lib.BwdArgs(t, t, t, t, t, t, t, t, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                     1, 8, 8, 64, 128, _lib.SSA_DTYPE_BF16, 1, 0.088)
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "field,value,status",
    [
        ("heads_kv", 3, _lib.SSA_ERR_SHAPE),        # Hq % Hkv != 0
        ("batch", 0, _lib.SSA_ERR_SHAPE),
        ("seqlen", 0, _lib.SSA_ERR_SHAPE),
        ("head_dim", 96, _lib.SSA_ERR_HEAD_DIM),
        ("head_dim", 512, _lib.SSA_ERR_HEAD_DIM),   # the largest is 256
        ("head_dim", 16, _lib.SSA_ERR_HEAD_DIM),    # bf16: D = 16 runs padded in Python, not here
        ("dtype", 7, _lib.SSA_ERR_DTYPE),
        ("m", None, _lib.SSA_ERR_NULL_POINTER),
        ("ssa_n", None, _lib.SSA_ERR_NULL_POINTER),
        ("q", _lib.Tensor4(FAKE + 2, 0, 0, 128), _lib.SSA_ERR_ALIGNMENT),
        ("k", _lib.Tensor4(FAKE, 0, 0, 100), _lib.SSA_ERR_ALIGNMENT),
        ("k", _lib.Tensor4(FAKE, 0, 0, 1 << 24), _lib.SSA_ERR_ALIGNMENT),
        ("v", _lib.Tensor4(FAKE, -128, 0, 128), _lib.SSA_ERR_ALIGNMENT),
        ("v", _lib.Tensor4(None, 0, 0, 128), _lib.SSA_ERR_NULL_POINTER),
    ],
)
def test_fwd_validation(field, value, status):
    a = _fwd_args(**{field: value})
    assert _lib.lib().ssa_fwd(ctypes.byref(a), None) == status


def test_fp32_head_dims():
    """fp32 takes head dims 16..256 (powers of two); other head dims stay refused."""
    for D in (48, 96, 512, 8):
        a = _fwd_args(dtype=_lib.SSA_DTYPE_FP32, head_dim=D)
        assert _lib.lib().ssa_fwd(ctypes.byref(a), None) == _lib.SSA_ERR_HEAD_DIM, D
        b = _bwd_args(dtype=_lib.SSA_DTYPE_FP32, head_dim=D)
        assert _lib.lib().ssa_bwd(ctypes.byref(b), None) == _lib.SSA_ERR_HEAD_DIM, D


def test_size_limits():
    """Shapes whose grid or row arithmetic would leave int32 are refused before any launch:
    seqlen > 2^30, more than INT32_MAX dense query rows, huge decode caches; the size
    queries return 0 for them instead of an overflowed value."""
    lib = _lib.lib()
    for over in ({"seqlen": (1 << 30) + 1}, {"batch": 1 << 16, "heads_q": 1 << 10, "heads_kv": 1 << 10},
                 {"seqlen": 2**31 - 1}):
        a = _fwd_args(**over)
        assert lib.ssa_fwd(ctypes.byref(a), None) == _lib.SSA_ERR_SHAPE, over
        b = _bwd_args(**over)
        assert lib.ssa_bwd(ctypes.byref(b), None) == _lib.SSA_ERR_SHAPE, over
    assert lib.ssa_bwd_ds_workspace_bytes(1 << 16, 1 << 10, 4096, 1) == 0
    assert lib.ssa_bwd_ds_workspace_bytes(2**31 - 1, 2**31 - 1, 2**31 - 1, 1) == 0
    assert lib.ssa_bwd_partials_count(2**31 - 1, 2**31 - 1, 1 << 30) == 0
    assert lib.ssa_varlen_bwd_ds_workspace_bytes(2**31 - 1, 2**31 - 1, 1 << 30, 2**31 - 1, 1) == 0
    assert lib.ssa_decode_num_splits(1, 8, 8, 2**31 - 1, 0) == 0
    assert lib.ssa_decode_num_splits(1, 8, 8, 4096, 2**31 - 1) == 32  # more splits than 128-key blocks: clamped
    assert lib.ssa_bwd_ds_workspace_bytes(4, 16, 4096, 1) == 4 * 16 * 128 * 129 * 1024
    # the status text names the size limits a caller may have hit
    text = _lib.status_text(_lib.SSA_ERR_SHAPE)
    for limit in ("2^30", "2^28", "2^31 - 1", "query rows"):
        assert limit in text, (limit, text)


def test_fwd_null_args():
    assert _lib.lib().ssa_fwd(None, None) == _lib.SSA_ERR_NULL_POINTER


@pytest.mark.parametrize("entry", ["ssa_bwd", "ssa_bwd_dkdv", "ssa_bwd_dq", "ssa_bwd_reduce"])
@pytest.mark.parametrize(
    "field,value,status",
    [
        ("heads_kv", 5, _lib.SSA_ERR_SHAPE),
        ("head_dim", 16, _lib.SSA_ERR_HEAD_DIM),    # D = 16 only with fp32
        ("dtype", 3, _lib.SSA_ERR_DTYPE),
        ("partials", None, _lib.SSA_ERR_NULL_POINTER),
        ("dn", None, _lib.SSA_ERR_NULL_POINTER),
        ("dq", _lib.Tensor4(FAKE, 4, 0, 128), _lib.SSA_ERR_ALIGNMENT),
        ("ds_workspace", FAKE + 8, _lib.SSA_ERR_ALIGNMENT),
    ],
)
def test_bwd_validation(entry, field, value, status):
    a = _bwd_args(**{field: value})
    assert getattr(_lib.lib(), entry)(ctypes.byref(a), None) == status


def test_preprocess_validation_needs_only_out_dout_delta():
    a = _bwd_args(q=_lib.Tensor4(None, 0, 0, 0), partials=None, dn=None, head_dim=48)
    assert _lib.lib().ssa_bwd_preprocess(ctypes.byref(a), None) == _lib.SSA_ERR_HEAD_DIM
    a = _bwd_args(delta=None)
    assert _lib.lib().ssa_bwd_preprocess(ctypes.byref(a), None) == _lib.SSA_ERR_NULL_POINTER


def test_status_maps_to_python_exceptions():
    with pytest.raises(ValueError, match="head_dim"):
        _lib.check(_lib.SSA_ERR_HEAD_DIM, "ssa_fwd")
    with pytest.raises(RuntimeError, match="launch"):
        _lib.check(_lib.SSA_ERR_LAUNCH, "ssa_fwd")
    _lib.check(_lib.SSA_OK, "ssa_fwd")


def _varlen_fwd_args(**over):
    a = _lib.VarlenFwdArgs(_fwd_args(), ctypes.c_void_p(FAKE), 1000)
    a.dense.seqlen = 256
    for key, val in over.items():
        setattr(a, key, val)
    return a


@pytest.mark.parametrize(
    "field,value,status",
    [
        ("cu_seqlens", None, _lib.SSA_ERR_NULL_POINTER),
        ("total_tokens", 0, _lib.SSA_ERR_CU_SEQLENS),
        ("total_tokens", 100, _lib.SSA_ERR_CU_SEQLENS),  # max_seqlen (256) > total_tokens
    ],
)
def test_varlen_fwd_validation(field, value, status):
    a = _varlen_fwd_args(**{field: value})
    assert _lib.lib().ssa_varlen_fwd(ctypes.byref(a), None) == status


def test_varlen_null_args():
    assert _lib.lib().ssa_varlen_fwd(None, None) == _lib.SSA_ERR_NULL_POINTER
    assert _lib.lib().ssa_varlen_bwd(None, None) == _lib.SSA_ERR_NULL_POINTER


@pytest.mark.parametrize(
    "B,Hq,Hkv,cap,req,splits",
    [
        (1, 16, 16, 4096, 0, 16),   # 16 units: 256 / 16 = 16 splits of 256 keys
        (1, 8, 8, 4096, 0, 16),     # 8 units: 32 wanted, capped at 4096 / 256 = 16
        (4, 16, 16, 4096, 0, 4),    # 64 units: 4 splits of 1024 keys
        (64, 16, 16, 4096, 0, 1),   # 1024 units fill the GPU already
        (1, 16, 16, 100, 0, 1),     # too short to split
        (1, 8, 8, 1000, 3, 3),      # 3 x 384 keys
        (1, 8, 8, 1000, 1000, 8),   # at most one split per 128 keys
        (2, 64, 1, 300, 1, 1),
    ],
)
def test_decode_num_splits(B, Hq, Hkv, cap, req, splits):
    lib = _lib.lib()
    assert lib.ssa_decode_num_splits(B, Hq, Hkv, cap, req) == splits
    ws = lib.ssa_decode_workspace_bytes(B, Hq, Hkv, cap, 128, req)
    if splits == 1:
        assert ws == 0
    else:  # (m, l) and acc[D] per record, fp32, (m, l) block padded to 16 bytes
        recs = B * Hq * splits
        assert ws == ((2 * recs + 3) // 4 * 4 + recs * 128) * 4


def test_decode_sizes_reject_bad_shapes():
    lib = _lib.lib()
    for args in ((0, 8, 8, 64, 0), (1, 8, 3, 64, 0), (1, 8, 8, 0, 0), (1, 8, 8, 64, -1)):
        assert lib.ssa_decode_num_splits(*args) == 0
        assert lib.ssa_decode_workspace_bytes(*args[:4], 128, args[4]) == 0
    assert lib.ssa_decode_workspace_bytes(4, 16, 16, 4096, 96, 0) == 0


def _decode_args(**kw):
    q = _lib.Tensor4(FAKE, 8 * 128, 128, 0)
    kc = _lib.Tensor4(FAKE, 8 * 4096 * 128, 4096 * 128, 128)
    a = _lib.DecodeArgs(q, kc, kc, q, None, FAKE, FAKE, FAKE, 4, 8, 8, 4096, 128, _lib.SSA_DTYPE_BF16, 0, 0.088,
                        FAKE)
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "field,value,status",
    [
        ("heads_kv", 3, _lib.SSA_ERR_SHAPE),
        ("capacity", 0, _lib.SSA_ERR_SHAPE),
        ("num_splits", -2, _lib.SSA_ERR_SHAPE),
        ("head_dim", 48, _lib.SSA_ERR_HEAD_DIM),
        ("dtype", 3, _lib.SSA_ERR_DTYPE),
        ("dtype", _lib.SSA_DTYPE_FP32, _lib.SSA_ERR_DTYPE),   # decode: bf16 / fp16 only
        ("cache_seqlens", None, _lib.SSA_ERR_NULL_POINTER),
        ("ssa_b", None, _lib.SSA_ERR_NULL_POINTER),
        ("workspace", None, _lib.SSA_ERR_NULL_POINTER),   # 4 x 8 heads x 4096 keys needs splits
        ("workspace", FAKE + 4, _lib.SSA_ERR_ALIGNMENT),
        ("k_cache", _lib.Tensor4(FAKE, 0, 0, 132), _lib.SSA_ERR_ALIGNMENT),
        ("v_cache", _lib.Tensor4(None, 0, 0, 128), _lib.SSA_ERR_NULL_POINTER),
        ("out", _lib.Tensor4(FAKE + 8, 0, 0, 0), _lib.SSA_ERR_ALIGNMENT),
    ],
)
def test_decode_validation(field, value, status):
    a = _decode_args(**{field: value})
    assert _lib.lib().ssa_decode(ctypes.byref(a), None) == status


def test_decode_null_args():
    assert _lib.lib().ssa_decode(None, None) == _lib.SSA_ERR_NULL_POINTER


def _rope_args(**kw):
    a = _lib.RopeArgs(FAKE, 16 * 128, 128, 128 * 0 + 128, FAKE, FAKE, FAKE, 4, 1, 16, 128, 0, 0)
    a.x_stride_h = 128
    a.x_stride_b = 16 * 128
    a.x_stride_s = 16 * 128
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "field,value,status",
    [
        ("x", None, 1), ("y", None, 1), ("cos", None, 1), ("sin", None, 1),
        ("seqlen", 0, 2), ("heads", -1, 2), ("head_dim", 96, 2), ("head_dim", 32, 2),
        ("dtype", 2, 3),
        ("x", FAKE + 4, 4), ("cos", FAKE + 8, 4), ("x_stride_h", 130, 4), ("x_stride_s", -128, 4),
    ],
)
def test_rope_validation(field, value, status):
    """ssa_rope (include/ssa_decoder_ops.h) rejects bad arguments on the host."""
    a = _rope_args(**{field: value})
    assert _lib.lib().ssa_rope(ctypes.byref(a), None) == status



def test_rmsnorm_validation_and_workspace():
    """ssa_rmsnorm_* (include/ssa_decoder_ops.h) reject bad arguments on the host."""
    lib = _lib.lib()
    assert lib.ssa_rmsnorm_workspace_floats(16384, 2048) == 256 * 2048
    assert lib.ssa_rmsnorm_workspace_floats(65, 8) == 2 * 8
    assert lib.ssa_rmsnorm_workspace_floats(0, 8) == 0
    f = _lib.RmsNormFwdArgs(FAKE, FAKE, FAKE, FAKE, 4, 2048, 0, 1e-5)
    for field, value, status in (("x", None, 1), ("rows", 0, 2), ("hidden", 4100, 2), ("hidden", 6, 2),
                                 ("out_dtype", 3, 3), ("x", FAKE + 8, 4), ("y", FAKE + 2, 4)):
        a = _lib.RmsNormFwdArgs(FAKE, FAKE, FAKE, FAKE, 4, 2048, 0, 1e-5)
        setattr(a, field, value)
        assert lib.ssa_rmsnorm_fwd(ctypes.byref(a), None) == status, field
    for field, value, status in (("dy", None, 1), ("dx", None, 1), ("workspace", None, 1), ("hidden", 0, 2),
                                 ("dy_dtype", 5, 3), ("dx", FAKE + 4, 4)):
        a = _lib.RmsNormBwdArgs(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 2048, 0)
        setattr(a, field, value)
        assert lib.ssa_rmsnorm_bwd(ctypes.byref(a), None) == status, field
    assert f.hidden == 2048


def test_swiglu_validation():
    """ssa_swiglu (include/ssa_decoder_ops.h) rejects bad arguments on the host."""
    lib = _lib.lib()
    for field, value, status in (("z", None, 1), ("out", None, 1), ("rows", 0, 2), ("ffn", 6, 2),
                                 ("dtype", 2, 3), ("z", FAKE + 4, 4)):
        a = _lib.SwigluArgs(FAKE, None, FAKE, 4, 64, 0, 0)
        setattr(a, field, value)
        assert lib.ssa_swiglu(ctypes.byref(a), None) == status, field
    a = _lib.SwigluArgs(FAKE, None, FAKE, 4, 64, 0, 1)  # backward needs dh
    assert lib.ssa_swiglu(ctypes.byref(a), None) == 1



def test_cross_entropy_validation():
    """ssa_cross_entropy (include/ssa_decoder_ops.h) rejects bad arguments on the host."""
    lib = _lib.lib()
    for field, value, status in (("logits", None, 1), ("loss", None, 1), ("rows", 0, 2), ("vocab", 6, 2),
                                 ("dtype", 2, 3), ("logits", FAKE + 2, 4)):
        a = _lib.CrossEntropyArgs(FAKE, FAKE, FAKE, FAKE, None, None, 4, 64, 0, 0)
        setattr(a, field, value)
        assert lib.ssa_cross_entropy(ctypes.byref(a), None) == status, field
    a = _lib.CrossEntropyArgs(FAKE, FAKE, None, FAKE, None, FAKE, 4, 64, 0, 1)  # backward needs scale
    assert lib.ssa_cross_entropy(ctypes.byref(a), None) == 1


@pytest.mark.parametrize(
    "field,value,status",
    [
        ("heads_kv", 5, _lib.SSA_ERR_SHAPE),
        ("head_dim", 16, _lib.SSA_ERR_HEAD_DIM),    # D = 16 only with fp32
        ("dtype", 3, _lib.SSA_ERR_DTYPE),
        ("dn", None, _lib.SSA_ERR_NULL_POINTER),
        ("m", None, _lib.SSA_ERR_NULL_POINTER),
        ("dq", _lib.Tensor4(FAKE, 4, 0, 128), _lib.SSA_ERR_ALIGNMENT),
    ],
)
def test_bwd_noalloc_validation(field, value, status):
    a = _bwd_args(**{field: value})
    assert _lib.lib().ssa_bwd_noalloc(ctypes.byref(a), None) == status


def test_bwd_noalloc_rejects_problems_beyond_its_scratch():
    """Delta (4 B per query row, rounded to 256 B) plus the partials (8 B per
    128-key block and kv-head) must fit the 16 MiB static scratch; larger
    problems are refused on the host, before any device call (this runs
    without a GPU), and the caller's own workspace fields are never required."""
    lim = 16 << 20
    a = _bwd_args(delta=None, partials=None, ds_workspace=None)
    assert _lib.lib().ssa_bwd_noalloc(None, None) == _lib.SSA_ERR_NULL_POINTER
    # B * Hq * N * 4 bytes of Delta alone above the limit
    a.batch, a.heads_q, a.heads_kv, a.seqlen = 64, 16, 16, 4097
    assert 64 * 16 * 4097 * 4 > lim
    assert _lib.lib().ssa_bwd_noalloc(ctypes.byref(a), None) == _lib.SSA_ERR_SCRATCH
    # just above: Delta exactly 16 MiB leaves no room for the partials
    a.batch, a.heads_q, a.heads_kv, a.seqlen = 64, 16, 16, 4096
    assert 64 * 16 * 4096 * 4 == lim
    assert _lib.lib().ssa_bwd_noalloc(ctypes.byref(a), None) == _lib.SSA_ERR_SCRATCH
    assert "scratch" in _lib.status_text(_lib.SSA_ERR_SCRATCH)


def test_hazard_scan_flags_short_waits():
    """SSA/_hazards.py, the build's wait-state check, on hand-written sequences:
    a VALU write of an SGPR needs 5 wait states before a vector-memory
    instruction reads it (descriptor or offset), an SALU write of M0 one
    before an LDS DMA; a label in between does not hide a fall-through path."""
    from SSA import _hazards

    def sites(body):
        return _hazards.scan_asm("_Zk:\n" + "\n".join("\t" + ln for ln in body))

    bad_off = ["v_readfirstlane_b32 s5, v1", "s_nop 0", "buffer_load_dwordx4 v2, s[8:11], s5 offen lds"]
    assert [s[1:3] for s in sites(bad_off)] == [(1, 5)]
    ok_off = ["v_readfirstlane_b32 s5, v1", "s_nop 4", "buffer_load_dwordx4 v2, s[8:11], s5 offen lds"]
    assert sites(ok_off) == []
    bad_rsrc = ["v_readlane_b32 s11, v180, 3", "s_add_i32 s4, s4, 1", ".LBB0_2:", "s_mov_b32 s6, 0",
                "buffer_store_dwordx2 v[4:5], v2, s[8:11], s4 offen offset:8"]
    assert [s[1:3] for s in sites(bad_rsrc)] == [(2, 5)]
    bad_m0 = ["s_add_i32 m0, s3, 0x400", "global_load_lds_dwordx4 v[2:3], off"]
    assert [s[1:3] for s in sites(bad_m0)] == [(0, 1)]
    assert sites(["s_mov_b32 m0, s3", "s_nop 0", "global_load_lds_dwordx4 v[2:3], off"]) == []
    # the form the tile loads had before: M0 written right before the load does
    # not hide a VALU write of the descriptor two instructions back
    both = ["v_readlane_b32 s11, v152, 20", "s_mov_b32 m0, s3", "s_nop 0",
            "buffer_load_dwordx4 v2, s[8:11], s5 offen lds"]
    assert [s[1:3] for s in sites(both)] == [(2, 5)]
    # an SGPR the memory instruction does not read, and a VALU write far enough back
    assert sites(["v_readfirstlane_b32 s7, v1", "buffer_load_dwordx4 v2, s[8:11], s5 offen lds"]) == []
    far = ["v_readfirstlane_b32 s5, v1"] + ["v_add_f32_e32 v3, v3, v3"] * 5 + [
        "buffer_load_dwordx4 v2, s[8:11], s5 offen lds"]
    assert sites(far) == []


def test_hazard_scan_flags_store_data_overwrite():
    """The store-data rule: a VALU write of a data VGPR of a preceding
    16-byte store needs 2 wait states (global data is the second operand,
    buffer data the first); 8-byte stores, SGPR-destination VALU forms and
    writes of other registers are not hazards."""
    from SSA import _hazards

    def sites(body):
        return [s[1:3] for s in _hazards.scan_asm("_Zk:\n" + "\n".join("\t" + ln for ln in body))]

    g = "global_store_dwordx4 v[10:11], v[4:7], off offset:16 nt"
    assert sites([g, "s_nop 0", "v_bitop3_b32 v4, v3, v186, 3 bitop3:0x6c"]) == [(1, 2)]
    assert sites([g, "v_mov_b32_e32 v7, 0"]) == [(0, 2)]
    assert sites([g, "s_nop 1", "v_mov_b32_e32 v7, 0"]) == []
    assert sites([g, "s_nop 0", "v_mov_b32_e32 v10, 0"]) == []  # the address, not the data
    assert sites([g, "v_readfirstlane_b32 s4, v5", "v_cmp_gt_i32_e64 s[2:3], v4, v6"]) == []
    b = "buffer_store_dwordx4 v[20:23], v2, s[8:11], s4 offen offset:512 nt"
    assert sites([b, "s_nop 0", "v_add_u32_e32 v21, 1, v21"]) == [(1, 2)]
    assert sites(["global_store_dwordx2 v[10:11], v[4:5], off", "v_mov_b32_e32 v4, 0"]) == []
    # the instruction after an unconditional transfer is not the store's successor,
    # while a plain label (a fall-through) still is
    assert sites([g, ".LBB0_7:", "s_endpgm", ".LBB0_8:", "v_add_u32_e32 v4, s26, v105"]) == []
    assert sites([g, "s_branch .LBB0_9", ".LBB0_8:", "v_add_u32_e32 v4, s26, v105"]) == []
    assert sites([g, ".LBB0_8:", "v_add_u32_e32 v4, s26, v105"]) == [(0, 2)]


def test_agpr_scan_follows_every_path():
    """SSA/_hazards.py's check of the inline-assembly AGPR accumulations:
    in-place form after its own s_nop, and no other access to the block
    within 19 wait states of the last accumulation on any path (a loop's
    back edge and a branch around the fence included)."""
    from SSA import _hazards

    def acc(dst="a[0:15]", src_c="a[0:15]", nop="s_nop 1"):
        return [";;#ASMSTART", nop, f"v_mfma_f32_32x32x16_bf16 {dst}, v[2:5], v[6:9], {src_c}", ";;#ASMEND"]

    fence = [";;#ASMSTART", "s_nop 7", "s_nop 7", "s_nop 7", ";;#ASMEND"]

    def sites(body):
        text = "_Zk:\n" + "\n".join(ln if ln.startswith(".L") else "\t" + ln for ln in body) + "\n.Lfunc_end0:\n"
        return [(s[1], s[2], s[3].split()[0]) for s in _hazards.scan_agpr(text)]

    loop = ["v_accvgpr_write_b32 a0, 0", ".LBB0_1:", *acc(), "v_add_f32_e32 v3, v3, v3",
            "s_cbranch_scc1 .LBB0_1"]
    assert sites(loop + fence + ["v_accvgpr_read_b32 v10, a3", "s_endpgm"]) == []
    # the read without the fence: 2 wait states after the accumulation
    assert sites(loop + ["v_accvgpr_read_b32 v10, a3", "s_endpgm"]) == [(2, 19, "v_accvgpr_read_b32")]
    # a branch that skips the fence reaches the read 3 wait states after it
    skip = loop + ["s_cbranch_vccnz .LBB0_3"] + fence + [".LBB0_3:", "v_accvgpr_read_b32 v10, a3", "s_endpgm"]
    assert sites(skip) == [(3, 19, "v_accvgpr_read_b32")]
    # an access of another block is not constrained; the loop's back edge is
    # (a copy at the top of the loop, 2 wait states after the previous pass)
    assert sites(loop + ["v_accvgpr_read_b32 v10, a16", "s_endpgm"]) == []
    back = ["v_accvgpr_write_b32 a0, 0", ".LBB0_1:", "v_accvgpr_read_b32 v11, a5", *acc(),
            "v_add_f32_e32 v3, v3, v3", "s_cbranch_scc1 .LBB0_1", *fence, "s_endpgm"]
    assert sites(back) == [(2, 19, "v_accvgpr_read_b32")]
    # an accumulation without its NOP, or not in place
    assert sites([*acc(nop="v_add_f32_e32 v4, v4, v4"), *fence, "s_endpgm"]) == [(0, 2, "v_mfma_f32_32x32x16_bf16")]
    assert sites([*acc(dst="a[16:31]"), *fence, "s_endpgm"]) == [(0, 2, "v_mfma_f32_32x32x16_bf16")]
    # a compiler-issued MFMA is the compiler's business
    assert sites(["v_mfma_f32_32x32x16_bf16 a[0:15], v[2:5], v[6:9], a[0:15]",
                  "v_accvgpr_read_b32 v10, a3", "s_endpgm"]) == []
    # ... except that its VGPR result may not feed an accumulation too soon,
    # on any path (here around a loop: written at the bottom, read at the top)
    mfma_v = "v_mfma_f32_32x32x16_bf16 v[0:15], v[20:23], v[24:27], 0"
    assert sites([mfma_v, "s_nop 7", *acc(), *fence, "s_endpgm"]) == [(10, 19, "v_mfma_f32_32x32x16_bf16")]
    assert sites([mfma_v, "s_nop 7", "s_nop 7", "s_nop 3", *acc(), *fence, "s_endpgm"]) == []
    around = [".LBB0_1:", *acc(), "v_add_f32_e32 v30, v30, v30", mfma_v, "s_cbranch_scc1 .LBB0_1", *fence, "s_endpgm"]
    assert sites(around) == [(3, 19, "v_mfma_f32_32x32x16_bf16")]


_ACC_PROBE = r"""
#include "ssa_common.hpp"
using namespace ssa;
__global__ void acc_probe(float* o, const bf16x8* a) {
  f32x16 c[1] = {f32x16{}}, d[1] = {f32x16{}};
  for (int t = 0; t < 4; ++t) {
    mfma32_acc(c[0], a[threadIdx.x + 128 * t], a[threadIdx.x + 64 + 128 * t]);
    mfma32_acc(d[0], a[threadIdx.x + 64 + 128 * t], a[threadIdx.x + 128 * t]);
  }
#ifdef FENCE
  acc_fence(c, d);
#endif
  for (int i = 0; i < 16; ++i) o[threadIdx.x * 16 + i] = c[0][i] + d[0][i];
}
"""


def test_agpr_scan_on_compiled_accumulation(tmp_path):
    """The accumulation helpers of csrc/ssa_common.hpp through the real
    compiler: without acc_fence() the compiler reads the accumulators right
    after the last inline-assembly MFMA (it does not know the statement is an
    MFMA), and the build's scan reports it; with the fence the scan is clean."""
    import subprocess

    from SSA import _build, _hazards

    try:
        hipcc = _build._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    src = tmp_path / "probe.hip"
    src.write_text(_ACC_PROBE)
    found = {}
    for tag, extra in (("plain", []), ("fenced", ["-DFENCE"])):
        out = tmp_path / f"{tag}.s"
        cmd = [hipcc, *_build.HIPCC_FLAGS, *_build.SOURCE_FLAGS["ssa_bwd.hip"], f"-I{_build.CSRC}", *extra,
               "--cuda-device-only", "-S", str(src), "-o", str(out)]
        subprocess.run(cmd, check=True, capture_output=True, text=True)
        found[tag] = _hazards.scan_agpr(out.read_text())
    assert found["fenced"] == []
    assert found["plain"] and all(ws < need and ins.startswith("v_accvgpr_read") for _, ws, need, ins in found["plain"])


def test_built_device_assembly_has_no_short_waits():
    """The assembly the last build() checked (luciole-1b_amd/_build/*.gfx950.s),
    re-scanned: no vector-memory instruction reads a register too soon."""
    from SSA import _hazards

    asms = sorted((ROOT / "luciole-1b_amd" / "_build").glob("*.gfx950.s"))
    if not asms:
        pytest.skip("no device assembly: run build() first")
    assert _hazards.check_files(asms) == []


def test_ds_workspace_policy(monkeypatch):
    """The Python layer's dS' workspace policy: on for every head dim within
    SSA_BWD_DS_MAX_BYTES, forced either way by SSA_BWD_DS or the ds argument."""
    from SSA.ssa_hip_kernel import _use_ds_workspace

    monkeypatch.delenv("SSA_BWD_DS", raising=False)
    monkeypatch.delenv("SSA_BWD_DS_MAX_BYTES", raising=False)
    for D in (32, 64, 128):
        assert _use_ds_workspace(1 << 30, D, None)
        assert not _use_ds_workspace(17 << 30, D, None)     # above the 16 GiB default cap
        assert not _use_ds_workspace(1 << 20, D, False) and _use_ds_workspace(17 << 30, D, True)
    monkeypatch.setenv("SSA_BWD_DS_MAX_BYTES", str(1 << 20))
    assert not _use_ds_workspace(1 << 21, 64, None) and _use_ds_workspace(1 << 20, 64, None)
    monkeypatch.setenv("SSA_BWD_DS", "0")
    assert not _use_ds_workspace(1 << 10, 128, None)
    monkeypatch.setenv("SSA_BWD_DS", "1")
    assert _use_ds_workspace(1 << 40, 32, None)


def test_ds_workspace_policy_leaves_headroom(monkeypatch):
    """Given a device, the automatic policy also keeps the workspace within half
    of the device's headroom (driver-free plus allocator-cached memory), so a
    large transient dS' never crowds out a training step: above it dq
    recomputes.  Forcing (SSA_BWD_DS=1 or ds=True) overrides it."""
    import SSA.ssa_hip_kernel as hk

    monkeypatch.delenv("SSA_BWD_DS", raising=False)
    monkeypatch.delenv("SSA_BWD_DS_MAX_BYTES", raising=False)
    monkeypatch.setattr(hk, "_device_headroom", lambda device: 8 << 30)
    assert hk._use_ds_workspace(4 << 30, 128, None, "cuda:0")
    assert not hk._use_ds_workspace((4 << 30) + 1, 128, None, "cuda:0")
    assert hk._use_ds_workspace(6 << 30, 128, True, "cuda:0")
    assert hk._use_ds_workspace(6 << 30, 128, None)          # no device: the byte cap alone
    monkeypatch.setattr(hk, "_device_headroom", lambda device: None)  # unknown: the cap alone
    assert hk._use_ds_workspace(6 << 30, 128, None, "cuda:0")
    monkeypatch.setenv("SSA_BWD_DS", "1")
    monkeypatch.setattr(hk, "_device_headroom", lambda device: 0)
    assert hk._use_ds_workspace(6 << 30, 128, None, "cuda:0")


def test_ds_path_by_dtype_and_head_dim():
    """Only the matrix-core kernels (bf16 / fp16, head dims up to 128) use a dS'
    workspace; fp32 and head dim 256 run the vector-ALU kernels, whose dq recomputes."""
    import torch

    from SSA.ssa_hip_kernel import _has_ds_path

    assert _has_ds_path(torch.bfloat16, 128) and _has_ds_path(torch.float16, 32)
    assert not _has_ds_path(torch.bfloat16, 256) and not _has_ds_path(torch.float32, 64)
