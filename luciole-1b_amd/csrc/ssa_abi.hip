// C ABI of libssa_mi355x.so: host-side validation and dispatch.
//
// Mirrors the checks of the reference launch layer
// (training/train/train_ssa_triton/SSA/ssa_triton_kernel.py:748-764, 802-809,
// 852-857) as status codes, plus the layout requirements of these kernels.
// Nothing is launched unless every check passes.
#include <stdint.h>

#include "../../include/ssa_mi355x.h"
#include "ssa_launch.hpp"

namespace {

using ssa::Tensor4;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int32_t check_tensor(const ssa_tensor4& t, bool required) {
  if (t.ptr == nullptr) return required ? SSA_ERR_NULL_POINTER : SSA_OK;
  if (!aligned16(t.ptr)) return SSA_ERR_ALIGNMENT;
  if ((t.stride_b % 8) != 0 || (t.stride_h % 8) != 0 || (t.stride_s % 8) != 0) return SSA_ERR_ALIGNMENT;
  if (t.stride_b < 0 || t.stride_h < 0 || t.stride_s < 0) return SSA_ERR_ALIGNMENT;
  // Tile loads address rows with 32-bit byte offsets from a per-tile base.
  if (t.stride_s >= (1ll << 24)) return SSA_ERR_ALIGNMENT;
  return SSA_OK;
}

// Sizes every launcher can take with int32 arithmetic: sequence lengths up
// to 2^30 (so N + tile - 1 fits), at most 2^28 units of 128 rows per grid
// (the smallest workgroup covers 64 rows, so every grid size fits), and --
// checked separately -- at most INT32_MAX query rows per launch over dense
// batches (B * Hq * N) and packed streams (Hq * T), the rows the Delta kernels
// cover.
constexpr int64_t kMaxSeqlen = 1ll << 30;
constexpr int64_t kMaxGridUnits = 1ll << 28;

bool shape_ok(int32_t B, int32_t Hq, int32_t Hkv, int32_t N) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || N <= 0 || N > kMaxSeqlen) return false;
  if (Hq % Hkv != 0) return false;
  const int64_t bh = static_cast<int64_t>(B) * Hq;
  return bh <= kMaxGridUnits && bh * ((static_cast<int64_t>(N) + 127) / 128) <= kMaxGridUnits;
}

bool rows_ok(int64_t a, int64_t b, int64_t c) {
  return a > 0 && b > 0 && c > 0 && a * b <= INT32_MAX && a * b * c <= INT32_MAX;
}

// a * b for non-negative operands, or -1 when either is negative or the
// product does not fit int64.
int64_t mul_or_neg(int64_t a, int64_t b) {
  int64_t r = 0;
  return (a < 0 || b < 0 || __builtin_mul_overflow(a, b, &r)) ? -1 : r;
}

int32_t check_common(int32_t B, int32_t Hq, int32_t Hkv, int32_t N, int32_t D, int32_t dtype, bool packed) {
  if (!shape_ok(B, Hq, Hkv, N)) return SSA_ERR_SHAPE;
  if (!packed && !rows_ok(B, Hq, N)) return SSA_ERR_SHAPE;
  if (dtype != SSA_DTYPE_BF16 && dtype != SSA_DTYPE_FP16 && dtype != SSA_DTYPE_FP32) return SSA_ERR_DTYPE;
  if (D != 32 && D != 64 && D != 128 && D != 256 && !(D == 16 && dtype == SSA_DTYPE_FP32)) return SSA_ERR_HEAD_DIM;
  return SSA_OK;
}

Tensor4 to_t4(const ssa_tensor4& t) { return Tensor4{t.ptr, t.stride_b, t.stride_h, t.stride_s}; }

#define SSA_TRY(expr)                 \
  do {                                \
    const int32_t st_ = (expr);       \
    if (st_ != SSA_OK) return st_;    \
  } while (0)

int32_t fill_fwd(const ssa_fwd_args* a, ssa::FwdParams* p, bool packed) {
  if (a == nullptr) return SSA_ERR_NULL_POINTER;
  SSA_TRY(check_common(a->batch, a->heads_q, a->heads_kv, a->seqlen, a->head_dim, a->dtype, packed));
  SSA_TRY(check_tensor(a->q, true));
  SSA_TRY(check_tensor(a->k, true));
  SSA_TRY(check_tensor(a->v, true));
  SSA_TRY(check_tensor(a->out, true));
  if (a->m == nullptr || a->ssa_n == nullptr || a->ssa_b == nullptr) return SSA_ERR_NULL_POINTER;
  p->q = to_t4(a->q);
  p->k = to_t4(a->k);
  p->v = to_t4(a->v);
  p->o = to_t4(a->out);
  p->m = a->m;
  p->n_ptr = a->ssa_n;
  p->b_ptr = a->ssa_b;
  p->B = a->batch;
  p->Hq = a->heads_q;
  p->Hkv = a->heads_kv;
  p->N = a->seqlen;
  p->scale = a->softmax_scale;
  p->cu_seqlens = nullptr;
  p->T = 0;
  return SSA_OK;
}

// Packed batches: the document table itself lives on the device and is only
// clamped there (see SeqView); the host checks what it can see.
int32_t check_varlen(int32_t docs, int32_t heads_q, int32_t max_seqlen, const int32_t* cu, int32_t total) {
  if (cu == nullptr) return SSA_ERR_NULL_POINTER;
  if (total <= 0 || docs <= 0 || max_seqlen <= 0 || max_seqlen > total) return SSA_ERR_CU_SEQLENS;
  if (!rows_ok(heads_q, total, 1)) return SSA_ERR_SHAPE;
  return SSA_OK;
}

int32_t launch_status(hipError_t e) { return e == hipSuccess ? SSA_OK : SSA_ERR_LAUNCH; }

bool decode_shape_ok(int32_t B, int32_t Hq, int32_t Hkv, int32_t cap, int32_t requested) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || cap <= 0 || cap > kMaxSeqlen || requested < 0 || Hq % Hkv != 0) return false;
  if (static_cast<int64_t>(B) * Hq >= (1ll << 30)) return false;
  // one workgroup per (batch, kv-head, group of 32 q-heads, split): int32 grid
  const int64_t units = static_cast<int64_t>(B) * Hkv * ((Hq / Hkv + 31ll) / 32);
  return units * ((static_cast<int64_t>(cap) + 127) / 128) < (1ll << 30);
}

// Decode workspace: (m, l) pairs of every (batch, q-head, split) record,
// padded to 16 bytes, then the records' acc[D].
int64_t decode_ml_floats(int64_t recs) { return (2 * recs + 3) & ~static_cast<int64_t>(3); }
int64_t decode_ws_bytes(int32_t B, int32_t Hq, int32_t D, int32_t splits) {
  if (splits <= 1) return 0;
  const int64_t recs = static_cast<int64_t>(B) * Hq * splits;
  return (decode_ml_floats(recs) + recs * D) * 4;
}

}  // namespace

namespace ssa {

// Validation and parameters of the backward entry points.  with_workspaces =
// false (ssa_bwd_noalloc) ignores delta, partials and ds_workspace: the
// caller of that entry point supplies them from its own storage.
int32_t fill_bwd_params(const ssa_bwd_args* a, BwdParams* p, bool preprocess_only, bool with_workspaces,
                        bool packed) {
  if (a == nullptr) return SSA_ERR_NULL_POINTER;
  SSA_TRY(check_common(a->batch, a->heads_q, a->heads_kv, a->seqlen, a->head_dim, a->dtype, packed));
  SSA_TRY(check_tensor(a->out, true));
  SSA_TRY(check_tensor(a->dout, true));
  if (with_workspaces && a->delta == nullptr) return SSA_ERR_NULL_POINTER;
  if (!preprocess_only) {
    SSA_TRY(check_tensor(a->q, true));
    SSA_TRY(check_tensor(a->k, true));
    SSA_TRY(check_tensor(a->v, true));
    SSA_TRY(check_tensor(a->dq, true));
    SSA_TRY(check_tensor(a->dk, true));
    SSA_TRY(check_tensor(a->dv, true));
    if (a->m == nullptr || (with_workspaces && a->partials == nullptr) || a->dn == nullptr || a->db == nullptr ||
        a->ssa_n == nullptr || a->ssa_b == nullptr)
      return SSA_ERR_NULL_POINTER;
  }
  p->q = to_t4(a->q);
  p->k = to_t4(a->k);
  p->v = to_t4(a->v);
  p->o = to_t4(a->out);
  p->dout = to_t4(a->dout);
  p->dq = to_t4(a->dq);
  p->dk = to_t4(a->dk);
  p->dv = to_t4(a->dv);
  p->m = a->m;
  p->delta = a->delta;
  p->partials = a->partials;
  p->dn = a->dn;
  p->db = a->db;
  p->n_ptr = a->ssa_n;
  p->b_ptr = a->ssa_b;
  p->B = a->batch;
  p->Hq = a->heads_q;
  p->Hkv = a->heads_kv;
  p->N = a->seqlen;
  p->scale = a->softmax_scale;
  p->cu_seqlens = nullptr;
  p->T = 0;
  if (with_workspaces && !preprocess_only && a->ds_workspace != nullptr && !aligned16(a->ds_workspace))
    return SSA_ERR_ALIGNMENT;
  p->ds = (preprocess_only || !with_workspaces) ? nullptr : a->ds_workspace;
  return SSA_OK;
}

// dQ then the dn / db reduction: on the workspace path (the matrix-core
// kernels with a dS' workspace) the dQ pass's first workgroup does the
// reduction, so it needs no launch of its own.
int32_t run_dq_and_reduce(const BwdParams& p, int dtype, int D, bool causal, hipStream_t s) {
  BwdParams pq = p;
  pq.fuse_reduce = p.ds != nullptr && !use_f32(dtype, D);
  SSA_TRY(launch_status(launch_bwd_dq(pq, dtype, D, causal, s)));
  return pq.fuse_reduce ? SSA_OK : launch_status(launch_reduce_partials(p, s));
}

// The whole backward on one stream: preprocess, dK/dV, dQ, reduction.
int32_t run_bwd(const BwdParams& p, int dtype, int D, bool causal, hipStream_t s) {
  SSA_TRY(launch_status(launch_bwd_preprocess(p, dtype, D, s)));
  SSA_TRY(launch_status(launch_bwd_dkdv(p, dtype, D, causal, s)));
  return run_dq_and_reduce(p, dtype, D, causal, s);
}

}  // namespace ssa

extern "C" {

int32_t ssa_abi_version(void) { return SSA_ABI_VERSION; }

const char* ssa_status_string(int32_t status) {
  switch (status) {
    case SSA_OK: return "ok";
    case SSA_ERR_NULL_POINTER: return "a required pointer is NULL";
    case SSA_ERR_SHAPE:
      return "invalid shape (batch, heads, seqlen must be > 0 and Hq % Hkv == 0; size limits: seqlen and decode "
             "capacity <= 2^30, batch * heads_q * ceil(seqlen / 128) <= 2^28, at most 2^31 - 1 query rows per "
             "launch: batch * heads_q * seqlen, or heads_q * total_tokens for packed sequences)";
    case SSA_ERR_HEAD_DIM: return "unsupported head_dim (supported: 32, 64, 128, 256; fp32 also 16)";
    case SSA_ERR_DTYPE: return "unsupported dtype (supported: bf16, fp16, fp32; the decode step bf16, fp16)";
    case SSA_ERR_ALIGNMENT:
      return "unsupported tensor layout (base pointer 16-byte aligned, strides non-negative multiples of 8 "
             "elements, row stride below 2^24 elements)";
    case SSA_ERR_LAUNCH: return "HIP kernel launch failed";
    case SSA_ERR_CU_SEQLENS:
      return "invalid packed-sequence arguments (total_tokens, documents and max_seqlen must be > 0, "
             "max_seqlen <= total_tokens)";
    case SSA_ERR_SCRATCH:
      return "problem too large for the static scratch of ssa_bwd_noalloc (Delta plus the dn/db partials "
             "must fit SSA_NOALLOC_SCRATCH_BYTES)";
    default: return "unknown status";
  }
}

int64_t ssa_bwd_partials_count(int32_t batch, int32_t heads_kv, int32_t seqlen) {
  if (!shape_ok(batch, heads_kv, heads_kv, seqlen)) return 0;
  return 2ll * batch * heads_kv * ssa::dkdv_key_blocks(seqlen);
}

int64_t ssa_bwd_ds_workspace_bytes(int32_t batch, int32_t heads_q, int32_t seqlen, int32_t causal) {
  if (!shape_ok(batch, heads_q, heads_q, seqlen) || !rows_ok(batch, heads_q, seqlen)) return 0;
  const int64_t tiles = mul_or_neg(static_cast<int64_t>(batch) * heads_q, ssa::ds_tiles_per_head(seqlen, causal != 0));
  const int64_t bytes = mul_or_neg(tiles, 1024);
  return bytes < 0 ? 0 : bytes;
}

int64_t ssa_varlen_bwd_ds_workspace_bytes(int32_t batch, int32_t heads_q, int32_t max_seqlen, int32_t total_tokens,
                                          int32_t causal) {
  if (!shape_ok(batch, heads_q, heads_q, max_seqlen) || total_tokens < max_seqlen ||
      !rows_ok(heads_q, total_tokens, 1))
    return 0;
  // ds_packed_tiles() = (T / 32 + B) * Hq * ds_slot_tiles(Nmax), multiplied with overflow checks
  const int64_t slots = static_cast<int64_t>(total_tokens / 32) + batch;
  const int64_t tiles = mul_or_neg(slots * heads_q, ssa::ds_slot_tiles(max_seqlen, causal != 0));
  const int64_t bytes = mul_or_neg(tiles, 1024);
  return bytes < 0 ? 0 : bytes;
}

int32_t ssa_decode_num_splits(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t capacity,
                              int32_t requested) {
  if (!decode_shape_ok(batch, heads_q, heads_kv, capacity, requested)) return 0;
  return ssa::decode_splits(batch, heads_q, heads_kv, capacity, requested);
}

int64_t ssa_decode_workspace_bytes(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t capacity,
                                   int32_t head_dim, int32_t requested) {
  if (!decode_shape_ok(batch, heads_q, heads_kv, capacity, requested)) return 0;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128) return 0;
  return decode_ws_bytes(batch, heads_q, head_dim,
                         ssa::decode_splits(batch, heads_q, heads_kv, capacity, requested));
}

int32_t ssa_decode(const ssa_decode_args* a, void* stream) {
  if (a == nullptr) return SSA_ERR_NULL_POINTER;
  if (!decode_shape_ok(a->batch, a->heads_q, a->heads_kv, a->capacity, a->num_splits)) return SSA_ERR_SHAPE;
  if (a->head_dim != 32 && a->head_dim != 64 && a->head_dim != 128) return SSA_ERR_HEAD_DIM;
  if (a->dtype != SSA_DTYPE_BF16 && a->dtype != SSA_DTYPE_FP16) return SSA_ERR_DTYPE;
  SSA_TRY(check_tensor(a->q, true));
  SSA_TRY(check_tensor(a->k_cache, true));
  SSA_TRY(check_tensor(a->v_cache, true));
  SSA_TRY(check_tensor(a->out, true));
  if (a->cache_seqlens == nullptr || a->ssa_n == nullptr || a->ssa_b == nullptr) return SSA_ERR_NULL_POINTER;
  ssa::DecodeParams p{};
  p.splits = ssa::decode_splits(a->batch, a->heads_q, a->heads_kv, a->capacity, a->num_splits);
  p.split_keys = ssa::decode_split_keys(a->capacity, p.splits);
  if (p.splits > 1) {
    if (a->workspace == nullptr) return SSA_ERR_NULL_POINTER;
    if (!aligned16(a->workspace)) return SSA_ERR_ALIGNMENT;
    const int64_t recs = static_cast<int64_t>(a->batch) * a->heads_q * p.splits;
    p.ws_ml = static_cast<float*>(a->workspace);
    p.ws_acc = p.ws_ml + decode_ml_floats(recs);
  }
  p.q = to_t4(a->q);
  p.k = to_t4(a->k_cache);
  p.v = to_t4(a->v_cache);
  p.o = to_t4(a->out);
  p.m = a->m;
  p.seqlens = a->cache_seqlens;
  p.n_ptr = a->ssa_n;
  p.b_ptr = a->ssa_b;
  p.B = a->batch;
  p.Hq = a->heads_q;
  p.Hkv = a->heads_kv;
  p.cap = a->capacity;
  p.scale = a->softmax_scale;
  return launch_status(ssa::launch_decode(p, a->dtype, a->head_dim, static_cast<hipStream_t>(stream)));
}

int32_t ssa_fwd(const ssa_fwd_args* a, void* stream) {
  ssa::FwdParams p{};
  SSA_TRY(fill_fwd(a, &p, false));
  return launch_status(
      ssa::launch_fwd(p, a->dtype, a->head_dim, a->causal != 0, static_cast<hipStream_t>(stream)));
}

int32_t ssa_varlen_fwd(const ssa_varlen_fwd_args* va, void* stream) {
  if (va == nullptr) return SSA_ERR_NULL_POINTER;
  const ssa_fwd_args* a = &va->dense;
  ssa::FwdParams p{};
  SSA_TRY(fill_fwd(a, &p, true));
  SSA_TRY(check_varlen(a->batch, a->heads_q, a->seqlen, va->cu_seqlens, va->total_tokens));
  p.cu_seqlens = va->cu_seqlens;
  p.T = va->total_tokens;
  hipStream_t s = static_cast<hipStream_t>(stream);
  SSA_TRY(launch_status(ssa::launch_fwd(p, a->dtype, a->head_dim, a->causal != 0, s)));
  ssa::VarlenFill f{};
  f.t[0] = p.o;
  f.heads[0] = a->heads_q;
  f.ntensors = 1;
  f.m = a->m;
  f.m_heads = a->heads_q;
  f.cu = va->cu_seqlens;
  f.B = a->batch;
  f.T = va->total_tokens;
  f.Nmax = a->seqlen;
  f.D = a->head_dim;
  f.esize = a->dtype == SSA_DTYPE_FP32 ? 4 : 2;
  return launch_status(ssa::launch_varlen_fill(f, s));
}

int32_t ssa_varlen_bwd(const ssa_varlen_bwd_args* va, void* stream) {
  if (va == nullptr) return SSA_ERR_NULL_POINTER;
  const ssa_bwd_args* a = &va->dense;
  ssa::BwdParams p{};
  SSA_TRY(ssa::fill_bwd_params(a, &p, false, true, true));
  SSA_TRY(check_varlen(a->batch, a->heads_q, a->seqlen, va->cu_seqlens, va->total_tokens));
  p.cu_seqlens = va->cu_seqlens;
  p.T = va->total_tokens;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool causal = a->causal != 0;
  // Delta over the whole token stream: one sequence of T rows, [H, T] layout.
  ssa::BwdParams pre = p;
  pre.cu_seqlens = nullptr;
  pre.B = 1;
  pre.N = va->total_tokens;
  SSA_TRY(launch_status(ssa::launch_bwd_preprocess(pre, a->dtype, a->head_dim, s)));
  SSA_TRY(launch_status(ssa::launch_bwd_dkdv(p, a->dtype, a->head_dim, causal, s)));
  SSA_TRY(ssa::run_dq_and_reduce(p, a->dtype, a->head_dim, causal, s));
  ssa::VarlenFill f{};
  f.t[0] = p.dq;
  f.t[1] = p.dk;
  f.t[2] = p.dv;
  f.heads[0] = a->heads_q;
  f.heads[1] = f.heads[2] = a->heads_kv;
  f.ntensors = 3;
  f.cu = va->cu_seqlens;
  f.B = a->batch;
  f.T = va->total_tokens;
  f.Nmax = a->seqlen;
  f.D = a->head_dim;
  f.esize = a->dtype == SSA_DTYPE_FP32 ? 4 : 2;
  return launch_status(ssa::launch_varlen_fill(f, s));
}

int32_t ssa_bwd_preprocess(const ssa_bwd_args* a, void* stream) {
  ssa::BwdParams p{};
  SSA_TRY(ssa::fill_bwd_params(a, &p, true, true, false));
  return launch_status(ssa::launch_bwd_preprocess(p, a->dtype, a->head_dim, static_cast<hipStream_t>(stream)));
}

int32_t ssa_bwd_dkdv(const ssa_bwd_args* a, void* stream) {
  ssa::BwdParams p{};
  SSA_TRY(ssa::fill_bwd_params(a, &p, false, true, false));
  return launch_status(
      ssa::launch_bwd_dkdv(p, a->dtype, a->head_dim, a->causal != 0, static_cast<hipStream_t>(stream)));
}

int32_t ssa_bwd_dq(const ssa_bwd_args* a, void* stream) {
  ssa::BwdParams p{};
  SSA_TRY(ssa::fill_bwd_params(a, &p, false, true, false));
  return launch_status(
      ssa::launch_bwd_dq(p, a->dtype, a->head_dim, a->causal != 0, static_cast<hipStream_t>(stream)));
}

int32_t ssa_bwd_reduce(const ssa_bwd_args* a, void* stream) {
  ssa::BwdParams p{};
  SSA_TRY(ssa::fill_bwd_params(a, &p, false, true, false));
  return launch_status(ssa::launch_reduce_partials(p, static_cast<hipStream_t>(stream)));
}

int32_t ssa_bwd(const ssa_bwd_args* a, void* stream) {
  ssa::BwdParams p{};
  SSA_TRY(ssa::fill_bwd_params(a, &p, false, true, false));
  return ssa::run_bwd(p, a->dtype, a->head_dim, a->causal != 0, static_cast<hipStream_t>(stream));
}

}  // extern "C"
