// Host-side launchers implemented in the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>

#include "ssa_common.hpp"

namespace ssa {

// dtype: 0 = bf16, 1 = fp16 (D in {32, 64, 128, 256}), 2 = fp32 (D in {16,
// 32, 64, 128, 256}); validated by the caller.  Which kernels run: use_f32().
hipError_t launch_fwd(const FwdParams& p, int dtype, int D, bool causal, hipStream_t stream);
hipError_t launch_bwd_preprocess(const BwdParams& p, int dtype, int D, hipStream_t stream);
hipError_t launch_bwd_dkdv(const BwdParams& p, int dtype, int D, bool causal, hipStream_t stream);
// dK/dV with two waves per SIMD (ssa_bwd_dkdv2w.hip): bf16 / fp16, D in {32, 64, 128}.
hipError_t launch_bwd_dkdv2w(const BwdParams& p, int dtype, int D, bool causal, bool off32, hipStream_t stream);
hipError_t launch_bwd_dq(const BwdParams& p, int dtype, int D, bool causal, hipStream_t stream);
// dQ from the dS' workspace (ssa_bwd_dq.hip): bf16 / fp16, D in {32, 64, 128}.
hipError_t launch_bwd_dq_ds(const BwdParams& p, int dtype, int D, bool causal, hipStream_t stream);
hipError_t launch_reduce_partials(const BwdParams& p, hipStream_t stream);

hipError_t launch_decode(const DecodeParams& p, int dtype, int D, hipStream_t stream);

// The fp32-arithmetic vector-ALU kernels (ssa_f32.hip) run fp32 inputs at
// every head dim and bf16 / fp16 inputs at head dim 256; the matrix-core
// kernels run bf16 / fp16 at 32, 64 and 128.  The vector-ALU backward does
// not use the dS' workspace (its dQ recomputes).
constexpr int kDtypeF32 = 2;
inline bool use_f32(int dtype, int D) { return dtype == kDtypeF32 || D == 256; }
hipError_t launch_fwd_f32(const FwdParams& p, int dtype, int D, bool causal, hipStream_t stream);
hipError_t launch_bwd_preprocess_f32(const BwdParams& p, int dtype, int D, hipStream_t stream);
hipError_t launch_bwd_dkdv_f32(const BwdParams& p, int dtype, int D, bool causal, hipStream_t stream);
hipError_t launch_bwd_dq_f32(const BwdParams& p, int dtype, int D, bool causal, hipStream_t stream);

}  // namespace ssa

struct ssa_bwd_args;  // include/ssa_mi355x.h

namespace ssa {

// Backward entry points (ssa_abi.hip): validation + parameters, and the four
// launches of a whole backward in order.  with_workspaces = false leaves
// delta, partials and ds unset for a caller that supplies them itself;
// packed = true skips the dense row-count limit (a packed stream's rows are
// checked against its token count instead).
int32_t fill_bwd_params(const ssa_bwd_args* a, BwdParams* p, bool preprocess_only, bool with_workspaces,
                        bool packed);
int32_t run_bwd(const BwdParams& p, int dtype, int D, bool causal, hipStream_t s);
int32_t run_dq_and_reduce(const BwdParams& p, int dtype, int D, bool causal, hipStream_t s);

// Packed batches: write the token rows no document covers (ssa_varlen_fill.hip):
// up to three [T, H, D] tensors of esize-byte elements (rows set to 0) and
// optionally an [m_heads, T] fp32 normaliser (set to -inf).
struct VarlenFill {
  Tensor4 t[3];
  int heads[3];
  int ntensors;
  float* m;
  int m_heads;
  const int* cu;
  int B, T, Nmax, D;
  int esize;  // bytes per element: 2 (bf16 / fp16) or 4 (fp32)
};
hipError_t launch_varlen_fill(const VarlenFill& f, hipStream_t stream);

// Decode key splits.  A split covers decode_split_keys() keys (a multiple of
// 128); the default asks for about 256 workgroups (one per CU: a second
// round of workgroups costs more than the longer splits save) but no split
// shorter than 256 keys.
inline int decode_split_keys(int cap, int splits) {
  const int64_t sk = (static_cast<int64_t>(cap) + splits - 1) / splits;
  return static_cast<int>((sk + 127) / 128 * 128);
}
inline int decode_splits(int B, int Hq, int Hkv, int cap, int requested) {
  int want = requested;
  if (want <= 0) {
    const int64_t units = static_cast<int64_t>(B) * Hkv * ((Hq / Hkv + 31ll) / 32);
    const int64_t most = (cap + 255ll) / 256;
    const int64_t w = (256 + units - 1) / units;
    want = static_cast<int>(w < most ? w : most);
    if (want < 1) want = 1;
  }
  const int64_t sk = decode_split_keys(cap, want);
  return static_cast<int>((cap + sk - 1) / sk);
}

// Number of key blocks of the dK/dV kernel (each writes one dn and one db partial).
__host__ __device__ inline int dkdv_key_blocks(int N) { return (N + 127) / 128; }

// dS' workspace: per (b, q-head) a sequence of 1 KB tiles, each 32 queries x
// 16 keys of dS' in bf16/fp16, 16 bytes per lane of the writing wave (lane
// 16 g + kl: key kl, queries 16 t + 4 g + (0..3) in elements 4 t ..).  Query
// tile qi (rows 32 qi ..) holds key tiles kj = 0 .. 2 qi + 1 under the causal
// mask (the triangle), kj = 0 .. 2 nq32 - 1 without it.
__host__ __device__ inline int64_t ds_tiles_per_head(int N, bool causal) {
  const int64_t nq = (N + 31) / 32;
  return causal ? nq * (nq + 1) : 2 * nq * nq;
}
__host__ __device__ inline int64_t ds_row_offset(int qi, int N, bool causal) {
  const int64_t q = qi;
  return causal ? q * (q + 1) : q * 2 * ((N + 31) / 32);
}

// Packed batches (longest document Nmax, T tokens): document b, first token
// s0, length L, owns the tiles from ((s0 / 32) + b) * Hq * ds_slot_tiles(Nmax)
// on, its heads' ds_tiles_per_head(L) tiles one after another.  That range
// holds ceil(L / 32) slots of Hq * ds_slot_tiles(Nmax) tiles, at least the
// Hq triangles (nq (nq + 1) <= nq (nq_max + 1), 2 nq^2 <= nq 2 nq_max), and
// s0 / 32 + b grows by at least ceil(L / 32) from one document to the next,
// so documents do not overlap.  For any table clamped to [0, T]
// (s0 + L <= T), floor(s0 / 32) + ceil(L / 32) <= floor(T / 32) + 1, so every
// tile lies below (T / 32 + B) slots: ds_packed_tiles().
__host__ __device__ inline int64_t ds_slot_tiles(int Nmax, bool causal) {
  const int64_t nq = (Nmax + 31) / 32;
  return causal ? nq + 1 : 2 * nq;
}
__host__ __device__ inline int64_t ds_packed_tiles(int B, int Hq, int T, int Nmax, bool causal) {
  return (static_cast<int64_t>(T / 32) + B) * Hq * ds_slot_tiles(Nmax, causal);
}
// First workspace tile of (sequence b, q-head h): packed (tok0 = s0, N = L)
// or dense (N = Nmax).
__host__ __device__ inline int64_t ds_head_tile(bool packed, int64_t tok0, int b, int h, int Hq, int N, int Nmax,
                                                bool causal) {
  if (packed) return ((tok0 >> 5) + b) * Hq * ds_slot_tiles(Nmax, causal) + h * ds_tiles_per_head(N, causal);
  return (static_cast<int64_t>(b) * Hq + h) * ds_tiles_per_head(Nmax, causal);
}

}  // namespace ssa
