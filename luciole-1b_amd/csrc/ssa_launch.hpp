// Host-side launchers implemented in the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>

#include "ssa_common.hpp"

namespace ssa {

// dtype: 0 = bf16, 1 = fp16.  D in {32, 64, 128} (validated by the caller).
hipError_t launch_fwd(const FwdParams& p, int dtype, int D, bool causal, hipStream_t stream);
hipError_t launch_bwd_preprocess(const BwdParams& p, int dtype, int D, hipStream_t stream);
hipError_t launch_bwd_dkdv(const BwdParams& p, int dtype, int D, bool causal, hipStream_t stream);
hipError_t launch_bwd_dq(const BwdParams& p, int dtype, int D, bool causal, hipStream_t stream);
hipError_t launch_reduce_partials(const BwdParams& p, hipStream_t stream);

hipError_t launch_decode(const DecodeParams& p, int dtype, int D, hipStream_t stream);

// Decode key splits.  A split covers decode_split_keys() keys (a multiple of
// 128); the default asks for about 256 workgroups (one per CU: a second
// round of workgroups costs more than the longer splits save) but no split
// shorter than 256 keys.
inline int decode_split_keys(int cap, int splits) {
  const int sk = (cap + splits - 1) / splits;
  return (sk + 127) / 128 * 128;
}
inline int decode_splits(int B, int Hq, int Hkv, int cap, int requested) {
  int want = requested;
  if (want <= 0) {
    const int64_t units = static_cast<int64_t>(B) * Hkv * ((Hq / Hkv + 31) / 32);
    const int64_t most = (cap + 255) / 256;
    const int64_t w = (256 + units - 1) / units;
    want = static_cast<int>(w < most ? w : most);
    if (want < 1) want = 1;
  }
  const int sk = decode_split_keys(cap, want);
  return (cap + sk - 1) / sk;
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

}  // namespace ssa
