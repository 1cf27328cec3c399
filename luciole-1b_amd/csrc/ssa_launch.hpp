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

// Number of key blocks of the dK/dV kernel (each writes one dn and one db partial).
__host__ __device__ inline int dkdv_key_blocks(int N) { return (N + 127) / 128; }

}  // namespace ssa
