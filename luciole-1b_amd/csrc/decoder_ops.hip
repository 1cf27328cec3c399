// Fused element-wise operators of the SSA decoder layer around the attention
// path (gfx950): rotary position embedding.  One HBM pass per call in the
// input dtype; the unfused PyTorch form makes six fp32 passes.
//
// Rotate-half RoPE (Megatron's default, non-interleaved), per (s, b, h) row of
// D values, i < D / 2, with c = cos[s][i], t = sin[s][i]:
//   y[i]         = x[i] c - x[i + D/2] t
//   y[i + D/2]   = x[i + D/2] c + x[i] t
// The inverse (the backward: the transpose of a rotation) uses -t.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ssa_decoder_ops.h"

namespace {

template <typename T>
struct Pack4 {
  typedef T type __attribute__((ext_vector_type(4)));
};

// One thread: 4 frequencies (8 values) of one row.  Rows are (s, b, h) in
// that order; x has strides (ss, sb, sh) and stride 1 over D, y is
// contiguous [S, B, H, D].
template <typename T, int D>
__global__ __launch_bounds__(256) void rope_kernel(const T* __restrict__ x, int64_t ss, int64_t sb, int64_t sh,
                                                   T* __restrict__ y, const float* __restrict__ cs,
                                                   const float* __restrict__ sn, int S, int B, int H, float sign) {
  typedef typename Pack4<T>::type v4;
  typedef float f4 __attribute__((ext_vector_type(4)));
  constexpr int TPR = D / 8;  // threads per row
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t row = gid / TPR;
  const int i = static_cast<int>(gid % TPR) * 4;
  if (row >= static_cast<int64_t>(S) * B * H) return;
  const int h = static_cast<int>(row % H);
  const int64_t sbi = row / H;
  const int b = static_cast<int>(sbi % B), s = static_cast<int>(sbi / B);
  const T* xr = x + s * ss + b * sb + h * sh;
  const v4 x1 = *reinterpret_cast<const v4*>(xr + i);
  const v4 x2 = *reinterpret_cast<const v4*>(xr + i + D / 2);
  const f4 c = *reinterpret_cast<const f4*>(cs + static_cast<int64_t>(s) * (D / 2) + i);
  const f4 t = *reinterpret_cast<const f4*>(sn + static_cast<int64_t>(s) * (D / 2) + i);
  v4 y1, y2;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a = static_cast<float>(x1[e]), bb = static_cast<float>(x2[e]), te = sign * t[e];
    y1[e] = static_cast<T>(a * c[e] - bb * te);
    y2[e] = static_cast<T>(bb * c[e] + a * te);
  }
  T* yr = y + row * D;
  *reinterpret_cast<v4*>(yr + i) = y1;
  *reinterpret_cast<v4*>(yr + i + D / 2) = y2;
}

template <typename T>
hipError_t launch_rope(const ssa_rope_args* a, hipStream_t st) {
  const int64_t rows = static_cast<int64_t>(a->seqlen) * a->batch * a->heads;
  const int64_t threads = rows * (a->head_dim / 8);
  const int grid = static_cast<int>((threads + 255) / 256);
  const T* x = static_cast<const T*>(a->x);
  T* y = static_cast<T*>(a->y);
  const float sign = a->inverse ? -1.f : 1.f;
  switch (a->head_dim) {
    case 64:
      hipLaunchKernelGGL((rope_kernel<T, 64>), dim3(grid), dim3(256), 0, st, x, a->x_stride_s, a->x_stride_b,
                         a->x_stride_h, y, a->cos, a->sin, a->seqlen, a->batch, a->heads, sign);
      break;
    case 128:
      hipLaunchKernelGGL((rope_kernel<T, 128>), dim3(grid), dim3(256), 0, st, x, a->x_stride_s, a->x_stride_b,
                         a->x_stride_h, y, a->cos, a->sin, a->seqlen, a->batch, a->heads, sign);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

}  // namespace

extern "C" int32_t ssa_rope(const ssa_rope_args* a, void* stream) {
  if (a == nullptr || a->x == nullptr || a->y == nullptr || a->cos == nullptr || a->sin == nullptr)
    return SSA_OPS_ERR_NULL_POINTER;
  if (a->seqlen <= 0 || a->batch <= 0 || a->heads <= 0) return SSA_OPS_ERR_SHAPE;
  if (a->head_dim != 64 && a->head_dim != 128) return SSA_OPS_ERR_SHAPE;
  if (a->dtype != 0 && a->dtype != 1) return SSA_OPS_ERR_DTYPE;
  if (a->x_stride_s < 0 || a->x_stride_b < 0 || a->x_stride_h < 0) return SSA_OPS_ERR_ALIGNMENT;
  // 8-byte vector accesses: every row start and the tables 4-element aligned
  if (!aligned(a->x, 8) || !aligned(a->y, 8) || !aligned(a->cos, 16) || !aligned(a->sin, 16) ||
      (a->x_stride_s % 4) != 0 || (a->x_stride_b % 4) != 0 || (a->x_stride_h % 4) != 0)
    return SSA_OPS_ERR_ALIGNMENT;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const hipError_t e = a->dtype == 0 ? launch_rope<__bf16>(a, st) : launch_rope<_Float16>(a, st);
  return e == hipSuccess ? SSA_OPS_OK : SSA_OPS_ERR_LAUNCH;
}
