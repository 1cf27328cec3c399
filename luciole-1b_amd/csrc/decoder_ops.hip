// Fused element-wise operators of the SSA decoder layer around the attention
// path (gfx950): rotary position embedding (one HBM pass per call in the
// input dtype; the unfused PyTorch form makes six fp32 passes), RMSNorm
// (one pass forward, one backward, plus a fixed-order weight-gradient sum),
// the SwiGLU gate (one pass each way) and the output layer's cross-entropy
// (one pass over the logits each way, no fp32 copy of them).
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

// ---------------------------------------------------------------------------
// RMSNorm over rows of H fp32 values: r = (mean(x^2) + eps)^-1/2,
// y = (x r) w in the output dtype.  Backward, with g = dy w and xh = x r:
//   dx = r (g - xh sum(g xh) / H),  dw = sum over rows of dy xh.
constexpr int kNormThreads = 256;
constexpr int kNormBwdRows = 64;  // rows per backward workgroup (one dw partial each)

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();  // red is reused by consecutive calls
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

template <typename TO>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_fwd_kernel(const float* __restrict__ x,
                                                                   const float* __restrict__ w,
                                                                   TO* __restrict__ y, float* __restrict__ rstd,
                                                                   int H, float eps) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * H;
  float ss = 0.f;
  for (int c = threadIdx.x * 4; c < H; c += kNormThreads * 4) {
    const f4 v = *reinterpret_cast<const f4*>(xr + c);
    ss += (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
  }
  const float r = rsqrtf(block_sum(ss, red) / H + eps);
  TO* yr = y + row * H;
  for (int c = threadIdx.x * 4; c < H; c += kNormThreads * 4) {
    const f4 v = *reinterpret_cast<const f4*>(xr + c);
    const f4 wv = *reinterpret_cast<const f4*>(w + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) yr[c + e] = static_cast<TO>(v[e] * r * wv[e]);
  }
  if (threadIdx.x == 0) rstd[row] = r;
}

template <typename TG>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_bwd_kernel(const float* __restrict__ x,
                                                                   const float* __restrict__ w,
                                                                   const TG* __restrict__ dy,
                                                                   const float* __restrict__ rstd,
                                                                   float* __restrict__ dx, float* __restrict__ dw_part,
                                                                   int T, int H) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  constexpr int MAXC = 4;  // column groups of 4 per thread: H <= 4 * 4 * 256
  __shared__ float red[4];
  f4 acc[MAXC];
#pragma unroll
  for (int k = 0; k < MAXC; ++k) acc[k] = f4{0.f, 0.f, 0.f, 0.f};
  const int r0 = blockIdx.x * kNormBwdRows;
  const int r1 = min(T, r0 + kNormBwdRows);
  for (int row = r0; row < r1; ++row) {
    const float* xr = x + static_cast<int64_t>(row) * H;
    const TG* gr = dy + static_cast<int64_t>(row) * H;
    const float r = rstd[row];
    f4 xh[MAXC], g[MAXC], gy[MAXC];
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
      const int c = (threadIdx.x + k * kNormThreads) * 4;
      if (c < H) {
        const f4 v = *reinterpret_cast<const f4*>(xr + c);
        const f4 wv = *reinterpret_cast<const f4*>(w + c);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          gy[k][e] = static_cast<float>(gr[c + e]);
          xh[k][e] = v[e] * r;
          g[k][e] = gy[k][e] * wv[e];
          dot += g[k][e] * xh[k][e];
        }
      }
    }
    const float m = block_sum(dot, red) / H;
    float* dxr = dx + static_cast<int64_t>(row) * H;
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
      const int c = (threadIdx.x + k * kNormThreads) * 4;
      if (c < H) {
        f4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[e] = r * (g[k][e] - xh[k][e] * m);
          acc[k][e] += gy[k][e] * xh[k][e];
        }
        *reinterpret_cast<f4*>(dxr + c) = o;
      }
    }
  }
  float* part = dw_part + static_cast<int64_t>(blockIdx.x) * H;
#pragma unroll
  for (int k = 0; k < MAXC; ++k) {
    const int c = (threadIdx.x + k * kNormThreads) * 4;
    if (c < H) *reinterpret_cast<f4*>(part + c) = acc[k];
  }
}

// dw[c] = sum over partials b (in order) of dw_part[b][c]
__global__ __launch_bounds__(256) void rmsnorm_dw_kernel(const float* __restrict__ dw_part, float* __restrict__ dw,
                                                         int nparts, int H) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= H) return;
  float s = 0.f;
  for (int b = 0; b < nparts; ++b) s += dw_part[static_cast<int64_t>(b) * H + c];
  dw[c] = s;
}

// ---------------------------------------------------------------------------
// SwiGLU of the MLP: z = [gate | up] rows of 2F values (the fc1 output), h =
// silu(gate) up with silu(g) = g sigmoid(g), in fp32, rounded once.
// Backward from dh: with s = sigmoid(g), d_up = dh silu(g) and
// d_gate = dh up s (1 + g (1 - s)), written as the [d_gate | d_up] rows of dz.
template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(const T* __restrict__ z, const T* __restrict__ dh,
                                                     T* __restrict__ out, int64_t T_rows, int F, int backward) {
  typedef typename Pack4<T>::type v4;
  const int q = F / 4;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= T_rows * q) return;
  const int64_t row = gid / q;
  const int c = static_cast<int>(gid % q) * 4;
  const T* zr = z + row * 2 * F;
  const v4 g = *reinterpret_cast<const v4*>(zr + c);
  const v4 u = *reinterpret_cast<const v4*>(zr + F + c);
  if (!backward) {
    v4 h;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float gf = static_cast<float>(g[e]);
      h[e] = static_cast<T>(gf / (1.f + __expf(-gf)) * static_cast<float>(u[e]));
    }
    *reinterpret_cast<v4*>(out + row * F + c) = h;
  } else {
    const v4 d = *reinterpret_cast<const v4*>(dh + row * F + c);
    v4 dg, du;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float gf = static_cast<float>(g[e]), uf = static_cast<float>(u[e]), df = static_cast<float>(d[e]);
      const float sg = 1.f / (1.f + __expf(-gf));
      du[e] = static_cast<T>(df * gf * sg);
      dg[e] = static_cast<T>(df * uf * sg * (1.f + gf * (1.f - sg)));
    }
    T* orow = out + row * 2 * F;
    *reinterpret_cast<v4*>(orow + c) = dg;
    *reinterpret_cast<v4*>(orow + F + c) = du;
  }
}

// ---------------------------------------------------------------------------
// Cross-entropy over rows of V logits (bf16/fp16), one workgroup per row.
// Forward: lse = log sum exp (one pass, running max per thread, merged across
// the workgroup); loss = lse - logit[label] (0 for label < 0).  Backward:
// dlogit = (exp(logit - lse) - [v == label]) * scale, 0 for an ignored row.
__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
  const float mm = fmaxf(m, m2);
  s = (m == -INFINITY ? 0.f : s * __expf(m - mm)) + (m2 == -INFINITY ? 0.f : s2 * __expf(m2 - mm));
  m = mm;
}

template <typename T>
__global__ __launch_bounds__(256) void xent_fwd_kernel(const T* __restrict__ logits, const int64_t* __restrict__ labels,
                                                       float* __restrict__ loss, float* __restrict__ lse, int V) {
  typedef typename Pack4<T>::type v4;
  __shared__ float sm[4], ss[4];
  const int64_t row = blockIdx.x;
  const T* lr = logits + row * V;
  float m = -INFINITY, s = 0.f;
  for (int c = threadIdx.x * 4; c < V; c += 256 * 4) {
    const v4 x = *reinterpret_cast<const v4*>(lr + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) lse_merge(m, s, static_cast<float>(x[e]), 1.f);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) lse_merge(m, s, __shfl_xor(m, off, 64), __shfl_xor(s, off, 64));
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sm[wave] = m;
    ss[wave] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = sm[0], S = ss[0];
    for (int w = 1; w < 4; ++w) lse_merge(M, S, sm[w], ss[w]);
    const float l = M + __logf(S);
    lse[row] = l;
    const int64_t lab = labels[row];
    loss[row] = (lab >= 0 && lab < V) ? l - static_cast<float>(lr[lab]) : 0.f;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void xent_bwd_kernel(const T* __restrict__ logits, const int64_t* __restrict__ labels,
                                                       const float* __restrict__ lse, const float* __restrict__ scale,
                                                       T* __restrict__ dlogits, int V) {
  typedef typename Pack4<T>::type v4;
  const int64_t row = blockIdx.x;
  const int64_t lab = labels[row];
  const bool valid = lab >= 0 && lab < V;
  const float l = lse[row], g = valid ? *scale : 0.f;
  const T* lr = logits + row * V;
  T* dr = dlogits + row * V;
  for (int c = threadIdx.x * 4; c < V; c += 256 * 4) {
    const v4 x = *reinterpret_cast<const v4*>(lr + c);
    v4 d;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p = __expf(static_cast<float>(x[e]) - l) - (c + e == lab ? 1.f : 0.f);
      d[e] = static_cast<T>(p * g);
    }
    *reinterpret_cast<v4*>(dr + c) = d;
  }
}

int32_t check_norm(const void* x, const void* w, const void* a, const void* b, int32_t T, int32_t H, int32_t dtype) {
  if (x == nullptr || w == nullptr || a == nullptr || b == nullptr) return SSA_OPS_ERR_NULL_POINTER;
  if (T <= 0 || H <= 0 || H % 4 != 0 || H > 4 * 4 * kNormThreads) return SSA_OPS_ERR_SHAPE;
  if (dtype != 0 && dtype != 1 && dtype != 2) return SSA_OPS_ERR_DTYPE;
  if (!aligned(x, 16) || !aligned(w, 16)) return SSA_OPS_ERR_ALIGNMENT;
  return SSA_OPS_OK;
}

}  // namespace

extern "C" int32_t ssa_rope(const ssa_rope_args* a, void* stream) {
  if (a == nullptr || a->x == nullptr || a->y == nullptr || a->cos == nullptr || a->sin == nullptr)
    return SSA_OPS_ERR_NULL_POINTER;
  if (a->seqlen <= 0 || a->batch <= 0 || a->heads <= 0) return SSA_OPS_ERR_SHAPE;
  // (token, head) rows fit int32, so the grid of head_dim / 8 threads per row fits too
  const int64_t sb = static_cast<int64_t>(a->seqlen) * a->batch;
  if (sb > INT32_MAX || sb * a->heads > INT32_MAX) return SSA_OPS_ERR_SHAPE;
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

extern "C" int64_t ssa_rmsnorm_workspace_floats(int32_t rows, int32_t hidden) {
  if (rows <= 0 || hidden <= 0) return 0;
  return (static_cast<int64_t>(rows) + kNormBwdRows - 1) / kNormBwdRows * hidden;
}

extern "C" int32_t ssa_rmsnorm_fwd(const ssa_rmsnorm_fwd_args* a, void* stream) {
  if (a == nullptr) return SSA_OPS_ERR_NULL_POINTER;
  const int32_t st = check_norm(a->x, a->weight, a->y, a->rstd, a->rows, a->hidden, a->out_dtype);
  if (st != SSA_OPS_OK) return st;
  if (!aligned(a->y, 8)) return SSA_OPS_ERR_ALIGNMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float* x = static_cast<const float*>(a->x);
  const float* w = static_cast<const float*>(a->weight);
  switch (a->out_dtype) {
    case 0: hipLaunchKernelGGL(rmsnorm_fwd_kernel<__bf16>, dim3(a->rows), dim3(kNormThreads), 0, s, x, w,
                               static_cast<__bf16*>(a->y), a->rstd, a->hidden, a->eps); break;
    case 1: hipLaunchKernelGGL(rmsnorm_fwd_kernel<_Float16>, dim3(a->rows), dim3(kNormThreads), 0, s, x, w,
                               static_cast<_Float16*>(a->y), a->rstd, a->hidden, a->eps); break;
    default: hipLaunchKernelGGL(rmsnorm_fwd_kernel<float>, dim3(a->rows), dim3(kNormThreads), 0, s, x, w,
                                static_cast<float*>(a->y), a->rstd, a->hidden, a->eps); break;
  }
  return hipGetLastError() == hipSuccess ? SSA_OPS_OK : SSA_OPS_ERR_LAUNCH;
}

extern "C" int32_t ssa_rmsnorm_bwd(const ssa_rmsnorm_bwd_args* a, void* stream) {
  if (a == nullptr) return SSA_OPS_ERR_NULL_POINTER;
  const int32_t st = check_norm(a->x, a->weight, a->dy, a->rstd, a->rows, a->hidden, a->dy_dtype);
  if (st != SSA_OPS_OK) return st;
  if (a->dx == nullptr || a->dweight == nullptr || a->workspace == nullptr) return SSA_OPS_ERR_NULL_POINTER;
  if (!aligned(a->dx, 16) || !aligned(a->workspace, 16) || !aligned(a->dy, 8)) return SSA_OPS_ERR_ALIGNMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nparts = static_cast<int>((static_cast<int64_t>(a->rows) + kNormBwdRows - 1) / kNormBwdRows);
  const float* x = static_cast<const float*>(a->x);
  const float* w = static_cast<const float*>(a->weight);
  switch (a->dy_dtype) {
    case 0: hipLaunchKernelGGL(rmsnorm_bwd_kernel<__bf16>, dim3(nparts), dim3(kNormThreads), 0, s, x, w,
                               static_cast<const __bf16*>(a->dy), a->rstd, a->dx, a->workspace, a->rows,
                               a->hidden); break;
    case 1: hipLaunchKernelGGL(rmsnorm_bwd_kernel<_Float16>, dim3(nparts), dim3(kNormThreads), 0, s, x, w,
                               static_cast<const _Float16*>(a->dy), a->rstd, a->dx, a->workspace, a->rows,
                               a->hidden); break;
    default: hipLaunchKernelGGL(rmsnorm_bwd_kernel<float>, dim3(nparts), dim3(kNormThreads), 0, s, x, w,
                                static_cast<const float*>(a->dy), a->rstd, a->dx, a->workspace, a->rows,
                                a->hidden); break;
  }
  if (hipGetLastError() != hipSuccess) return SSA_OPS_ERR_LAUNCH;
  hipLaunchKernelGGL(rmsnorm_dw_kernel, dim3((a->hidden + 255) / 256), dim3(256), 0, s, a->workspace, a->dweight,
                     nparts, a->hidden);
  return hipGetLastError() == hipSuccess ? SSA_OPS_OK : SSA_OPS_ERR_LAUNCH;
}

extern "C" int32_t ssa_swiglu(const ssa_swiglu_args* a, void* stream) {
  if (a == nullptr || a->z == nullptr || a->out == nullptr || (a->backward && a->dh == nullptr))
    return SSA_OPS_ERR_NULL_POINTER;
  if (a->rows <= 0 || a->ffn <= 0 || a->ffn % 4 != 0) return SSA_OPS_ERR_SHAPE;
  const int64_t threads = static_cast<int64_t>(a->rows) * (a->ffn / 4);  // one per 4 outputs
  if ((threads + 255) / 256 > INT32_MAX) return SSA_OPS_ERR_SHAPE;
  if (a->dtype != 0 && a->dtype != 1) return SSA_OPS_ERR_DTYPE;
  if (!aligned(a->z, 8) || !aligned(a->out, 8) || (a->backward && !aligned(a->dh, 8))) return SSA_OPS_ERR_ALIGNMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int grid = static_cast<int>((threads + 255) / 256);
  if (a->dtype == 0)
    hipLaunchKernelGGL(swiglu_kernel<__bf16>, dim3(grid), dim3(256), 0, s, static_cast<const __bf16*>(a->z),
                       static_cast<const __bf16*>(a->dh), static_cast<__bf16*>(a->out), static_cast<int64_t>(a->rows),
                       a->ffn, a->backward);
  else
    hipLaunchKernelGGL(swiglu_kernel<_Float16>, dim3(grid), dim3(256), 0, s, static_cast<const _Float16*>(a->z),
                       static_cast<const _Float16*>(a->dh), static_cast<_Float16*>(a->out),
                       static_cast<int64_t>(a->rows), a->ffn, a->backward);
  return hipGetLastError() == hipSuccess ? SSA_OPS_OK : SSA_OPS_ERR_LAUNCH;
}

extern "C" int32_t ssa_cross_entropy(const ssa_cross_entropy_args* a, void* stream) {
  if (a == nullptr || a->logits == nullptr || a->labels == nullptr || a->lse == nullptr) return SSA_OPS_ERR_NULL_POINTER;
  if (!a->backward && a->loss == nullptr) return SSA_OPS_ERR_NULL_POINTER;
  if (a->backward && (a->scale == nullptr || a->dlogits == nullptr)) return SSA_OPS_ERR_NULL_POINTER;
  if (a->rows <= 0 || a->vocab <= 0 || a->vocab % 4 != 0) return SSA_OPS_ERR_SHAPE;
  if (a->dtype != 0 && a->dtype != 1) return SSA_OPS_ERR_DTYPE;
  if (!aligned(a->logits, 8) || (a->backward && !aligned(a->dlogits, 8))) return SSA_OPS_ERR_ALIGNMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t* lab = static_cast<const int64_t*>(a->labels);
  if (!a->backward) {
    if (a->dtype == 0)
      hipLaunchKernelGGL(xent_fwd_kernel<__bf16>, dim3(a->rows), dim3(256), 0, s,
                         static_cast<const __bf16*>(a->logits), lab, a->loss, a->lse, a->vocab);
    else
      hipLaunchKernelGGL(xent_fwd_kernel<_Float16>, dim3(a->rows), dim3(256), 0, s,
                         static_cast<const _Float16*>(a->logits), lab, a->loss, a->lse, a->vocab);
  } else {
    if (a->dtype == 0)
      hipLaunchKernelGGL(xent_bwd_kernel<__bf16>, dim3(a->rows), dim3(256), 0, s,
                         static_cast<const __bf16*>(a->logits), lab, a->lse, a->scale,
                         static_cast<__bf16*>(a->dlogits), a->vocab);
    else
      hipLaunchKernelGGL(xent_bwd_kernel<_Float16>, dim3(a->rows), dim3(256), 0, s,
                         static_cast<const _Float16*>(a->logits), lab, a->lse, a->scale,
                         static_cast<_Float16*>(a->dlogits), a->vocab);
  }
  return hipGetLastError() == hipSuccess ? SSA_OPS_OK : SSA_OPS_ERR_LAUNCH;
}
