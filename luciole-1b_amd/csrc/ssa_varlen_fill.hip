// Packed (varlen) batches: rows of the token stream that no document covers.
//
// A token is covered when it lies in [s0, s0 + min(L, max_seqlen)) of some
// document (s0 = cu[i], L = cu[i+1] - cu[i], both clamped to [0, T] as
// SeqView clamps them).  The attention kernels write only covered rows; the
// others -- tokens after cu[batch] < T, before cu[0] > 0, and the tail of a
// document longer than max_seqlen -- would keep whatever the caller's
// allocation held, and in training those rows of dq / dk / dv reach the QKV
// weight gradient.  This kernel writes them: output rows 0 and m = -inf (a
// row with no keys) after the forward, gradient rows 0 after the backward.
//
// One workgroup per gap: workgroup 0 the tokens before the first document,
// workgroup 1 + i the gap after document i's covered part (up to the next
// document's start, i.e. cu[i+1]), workgroup B + 1 the tokens after the last
// document.  For a nondecreasing table these ranges are disjoint from every
// covered row; a malformed table gives wrong results (as elsewhere) but every
// store stays inside [0, T).  A well-formed table with no gaps costs one
// launch whose workgroups exit at once.
#include "ssa_common.hpp"
#include "ssa_launch.hpp"

namespace ssa {

__device__ __forceinline__ int clamp_tok(int x, int lo, int hi) { return x < lo ? lo : (x > hi ? hi : x); }

__global__ __launch_bounds__(256) void ssa_varlen_fill_kernel(VarlenFill f) {
  const int w = blockIdx.x;
  int a, e;
  if (w == 0) {
    a = 0;
    e = clamp_tok(f.cu[0], 0, f.T);
  } else if (w <= f.B) {
    const int i = w - 1;
    const int s0 = clamp_tok(f.cu[i], 0, f.T);
    const int s1 = clamp_tok(f.cu[i + 1], s0, f.T);
    a = s0 + (s1 - s0 < f.Nmax ? s1 - s0 : f.Nmax);
    e = s1;
  } else {
    const int s0 = clamp_tok(f.cu[f.B - 1], 0, f.T);  // the last document, clamped like SeqView
    a = clamp_tok(f.cu[f.B], s0, f.T);
    e = f.T;
  }
  if (a >= e) return;
  const int rows = e - a;
  const int cpr = f.D * f.esize / 16;  // 16-byte chunks per (token, head) row
  for (int j = 0; j < f.ntensors; ++j) {
    const Tensor4& t = f.t[j];
    const int H = f.heads[j];
    const int64_t items = static_cast<int64_t>(rows) * H * cpr;
    for (int64_t it = threadIdx.x; it < items; it += blockDim.x) {
      const int c = static_cast<int>(it % cpr);
      const int64_t th = it / cpr;
      const int h = static_cast<int>(th % H);
      const int tok = a + static_cast<int>(th / H);
      char* p = static_cast<char*>(const_cast<void*>(t.ptr)) + ((tok * t.ss + h * t.sh) * f.esize + c * 16);
      *reinterpret_cast<u32x4*>(p) = u32x4{0u, 0u, 0u, 0u};
    }
  }
  if (f.m != nullptr) {
    const int64_t items = static_cast<int64_t>(rows) * f.m_heads;
    for (int64_t it = threadIdx.x; it < items; it += blockDim.x) {
      const int h = static_cast<int>(it / rows);
      const int tok = a + static_cast<int>(it % rows);
      f.m[static_cast<int64_t>(h) * f.T + tok] = -__builtin_inff();
    }
  }
}

hipError_t launch_varlen_fill(const VarlenFill& f, hipStream_t stream) {
  hipLaunchKernelGGL(ssa_varlen_fill_kernel, dim3(f.B + 2), dim3(256), 0, stream, f);
  return hipGetLastError();
}

}  // namespace ssa
