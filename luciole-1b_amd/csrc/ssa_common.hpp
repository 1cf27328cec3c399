// Shared device helpers for the gfx950 SSA attention kernels.
//
// Matrix-core conventions used by every kernel (v_mfma_f32_32x32x16_{bf16,f16},
// wave64):
//   A operand  (32 x 16): lane l holds row (l % 32), 8 k-slots of half (l / 32)
//   B operand  (16 x 32): lane l holds column (l % 32), the same 8 k-slots
//   C/D        (32 x 32): lane l holds column (l % 32) and rows
//                         8*(r/4) + 4*(l/32) + (r%4), r = 0..15
// The contraction is over k-slots, so any bijection between (half, slot) and
// the logical k index works as long as A and B use the same one.  The kernels
// exploit this: an accumulator tile whose 16 rows per lane are
// {0-3, 8-11, 16-19, 24-27} (+4 for the upper half) feeds the next MFMA as an
// A or B operand directly, with k-step ks taking accumulator entries 8ks..8ks+7,
// and the other operand is gathered with the matching row order (crow()).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ssa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <typename T>
struct Vec8;
template <>
struct Vec8<__bf16> {
  typedef bf16x8 type;
};
template <>
struct Vec8<_Float16> {
  typedef f16x8 type;
};

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// c += a b into a block that lives in accumulation registers (AGPRs) from its
// zero initialisation to acc_fence().  A kernel that keeps long-lived
// accumulators this way lets the compiler place every builtin MFMA result in
// arch VGPRs (ssa_bwd.hip is built with -amdgpu-mfma-vgpr-form), where the
// VALU reads it without a copy.  The compiler does not see inside the asm, so
// its two hazards are covered here and checked on the built assembly
// (SSA/_hazards.py): the s_nop gives the 2 wait states a VALU write of a
// source (or of the zeroed accumulator) needs before the matrix core reads it;
// acc_fence() puts 24 wait states between the last accumulation and any other
// access to the block.  Only these two statements may touch the block.
__device__ __forceinline__ void mfma32_acc(f32x16& c, bf16x8 a, bf16x8 b) {
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma32_acc(f32x16& c, f16x8 a, f16x8 b) {
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
// After the last mfma32_acc on x and y, before their values are read.  The
// volatile statements keep their order, and each one names its blocks as
// read-write, so every read of x[i] / y[i] follows the NOPs.
template <int N>
__device__ __forceinline__ void acc_fence(f32x16 (&x)[N], f32x16 (&y)[N]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+a"(x[0]), "+a"(y[0]));
#pragma unroll
  for (int i = 1; i < N; ++i) asm volatile("" : "+a"(x[i]), "+a"(y[i]));
}

// Row (within a 32-row accumulator block) held in accumulator entry r by lane half hh.
__device__ __forceinline__ int crow(int r, int hh) { return ((r >> 2) << 3) + (hh << 2) + (r & 3); }

template <typename V>
__device__ __forceinline__ V load16(const void* p) {
  return __builtin_bit_cast(V, *reinterpret_cast<const u32x4*>(p));
}

template <typename V>
__device__ __forceinline__ V zero8() {
  return __builtin_bit_cast(V, u32x4{0u, 0u, 0u, 0u});
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// Value barrier: `x` is computed before this point (an empty side-effecting
// statement that stays in order with scheduling fences, so a value computed
// for a later use is not moved past them).
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }

// Value of `x` in the lane 32 positions away (the other half of the wave).
__device__ __forceinline__ float swap_halves(float x) { return __shfl_xor(x, 32, 64); }

// max / sum of x over the lane pair (l, l ^ 32), in every lane: one
// v_permlane32_swap (which leaves {x[l % 32], x[l % 32 + 32]} in its two
// results in every lane) and one op, no LDS.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Workgroups are dispatched round-robin over the 8 XCDs (block id % 8).  This
// bijection on [0, total) gives each XCD a contiguous range of logical block
// indices, so logical neighbours (same head) share one XCD's L2.
__host__ __device__ __forceinline__ int xcd_remap(int bid, int total) {
  const int q = total >> 3, r = total & 7;
  const int x = bid & 7, j = bid >> 3;
  return x * q + (x < r ? x : r) + j;
}

// Dispatch order of a grid of nhb x nblk workgroups (nhb (sequence, head)
// pairs, nblk blocks each, block weights falling with rank under a causal
// mask).  Logical block L maps to (hb, rank), rank 0 the heaviest: groups of
// `group` consecutive hb hand out their blocks heaviest first, alternating
// between the members of the group.  Each XCD dispatches its range of L in
// order to whichever CU frees first, so with group = 2 this is
// longest-processing-time-first list scheduling over a pair of heads, and the
// workgroups that finish last are light ones (one head at a time leaves the
// heaviest blocks of the last head of a range starting late: up to a sixth of
// the kernel as idle tail).  Packed batches use group = 1: there the members
// of a pair are documents of different lengths, whose block weights the rank
// does not describe (measured: pairs cost the packed benchmark 15 %).
constexpr int kOrderGroup = 2;
__host__ __device__ __forceinline__ void dispatch_order(int L, int nhb, int nblk, int group, int& hb, int& rank) {
  const int g = L / (group * nblk), r = L - g * group * nblk;
  const int gs = group < nhb - g * group ? group : nhb - g * group;  // >= 1 for L < nhb * nblk
  hb = g * group + r % gs;
  rank = r / gs;
}

struct Tensor4 {
  const void* ptr;
  int64_t sb, sh, ss;
};

// Dense batches: B sequences of length N, sequence b at element offset
// b * sb of each tensor, row-normaliser M / Delta of (b, h) at (b H + h) N.
// Packed (varlen) batches: cu_seqlens != nullptr, B documents of a [T, H, D]
// token stream, document b = tokens [cu[b], cu[b+1]) (N = the longest),
// M / Delta laid out [H, T].
struct FwdParams {
  Tensor4 q, k, v, o;
  float* m;
  const float* n_ptr;
  const float* b_ptr;
  int B, Hq, Hkv, N;
  float scale;
  const int* cu_seqlens;
  int T;
};

struct BwdParams {
  Tensor4 q, k, v, o, dout, dq, dk, dv;
  const float* m;
  float* delta;
  float* partials;  // [2][B*Hkv*nkb]: dn terms then db terms
  float* dn;
  float* db;
  const float* n_ptr;
  const float* b_ptr;
  int B, Hq, Hkv, N;
  float scale;
  const int* cu_seqlens;
  int T;
  // Optional dS' workspace (dense batches): when set, dK/dV writes the
  // gradient tiles there and dQ is a product with K instead of a recompute.
  void* ds;
  // Workspace dQ pass only: its workgroup 0 also sums the dn / db partials
  // (the reduction of ssa_reduce_partials_kernel, bit for bit), so the whole
  // backward needs no separate reduction launch.
  int fuse_reduce;
};

// Decode against a KV cache: q / o [B, Hq, 1, D] (row stride unused), k / v
// [B, Hkv, cap, D]; sequence b attends keys [0, seqlens[b]) (clamped to
// [0, cap]).  With splits > 1 every (b, q-head, split) leaves an unnormalised
// partial (m, l, acc[D]) in ws_ml / ws_acc for the merge kernel.
struct DecodeParams {
  Tensor4 q, k, v, o;
  float* m;  // optional [B, Hq]
  const int* seqlens;
  const float* n_ptr;
  const float* b_ptr;
  float* ws_ml;   // [B * Hq * splits][2]
  float* ws_acc;  // [B * Hq * splits][D]
  int B, Hq, Hkv, cap, splits, split_keys;
  float scale;
};

// An entry of a table every lane of the workgroup reads at the same index
// (the packed batches' document table), read through the global address
// space: a scalar load with a wave-uniform result even where the compiler
// cannot trace the pointer back to a kernel argument.
__host__ __device__ __forceinline__ int load_table_entry(const int* t, int i) {
#if defined(__HIP_DEVICE_COMPILE__)
  return ((const __attribute__((address_space(1))) int*)t)[i];
#else
  return t[i];
#endif
}

// The sequence a workgroup works on.  For packed batches the document table
// is clamped to [0, T] and the length to N, so any table keeps every access
// inside the token stream.
struct SeqView {
  int N;         // length of this sequence
  int64_t tok0;  // packed: first token of the document
  bool packed;
  __host__ __device__ __forceinline__ SeqView() : N(0), tok0(0), packed(false) {}
  __host__ __device__ __forceinline__ SeqView(const int* cu, int T, int Nmax, int b) {
    packed = cu != nullptr;
    if (packed) {
      int s0 = load_table_entry(cu, b), s1 = load_table_entry(cu, b + 1);
      s0 = s0 < 0 ? 0 : (s0 > T ? T : s0);
      s1 = s1 < s0 ? s0 : (s1 > T ? T : s1);
      tok0 = s0;
      N = s1 - s0 < Nmax ? s1 - s0 : Nmax;
    } else {
      tok0 = 0;
      N = Nmax;
    }
  }
  // element offset of the sequence in a tensor (before the head offset)
  __host__ __device__ __forceinline__ int64_t off(const Tensor4& t, int b) const { return packed ? tok0 * t.ss : b * t.sb; }
  // index of row 0 of (b, h) in M / Delta
  __host__ __device__ __forceinline__ int64_t mrow(int b, int h, int H, int T, int Nmax) const {
    return packed ? static_cast<int64_t>(h) * T + tok0 : (static_cast<int64_t>(b) * H + h) * Nmax;
  }
};

constexpr float kLn2 = 0.69314718055994530942f;
// Lazy rescaling threshold (log2 units): the running max used for exp2 is only
// moved when a new row max exceeds it by more than this, so p <= 2^kRescaleTau.
constexpr float kRescaleTau = 8.0f;
// The pipelined forward tests instead the sum of each lane's p against this
// bound: every p is at most that sum, and any finite m with p <= 2^20 keeps
// the fp32 sums far from overflow while M = m + log2(l) stays exact.
constexpr float kPsumLimit = 1048576.0f;

// dn, db = fixed-order sums of the per-workgroup partials: threads 0 .. 255
// of the calling workgroup Kahan-sum strided slices, then a fixed tree; every
// thread of the workgroup reaches the barriers.
__device__ __forceinline__ void reduce_partials_body(const float* partials, int64_t count, float* dn, float* db,
                                                     float (*sh)[256], int tid) {
  if (tid < 256) {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const float* src = partials + w * count;
      float acc = 0.f, comp = 0.f;
      for (int64_t i = tid; i < count; i += 256) {
        const float y = src[i] - comp, t = acc + y;
        comp = (t - acc) - y;
        acc = t;
      }
      sh[w][tid] = acc;
    }
  }
  __syncthreads();
  for (int stride = 128; stride > 0; stride >>= 1) {
    if (tid < stride) {
      sh[0][tid] += sh[0][tid + stride];
      sh[1][tid] += sh[1][tid + stride];
    }
    __syncthreads();
  }
  if (tid == 0) {
    *dn = sh[0][0];
    *db = sh[1][0];
  }
}

}  // namespace ssa
