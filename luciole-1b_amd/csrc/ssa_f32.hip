// SSA attention forward and backward with fp32 arithmetic, on the vector ALU:
// the kernels of fp32 inputs at every head dim, and of bf16 / fp16 inputs at
// head dim 256 (the matrix-core kernels cover bf16 / fp16 at 32, 64 and 128).
//
// The reference runs its Triton kernels on fp32 tensors with fp32 operands in
// the dot products (MATMUL_PRECISION = tl.float32,
// training/train/train_ssa_triton/SSA/ssa_triton_kernel.py:766-772, 819-825)
// and checks them to atol 5e-4 / rtol 1e-3 and scalar 5e-5 + 1e-4 |ref|
// (check_ssa_triton_parity.py:1064-1069), a bar that no bf16 rounding of the
// operands meets.  These kernels keep every product in fp32 FMA and every
// transcendental in the hardware's f32 exp2 / log2 / rcp.  They follow the
// equations of ssa_fwd.hip / ssa_bwd.hip with simple structures: each row of
// the register-resident operand is split over P adjacent lanes (P = D / 32
// from head dim 64 on, so a lane holds at most 32 columns of each row; the
// partial dot products meet by butterfly shuffles), and the other operand's
// rows are shared through LDS, converted to fp32 on the way in, and read as
// broadcasts.  bf16 / fp16 elements are widened on load and rounded to
// nearest even on store.  Masks, GQA, packed sequences and the dn / db
// partials (one per 128-key block, the layout ssa_reduce_partials_kernel
// sums) are those of the matrix-core path; the reference accepts every
// power-of-two head dim (ssa_triton_kernel.py:761-764), and head dim 256 is
// the largest its Triton tiles hold.
#include "ssa_common.hpp"
#include "ssa_launch.hpp"

namespace ssa {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Four consecutive elements of T as fp32 (16-byte or 8-byte aligned: columns
// are multiples of 4, rows 16-byte aligned), and back.
__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ void st4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
template <typename T>
__device__ __forceinline__ f32x4 ld4(const T* p) {
  typedef T t4 __attribute__((ext_vector_type(4)));
  const t4 x = *reinterpret_cast<const t4*>(p);
  return f32x4{static_cast<float>(x[0]), static_cast<float>(x[1]), static_cast<float>(x[2]),
               static_cast<float>(x[3])};
}
template <typename T>
__device__ __forceinline__ void st4(T* p, f32x4 v) {
  typedef T t4 __attribute__((ext_vector_type(4)));
  *reinterpret_cast<t4*>(p) = t4{static_cast<T>(v[0]), static_cast<T>(v[1]), static_cast<T>(v[2]),
                                 static_cast<T>(v[3])};
}

// sL = sign(x) log2(1 + c|x|) for a raw score x = q.k, c = scale b; u1 = 1 + c|x|
__device__ __forceinline__ float ssa_sl(float x, float u1) { return copysignf(fast_log2(u1), x); }

constexpr int kF32Rows = 64;   // query rows per forward workgroup
constexpr int kF32Tile = 32;   // rows per LDS tile of the streamed operand
constexpr int kF32Pair = 128;  // keys (dK/dV) or queries (dQ) per backward workgroup

// Lanes per row: the forward splits rows from head dim 64 on, the backward
// (which holds two or three row operands per lane) always.
template <int D>
constexpr int fwd_parts() {
  return D >= 64 ? D / 32 : 1;
}
template <int D>
constexpr int bwd_parts() {
  return D >= 64 ? D / 32 : 2;
}
// Rows of the backward block held at once: all 128 up to head dim 128; at 256
// (8 lanes per row) 64, in two passes, so that a workgroup stays at 512 lanes
// and each lane keeps its four 32-column row shares (128 registers) in the
// 256 registers of two waves per SIMD.
template <int D>
constexpr int bwd_rows() {
  return D >= 256 ? 64 : kF32Pair;
}
template <int D>
constexpr int fwd_threads() {
  return kF32Rows * fwd_parts<D>();
}
template <int D>
constexpr int bwd_threads() {
  return bwd_rows<D>() * bwd_parts<D>();
}

// Dot product of a lane's CP four-column chunks with the same chunks of an
// LDS row.
template <int CP>
__device__ __forceinline__ float part_dot(const f32x4* reg, const f32x4* lds) {
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CP; ++c) {
    const f32x4 x = lds[c];
    s = fmaf(reg[c].x, x.x, s);
    s = fmaf(reg[c].y, x.y, s);
    s = fmaf(reg[c].z, x.z, s);
    s = fmaf(reg[c].w, x.w, s);
  }
  return s;
}

// Sum over the P adjacent lanes of a row (P in {1, 2, 4, 8}); every lane gets it.
template <int P>
__device__ __forceinline__ float sum_parts(float x) {
  if constexpr (P >= 2) x += __shfl_xor(x, 1, 64);
  if constexpr (P >= 4) x += __shfl_xor(x, 2, 64);
  if constexpr (P >= 8) x += __shfl_xor(x, 4, 64);
  return x;
}

// ---------------------------------------------------------------------------
// Forward: P lanes = one query row, the lane's share of q and of the
// accumulator in registers, K / V tiles of 32 keys in LDS; exact running max
// (online softmax in base 2), the same in the P lanes of a row.
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(fwd_threads<D>()) void ssa_fwd_f32_kernel(FwdParams p) {
  constexpr int P = fwd_parts<D>(), C4 = D / 4, CP = C4 / P, NT = fwd_threads<D>();
  __shared__ f32x4 ks[kF32Tile * C4], vs[kF32Tile * C4];
  const int tid = threadIdx.x, part = tid % P;
  const int nqb = (p.N + kF32Rows - 1) / kF32Rows;
  const int qb = blockIdx.x % nqb, bh = blockIdx.x / nqb;
  const int b = bh % p.B, h = bh / p.B, hk = h / (p.Hq / p.Hkv);
  const SeqView sv(p.cu_seqlens, p.T, p.N, b);
  const int N = sv.N;
  const int q0 = qb * kF32Rows;
  if (q0 >= N) return;  // packed: past the end of a shorter document
  const int i = q0 + tid / P;
  const T* qg = static_cast<const T*>(p.q.ptr) + sv.off(p.q, b) + h * p.q.sh;
  const T* kg = static_cast<const T*>(p.k.ptr) + sv.off(p.k, b) + hk * p.k.sh;
  const T* vg = static_cast<const T*>(p.v.ptr) + sv.off(p.v, b) + hk * p.v.sh;
  T* og = static_cast<T*>(const_cast<void*>(p.o.ptr)) + sv.off(p.o, b) + h * p.o.sh;
  const float n = *p.n_ptr, bv = *p.b_ptr, c = p.scale * bv;

  f32x4 qv[CP], acc[CP];
#pragma unroll
  for (int c4 = 0; c4 < CP; ++c4) {
    qv[c4] = i < N ? ld4(qg + i * p.q.ss + 4 * (part * CP + c4)) : f32x4{0.f, 0.f, 0.f, 0.f};
    acc[c4] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float m = -__builtin_inff(), l = 0.f;
  const int kv_end = CAUSAL ? min(N, q0 + kF32Rows) : N;
  for (int k0 = 0; k0 < kv_end; k0 += kF32Tile) {
    __syncthreads();  // the previous tile is consumed
    for (int idx = tid; idx < kF32Tile * C4; idx += NT) {
      const int row = min(k0 + idx / C4, N - 1), c4 = idx % C4;
      ks[idx] = ld4(kg + row * p.k.ss + 4 * c4);
      vs[idx] = ld4(vg + row * p.v.ss + 4 * c4);
    }
    __syncthreads();
    const int kn = min(kF32Tile, kv_end - k0);
    for (int j = 0; j < kn; ++j) {
      const float s = sum_parts<P>(part_dot<CP>(qv, ks + j * C4 + part * CP));
      if (i < N && (!CAUSAL || k0 + j <= i)) {
        const float t2 = n * ssa_sl(s, fmaf(c, fabsf(s), 1.f));
        if (t2 > m) {  // the running max moves: rescale what is summed so far
          const float alpha = fast_exp2(m - t2);
          l *= alpha;
#pragma unroll
          for (int c4 = 0; c4 < CP; ++c4) acc[c4] *= alpha;
          m = t2;
        }
        const float pv = fast_exp2(t2 - m);
        l += pv;
        const f32x4* vrow = vs + j * C4 + part * CP;
#pragma unroll
        for (int c4 = 0; c4 < CP; ++c4) acc[c4] += pv * vrow[c4];
      }
    }
  }
  if (i < N) {
    const float inv = 1.f / l;  // every row has a key (causal: itself)
#pragma unroll
    for (int c4 = 0; c4 < CP; ++c4) st4(og + i * p.o.ss + 4 * (part * CP + c4), acc[c4] * inv);
    if (part == 0) p.m[sv.mrow(b, h, p.Hq, p.T, p.N) + i] = m + log2f(l);
  }
}

// Delta = rowsum(dO * O): D / 4 lanes per row, 4-element loads, butterfly.
template <typename T, int D>
__global__ __launch_bounds__(256) void ssa_bwd_preprocess_f32_kernel(BwdParams p) {
  constexpr int LPR = D / 4, RPB = 256 / LPR;
  const int tid = threadIdx.x;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + tid / LPR;
  const int sub = tid % LPR;
  const int64_t total = static_cast<int64_t>(p.B) * p.Hq * p.N;
  float acc = 0.f;
  if (row < total) {
    const int s = static_cast<int>(row % p.N);
    const int64_t bh = row / p.N;
    const int h = static_cast<int>(bh % p.Hq), b = static_cast<int>(bh / p.Hq);
    const f32x4 o = ld4(static_cast<const T*>(p.o.ptr) + b * p.o.sb + h * p.o.sh + s * p.o.ss + 4 * sub);
    const f32x4 g = ld4(static_cast<const T*>(p.dout.ptr) + b * p.dout.sb + h * p.dout.sh + s * p.dout.ss + 4 * sub);
    acc = fmaf(o.x, g.x, fmaf(o.y, g.y, fmaf(o.z, g.z, o.w * g.w)));
  }
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (row < total && sub == 0) p.delta[row] = acc;
}

// ---------------------------------------------------------------------------
// dK, dV (+ dn / db partials) for 128 keys of one (batch, kv-head), in passes
// of bwd_rows<D>() keys: P lanes per key, each holding its share of k, v, dK,
// dV; Q / dO tiles of 32 rows,
// with M and Delta, in LDS, over every q-head of the GQA group.  Per valid
// pair, as in ssa_bwd.hip: P = exp2(n sL - M), dT = P (dP - Delta),
// dS' = dT / (1 + c|x|), dV += P dO, dK += dS' q (scaled by scale n b at the
// end), dn += ln2 dT sL, db += n scale dS' x.
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(bwd_threads<D>()) void ssa_bwd_dkdv_f32_kernel(BwdParams p) {
  constexpr int P = bwd_parts<D>(), C4 = D / 4, CP = C4 / P, NT = bwd_threads<D>(), NWV = NT / 64;
  constexpr int ROWS = bwd_rows<D>();
  __shared__ f32x4 qs[kF32Tile * C4], dos[kF32Tile * C4];
  __shared__ float ms[kF32Tile], dls[kF32Tile];
  __shared__ float red[2][NWV];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, part = tid % P;
  const int nkb = dkdv_key_blocks(p.N);
  const int kb = blockIdx.x % nkb, bhk = blockIdx.x / nkb;
  const int b = bhk % p.B, hk = bhk / p.B;
  const int G = p.Hq / p.Hkv;
  const SeqView sv(p.cu_seqlens, p.T, p.N, b);
  const int N = sv.N;
  const int64_t PP = static_cast<int64_t>(p.B) * p.Hkv * nkb;
  if (kb * kF32Pair >= N) {  // packed: past the end of a shorter document
    if (tid == 0) {
      p.partials[static_cast<int64_t>(bhk) * nkb + kb] = 0.f;
      p.partials[PP + static_cast<int64_t>(bhk) * nkb + kb] = 0.f;
    }
    return;
  }
  const T* kg = static_cast<const T*>(p.k.ptr) + sv.off(p.k, b) + hk * p.k.sh;
  const T* vg = static_cast<const T*>(p.v.ptr) + sv.off(p.v, b) + hk * p.v.sh;
  const float n = *p.n_ptr, bv = *p.b_ptr, c = p.scale * bv;
  float dn_acc = 0.f, dn_c = 0.f, db_acc = 0.f, db_c = 0.f;  // Kahan sums (lanes with part == 0)
  // ROWS keys at a time (one pass up to head dim 128, two at 256)
  const int kend = min(N, kb * kF32Pair + kF32Pair);
  for (int k0 = kb * kF32Pair; k0 < kend; k0 += ROWS) {
    const int key = k0 + tid / P;
    f32x4 kh[CP], vh[CP], dkh[CP], dvh[CP];
#pragma unroll
    for (int c4 = 0; c4 < CP; ++c4) {
      const int col = 4 * (part * CP + c4);
      kh[c4] = key < N ? ld4(kg + key * p.k.ss + col) : f32x4{0.f, 0.f, 0.f, 0.f};
      vh[c4] = key < N ? ld4(vg + key * p.v.ss + col) : f32x4{0.f, 0.f, 0.f, 0.f};
      dkh[c4] = dvh[c4] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int qstart = CAUSAL ? k0 : 0;
    for (int g = 0; g < G; ++g) {
      const int h = hk * G + g;
      const T* qg = static_cast<const T*>(p.q.ptr) + sv.off(p.q, b) + h * p.q.sh;
      const T* dog = static_cast<const T*>(p.dout.ptr) + sv.off(p.dout, b) + h * p.dout.sh;
      const int64_t mr = sv.mrow(b, h, p.Hq, p.T, p.N);
      for (int q0 = qstart; q0 < N; q0 += kF32Tile) {
        __syncthreads();  // the previous tile is consumed
        for (int idx = tid; idx < kF32Tile * C4; idx += NT) {
          const int row = min(q0 + idx / C4, N - 1), c4 = idx % C4;
          qs[idx] = ld4(qg + row * p.q.ss + 4 * c4);
          dos[idx] = ld4(dog + row * p.dout.ss + 4 * c4);
        }
        if (tid < kF32Tile) {
          const int row = min(q0 + tid, N - 1);
          ms[tid] = p.m[mr + row];
          dls[tid] = p.delta[mr + row];
        }
        __syncthreads();
        const int qn = min(kF32Tile, N - q0);
        for (int r = 0; r < qn; ++r) {
          const int qi = q0 + r;
          const f32x4* qrow = qs + r * C4 + part * CP;
          const f32x4* drow = dos + r * C4 + part * CP;
          const float s = sum_parts<P>(part_dot<CP>(kh, qrow));
          const float dp = sum_parts<P>(part_dot<CP>(vh, drow));
          if (key < N && (!CAUSAL || key <= qi)) {
            const float u1 = fmaf(c, fabsf(s), 1.f);
            const float sl = ssa_sl(s, u1);
            const float pv = fast_exp2(fmaf(n, sl, -ms[r]));
            const float dt = pv * (dp - dls[r]);
            const float dsp = dt * fast_rcp(u1);
#pragma unroll
            for (int c4 = 0; c4 < CP; ++c4) {
              dvh[c4] += pv * drow[c4];
              dkh[c4] += dsp * qrow[c4];
            }
            if (part == 0) {
              const float y = dt * sl - dn_c, t = dn_acc + y;
              dn_c = (t - dn_acc) - y;
              dn_acc = t;
              const float y2 = dsp * s - db_c, t2 = db_acc + y2;
              db_c = (t2 - db_acc) - y2;
              db_acc = t2;
            }
          }
        }
      }
    }
    if (key < N) {
      const float ks_ = p.scale * n * bv;
      T* dkr = static_cast<T*>(const_cast<void*>(p.dk.ptr)) + sv.off(p.dk, b) + hk * p.dk.sh + key * p.dk.ss;
      T* dvr = static_cast<T*>(const_cast<void*>(p.dv.ptr)) + sv.off(p.dv, b) + hk * p.dv.sh + key * p.dv.ss;
#pragma unroll
      for (int c4 = 0; c4 < CP; ++c4) {
        const int col = 4 * (part * CP + c4);
        st4(dkr + col, dkh[c4] * ks_);
        st4(dvr + col, dvh[c4]);
      }
    }
  }
  // dn / db partial of this key block: lane butterfly, then the waves in order
  float pdn = dn_acc - dn_c, pdb = db_acc - db_c;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    pdn += __shfl_xor(pdn, off, 64);
    pdb += __shfl_xor(pdb, off, 64);
  }
  if (lane == 0) {
    red[0][wave] = pdn;
    red[1][wave] = pdb;
  }
  __syncthreads();
  if (tid == 0) {
    float sdn = 0.f, sdb = 0.f;
#pragma unroll
    for (int w = 0; w < NWV; ++w) {
      sdn += red[0][w];
      sdb += red[1][w];
    }
    p.partials[static_cast<int64_t>(bhk) * nkb + kb] = kLn2 * sdn;
    p.partials[PP + static_cast<int64_t>(bhk) * nkb + kb] = n * p.scale * sdb;
  }
}

// ---------------------------------------------------------------------------
// dQ for 128 query rows of one (batch, q-head), in passes of bwd_rows<D>()
// rows: P lanes per row, each holding its share of q, dO and dQ; K / V tiles of 32 keys in LDS; the scores and dP
// are recomputed (dQ += scale n b dS' k).
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(bwd_threads<D>()) void ssa_bwd_dq_f32_kernel(BwdParams p) {
  constexpr int P = bwd_parts<D>(), C4 = D / 4, CP = C4 / P, NT = bwd_threads<D>(), ROWS = bwd_rows<D>();
  __shared__ f32x4 ks[kF32Tile * C4], vs[kF32Tile * C4];
  const int tid = threadIdx.x, part = tid % P;
  const int nqb = (p.N + kF32Pair - 1) / kF32Pair;
  const int qb = blockIdx.x % nqb, bh = blockIdx.x / nqb;
  const int b = bh % p.B, h = bh / p.B, hk = h / (p.Hq / p.Hkv);
  const SeqView sv(p.cu_seqlens, p.T, p.N, b);
  const int N = sv.N;
  if (qb * kF32Pair >= N) return;
  const T* qg = static_cast<const T*>(p.q.ptr) + sv.off(p.q, b) + h * p.q.sh;
  const T* dog = static_cast<const T*>(p.dout.ptr) + sv.off(p.dout, b) + h * p.dout.sh;
  const T* kg = static_cast<const T*>(p.k.ptr) + sv.off(p.k, b) + hk * p.k.sh;
  const T* vg = static_cast<const T*>(p.v.ptr) + sv.off(p.v, b) + hk * p.v.sh;
  const int64_t mr = sv.mrow(b, h, p.Hq, p.T, p.N);
  const float n = *p.n_ptr, bv = *p.b_ptr, c = p.scale * bv;
  // ROWS query rows at a time (one pass up to head dim 128, two at 256)
  const int qend = min(N, qb * kF32Pair + kF32Pair);
  for (int q0 = qb * kF32Pair; q0 < qend; q0 += ROWS) {
    const int i = q0 + tid / P;
    f32x4 qh[CP], doh[CP], dqh[CP];
#pragma unroll
    for (int c4 = 0; c4 < CP; ++c4) {
      const int col = 4 * (part * CP + c4);
      qh[c4] = i < N ? ld4(qg + i * p.q.ss + col) : f32x4{0.f, 0.f, 0.f, 0.f};
      doh[c4] = i < N ? ld4(dog + i * p.dout.ss + col) : f32x4{0.f, 0.f, 0.f, 0.f};
      dqh[c4] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const float mi = i < N ? p.m[mr + i] : 0.f, di = i < N ? p.delta[mr + i] : 0.f;
    const int kv_end = CAUSAL ? min(N, q0 + ROWS) : N;
    for (int k0 = 0; k0 < kv_end; k0 += kF32Tile) {
      __syncthreads();  // the previous tile is consumed
      for (int idx = tid; idx < kF32Tile * C4; idx += NT) {
        const int row = min(k0 + idx / C4, N - 1), c4 = idx % C4;
        ks[idx] = ld4(kg + row * p.k.ss + 4 * c4);
        vs[idx] = ld4(vg + row * p.v.ss + 4 * c4);
      }
      __syncthreads();
      const int kn = min(kF32Tile, kv_end - k0);
      for (int j = 0; j < kn; ++j) {
        const f32x4* krow = ks + j * C4 + part * CP;
        const float s = sum_parts<P>(part_dot<CP>(qh, krow));
        const float dp = sum_parts<P>(part_dot<CP>(doh, vs + j * C4 + part * CP));
        if (i < N && (!CAUSAL || k0 + j <= i)) {
          const float u1 = fmaf(c, fabsf(s), 1.f);
          const float pv = fast_exp2(fmaf(n, ssa_sl(s, u1), -mi));
          const float dsp = pv * (dp - di) * fast_rcp(u1);
#pragma unroll
          for (int c4 = 0; c4 < CP; ++c4) dqh[c4] += dsp * krow[c4];
        }
      }
    }
    if (i < N) {
      const float qs_ = p.scale * n * bv;
      T* dqr = static_cast<T*>(const_cast<void*>(p.dq.ptr)) + sv.off(p.dq, b) + h * p.dq.sh + i * p.dq.ss;
#pragma unroll
      for (int c4 = 0; c4 < CP; ++c4) st4(dqr + 4 * (part * CP + c4), dqh[c4] * qs_);
    }
  }
}

// One launch of KERNEL<T, DD, CAUSAL> with THREADS<DD>() threads.
#define SSA_F32_LAUNCH(KERNEL, THREADS, T, DD, GRID, P, CAUSAL, S)                                 \
  do {                                                                                             \
    if (CAUSAL) hipLaunchKernelGGL((KERNEL<T, DD, true>), dim3(GRID), dim3(THREADS<DD>()), 0, S, P); \
    else hipLaunchKernelGGL((KERNEL<T, DD, false>), dim3(GRID), dim3(THREADS<DD>()), 0, S, P);      \
  } while (0)

// The head dims of each element type: fp32 at 16-256, bf16 / fp16 at 256
// (their other head dims run on the matrix-core kernels).
#define SSA_F32_DISPATCH(KERNEL, THREADS, GRID, P, DTYPE, D, CAUSAL, S)                         \
  if (DTYPE == kDtypeF32) {                                                                     \
    switch (D) {                                                                                \
      case 16: SSA_F32_LAUNCH(KERNEL, THREADS, float, 16, GRID, P, CAUSAL, S); break;           \
      case 32: SSA_F32_LAUNCH(KERNEL, THREADS, float, 32, GRID, P, CAUSAL, S); break;           \
      case 64: SSA_F32_LAUNCH(KERNEL, THREADS, float, 64, GRID, P, CAUSAL, S); break;           \
      case 128: SSA_F32_LAUNCH(KERNEL, THREADS, float, 128, GRID, P, CAUSAL, S); break;         \
      case 256: SSA_F32_LAUNCH(KERNEL, THREADS, float, 256, GRID, P, CAUSAL, S); break;         \
      default: return hipErrorInvalidValue;                                                     \
    }                                                                                           \
  } else if (D == 256) {                                                                        \
    if (DTYPE == 0) SSA_F32_LAUNCH(KERNEL, THREADS, __bf16, 256, GRID, P, CAUSAL, S);           \
    else SSA_F32_LAUNCH(KERNEL, THREADS, _Float16, 256, GRID, P, CAUSAL, S);                    \
  } else {                                                                                      \
    return hipErrorInvalidValue;                                                                \
  }

template <typename T, int D>
static void launch_pre(const BwdParams& p, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.N;
  const int rpb = 256 / (D / 4);
  const int grid = static_cast<int>((rows + rpb - 1) / rpb);
  hipLaunchKernelGGL((ssa_bwd_preprocess_f32_kernel<T, D>), dim3(grid), dim3(256), 0, s, p);
}

}  // namespace

hipError_t launch_fwd_f32(const FwdParams& p, int dtype, int D, bool causal, hipStream_t s) {
  const int grid = (p.N + kF32Rows - 1) / kF32Rows * p.B * p.Hq;
  SSA_F32_DISPATCH(ssa_fwd_f32_kernel, fwd_threads, grid, p, dtype, D, causal, s)
  return hipGetLastError();
}

hipError_t launch_bwd_preprocess_f32(const BwdParams& p, int dtype, int D, hipStream_t s) {
  if (dtype == kDtypeF32) {
    switch (D) {
      case 16: launch_pre<float, 16>(p, s); break;
      case 32: launch_pre<float, 32>(p, s); break;
      case 64: launch_pre<float, 64>(p, s); break;
      case 128: launch_pre<float, 128>(p, s); break;
      case 256: launch_pre<float, 256>(p, s); break;
      default: return hipErrorInvalidValue;
    }
  } else if (D == 256) {
    if (dtype == 0)
      launch_pre<__bf16, 256>(p, s);
    else
      launch_pre<_Float16, 256>(p, s);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_bwd_dkdv_f32(const BwdParams& p, int dtype, int D, bool causal, hipStream_t s) {
  const int grid = dkdv_key_blocks(p.N) * p.B * p.Hkv;
  SSA_F32_DISPATCH(ssa_bwd_dkdv_f32_kernel, bwd_threads, grid, p, dtype, D, causal, s)
  return hipGetLastError();
}

hipError_t launch_bwd_dq_f32(const BwdParams& p, int dtype, int D, bool causal, hipStream_t s) {
  const int grid = (p.N + kF32Pair - 1) / kF32Pair * p.B * p.Hq;
  SSA_F32_DISPATCH(ssa_bwd_dq_f32_kernel, bwd_threads, grid, p, dtype, D, causal, s)
  return hipGetLastError();
}

}  // namespace ssa
