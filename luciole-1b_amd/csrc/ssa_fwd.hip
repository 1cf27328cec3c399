// SSA attention forward for gfx950.
//
// Replaces _ssa_attn_fwd / _ssa_attn_fwd_inner
// (training/train/train_ssa_triton/SSA/ssa_triton_kernel.py:40-260).
//
// One workgroup = 4 waves = 128 query rows of one (batch, q-head); each wave
// owns 32 query rows.  K/V tiles of 64 keys are staged through LDS and shared
// by the 4 waves.  Everything is computed transposed so that a query row lives
// in a single lane pair (l, l+32):
//   S^T = K Q^T      (A = K rows from LDS, B = Q^T fragment held in registers)
//   O^T += V^T P^T   (A = V^T gathered from LDS, B = P^T straight from S^T)
// Row max / row sum therefore need one exchange between the two wave halves.
//
// SSA transform in base 2: t2 = n * sign(s) * log2(1 + b|s|) = t / ln 2, with
// s = scale * q.k.  Because t2 is monotone in s (increasing for n >= 0,
// decreasing for n < 0), the row max of t2 is t2 at the row max (or min) of
// s, so the max is taken on the raw scores and p = exp2(n * sL - m) is a
// single fma + exp.  The running max moves lazily (kRescaleTau); the stored
// normaliser M = m + log2(l) is exact either way.
#include "ssa_common.hpp"
#include "ssa_launch.hpp"

namespace ssa {

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void ssa_fwd_kernel(FwdParams p) {
  constexpr int BM = 128, BN = 64, LDSD = D + 8;
  constexpr int ND16 = D / 16, ND32 = D / 32;
  constexpr int CH_PER_ROW = D / 8;              // 16-byte chunks per row
  constexpr int CH_PER_T = BN * CH_PER_ROW / 256;  // chunks per thread per tile
  typedef typename Vec8<T>::type v8;

  __shared__ __attribute__((aligned(16))) T k_lds[BN * LDSD];
  __shared__ __attribute__((aligned(16))) T v_lds[BN * LDSD];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hh = lane >> 5;
  const int nqb = (p.N + BM - 1) / BM;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = L / nqb;
  const int qb = nqb - 1 - (L % nqb);  // heaviest (last) query block first
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h / (p.Hq / p.Hkv);

  const T* qg = static_cast<const T*>(p.q.ptr) + b * p.q.sb + h * p.q.sh;
  const T* kg = static_cast<const T*>(p.k.ptr) + b * p.k.sb + hk * p.k.sh;
  const T* vg = static_cast<const T*>(p.v.ptr) + b * p.v.sb + hk * p.v.sh;
  T* og = static_cast<T*>(const_cast<void*>(p.o.ptr)) + b * p.o.sb + h * p.o.sh;

  const float n = *p.n_ptr;
  const float c = p.scale * *p.b_ptr;  // u = c * |q.k|
  const float sgn = n >= 0.f ? 1.f : -1.f;
  const int N = p.N;
  const int q0 = qb * BM;
  const int wq0 = q0 + wave * 32;
  const int qrow = wq0 + l32;

  v8 qf[ND16];
#pragma unroll
  for (int ds = 0; ds < ND16; ++ds)
    qf[ds] = qrow < N ? load16<v8>(qg + qrow * p.q.ss + ds * 16 + 8 * hh) : zero8<v8>();

  f32x16 acc[ND32];
#pragma unroll
  for (int i = 0; i < ND32; ++i) acc[i] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  const int kv_end = CAUSAL ? min(N, q0 + BM) : N;
  const int ntiles = (kv_end + BN - 1) / BN;

  u32x4 kreg[CH_PER_T], vreg[CH_PER_T];
  auto gload = [&](int tile) {
#pragma unroll
    for (int i = 0; i < CH_PER_T; ++i) {
      const int ch = tid + i * 256;
      const int row = ch / CH_PER_ROW, col = (ch % CH_PER_ROW) * 8;
      const int key = tile * BN + row;
      if (key < N) {
        kreg[i] = *reinterpret_cast<const u32x4*>(kg + key * p.k.ss + col);
        vreg[i] = *reinterpret_cast<const u32x4*>(vg + key * p.v.ss + col);
      } else {
        kreg[i] = u32x4{0u, 0u, 0u, 0u};
        vreg[i] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };

  gload(0);
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < CH_PER_T; ++i) {
      const int ch = tid + i * 256;
      const int row = ch / CH_PER_ROW, col = (ch % CH_PER_ROW) * 8;
      *reinterpret_cast<u32x4*>(&k_lds[row * LDSD + col]) = kreg[i];
      *reinterpret_cast<u32x4*>(&v_lds[row * LDSD + col]) = vreg[i];
    }
    __syncthreads();
    if (t + 1 < ntiles) gload(t + 1);

    const int kbase = t * BN;
    bool active[2];
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int kstart = kbase + kb * 32;
      active[kb] = kstart < N && (!CAUSAL || kstart <= wq0 + 31);
      s[kb] = f32x16{};
      if (active[kb]) {
#pragma unroll
        for (int ds = 0; ds < ND16; ++ds) {
          const v8 a = load16<v8>(&k_lds[(kb * 32 + l32) * LDSD + ds * 16 + 8 * hh]);
          s[kb] = mfma32(a, qf[ds], s[kb]);
        }
      }
    }

    // Row max over valid keys, on sgn * s (monotone image of t2).
    float zmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      if (!active[kb]) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kbase + kb * 32 + crow(r, hh);
        const bool valid = key < N && (!CAUSAL || key <= qrow);
        if (valid) zmax = fmaxf(zmax, sgn * s[kb][r]);
      }
    }
    zmax = fmaxf(zmax, swap_halves(zmax));
    float t2max = -INFINITY;
    if (zmax != -INFINITY) {
      const float sst = sgn * zmax;
      t2max = n * copysignf(fast_log2(fmaf(c, fabsf(sst), 1.f)), sst);
    }
    if (__any(t2max > m_run + kRescaleTau)) {
      const float mnew = fmaxf(m_run, t2max);
      const float alpha = mnew == -INFINITY ? 1.f : fast_exp2(m_run - mnew);
#pragma unroll
      for (int i = 0; i < ND32; ++i) acc[i] *= alpha;
      l_run *= alpha;
      m_run = mnew;
    }

    v8 pb[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kbase + kb * 32 + crow(r, hh);
        const bool valid = active[kb] && key < N && (!CAUSAL || key <= qrow);
        const float x = s[kb][r];
        const float sl = copysignf(fast_log2(fmaf(c, fabsf(x), 1.f)), x);
        const float pv = valid ? fast_exp2(fmaf(n, sl, -m_run)) : 0.f;
        l_run += pv;
        pb[kb][r >> 3][r & 7] = static_cast<T>(pv);
      }
    }

#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      if (!active[kb]) continue;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int db = 0; db < ND32; ++db) {
          v8 va;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int krow = kb * 32 + ks * 16 + crow(e, hh);
            va[e] = v_lds[krow * LDSD + db * 32 + l32];
          }
          acc[db] = mfma32(va, pb[kb][ks], acc[db]);
        }
      }
    }
  }

  const float l_tot = l_run + swap_halves(l_run);
  const float l_safe = l_tot > 0.f ? l_tot : 1.f;
  const float inv = 1.f / l_safe;
  if (qrow < N) {
#pragma unroll
    for (int db = 0; db < ND32; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + g * 8 + 4 * hh;
        T* dst = og + qrow * p.o.ss + d0;
        typedef T t4 __attribute__((ext_vector_type(4)));
        t4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = static_cast<T>(acc[db][4 * g + e] * inv);
        *reinterpret_cast<t4*>(dst) = o4;
      }
    }
    if (hh == 0) p.m[static_cast<int64_t>(bh) * N + qrow] = m_run + log2f(l_safe);
  }
}

template <typename T, int D, bool CAUSAL>
static hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
  const int nqb = (p.N + 127) / 128;
  const int grid = nqb * p.B * p.Hq;
  hipLaunchKernelGGL((ssa_fwd_kernel<T, D, CAUSAL>), dim3(grid), dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_fwd_dt(const FwdParams& p, int D, bool causal, hipStream_t s) {
  switch (D) {
    case 32: return causal ? launch_fwd_t<T, 32, true>(p, s) : launch_fwd_t<T, 32, false>(p, s);
    case 64: return causal ? launch_fwd_t<T, 64, true>(p, s) : launch_fwd_t<T, 64, false>(p, s);
    case 128: return causal ? launch_fwd_t<T, 128, true>(p, s) : launch_fwd_t<T, 128, false>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_fwd(const FwdParams& p, int dtype, int D, bool causal, hipStream_t stream) {
  if (dtype == 0) return launch_fwd_dt<__bf16>(p, D, causal, stream);
  return launch_fwd_dt<_Float16>(p, D, causal, stream);
}

}  // namespace ssa
