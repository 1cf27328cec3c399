// SSA attention forward for gfx950.
//
// Replaces _ssa_attn_fwd / _ssa_attn_fwd_inner
// (training/train/train_ssa_triton/SSA/ssa_triton_kernel.py:40-260).
//
// One workgroup = 4 waves = 128 query rows of one (batch, q-head); each wave
// owns 32 query rows.  K/V tiles of 64 keys are double-buffered in LDS,
// filled by direct-to-LDS loads and shared by the 4 waves (one barrier per
// tile).  Everything is computed transposed so that a query row lives in a
// single lane pair (l, l+32):
//   S^T = K Q^T      (A = K rows from LDS, B = Q^T fragment held in registers)
//   O^T += V^T P^T   (A = V^T via LDS transpose reads, B = P^T straight from S^T)
// Row max / row sum therefore need one exchange between the two wave halves.
//
// SSA transform in base 2: t2 = n * sign(s) * log2(1 + b|s|) = t / ln 2, with
// s = scale * q.k.  Because t2 is monotone in s (increasing for n >= 0,
// decreasing for n < 0), the row max of t2 is t2 at the row max (or min) of
// s, so the max is taken on the raw scores and p = exp2(n * sL - m) is a
// single fma + exp.  The running max moves lazily (kRescaleTau); the stored
// normaliser M = m + log2(l) is exact either way.  Masks are evaluated only on
// the diagonal tile and the sequence-end tile.
#include <type_traits>

#include "ssa_common.hpp"
#include "ssa_launch.hpp"
#include "ssa_tile.hpp"

namespace ssa {

namespace {

template <typename T, int D>
struct FwdTile {
  typedef typename Vec8<T>::type v8;
  typedef T v4 __attribute__((ext_vector_type(4)));
  static constexpr int ND16 = D / 16, ND32 = D / 32;

  // S^T for the 64 keys of the tile at `kl` (LDS byte address), blocks kb
  // that are not `active` are skipped.
  __device__ static __forceinline__ void scores(const RowBase<D>& rb, const v8* qf, const bool* active,
                                                f32x16* s) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = f32x16{};
      if (!active[kb]) continue;
#pragma unroll
      for (int ds = 0; ds < ND16; ++ds) {
        const v8 a = tile_read_row<D, v8>(rb, kb, ds);
        s[kb] = mfma32(a, qf[ds], s[kb]);
      }
    }
  }

  __device__ static __forceinline__ void pv(const TrBase<D>& tb, const v8 (*pb)[2], const bool* active,
                                            f32x16* acc) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      if (!active[kb]) continue;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int db = 0; db < ND32; ++db) {
          const v4 lo = tile_read_tr<D, v4>(tb, kb, ks, 0, db);
          const v4 hi = tile_read_tr<D, v4>(tb, kb, ks, 1, db);
          const v8 va = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          acc[db] = mfma32(va, pb[kb][ks], acc[db]);
        }
      }
    }
  }
};

template <typename T, int D, bool CAUSAL, bool NPOS>
__device__ __forceinline__ void fwd_body(const FwdParams& p, const int N, const int bh, const int qb, const int b,
                                         const int h, const int hk, char* smem) {
  typedef FwdTile<T, D> FT;
  typedef typename FT::v8 v8;
  constexpr int BM = 128, BN = 64;
  constexpr int TILE_BYTES = BN * D * 2;
  constexpr int ND16 = D / 16, ND32 = D / 32;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  const uint32_t lds0 = lds_addr(smem);
  const RowBase<D> rb(l32, hh);
  const TrBase<D> tb(lane);
  const LoadLane llk(lane, wave, p.k.ss), llv(lane, wave, p.v.ss);
  // buffer t: K at lds0 + t*2*TILE_BYTES, V right after
  const T* qg = static_cast<const T*>(p.q.ptr) + b * p.q.sb + h * p.q.sh;
  const char* kg = static_cast<const char*>(p.k.ptr) + (b * p.k.sb + hk * p.k.sh) * 2;
  const char* vg = static_cast<const char*>(p.v.ptr) + (b * p.v.sb + hk * p.v.sh) * 2;
  T* og = static_cast<T*>(const_cast<void*>(p.o.ptr)) + b * p.o.sb + h * p.o.sh;

  const float n = *p.n_ptr;
  const float c = p.scale * *p.b_ptr;  // u = c * |q.k|
  const int q0 = qb * BM;
  const int wq0 = q0 + wave * 32;
  const int qrow = wq0 + l32;

  const int kv_end = CAUSAL ? min(N, q0 + BM) : N;
  const int ntiles = (kv_end + BN - 1) / BN;
  // first tile that needs masks: the causal diagonal or the sequence end
  const int nfull = CAUSAL ? min(q0 / BN, N / BN) : N / BN;

  tile_load_async<D, BN, 4>(kg, p.k.ss, 0, N, lds0, wave, llk);
  tile_load_async<D, BN, 4>(vg, p.v.ss, 0, N, lds0 + TILE_BYTES, wave, llv);

  v8 qf[ND16];
#pragma unroll
  for (int ds = 0; ds < ND16; ++ds)
    qf[ds] = qrow < N ? load16<v8>(qg + qrow * p.q.ss + ds * 16 + 8 * hh) : zero8<v8>();

  f32x16 acc[ND32];
#pragma unroll
  for (int i = 0; i < ND32; ++i) acc[i] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  auto tile = [&](int t, auto masked_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const uint32_t kl = lds0 + (t & 1) * 2 * TILE_BYTES;
    const uint32_t vl = kl + TILE_BYTES;
    if (t + 1 < ntiles) {
      const uint32_t nk = lds0 + ((t + 1) & 1) * 2 * TILE_BYTES;
      const int r1 = (t + 1) * BN;
      if (r1 + BN <= N) {
        tile_load_pieces<D, BN, 4, false>(kg, p.k.ss, r1, N, nk, wave, llk);
        tile_load_pieces<D, BN, 4, false>(vg, p.v.ss, r1, N, nk + TILE_BYTES, wave, llv);
      } else {
        tile_load_pieces<D, BN, 4, true>(kg, p.k.ss, r1, N, nk, wave, llk);
        tile_load_pieces<D, BN, 4, true>(vg, p.v.ss, r1, N, nk + TILE_BYTES, wave, llv);
      }
    }
    const int kbase = t * BN;
    bool active[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int kstart = kbase + kb * 32;
      active[kb] = !MASKED || (kstart < N && (!CAUSAL || kstart <= wq0 + 31));
    }
    f32x16 s[2];
    FT::scores(at_tile(rb, kl), qf, active, s);

    // Row extreme of the raw scores over valid keys (max for n >= 0, min for n < 0).
    float z = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if (MASKED) {
          const int key = kbase + kb * 32 + crow(r, hh);
          const bool valid = active[kb] && key < N && (!CAUSAL || key <= qrow);
          if (!valid) s[kb][r] = NPOS ? -INFINITY : INFINITY;
        }
        z = fmaxf(z, NPOS ? s[kb][r] : -s[kb][r]);
      }
    }
    z = fmaxf(z, swap_halves(z));
    float t2max = -INFINITY;
    if (z != -INFINITY) {
      const float sst = NPOS ? z : -z;
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
    const float neg_m = -m_run;

    v8 pb[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = s[kb][r];
        const float sl = copysignf(fast_log2(fmaf(c, fabsf(x), 1.f)), x);
        float pv = fast_exp2(fmaf(n, sl, neg_m));
        if (MASKED) pv = (NPOS ? x == -INFINITY : x == INFINITY) ? 0.f : pv;
        l_run += pv;
        pb[kb][r >> 3][r & 7] = static_cast<T>(pv);
      }
    }
    FT::pv(at_tile(tb, vl), pb, active, acc);
  };
  for (int t = 0; t < nfull; ++t) tile(t, std::false_type{});
  for (int t = nfull; t < ntiles; ++t) tile(t, std::true_type{});

  const float l_tot = l_run + swap_halves(l_run);
  const float l_safe = l_tot > 0.f ? l_tot : 1.f;
  const float inv = 1.f / l_safe;
  if (qrow < N) {
#pragma unroll
    for (int db = 0; db < ND32; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + g * 8 + 4 * hh;
        typedef T t4 __attribute__((ext_vector_type(4)));
        t4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = static_cast<T>(acc[db][4 * g + e] * inv);
        *reinterpret_cast<t4*>(og + qrow * p.o.ss + d0) = o4;
      }
    }
    if (hh == 0) p.m[static_cast<int64_t>(bh) * N + qrow] = m_run + log2f(l_safe);
  }
}

}  // namespace

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void ssa_fwd_kernel(FwdParams p) {
  constexpr int BM = 128;
  __shared__ __attribute__((aligned(1024))) char smem[2 * 2 * 64 * D * 2];
  const int N = p.N;
  const int nqb = (N + BM - 1) / BM;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = L / nqb;
  const int qb = nqb - 1 - (L % nqb);  // heaviest (last) query block first
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h / (p.Hq / p.Hkv);
  if (*p.n_ptr >= 0.f)
    fwd_body<T, D, CAUSAL, true>(p, N, bh, qb, b, h, hk, smem);
  else
    fwd_body<T, D, CAUSAL, false>(p, N, bh, qb, b, h, hk, smem);
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
