// SSA attention forward for gfx950.
//
// Replaces _ssa_attn_fwd / _ssa_attn_fwd_inner
// (training/train/train_ssa_triton/SSA/ssa_triton_kernel.py:40-260).
//
// One workgroup = 8 waves = 256 query rows of one (batch, q-head); each wave
// owns 32 query rows, two waves share a SIMD.  K/V tiles of 64 keys live in
// four LDS buffers filled by direct-to-LDS loads two tiles ahead and shared by
// the 8 waves (one barrier per tile).  Everything is computed transposed so
// that a query row lives in a single lane pair (l, l+32):
//   S^T = K Q^T      (A = K rows from LDS, B = Q^T fragment held in registers)
//   O^T += V^T P^T   (A = V^T via LDS transpose reads, B = P^T straight from S^T)
// Row max / row sum therefore need one exchange between the two wave halves.
//
// SSA transform in base 2: t2 = n * sign(s) * log2(1 + b|s|) = t / ln 2, with
// s = scale * q.k.  Because t2 is monotone in s (increasing for n >= 0,
// decreasing for n < 0), the row max of t2 is t2 at the row max (or min) of
// s, so the max is taken on the raw scores and p = exp2(n * sL - m) is a
// single fma + exp.  The running max moves lazily (kRescaleTau in the masked
// iterations, which track the max; kPsumLimit in the pipelined ones, which
// only bound the sum of p); the stored normaliser M = m + log2(l) is exact
// either way.  Masks are evaluated only on the diagonal tiles and the
// sequence-end tile.
#include <type_traits>
#include <utility>

#include "ssa_common.hpp"
#include "ssa_launch.hpp"
#include "ssa_plan.hpp"
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

// ---------------------------------------------------------------------------
// Software-pipelined forward.  One workgroup = 8 waves = 256 query rows (32
// per wave), two waves per SIMD; K/V tiles of 64 keys in NB = 4 LDS buffers
// shared by all 8 waves, one barrier per tile.  Iteration i of a wave issues
//   MFMA : S_{i+1} = K_{i+1} Q^T   and   O^T += V_{i-1}^T P_{i-1}^T
//   VALU : SSA transform, online max / sum and P_i = exp2(...) of S_i
// with no dependence between the two streams inside the iteration, so each
// wave's instruction stream mixes matrix and vector work and the two waves
// of a SIMD overlap one another's.  The accumulator rescale for a moved
// running max is applied at the end of the iteration (after P_{i-1} V_{i-1}
// has been added at the old scale).  Tile t is loaded at the start of
// iteration t - 2 (its buffer last held tile t - 4, whose V was last read in
// iteration t - 3) and must be complete at the start of iteration t - 1.
template <typename T, int D, bool CAUSAL, bool NPOS>
__device__ __forceinline__ void fwd_sp_body(const FwdParams& p, const FwdPlan<D, CAUSAL>& pl, char* smem) {
  typedef FwdTile<T, D> FT;
  typedef typename FT::v8 v8;
  using Plan = FwdPlan<D, CAUSAL>;
  constexpr int BM = Plan::BM, BN = Plan::BN, NW = Plan::NW, NB = Plan::NB;
  constexpr int TILE = Plan::TILE, BUF = Plan::BUF;
  constexpr int ND16 = D / 16, ND32 = D / 32;
  constexpr int PER = (BN / 32 * BlockLayout<D>::IPB + NW - 1) / NW;  // loads per matrix per wave
  constexpr int LPT = 2 * PER;                                       // loads per tile per wave

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  const uint32_t lds0 = lds_addr(smem);
  const RowBase<D> rb(l32, hh);
  const TrBase<D> tb(lane);
  const LoadLane llk(lane, wave, p.k.ss), llv(lane, wave, p.v.ss);
  const SeqView& sv = pl.sv;
  const int N = pl.N, b = pl.b, h = pl.h;
  const T* qg = static_cast<const T*>(p.q.ptr) + sv.off(p.q, b) + h * p.q.sh;
  T* og = static_cast<T*>(const_cast<void*>(p.o.ptr)) + sv.off(p.o, b) + h * p.o.sh;

  const float n = *p.n_ptr;
  const float c = p.scale * *p.b_ptr;  // u = c * |q.k|
  const int q0 = pl.qb * BM;
  const int wq0 = q0 + wave * 32;
  const int qrow = wq0 + l32;

  const int NT = pl.NT;  // tiles streamed by the workgroup
  // tiles this wave computes on, and the first of them that needs masks
  const int Tw = wq0 >= N ? 0 : (CAUSAL ? (min(N, wq0 + 32) + BN - 1) / BN : NT);
  const int nfull = min(Tw, CAUSAL ? min(wq0 / BN, N / BN) : N / BN);

  auto load_tile = [&](int t) { pl.load_tile(t, lds0, wave, llk, llv); };

  v8 qf[ND16];
#pragma unroll
  for (int ds = 0; ds < ND16; ++ds)
    qf[ds] = qrow < N ? load16<v8>(qg + qrow * p.q.ss + ds * 16 + 8 * hh) : zero8<v8>();
  load_tile(0);
  load_tile(1);

  f32x16 acc[ND32];
#pragma unroll
  for (int i = 0; i < ND32; ++i) acc[i] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;
  f32x16 sc[2], sn[2];          // S_i, S_{i+1}
  v8 pc[2][2], pp[2][2];        // P_i, P_{i-1}
  bool ac[2] = {false, false};  // active 32-key blocks of tile i, i+1, i-1
  bool an[2] = {false, false}, ap[2] = {false, false};

  auto flags = [&](int t, bool* a, auto masked_tag) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int kstart = t * BN + kb * 32;
      a[kb] = !decltype(masked_tag)::value || (t < Tw && kstart < N && (!CAUSAL || kstart <= wq0 + 31));
    }
  };

  if (NT > 1)
    wait_vm<LPT>();
  else
    wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  flags(0, ac, std::true_type{});
  if (0 < Tw) FT::scores(at_tile(rb, lds0), qf, ac, sc);

  auto iteration = [&](int i, auto masked_tag, auto first_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool FIRST = decltype(first_tag)::value;  // i == 0: no P V product yet
    wait_vm<0>();  // tile i + 1
    __builtin_amdgcn_s_barrier();
    load_tile(i + 2);
    // matrix stream
    flags(i + 1, an, masked_tag);
    static constexpr bool all2[2] = {true, true};  // unmasked iterations: no run-time block tests
    if (!MASKED || i + 1 < Tw)
      FT::scores(at_tile(rb, lds0 + ((i + 1) & (NB - 1)) * BUF), qf, MASKED ? an : all2, sn);
    if (!FIRST && (!MASKED || i - 1 < Tw))
      FT::pv(at_tile(tb, lds0 + ((i - 1) & (NB - 1)) * BUF + TILE), pp, MASKED ? ap : all2, acc);
    // vector stream: P_i from S_i.  P is computed against the running max
    // m (no dependence on this tile's max, so it interleaves freely with the
    // MFMAs); the tile max is checked on a parallel chain and, when it exceeds
    // m by more than kRescaleTau (so exp2 could exceed 2^kRescaleTau), the rare
    // slow path below recomputes P with the new max and rescales.
    bool grow = false;
    float psum = 0.f;
    float t2max = -INFINITY;
    auto compute_p = [&](float neg_m) {
      float sum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float x = sc[kb][r];
          const float sl = copysignf(fast_log2(fmaf(c, fabsf(x), 1.f)), x);
          float pv = fast_exp2(fmaf(n, sl, neg_m));
          if (MASKED) pv = (NPOS ? x == -INFINITY : x == INFINITY) ? 0.f : pv;
          sum += pv;
          pc[kb][r >> 3][r & 7] = static_cast<T>(pv);
        }
      }
      return sum;
    };
    if (!MASKED || i < Tw) {
      const int kbase = i * BN;
      if (MASKED) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kbase + kb * 32 + crow(r, hh);
            const bool valid = ac[kb] && key < N && (!CAUSAL || key <= qrow);
            if (!valid) sc[kb][r] = NPOS ? -INFINITY : INFINITY;
          }
        }
      }
      psum = compute_p(-m_run);
      // Row extreme of the raw scores over valid keys (max for n >= 0, min for n < 0).
      float z = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) z = fmaxf(z, NPOS ? sc[kb][r] : -sc[kb][r]);
      }
      z = pair_max(z);
      const float sst = NPOS ? z : -z;
      t2max = z == -INFINITY ? -INFINITY : n * copysignf(fast_log2(fmaf(c, fabsf(sst), 1.f)), sst);
      grow = __any(t2max > m_run + kRescaleTau);
    }
    if (grow) {  // rare: the running max moves (always on a row's first tile)
      const float mnew = fmaxf(m_run, t2max);
      const float alpha = fast_exp2(mnew == -INFINITY ? 0.f : m_run - mnew);
      m_run = mnew;
      psum = compute_p(-m_run);
#pragma unroll
      for (int d = 0; d < ND32; ++d) acc[d] *= alpha;  // acc holds P V up to tile i - 1
      l_run *= alpha;
    }
    l_run += psum;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sc[kb] = sn[kb];
      ap[kb] = ac[kb];
      ac[kb] = an[kb];
      pp[kb][0] = pc[kb][0];
      pp[kb][1] = pc[kb][1];
    }
  };

  // Steady-state iteration (tiles i - 1, i, i + 1 unmasked) with the
  // instruction order fixed by the source: NG = D / 4 chunks, each = the LDS
  // operand reads of the MFMA two chunks ahead, one MFMA, and the vector work
  // of EPC = 32 / NG elements of S_i, fenced so that the compiler keeps the
  // mix.  Chunks g < NP add P_{i-1} V_{i-1} (ND32 independent chains) while the
  // elements of key block 0 of S_i are transformed; chunks g >= NP build
  // S_{i+1} (two independent chains) alongside key block 1, so P_{i-1} and the
  // first half of S_i are dead before S_{i+1} is allocated.  The rare slow
  // path (running max moves) recomputes S_i from K_i, still in LDS.  MASKED:
  // the same iteration on a tile that needs masks (the causal diagonal band,
  // the sequence end): p is zeroed outside the mask, in the pipeline and in
  // the slow path, and every MFMA runs (a masked block adds zeros).
  auto iteration_fast = [&](int i, auto masked_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    typedef T v4 __attribute__((ext_vector_type(4)));
    constexpr int NP = 4 * ND32, NS = 2 * ND16, NG = NP + NS, EPC = 32 / NG;
    wait_vm<0>();  // tile i + 1
    __builtin_amdgcn_s_barrier();
    load_tile(i + 2);
    const RowBase<D> kr = at_tile(rb, lds0 + ((i + 1) & (NB - 1)) * BUF);
    const TrBase<D> vt = at_tile(tb, lds0 + ((i - 1) & (NB - 1)) * BUF + TILE);
    const float neg_m = -m_run;
    float psum = 0.f;
    v8 ops[3];
    auto read = [&](auto gc) {
      constexpr int G = decltype(gc)::value;
      if constexpr (G < NP) {
        constexpr int db = G % ND32, ks = (G / ND32) % 2, kb = G / (2 * ND32);
        const v4 lo = tile_read_tr<D, v4>(vt, kb, ks, 0, db);
        const v4 hi = tile_read_tr<D, v4>(vt, kb, ks, 1, db);
        ops[G % 3] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      } else if constexpr (G < NG) {
        constexpr int H = G - NP;
        ops[G % 3] = tile_read_row<D, v8>(kr, H & 1, H >> 1);
      }
    };
    // Element pipeline, three stages on different elements per chunk:
    //   A: u = 1 + c|x|, L = log2(u)
    //   B: t = n copysign(L, x) - m, p = exp2(t)
    //   C: sum and bf16 conversion of p
    // chunk g runs A on elements of chunk g + 2, B on g + 1, C on g.
    float Lv[32], pvv[32];
    auto stage_a = [&](auto ec) {
      constexpr int E = decltype(ec)::value;
      if constexpr (E < 32) {
        const float x = sc[E / 16][E % 16];
        Lv[E] = fast_log2(fmaf(c, fabsf(x), 1.f));
        pin(Lv[E]);
      }
    };
    // Element (kb, r) of S_i holds key i BN + 32 kb + crow(r, hh), crow(r, hh) =
    // crow(r, 0) + 4 hh; it is valid (key < N and, causal, key <= qrow) when
    // crow(r, 0) <= lim[kb], a per-lane bound: one compare with a constant.
    int lim[2] = {0, 0};
    if constexpr (MASKED) {
      const int last = CAUSAL ? min(qrow, N - 1) : N - 1;
      lim[0] = last - i * BN - 4 * hh;
      lim[1] = lim[0] - 32;
    }
    auto valid_key = [&](int kb, int r) { return crow(r, 0) <= lim[kb]; };
    auto stage_b = [&](auto ec) {
      constexpr int E = decltype(ec)::value;
      if constexpr (E < 32) {
        const float x = sc[E / 16][E % 16];
        pvv[E] = fast_exp2(fmaf(n, copysignf(Lv[E], x), neg_m));
        if constexpr (MASKED) pvv[E] = valid_key(E / 16, E % 16) ? pvv[E] : 0.f;
        pin(pvv[E]);
      }
    };
    auto stage_c = [&](auto ec) {
      constexpr int E = decltype(ec)::value;
      psum += pvv[E];
      pin(psum);
      if constexpr (E % 2 == 1) {
        constexpr int kb = E / 16, r = E % 16;
        pc[kb][r >> 3][(r & 7) - 1] = static_cast<T>(pvv[E - 1]);
        pc[kb][r >> 3][r & 7] = static_cast<T>(pvv[E]);
      }
    };
    auto stages = [&](auto f, auto gc) {
      constexpr int G = decltype(gc)::value;
      [&]<int... e>(std::integer_sequence<int, e...>) {
        (f(std::integral_constant<int, G * EPC + e>{}), ...);
      }(std::make_integer_sequence<int, EPC>{});
    };
    auto chunk = [&](auto gc) {
      constexpr int G = decltype(gc)::value;
      read(std::integral_constant<int, G + 2>{});
      if constexpr (G < NP) {
        constexpr int db = G % ND32, ks = (G / ND32) % 2, kb = G / (2 * ND32);
        acc[db] = mfma32(ops[G % 3], pp[kb][ks], acc[db]);
      } else {
        constexpr int H = G - NP, kb = H & 1, ds = H >> 1;
        sn[kb] = mfma32(ops[G % 3], qf[ds], ds == 0 ? f32x16{} : sn[kb]);
      }
      if constexpr (G + 2 < NG) stages(stage_a, std::integral_constant<int, G + 2>{});
      if constexpr (G + 1 < NG) stages(stage_b, std::integral_constant<int, G + 1>{});
      stages(stage_c, std::integral_constant<int, G>{});
      __builtin_amdgcn_sched_barrier(0);
    };
    read(std::integral_constant<int, 0>{});
    read(std::integral_constant<int, 1>{});
    stages(stage_a, std::integral_constant<int, 0>{});
    stages(stage_a, std::integral_constant<int, 1>{});
    stages(stage_b, std::integral_constant<int, 0>{});
    [&]<int... G>(std::integer_sequence<int, G...>) {
      (chunk(std::integral_constant<int, G>{}), ...);
    }(std::make_integer_sequence<int, NG>{});
    // Every p of this lane is at most its sum, so one test per lane bounds
    // them all (and catches inf / NaN).  Rare: the running max must move.
    // The tile's true max then comes from S_i recomputed from K_i (still in
    // LDS), one 32-key block at a time (register pressure), and P is
    // recomputed against the new max.
    if (__any(!(psum <= kPsumLimit))) {
      const RowBase<D> ki = at_tile(rb, lds0 + (i & (NB - 1)) * BUF);
      float z = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        f32x16 so = f32x16{};
#pragma unroll
        for (int ds = 0; ds < ND16; ++ds) so = mfma32(tile_read_row<D, v8>(ki, kb, ds), qf[ds], so);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float zr = NPOS ? so[r] : -so[r];
          z = fmaxf(z, !MASKED || valid_key(kb, r) ? zr : -INFINITY);
        }
      }
      z = pair_max(z);
      const float sst = NPOS ? z : -z;
      const float t2max = n * copysignf(fast_log2(fmaf(c, fabsf(sst), 1.f)), sst);
      const float mnew = fmaxf(m_run, t2max);
      const float alpha = fast_exp2(mnew == -INFINITY ? 0.f : m_run - mnew);
      m_run = mnew;
#pragma unroll
      for (int d = 0; d < ND32; ++d) acc[d] *= alpha;
      l_run *= alpha;
      psum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        f32x16 so = f32x16{};
#pragma unroll
        for (int ds = 0; ds < ND16; ++ds) so = mfma32(tile_read_row<D, v8>(ki, kb, ds), qf[ds], so);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float x = so[r];
          const float sl = copysignf(fast_log2(fmaf(c, fabsf(x), 1.f)), x);
          float pv = fast_exp2(fmaf(n, sl, -m_run));
          if constexpr (MASKED) pv = valid_key(kb, r) ? pv : 0.f;
          psum += pv;
          pc[kb][r >> 3][r & 7] = static_cast<T>(pv);
        }
      }
    }
    l_run += psum;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sc[kb] = sn[kb];
      ap[kb] = ac[kb] = an[kb] = true;
      pp[kb][0] = pc[kb][0];
      pp[kb][1] = pc[kb][1];
    }
  };

  // Iterations with tile i + 1 < nfull keep every stream unmasked.
  iteration(0, std::true_type{}, std::true_type{});
  int i = 1;
  // Iterations whose tile i needs masks run the masked fast iteration while
  // tile i + 1 exists and this wave has valid keys in tile i; the last two
  // (and a wave's tiles past its rows) run the generic one.
  for (; i + 1 < nfull; ++i) iteration_fast(i, std::false_type{});
  for (; i + 1 < NT && i < Tw; ++i) iteration_fast(i, std::true_type{});
  for (; i <= NT; ++i) iteration(i, std::true_type{}, std::false_type{});

  const float l_tot = pair_sum(l_run);
  const float l_safe = l_tot > 0.f ? l_tot : 1.f;
  const float inv = 1.f / l_safe;
  // O rows through LDS (whole rows per store instruction): every wave is
  // past its last read of the K/V ring, which then holds 32 rows of 2 D bytes
  // per wave.
  __syncthreads();
  if (wq0 < N) {
    store_rows_via_lds<T, D>(
        acc, inv, [&](int r) { return lds0 + wave * (32 * D * 2) + r * (D * 2); },
        og + static_cast<int64_t>(wq0) * p.o.ss, p.o.ss, N - wq0, lane);
    if (qrow < N && hh == 0) p.m[sv.mrow(b, h, p.Hq, p.T, p.N) + qrow] = m_run + log2f(l_safe);
  }
}

}  // namespace

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(512) void ssa_fwd_kernel(FwdParams p) {
  using Plan = FwdPlan<D, CAUSAL>;
  __shared__ __attribute__((aligned(1024))) char smem[Plan::LDS_BYTES];
  const Plan pl(p, blockIdx.x, gridDim.x);
  if (pl.empty()) return;  // packed: past the end of a shorter document
  if (*p.n_ptr >= 0.f)
    fwd_sp_body<T, D, CAUSAL, true>(p, pl, smem);
  else
    fwd_sp_body<T, D, CAUSAL, false>(p, pl, smem);
}

template <typename T, int D, bool CAUSAL>
static hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
  const int grid = FwdPlan<D, CAUSAL>::grid(p);
  hipLaunchKernelGGL((ssa_fwd_kernel<T, D, CAUSAL>), dim3(grid), dim3(512), 0, stream, p);
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
  if (use_f32(dtype, D)) return launch_fwd_f32(p, dtype, D, causal, stream);
  if (dtype == 0) return launch_fwd_dt<__bf16>(p, D, causal, stream);
  return launch_fwd_dt<_Float16>(p, D, causal, stream);
}

}  // namespace ssa
