// SSA attention decode step for gfx950: one new query token per sequence
// against a KV cache.
//
// No reference kernel: the reference's generation loop re-runs the whole
// prefix through the forward for every new token
// (training/train/train_ssa_triton/generate_triton.py:315-331).  The result of
// this kernel is the last row of the causal forward over the cached prefix,
// i.e. the same SSA transform and base-2 online normaliser as
// _ssa_attn_fwd_inner (training/train/train_ssa_triton/SSA/ssa_triton_kernel.py:95-122).
//
// The step is an HBM stream over the cache (2 * L * D * 2 bytes per
// (sequence, kv-head)).  Work unit = (sequence b, kv-head, group of up to 32
// q-heads sharing it, key split); one workgroup per unit, NW waves, each wave
// streaming its own 32-key tiles (tile t of the split goes to wave t % NW)
// through a private LDS ring of NB tiles filled by direct-to-LDS loads NB - 1
// tiles ahead, so no barrier is needed until the end.  The stream is bound by
// the loads each CU keeps in flight: as many waves as 128 KB of rings allow
// (measured: 4 waves with 2-deep rings move 1.6x the bytes of 2 waves with
// 4-deep rings at D = 128), and one workgroup per CU.  The GQA group is the
// MFMA's 32-wide column dimension, so the cache is read once per kv-head:
//   S^T = K Q^T   (A = 32 keys from LDS, B = Q^T of the group in registers)
//   O^T += V^T P^T (A = V^T via LDS transpose reads, B = P^T from S^T)
// A lane pair (l, l + 32) holds one q-head.  The running max is exact (the
// tile max comes from the raw scores, as t is monotone in s).  At the end the
// waves merge (m, l, acc) through LDS; with one split the workgroup writes
// the output, otherwise an unnormalised partial that ssa_decode_merge_kernel
// combines in split order (deterministic).
#include "ssa_common.hpp"
#include "ssa_launch.hpp"
#include "ssa_plan.hpp"
#include "ssa_tile.hpp"

namespace ssa {

namespace {

// DecodeCfg, DecodePlan and block_load_wave: ssa_plan.hpp.

template <typename T, int D, bool NPOS>
__device__ __forceinline__ void decode_body(const DecodeParams& p, char* smem, const DecodePlan<D>& pl) {
  typedef DecodeCfg<D> C;
  typedef typename Vec8<T>::type v8;
  typedef T v4 __attribute__((ext_vector_type(4)));
  constexpr int NW = C::NW, NB = C::NB, ND16 = D / 16, ND32 = D / 32;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  const int b = pl.b, hk = pl.hk, qg = pl.qg, split = pl.split;
  const int G = p.Hq / p.Hkv;
  const int gq = min(32, G - qg * 32);  // q-heads of this group
  const int h0 = hk * G + qg * 32;      // first q-head of the group

  const int kbeg = pl.kbeg, kend = pl.kend;
  const int ntw = pl.tiles_of(wave);  // tiles of this wave

  const float n = *p.n_ptr;
  const float c = p.scale * *p.b_ptr;  // u = c * |q.k|

  v8 qf[ND16];
  {
    const T* qg_ptr = static_cast<const T*>(p.q.ptr) + b * p.q.sb + (h0 + l32) * p.q.sh;
#pragma unroll
    for (int ds = 0; ds < ND16; ++ds) qf[ds] = l32 < gq ? load16<v8>(qg_ptr + ds * 16 + 8 * hh) : zero8<v8>();
  }

  f32x16 acc[ND32];
#pragma unroll
  for (int d = 0; d < ND32; ++d) acc[d] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  if (ntw > 0) {
    const LoadLane lk0(lane, 0, p.k.ss), lk1(lane, 1, p.k.ss), lv0(lane, 0, p.v.ss), lv1(lane, 1, p.v.ss);
    const uint32_t ring = lds_addr(smem) + wave * NB * C::TB;
    const RowBase<D> rb(l32, hh);
    const TrBase<D> tb(lane);
    // The i-th tile of this wave; past the wave's last tile the rows clamp to
    // kend - 1 (loads into a free buffer, never read), so every iteration
    // issues the same number of loads and one wait count fits all.
    auto issue = [&](int i) { pl.issue(i, wave, ring, lk0, lk1, lv0, lv1); };
#pragma unroll
    for (int i = 0; i < NB - 1; ++i) issue(i);
    for (int i = 0; i < ntw; ++i) {
      wait_lgkm<0>();  // reads of tile i - 1, whose buffer the next issue overwrites
      issue(i + NB - 1);
      wait_vm<(NB - 1) * C::LPT>();  // tile i has landed
      const uint32_t buf = ring + (i % NB) * C::TB;
      const RowBase<D> kr = at_tile(rb, buf);
      const TrBase<D> vt = at_tile(tb, buf + C::BLOCK);
      f32x16 s = f32x16{};
#pragma unroll
      for (int ds = 0; ds < ND16; ++ds) s = mfma32(tile_read_row<D, v8>(kr, 0, ds), qf[ds], s);
      // keys of the tile at or past kend are masked (p = 0)
      const int key0 = kbeg + 32 * (wave + NW * i);
      float z = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if (key0 + crow(r, hh) >= kend) s[r] = NPOS ? -INFINITY : INFINITY;
        z = fmaxf(z, NPOS ? s[r] : -s[r]);
      }
      z = pair_max(z);
      const float sst = NPOS ? z : -z;
      const float t2max = z == -INFINITY ? -INFINITY : n * copysignf(fast_log2(fmaf(c, fabsf(sst), 1.f)), sst);
      const float mnew = fmaxf(m_run, t2max);
      const float alpha = fast_exp2(mnew == -INFINITY ? 0.f : m_run - mnew);
      m_run = mnew;
#pragma unroll
      for (int d = 0; d < ND32; ++d) acc[d] *= alpha;
      l_run *= alpha;
      v8 pb[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = s[r];
        const float sl = copysignf(fast_log2(fmaf(c, fabsf(x), 1.f)), x);
        float pv = fast_exp2(fmaf(n, sl, -m_run));
        pv = (NPOS ? x == -INFINITY : x == INFINITY) ? 0.f : pv;
        l_run += pv;
        pb[r >> 3][r & 7] = static_cast<T>(pv);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int db = 0; db < ND32; ++db) {
          const v4 lo = tile_read_tr<D, v4>(vt, 0, ks, 0, db);
          const v4 hi = tile_read_tr<D, v4>(vt, 0, ks, 1, db);
          acc[db] = mfma32(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), pb[ks], acc[db]);
        }
      }
    }
    wait_vm<0>();  // the trailing prefetches land before the ring is reused
  }
  const float l_tot = pair_sum(l_run);

  // Merge the waves: (m, l) per q-head and acc[q][d] through LDS, then one
  // thread per (q-head, d) combines them in wave order.
  __syncthreads();
  float* ml = reinterpret_cast<float*>(smem);                  // [NW][2][32]
  float* accs = reinterpret_cast<float*>(smem + C::ML_BYTES);  // [NW][32][ACC_LD]
  if (hh == 0) {
    ml[(wave * 2 + 0) * 32 + l32] = m_run;
    ml[(wave * 2 + 1) * 32 + l32] = l_tot;
  }
#pragma unroll
  for (int db = 0; db < ND32; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) accs[(wave * 32 + l32) * C::ACC_LD + db * 32 + crow(r, hh)] = acc[db][r];
  }
  __syncthreads();
  for (int e = tid; e < gq * D; e += NW * 64) {
    const int q = e / D, d = e - q * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, ml[(w * 2) * 32 + q]);
    float Ls = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float sc = fast_exp2(ml[(w * 2) * 32 + q] - M);
        Ls += ml[(w * 2 + 1) * 32 + q] * sc;
        O += accs[(w * 32 + q) * C::ACC_LD + d] * sc;
      }
    }
    const int hq = h0 + q;
    if (p.splits == 1) {
      const float l_safe = Ls > 0.f ? Ls : 1.f;
      const float inv = 1.f / l_safe;
      T* o = static_cast<T*>(const_cast<void*>(p.o.ptr)) + b * p.o.sb + hq * p.o.sh;
      o[d] = static_cast<T>(O * inv);
      if (d == 0 && p.m != nullptr) p.m[b * p.Hq + hq] = M + log2f(l_safe);
    } else {
      const int64_t rec = (static_cast<int64_t>(b) * p.Hq + hq) * p.splits + split;
      p.ws_acc[rec * D + d] = O;
      if (d == 0) {
        p.ws_ml[2 * rec] = M;
        p.ws_ml[2 * rec + 1] = Ls;
      }
    }
  }
}

}  // namespace

template <typename T, int D>
__global__ __launch_bounds__(DecodeCfg<D>::NW * 64) void ssa_decode_kernel(DecodeParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[DecodeCfg<D>::SMEM];
  const DecodePlan<D> pl(p, blockIdx.x);
  if (*p.n_ptr >= 0.f)
    decode_body<T, D, true>(p, smem, pl);
  else
    decode_body<T, D, false>(p, smem, pl);
}

// One thread per output element d of a (sequence, q-head): combine the split
// partials in split order, out = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M),
// in one pass with the running maximum (each split's loads are independent of
// the running state, so they can all be in flight at once).
template <typename T, int D>
__global__ __launch_bounds__(128) void ssa_decode_merge_kernel(DecodeParams p) {
  const int bh = blockIdx.x, d = threadIdx.x;
  const int b = bh / p.Hq, hq = bh - b * p.Hq;
  const int64_t rec0 = static_cast<int64_t>(bh) * p.splits;
  float M = -INFINITY, Ls = 0.f, O = 0.f;
  for (int s = 0; s < p.splits; ++s) {
    const float ms = p.ws_ml[2 * (rec0 + s)];
    const float ls = p.ws_ml[2 * (rec0 + s) + 1];
    const float as = d < D ? p.ws_acc[(rec0 + s) * D + d] : 0.f;
    if (ms == -INFINITY) continue;  // empty split: l = 0, acc = 0
    if (ms > M) {
      const float f = fast_exp2(M - ms);  // 0 while M is still -inf
      Ls = Ls * f + ls;
      O = O * f + as;
      M = ms;
    } else {
      const float f = fast_exp2(ms - M);
      Ls += ls * f;
      O += as * f;
    }
  }
  const float l_safe = Ls > 0.f ? Ls : 1.f;
  if (d < D) {
    T* o = static_cast<T*>(const_cast<void*>(p.o.ptr)) + b * p.o.sb + hq * p.o.sh;
    o[d] = static_cast<T>(O * (1.f / l_safe));
  }
  if (d == 0 && p.m != nullptr) p.m[bh] = M + log2f(l_safe);
}

template <typename T, int D>
static hipError_t launch_decode_t(const DecodeParams& p, hipStream_t s) {
  const int grid = DecodePlan<D>::grid(p);
  hipLaunchKernelGGL((ssa_decode_kernel<T, D>), dim3(grid), dim3(DecodeCfg<D>::NW * 64), 0, s, p);
  if (p.splits > 1) hipLaunchKernelGGL((ssa_decode_merge_kernel<T, D>), dim3(p.B * p.Hq), dim3(128), 0, s, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_decode_dt(const DecodeParams& p, int D, hipStream_t s) {
  switch (D) {
    case 32: return launch_decode_t<T, 32>(p, s);
    case 64: return launch_decode_t<T, 64>(p, s);
    case 128: return launch_decode_t<T, 128>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_decode(const DecodeParams& p, int dtype, int D, hipStream_t stream) {
  if (dtype == 0) return launch_decode_dt<__bf16>(p, D, stream);
  return launch_decode_dt<_Float16>(p, D, stream);
}

}  // namespace ssa
