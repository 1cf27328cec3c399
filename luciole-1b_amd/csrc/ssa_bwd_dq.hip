// SSA attention backward for gfx950: dQ from the dS' workspace (the dS' K
// pass), with the fixed-order dn / db reduction folded into its workgroup 0.
//
// Replaces the dQ half of _ssa_attn_bwd_dq
// (training/train/train_ssa_triton/SSA/ssa_triton_kernel.py:408-481): where
// the reference recomputes the scores, this pass reads the -dS' tiles the
// dK/dV kernel stored (ssa_bwd.hip) and multiplies them with K.
#include "ssa_common.hpp"
#include "ssa_launch.hpp"
#include "ssa_plan.hpp"
#include "ssa_tile.hpp"

namespace ssa {

// dQ from the dS' workspace written by the dK/dV kernel: dQ = scale n b dS' K,
// no recompute.  32 NW queries per workgroup (NW waves x 32), keys in tiles of
// 64.  Two LDS rings, both filled by direct-to-LDS loads: K tiles (L2-resident)
// NK buffers loaded PFK steps ahead; the four 1 KB dS' tiles of every wave
// (streamed from HBM) NDS buffers loaded PFD > PFK steps ahead.  At D = 128,
// NW = 8: 128 KB, one workgroup per CU, each K tile read once per 256 queries
// (4 % faster than two 4-wave workgroups per CU, which read K twice as often).  Step t issues K(t + PFK), then
// dS'(t + PFD), so dS'(t) is older than K(t) and one counted wait covers both:
// the loads issued after K(t) -- the 4 dS' loads of its own step and the
// KP + 4 of each of the PFK - 1 steps after it -- may be outstanding.  Every step issues the same
// loads unconditionally (addresses clamped into the workspace and the
// sequence), so the counts are exact.  Per wave the product is
// dQ^T += K^T dS'^T on 32x32x16 MFMAs: A = K^T by transpose reads (rows d,
// contraction over keys in the order 8 hi + 4 hh + e), B = the stored tile,
// transposed on the way out of LDS into that same key order.
template <typename T, int D, bool CAUSAL, int NW>
__global__ __launch_bounds__(NW * 64) void ssa_bwd_dq_ds_kernel(BwdParams p) {
  typedef typename Vec8<T>::type v8;
  typedef T v4 __attribute__((ext_vector_type(4)));
  using Loads = DqDsLoads<D, CAUSAL, NW>;
  constexpr int ND32 = D / 32;
  constexpr int NK = Loads::NK, PFK = Loads::PFK, PFD = Loads::PFD;
  constexpr int KTILE = Loads::KTILE, DSTAGE = Loads::DSTAGE, KP = Loads::KP;
  static_assert(NW * 64 >= 256, "the fused reduction needs 256 threads");
  __shared__ __attribute__((aligned(1024))) char smem[Loads::LDS_BYTES];

  // The backward's dn / db reduction, before this workgroup issues any load
  // (the partials are complete: dK/dV ran before this kernel), in the first
  // 2 KB of the ring, which the loads overwrite only after the barrier.
  if (p.fuse_reduce && blockIdx.x == 0) {
    const int64_t count = static_cast<int64_t>(p.B) * p.Hkv * dkdv_key_blocks(p.N);
    reduce_partials_body(p.partials, count, p.dn, p.db, reinterpret_cast<float(*)[256]>(smem), threadIdx.x);
    __syncthreads();
  }

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // dispatch, K tile and dS' tile loads (ssa_plan.hpp)
  const Loads ld(p, blockIdx.x, gridDim.x, wave, lane);
  if (ld.empty()) return;  // packed: past the end of a shorter document
  const int b = ld.b, h = ld.h, N = ld.N;
  const SeqView& sv = ld.sv;
  // the workspace holds -dS' (the dK/dV kernel's sign convention); n and b
  // are read before the stream starts (read after it, the two loads queue
  // behind the workspace traffic and hold the workgroup's end: 25 % of the
  // pass in the loads-only ablation)
  const float qscale = -(p.scale * *p.n_ptr * *p.b_ptr);
  const uint32_t lds0 = lds_addr(smem);
  const uint32_t lds_ds = lds0 + NK * KTILE;
  // K tiles: row-swizzled for D = 128 (whole-row loads), block-chunk-major otherwise
  constexpr bool ROWSWZ = Loads::ROWSWZ;
  const TrBase<D> tb(lane);
  const RowSwzTr rtb(lane);

  const int wq0 = ld.wq0;
  const int ntiles = ld.ntiles;
  // dS' tiles of this wave's query rows: kj < nkj (loads clamped to kj_max)
  const int nkj = ld.nkj;
  // A stored tile holds, in lane s = 16 g + kl, key kl and queries 16 t + 4 g +
  // (0..3) (elements 4 t ..).  LDS slot 16 g + m receives stored lane
  // 16 g + (m ^ 4 g) (the loads' lane order); the B operand (query L % 32,
  // keys 8 r + 4 hh + e) is then two transposed reads, lane i of group G
  // supplying key 8 r + 4 hh + i / 4, queries 16 (G & 1) + 4 (i % 4) .. + 3,
  // and each half-wave covers every bank once.
  uint32_t ds_rd[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int G = lane >> 4, i = lane & 15, gp = i & 3;
    const int key = 8 * r + 4 * (G >> 1) + (i >> 2);
    ds_rd[r] = static_cast<uint32_t>((16 * gp + (key ^ (4 * gp))) * 16 + 8 * (G & 1));
  }

  auto issue_k = [&](int t) { ld.issue_k(t, lds0); };
  auto issue_ds = [&](int t) { ld.issue_ds(t, lds0); };

  f32x16 dq[ND32];
#pragma unroll
  for (int i = 0; i < ND32; ++i) dq[i] = f32x16{};

  // virtual steps -PFD .. -1 of the issue schedule: K(s + PFK) if s + PFK >= 0, then dS'(s + PFD)
#pragma unroll
  for (int sv = -PFD; sv < 0; ++sv) {
    if (sv + PFK >= 0) issue_k(sv + PFK);
    issue_ds(sv + PFD);
  }
  for (int t = 0; t < ntiles; ++t) {
    wait_vm<4 + (PFK - 1) * (KP + 4)>();  // K(t), and the older dS'(t), of this wave
    __builtin_amdgcn_s_barrier();
    issue_k(t + PFK);
    issue_ds(t + PFD);
    const TrBase<D> tk = at_tile(tb, Loads::ktile(lds0, t));
    const RowSwzTr rk = at_tile(rtb, Loads::ktile(lds0, t));
    const uint32_t dsl = ld.dstage(lds0, t);
    typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      // tiles past the wave's last one hold clamped copies: multiply by zero
      // (no branch, so the reads of all four tiles can be issued together)
      v4 part[2];
#pragma unroll
      for (int r = 0; r < 2; ++r)
        part[r] = __builtin_bit_cast(v4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                                             (__attribute__((address_space(3))) bf16x4_t*)(uintptr_t)(
                                                 dsl + s4 * 1024 + ds_rd[r])));
      const v8 raw = __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7);
      const v8 dsv = 4 * t + s4 < nkj ? raw : zero8<v8>();
      const int blk = s4 >> 1, ks = s4 & 1;
#pragma unroll
      for (int db = 0; db < ND32; ++db) {
        v4 lo, hi;
        if constexpr (ROWSWZ) {
          lo = rowswz_read_tr<v4>(rk, blk, ks, 0, db);
          hi = rowswz_read_tr<v4>(rk, blk, ks, 1, db);
        } else {
          lo = tile_read_tr<D, v4>(tk, blk, ks, 0, db);
          hi = tile_read_tr<D, v4>(tk, blk, ks, 1, db);
        }
        dq[db] = mfma32(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), dsv, dq[db]);
      }
    }
  }
  wait_vm<0>();  // no direct-to-LDS load may outlive the workgroup

  // dQ rows through this wave's own dS' slots (its loads have all landed and
  // no other wave reads them): rows 0-15 in the slot of stage 0, rows 16-31 in
  // that of stage 1 (16 rows of D bf16 fill at most one 4 KB slot).
  static_assert(16 * D * 2 <= 4096, "16 dQ rows per dS' slot");
  T* dq0 = static_cast<T*>(const_cast<void*>(p.dq.ptr)) + sv.off(p.dq, b) + h * p.dq.sh;
  store_rows_via_lds<T, D>(
      dq, qscale, [&](int r) { return lds_ds + (r >> 4) * DSTAGE + wave * 4096 + (r & 15) * (D * 2); },
      dq0 + static_cast<int64_t>(min(wq0, N - 1)) * p.dq.ss, p.dq.ss, N - wq0, lane);
}


template <typename T, int D, bool CAUSAL>
static hipError_t dq_ds_t(const BwdParams& p, hipStream_t s) {
  constexpr int NW = dq_ds_waves<D>();
  const int grid = DqDsLoads<D, CAUSAL, NW>::grid(p);
  hipLaunchKernelGGL((ssa_bwd_dq_ds_kernel<T, D, CAUSAL, NW>), dim3(grid), dim3(NW * 64), 0, s, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t dq_ds_dt(const BwdParams& p, int D, bool causal, hipStream_t s) {
  switch (D) {
    case 32: return causal ? dq_ds_t<T, 32, true>(p, s) : dq_ds_t<T, 32, false>(p, s);
    case 64: return causal ? dq_ds_t<T, 64, true>(p, s) : dq_ds_t<T, 64, false>(p, s);
    case 128: return causal ? dq_ds_t<T, 128, true>(p, s) : dq_ds_t<T, 128, false>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_bwd_dq_ds(const BwdParams& p, int dtype, int D, bool causal, hipStream_t s) {
  return dtype == 0 ? dq_ds_dt<__bf16>(p, D, causal, s) : dq_ds_dt<_Float16>(p, D, causal, s);
}

}  // namespace ssa
