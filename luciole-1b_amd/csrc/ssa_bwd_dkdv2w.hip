// dK, dV (+ dn / db partials, optional dS' workspace) for gfx950 with two waves
// per SIMD.  Replaces _ssa_attn_bwd_dkdv (training/train/train_ssa_triton/SSA/
// ssa_triton_kernel.py:305-401, called from _ssa_attn_bwd :545-636); the math
// per valid (query i, key j) is that of ssa_bwd.hip's header.
//
// Why a second dK/dV kernel.  With 32 keys per wave at head dim 128 the dK/dV
// accumulators (128 registers) and the K / V fragments (64) leave no room for
// a second wave on a SIMD, and one in-order wave cannot hide its own LDS,
// transcendental and MFMA latencies.  Here a wave owns 16 keys: the
// accumulators take 64 registers and the fragments 32, and the whole wave
// fits in 256, so a workgroup of 8 waves (128 keys) runs two waves per SIMD.
//
// Products (v_mfma_f32_16x16x32, lane l = 16 g + i):
//   S  = Q K^T, dP = dO V^T per 16-query block qb of a 64-query step: lane l
//        holds key i, queries 16 qb + 4 g + (0..3); contraction over d in
//        k-steps of 32 (chunk 4 ks + sg(g) of the rows, sg = {0, 2, 1, 3}).
//   dV += P^T dO, dK += dS'^T Q per query half h (32 queries) and 16-column
//        block db: A = P^T from the lane's own elements (k-slot kk <->
//        query 32 h + 16 (kk / 4) + 4 g + kk % 4), B = dO or Q by two
//        transpose reads in that order.  The accumulator lane holds column
//        16 db + i of keys 4 g + (0..3).
// V is held negated and dP starts from Delta, so the dP accumulator is
// Delta - dP, and the per-pair terms are the negated ones (see ssa_bwd.hip).
//
// Q / dO / M / Delta tiles of 64 queries live in a ring of four LDS buffers;
// tile t is loaded two slots before it is first read (see SYNC below).
//
// The 16 elements of a step are the four 4-element blocks of S / dP.  A slot
// runs the element pipeline of step j one element per tick (16 ticks) and,
// between its stages, the MFMAs of three steps: dV/dK of the second query
// half of step j - 1, S/dP block 3 of step j, S/dP blocks 0-2 of step j + 1
// and dV/dK of the first half of step j.  Each S/dP block of step j + 1 is
// issued once the element pipeline is done with that block of step j, and each
// dV/dK half once its P / dS' operands are complete, so all of these live in
// one set of registers: nothing is copied between slots.
#include <type_traits>
#include <utility>

#include "ssa_common.hpp"
#include "ssa_launch.hpp"
#include "ssa_plan.hpp"
#include "ssa_tile.hpp"

namespace ssa {

__device__ __forceinline__ f32x4_t mfma16(bf16x8 a, bf16x8 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16(f16x8 a, f16x8 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Q / dO tiles of 64 rows in the Swz8 layout: two 32-row blocks, chunk-major
// (chunk c of a block is 512 contiguous bytes), row r of chunk c at position
// r ^ 8 (c & 1).  Measured LDS rules (ssa_tile.hpp) and the two fetches:
//   * S / dP operand rows (ds_read_b128): a 16-lane group reads one chunk of
//     16 consecutive rows, 256 contiguous bytes; the two groups of a half-wave
//     read chunks of the same parity (sg(g) & 1 = g >> 1), i.e. the same row
//     permutation;
//   * dV / dK operands (ds_read_b64_tr_b16): a half-wave reads 8 rows (two
//     aligned quads) of the chunk pair 2 db, 2 db + 1, whose swizzles differ
//     in bit 3, so the four (quad, chunk) pieces fall on four disjoint 64-byte
//     bank groups.
template <int D>
struct Swz8Tile {
  static constexpr int BLOCK = 32 * D * 2;
  static constexpr int TILE = 2 * BLOCK;
  // per-lane base of the operand-row fetch; + row_imm(qb, ks)
  static __device__ __forceinline__ uint32_t row_base(int lane) {
    const int g = lane >> 4, i = lane & 15;
    return static_cast<uint32_t>((2 * (g & 1) + (g >> 1)) * 512 + ((i ^ (8 * (g >> 1))) << 4));
  }
  static constexpr uint32_t row_imm(int qb, int ks) { return (qb >> 1) * BLOCK + ks * 4 * 512 + (qb & 1) * 256; }
  // per-lane base of the transpose fetch; + tr_imm(h, db, s): lane 16 g + i
  // receives column 16 db + i of rows 32 h + 16 s + 4 g + (0..3)
  static __device__ __forceinline__ uint32_t tr_base(int lane) {
    const int g = lane >> 4, i = lane & 15, cb = (i & 3) >> 1;
    return static_cast<uint32_t>(cb * 512 + (((4 * g + (i >> 2)) ^ (8 * cb)) << 4) + ((i & 1) << 3));
  }
  static constexpr uint32_t tr_imm(int h, int db, int s) { return h * BLOCK + db * 1024 + s * 256; }
};

template <typename V>
__device__ __forceinline__ V lds_v8(uint32_t addr) {
  return *(const __attribute__((address_space(3))) V*)(uintptr_t)addr;
}
template <typename V4>
__device__ __forceinline__ V4 lds_tr4(uint32_t addr) {
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(V4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                                    (__attribute__((address_space(3))) bf16x4_t*)(uintptr_t)addr));
}

// MFMA schedule of a slot: item index -> kind and tick.  Items in order:
//   H1: dV/dK of step j - 1, query half 1 (2 NDB: dV, dK per column block)
//   B3: S/dP block 3 of step j (2 NKS: S, dP per k-step)
//   B0, B1: S/dP blocks 0, 1 of step j + 1
//   H0a: dV/dK of step j, half 0, first NDB / 2 column blocks
//   B2: S/dP block 2 of step j + 1
//   H0b: the remaining column blocks of half 0
// An item runs at tick max(earliest, i TK / NG): block b of step j + 1 after
// tick 4 b + 4 (the last stage that reads S / dP elements 4 b .. 4 b + 3 of
// step j), half 0 of step j after tick 8 (its operands' last stage).
template <int D>
struct Sched2w {
  static constexpr int NKS = D / 32, NDB = D / 16;
  static constexpr int NH = 2 * NDB, NBK = 2 * NKS;
  static constexpr int NG = 2 * NH + 4 * NBK, TK = 16;
  enum Kind { H1, B3, B0, B1, H0, B2 };
  struct Item {
    int kind, k;  // k: index inside its group (dV/dK: 2 db + t; S/dP: 2 ks + t)
  };
  static constexpr Item item(int i) {
    if (i < NH) return {H1, i};
    i -= NH;
    if (i < NBK) return {B3, i};
    i -= NBK;
    if (i < NBK) return {B0, i};
    i -= NBK;
    if (i < NBK) return {B1, i};
    i -= NBK;
    if (i < NH / 2) return {H0, i};
    i -= NH / 2;
    if (i < NBK) return {B2, i};
    i -= NBK;
    return {H0, NH / 2 + i};
  }
  static constexpr int earliest(int kind) {
    return kind == B0 ? 5 : kind == B1 ? 9 : kind == H0 ? 9 : kind == B2 ? 13 : 0;
  }
  static constexpr int tick(int i) {
    const int u = i * TK / NG, e = earliest(item(i).kind);
    return u > e ? u : e;
  }
  static constexpr int first(int t) {  // first item at tick >= t
    int i = 0;
    while (i < NG && tick(i) < t) ++i;
    return i;
  }
};

// Pipeline variants (measured): kDeep synchronises at tick SYNC and loads
// tile j + 3 (two slots of load latency) instead of synchronising at the
// start of the slot and loading tile j + 2; kSwap lets the waves of the upper
// half (the second wave on each SIMD) issue each tick's vector stages before
// its MFMAs, so that the two waves of a SIMD start a tick on different units.
constexpr bool kDeep = false;
constexpr bool kSwap = false;
// Operand reads are issued kLead MFMAs ahead of the MFMA that consumes them.
constexpr int kLead = 2;
// kSpread: in the steady state each wave issues its loads of the next tile
// one at a time over the slot's ticks instead of all after the barrier.
constexpr bool kSpread = true;


template <typename T, int D, bool CAUSAL, bool DS, bool OFF32>
__global__ __launch_bounds__(512, 1) void ssa_bwd_dkdv2w_kernel(BwdParams p) {
  typedef typename Vec8<T>::type v8;
  typedef T v4 __attribute__((ext_vector_type(4)));
  using Loads = Dkdv2wLoads<D, CAUSAL, OFF32, kSpread>;
  using Plan = typename Loads::Plan;
  constexpr int NW = Loads::NW, KW = Loads::KW, NB = Loads::NB;
  using SC = Sched2w<D>;
  using TL = Swz8Tile<D>;
  constexpr int NKS = SC::NKS, NDB = SC::NDB;
  constexpr int TILE = TL::TILE;
  static_assert(TILE == Loads::TILE, "tile size");
  __shared__ __attribute__((aligned(1024))) char smem[Loads::LDS_BYTES];
  __shared__ float red[2][NW];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, i16 = lane & 15;
  // dispatch and step order (ssa_plan.hpp)
  const Plan pl(p, blockIdx.x, gridDim.x);
  const int nkb = pl.nkb, bhk = pl.bhk, kb = pl.kb, b = pl.b, hk = pl.hk, G = pl.G, N = pl.N;
  const SeqView& sv = pl.sv;
  if (pl.empty()) {  // packed: past the end of a shorter document
    if (tid == 0) {
      const int64_t P = static_cast<int64_t>(p.B) * p.Hkv * nkb;
      p.partials[static_cast<int64_t>(bhk) * nkb + kb] = 0.f;
      p.partials[P + static_cast<int64_t>(bhk) * nkb + kb] = 0.f;
    }
    return;
  }
  const float n = *p.n_ptr, bv = *p.b_ptr;
  const float c = p.scale * bv;
  const uint32_t lds0 = lds_addr(smem);

  const int k0 = pl.k0;
  const int k0w = k0 + wave * KW;
  const int key = k0w + i16;
  const T* kg = static_cast<const T*>(p.k.ptr) + sv.off(p.k, b) + hk * p.k.sh;
  const T* vg = static_cast<const T*>(p.v.ptr) + sv.off(p.v, b) + hk * p.v.sh;

  const int nsteps = pl.nsteps;
  const int per_m = pl.per_m, per_u = pl.per_u, nmasked = pl.nmasked;
  auto bufof = [&](int st) { return Loads::buf(lds0, st); };

  StepWalk wi(nmasked), wc(nmasked);
  // Q / dO / M / Delta loads of a step (ssa_plan.hpp); in the steady state
  // (kSpread) issue() only prepares a tile and issue_piece<K>() issues its
  // loads one at a time.
  Loads ld(p, pl, wave, lane);
  auto issue = [&](int st, const StepWalk& w) { ld.issue(pl, st, w, lds0); };
  // vector-memory operations per wave and tile that the waits below count:
  // Q and dO pieces (D = 32: one of the two), M, Delta
  constexpr int LPT = Loads::LPT;
  constexpr int NLD = Loads::NLD;
  auto issue_piece = [&](auto kc) { ld.template issue_piece<decltype(kc)::value>(N); };
  // deferred loads of the prologue's tiles are issued at once
  auto issue_all = [&](int st, const StepWalk& w) {
    issue(st, w);
    [&]<int... k>(std::integer_sequence<int, k...>) {
      (issue_piece(std::integral_constant<int, k>{}), ...);
    }(std::make_integer_sequence<int, NLD>{});
  };
  auto loads_of = [&](int st) { return st < nsteps ? LPT : 0; };
  // tiles 0 .. 2 (kDeep) or 0 .. 1 in flight
  constexpr int AHEAD = kDeep ? 3 : 2;
#pragma unroll
  for (int t = 0; t < AHEAD; ++t) {
    issue_all(t, wi);
    wi.next(per_m, per_u, G);
  }

  // K / V fragments (B operands of S / dP): key i16, columns 8 (4 ks + sg) ..
  const int sg = 2 * (g4 & 1) + (g4 >> 1);
  v8 kf[NKS], vf[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    const int col = 8 * (4 * ks + sg);
    kf[ks] = key < N ? load16<v8>(kg + key * p.k.ss + col) : zero8<v8>();
    vf[ks] = key < N ? __builtin_bit_cast(v8, __builtin_bit_cast(u32x4, load16<v8>(vg + key * p.v.ss + col)) ^
                                                  u32x4{0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u})
                     : zero8<v8>();
  }
  // The first slot runs dV/dK of "step -1" with zero P / dS' operands on
  // buffer NB - 1 (filled first at slot 0's synchronisation, after those
  // reads): zero its Q / dO tiles so that the products add exact zeros.
  {
    const uint32_t z = bufof(NB - 1);
#pragma unroll
    for (int o = tid * 16; o < 2 * TILE; o += 512 * 16)
      *(__attribute__((address_space(3))) u32x4*)(uintptr_t)(z + o) = u32x4{0u, 0u, 0u, 0u};
  }

  f32x4_t dk[NDB], dv[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) dk[i] = dv[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float dn_acc = 0.f, dn_c = 0.f, db_acc = 0.f, db_c = 0.f;
  f32x4_t s[4], dp[4];  // S and Delta - dP, one 4-element block per qb
  v8 pa[2], sa[2];      // P^T, -dS'^T operands per query half
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = dp[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int h = 0; h < 2; ++h) pa[h] = sa[h] = zero8<v8>();

  const uint32_t rowb = TL::row_base(lane), trb = TL::tr_base(lane);
  const uint32_t mlane = static_cast<uint32_t>(16 * g4);  // M / Delta rows 16 qb + 4 g ..

  auto kahan = [&](float tdn, float tdb) {
    const float y = tdn - dn_c, t = dn_acc + y;
    dn_c = (t - dn_acc) - y;
    dn_acc = t;
    const float y2 = tdb - db_c, t2 = db_acc + y2;
    db_c = (t2 - db_acc) - y2;
    db_acc = t2;
  };

  // dS' workspace: this wave's key tile k0w / 16 of query tiles qt (the
  // stored layout is the lane layout of sa[h]: lane 16 g + i holds key i,
  // queries 16 t + 4 g + (0..3) in elements 4 t ..).
  const Dkdv2wDsStores<CAUSAL, OFF32> dss(p, pl, k0w, lane);
  // Stores of step (g, q0), tiles hq = 0, 1 with mask bits `which`.
  auto ds_store = [&](int g, int q0, int which) {
#pragma unroll
    for (int hq = 0; hq < 2; ++hq)
      if (which & (1 << hq)) dss.store(g, q0, hq, __builtin_bit_cast(u32x4, sa[hq]));
  };
  auto ds_which = [&](int q0) { return dss.which(q0); };

  // ---- one slot: element pipeline of step j, MFMAs of steps j - 1, j, j + 1 ----
  // The workgroup synchronises once per slot, at tick SYNC: every wave is then
  // past its reads of tile j - 1 (the H1 products, ticks before SYNC), whose
  // buffer takes tile j + 3, and tile j + 1 (first read at SYNC, by the operand
  // reads of B0) has landed: issued two slots earlier, at the previous slot's
  // SYNC but one.  `npend` = the vector-memory operations this wave issued
  // after tile j + 1's loads (the dS' stores of slots j - 2 and j - 1 and the
  // loads of tile j + 2), which may stay in flight.  Returns the number of dS'
  // tiles stored.
  constexpr int SYNC = kDeep ? SC::tick(SC::NH + SC::NBK - kLead) : 0;
  static_assert(!kDeep || (SC::NH + SC::NBK >= kLead && SC::tick(SC::NH - 1) < SYNC),
                "tile j - 1 is read only before the synchronisation");
  auto slot = [&](int j, auto masked_tag, auto swap_tag, int npend) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool SWAP = decltype(swap_tag)::value;
    const int gq = wc.g;
    const int q0 = pl.template q0<false>(wc);
    const int qm = q0 + 4 * g4;  // query of element e: qm + 16 (e >> 2) + (e & 3)
    const uint32_t bprev = bufof(j - 1), bcur = bufof(j), bnext = bufof(j + 1);
    const uint32_t tr_prev = opaque(bprev + trb), tr_cur = opaque(bcur + trb);
    const uint32_t row_cur = opaque(bcur + rowb), row_next = opaque(bnext + rowb);
    const uint32_t m_cur = bcur + 2 * TILE + mlane;
    const uint32_t d_cur = m_cur + 256, d_next = bnext + 2 * TILE + 256 + mlane;

    constexpr int R = kLead + 1;  // operand ring
    v8 ops[R];
    // Delta rows of a dP block, read with its first operand: not into dp[qb]
    // itself, which the element pipeline may still read in that tick
    f32x4_t dinit[4];
    // operand of item I (read two items ahead of its MFMA)
    auto read = [&](auto ic) {
      constexpr int I = decltype(ic)::value;
      if constexpr (I < SC::NG) {
        constexpr auto it = SC::item(I);
        if constexpr (it.kind == SC::H1 || it.kind == SC::H0) {
          constexpr int h = it.kind == SC::H1 ? 1 : 0, db = it.k / 2, t = it.k % 2;
          const uint32_t base = (it.kind == SC::H1 ? tr_prev : tr_cur) + (t == 0 ? TILE : 0);  // dV reads dO
          const v4 lo = lds_tr4<v4>(base + TL::tr_imm(h, db, 0));
          const v4 hi = lds_tr4<v4>(base + TL::tr_imm(h, db, 1));
          ops[I % R] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        } else {
          constexpr int qb = it.kind == SC::B3 ? 3 : it.kind == SC::B0 ? 0 : it.kind == SC::B1 ? 1 : 2;
          constexpr int ks = it.k / 2, t = it.k % 2;
          const uint32_t base = (it.kind == SC::B3 ? row_cur : row_next) + (t == 1 ? TILE : 0);  // dP reads dO
          ops[I % R] = lds_v8<v8>(base + TL::row_imm(qb, ks));
          if constexpr (t == 1 && ks == 0)  // dP accumulator starts from Delta
            dinit[qb] = lds_read_f4((it.kind == SC::B3 ? d_cur : d_next) + 64 * qb);
        }
      }
    };
    auto mfma = [&](auto ic) {
      constexpr int I = decltype(ic)::value;
      constexpr auto it = SC::item(I);
      if constexpr (it.kind == SC::H1 || it.kind == SC::H0) {
        constexpr int h = it.kind == SC::H1 ? 1 : 0, db = it.k / 2, t = it.k % 2;
        if constexpr (t == 0)
          dv[db] = mfma16(pa[h], ops[I % R], dv[db]);
        else
          dk[db] = mfma16(sa[h], ops[I % R], dk[db]);
      } else {
        constexpr int qb = it.kind == SC::B3 ? 3 : it.kind == SC::B0 ? 0 : it.kind == SC::B1 ? 1 : 2;
        constexpr int ks = it.k / 2, t = it.k % 2;
        if constexpr (t == 0)
          s[qb] = mfma16(ops[I % R], kf[ks], ks == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : s[qb]);
        else
          dp[qb] = mfma16(ops[I % R], vf[ks], ks == 0 ? dinit[qb] : dp[qb]);
      }
    };

    // element pipeline: A(e) at tick e - 2, B(e) at e - 1, C1(e) at e, C2(e) at e + 1
    float Lv[16], rv[16], slv[16], pv[16], dtv[16], dsv[16];
    f32x4_t mq[4];
    float tdn = 0.f, tdb = 0.f;
    auto A = [&](int e) {
      const float x = s[e >> 2][e & 3];
      const float u1 = fmaf(c, fabsf(x), 1.f);
      Lv[e] = fast_log2(u1);
      rv[e] = fast_rcp(u1);
      pin(Lv[e]);
      pin(rv[e]);
    };
    auto B = [&](int e) {
      const float x = s[e >> 2][e & 3];
      slv[e] = copysignf(Lv[e], x);
      pv[e] = fast_exp2(fmaf(n, slv[e], -mq[e >> 2][e & 3]));
      if constexpr (MASKED) {
        const int qi = qm + 16 * (e >> 2) + (e & 3);
        const bool valid = qi < N && key < N && (!CAUSAL || key <= qi);
        pv[e] = valid ? pv[e] : 0.f;
      }
      pin(pv[e]);
    };
    auto C1 = [&](int e) {
      dtv[e] = pv[e] * dp[e >> 2][e & 3];
      dsv[e] = dtv[e] * rv[e];
      pin(dtv[e]);
      pin(dsv[e]);
    };
    auto C2 = [&](int e) {
      tdn = fmaf(dtv[e], slv[e], tdn);
      tdb = fmaf(dsv[e], s[e >> 2][e & 3], tdb);
      pin(tdn);
      pin(tdb);
      if (e & 1) {
        pa[e >> 3][(e & 7) - 1] = static_cast<T>(pv[e - 1]);
        pa[e >> 3][e & 7] = static_cast<T>(pv[e]);
        sa[e >> 3][(e & 7) - 1] = static_cast<T>(dsv[e - 1]);
        sa[e >> 3][e & 7] = static_cast<T>(dsv[e]);
      }
    };
    auto tick = [&](auto tc) {
      constexpr int t = decltype(tc)::value;
      constexpr int I0 = SC::first(t), I1 = SC::first(t + 1);
      if constexpr (t == SYNC) {
        wait_vm_dyn(npend);
        __builtin_amdgcn_s_barrier();
        issue(j + AHEAD, wi);
        wi.next(per_m, per_u, G);
      }
      // the deferred loads of that tile, one every other tick after it
      if constexpr (t > SYNC && (t - SYNC) % 2 == 1 && (t - SYNC) / 2 < NLD) {
        issue_piece(std::integral_constant<int, (t - SYNC) / 2>{});
      }
      auto products = [&]() {
        [&]<int... k>(std::integer_sequence<int, k...>) {
          ((read(std::integral_constant<int, I0 + k + kLead>{}), mfma(std::integral_constant<int, I0 + k>{})), ...);
        }(std::make_integer_sequence<int, I1 - I0>{});
      };
      // (stages first is always legal: it only moves the products later)
      if constexpr (!SWAP) products();
      // M of block qb two ticks before its first B stage (tick 4 qb - 1)
      if constexpr (t % 4 == 1 && t + 3 < 16) mq[(t + 3) >> 2] = lds_read_f4(m_cur + 64 * ((t + 3) >> 2));
      if (t + 2 < 16) A(t + 2);
      if (t + 1 < 16) B(t + 1);
      C1(t);
      if (t >= 1) C2(t - 1);
      if constexpr (SWAP) products();
      __builtin_amdgcn_sched_barrier(0);
    };
    mq[0] = lds_read_f4(m_cur);
    [&]<int... k>(std::integer_sequence<int, k...>) {
      (read(std::integral_constant<int, k>{}), ...);
    }(std::make_integer_sequence<int, kLead>{});
    A(0);
    A(1);
    B(0);
    __builtin_amdgcn_sched_barrier(0);
    [&]<int... t>(std::integer_sequence<int, t...>) {
      (tick(std::integral_constant<int, t>{}), ...);
    }(std::make_integer_sequence<int, SC::TK>{});
    // items past the last tick (none with the current schedule)
    [&]<int... k>(std::integer_sequence<int, k...>) {
      ((read(std::integral_constant<int, SC::first(SC::TK) + k + kLead>{}),
        mfma(std::integral_constant<int, SC::first(SC::TK) + k>{})), ...);
    }(std::make_integer_sequence<int, SC::NG - SC::first(SC::TK)>{});
    C2(15);
    kahan(tdn, tdb);
    // deferred loads the ticks did not reach (before the dS' stores, which
    // the next slot's wait count assumes come last)
    constexpr int LEFT = (14 - SYNC) / 2 + 1;  // first load with no tick (tick SYNC + 2 K + 1 > 15)
    [&]<int... k>(std::integer_sequence<int, k...>) {
      (issue_piece(std::integral_constant<int, LEFT + k>{}), ...);
    }(std::make_integer_sequence<int, (NLD > LEFT ? NLD - LEFT : 0)>{});
    int stored = 0;
    if constexpr (DS) {
      if constexpr (MASKED) {
        const int which = ds_which(q0);
        ds_store(gq, q0, which);
        stored = __builtin_popcount(which);
      } else {
        ds_store(gq, q0, 3);
        stored = 2;
      }
    }
    wc.next(per_m, per_u, G);
    return stored;
  };

  // prologue: tile 0 landed (tiles 1 and 2 may be in flight); S / dP blocks
  // 0-2 of step 0
  wait_vm_dyn(kDeep ? loads_of(1) + loads_of(2) : loads_of(1));
  __syncthreads();  // also orders the zeroed buffer before any read of it
  {
    const uint32_t row0 = opaque(bufof(0) + rowb);
    const uint32_t d0 = bufof(0) + 2 * TILE + 256 + mlane;
#pragma unroll
    for (int qb = 0; qb < 3; ++qb) {
      dp[qb] = lds_read_f4(d0 + 64 * qb);
      s[qb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        s[qb] = mfma16(lds_v8<v8>(row0 + TL::row_imm(qb, ks)), kf[ks], s[qb]);
        dp[qb] = mfma16(lds_v8<v8>(row0 + TILE + TL::row_imm(qb, ks)), vf[ks], dp[qb]);
      }
    }
  }
  int s1 = 0, s2 = 0;  // dS' stores of slots j - 1 and j - 2
  int j = 0;
  // vector-memory operations issued after tile j + 1's loads
  auto pending = [&](int j) { return kDeep ? s2 + loads_of(j + 2) + s1 : s1; };
  auto run = [&](int jend, auto masked_tag) __attribute__((always_inline)) {
    for (; j < jend; ++j) {
      int st;
      if (kSwap && wave >= NW / 2)
        st = slot(j, masked_tag, std::true_type{}, pending(j));
      else
        st = slot(j, masked_tag, std::false_type{}, pending(j));
      s2 = s1;
      s1 = st;
    }
  };
  run(min(nmasked, nsteps), std::true_type{});
  run(nsteps, std::false_type{});
  // drain: dV/dK of the last step's second query half
  wait_vm<0>();
  {
    const uint32_t tr_last = opaque(bufof(nsteps - 1) + trb);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const v4 dlo = lds_tr4<v4>(tr_last + TILE + TL::tr_imm(1, db, 0));
      const v4 dhi = lds_tr4<v4>(tr_last + TILE + TL::tr_imm(1, db, 1));
      const v4 qlo = lds_tr4<v4>(tr_last + TL::tr_imm(1, db, 0));
      const v4 qhi = lds_tr4<v4>(tr_last + TL::tr_imm(1, db, 1));
      dv[db] = mfma16(pa[1], __builtin_shufflevector(dlo, dhi, 0, 1, 2, 3, 4, 5, 6, 7), dv[db]);
      dk[db] = mfma16(sa[1], __builtin_shufflevector(qlo, qhi, 0, 1, 2, 3, 4, 5, 6, 7), dk[db]);
    }
  }

  // dK (scaled by scale n b; the accumulator holds -dK_raw) and dV: lane
  // 16 g + i holds column 16 db + i of keys k0w + 4 g + (0..3); staged as
  // whole rows in the wave's 16-row scratch of the (now idle) ring.
  __syncthreads();
  {
    const uint32_t tile = lds0 + wave * (16 * D * 2);
    auto slot_row = [&](int r) { return tile + r * (D * 2); };
    T* dkr = static_cast<T*>(const_cast<void*>(p.dk.ptr)) + sv.off(p.dk, b) + hk * p.dk.sh;
    T* dvr = static_cast<T*>(const_cast<void*>(p.dv.ptr)) + sv.off(p.dv, b) + hk * p.dv.sh;
    const int64_t k0r = static_cast<int64_t>(min(k0w, N - 1));
    const float kscale = -(p.scale * n * bv);
#pragma unroll
    for (int which = 0; which < 2; ++which) {
      const f32x4_t* acc = which == 0 ? dk : dv;
      const float sc = which == 0 ? kscale : 1.f;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g4 + e;
          *(__attribute__((address_space(3))) T*)(uintptr_t)(slot_row(r) + stage_off<D>(r, 16 * db + i16)) =
              static_cast<T>(acc[db][e] * sc);
        }
      T* dst = which == 0 ? dkr + k0r * p.dk.ss : dvr + k0r * p.dv.ss;
      const int64_t ss = which == 0 ? p.dk.ss : p.dv.ss;
      stage_to_rows<T, D, 16>(slot_row, dst, ss, N - k0w, lane);
    }
  }

  // dn / db partial of this workgroup: lane butterfly, then waves in order.
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
    const int64_t P = static_cast<int64_t>(p.B) * p.Hkv * nkb;
    const float sdn = ((red[0][0] + red[0][1]) + (red[0][2] + red[0][3])) +
                      ((red[0][4] + red[0][5]) + (red[0][6] + red[0][7]));
    const float sdb = ((red[1][0] + red[1][1]) + (red[1][2] + red[1][3])) +
                      ((red[1][4] + red[1][5]) + (red[1][6] + red[1][7]));
    p.partials[static_cast<int64_t>(bhk) * nkb + kb] = -kLn2 * sdn;
    p.partials[P + static_cast<int64_t>(bhk) * nkb + kb] = -(n * p.scale) * sdb;
  }
}

template <typename T, int D, bool CAUSAL>
static hipError_t dkdv2w_t(const BwdParams& p, bool off32, hipStream_t s) {
  const int grid = DkdvPlan<128, 64, CAUSAL>::grid(p);
  if (p.ds != nullptr) {
    if (off32)
      hipLaunchKernelGGL((ssa_bwd_dkdv2w_kernel<T, D, CAUSAL, true, true>), dim3(grid), dim3(512), 0, s, p);
    else
      hipLaunchKernelGGL((ssa_bwd_dkdv2w_kernel<T, D, CAUSAL, true, false>), dim3(grid), dim3(512), 0, s, p);
  } else {
    if (off32)
      hipLaunchKernelGGL((ssa_bwd_dkdv2w_kernel<T, D, CAUSAL, false, true>), dim3(grid), dim3(512), 0, s, p);
    else
      hipLaunchKernelGGL((ssa_bwd_dkdv2w_kernel<T, D, CAUSAL, false, false>), dim3(grid), dim3(512), 0, s, p);
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t dkdv2w_dt(const BwdParams& p, int D, bool causal, bool off32, hipStream_t s) {
  switch (D) {
    case 32: return causal ? dkdv2w_t<T, 32, true>(p, off32, s) : dkdv2w_t<T, 32, false>(p, off32, s);
    case 64: return causal ? dkdv2w_t<T, 64, true>(p, off32, s) : dkdv2w_t<T, 64, false>(p, off32, s);
    case 128: return causal ? dkdv2w_t<T, 128, true>(p, off32, s) : dkdv2w_t<T, 128, false>(p, off32, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_bwd_dkdv2w(const BwdParams& p, int dtype, int D, bool causal, bool off32, hipStream_t s) {
  return dtype == 0 ? dkdv2w_dt<__bf16>(p, D, causal, off32, s) : dkdv2w_dt<_Float16>(p, D, causal, off32, s);
}

}  // namespace ssa
