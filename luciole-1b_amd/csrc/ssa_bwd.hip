// SSA attention backward for gfx950: Delta preprocess, dK/dV (+ dn/db
// partials), dQ, and the fixed-order dn/db reduction.
//
// Replaces _ssa_attn_bwd_preprocess, _ssa_attn_bwd_dkdv, _ssa_attn_bwd_dq and
// _ssa_attn_bwd (training/train/train_ssa_triton/SSA/ssa_triton_kernel.py:
// 267-298, 305-401, 408-481, 488-719) and the dn_partial/db_partial sums
// (:894-895).  As in the reference, dQ is produced by its own pass, so no
// floating-point atomics are needed anywhere and the results are bitwise
// reproducible: either recomputing the scores (the reference's way) or, with
// a dS' workspace written by dK/dV, as a streaming product dS' K.
//
// Per valid (query i, key j), with s = scale * q_i.k_j, u = b|s|,
// sL = sign(s) log2(1+u) and M_i the base-2 normaliser saved by the forward:
//   P   = exp2(n sL - M_i)
//   dT  = P (dP - Delta_i)              dP = dO_i . v_j
//   dS' = dT / (1 + u)                  (dS = n b dS')
//   dV_j += P dO_i,  dK_j += scale n b dS' q_i,  dQ_i += scale n b dS' k_j
//   dn  += ln2 * dT sL,  db += n scale dS' (q_i.k_j)
// The constant factors (scale n b, ln2, n scale) are applied once at the end.
#include <stdlib.h>

#include <type_traits>

#include "ssa_common.hpp"
#include "ssa_launch.hpp"
#include "ssa_plan.hpp"
#include "ssa_tile.hpp"

namespace ssa {

// ---------------------------------------------------------------------------
// Delta_i = sum_d O_id dO_id (fp32).  HBM-bound: one 16-byte load of O and dO
// per lane, D/8 lanes per row, butterfly reduction inside the row group.
template <typename T, int D>
__global__ __launch_bounds__(256) void ssa_bwd_preprocess_kernel(BwdParams p) {
  constexpr int LPR = D / 8;         // lanes per row
  constexpr int RPB = 256 / LPR;     // rows per block
  typedef typename Vec8<T>::type v8;
  const int tid = threadIdx.x;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + tid / LPR;
  const int sub = tid % LPR;
  const int64_t total = static_cast<int64_t>(p.B) * p.Hq * p.N;
  float acc = 0.f;
  if (row < total) {
    const int s = static_cast<int>(row % p.N);
    const int64_t bh = row / p.N;
    const int h = static_cast<int>(bh % p.Hq), b = static_cast<int>(bh / p.Hq);
    const T* o = static_cast<const T*>(p.o.ptr) + b * p.o.sb + h * p.o.sh + s * p.o.ss + sub * 8;
    const T* g = static_cast<const T*>(p.dout.ptr) + b * p.dout.sb + h * p.dout.sh + s * p.dout.ss + sub * 8;
    const v8 ov = load16<v8>(o), gv = load16<v8>(g);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fmaf(static_cast<float>(ov[e]), static_cast<float>(gv[e]), acc);
  }
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (row < total && sub == 0) p.delta[row] = acc;
}

// ---------------------------------------------------------------------------
// dK, dV for a block of 128 keys (32 per wave) of one (batch, kv-head), looping
// over every q-head of the GQA group and every 32-query sub-tile at or after
// the keys (causal).  S = Q K^T is computed with the keys on the lane axis, so
// P^T and dS'^T come out of the accumulators already in A-operand order for
// dV += P^T dO and dK += dS'^T Q; the B operands (dO, Q with the query index
// as the contraction dimension) are LDS transpose reads of the same sub-tiles
// the S and dP products read row-wise.  K and V stay in registers, dK and dV
// accumulate in AGPRs.
//
// Sign convention: the V fragments are held negated and the dP product starts
// from Delta instead of zero, so its accumulator is Delta - dP = -(dP - Delta)
// with no vector instruction per element; every per-pair quantity derived
// from it (dT, dS', the dn / db terms) is therefore the negated one, and the
// sign is restored where those sums leave the kernel (the dK scale, the dn / db
// partials, and the dS' workspace, which holds -dS' for the dQ pass).
//
// Software pipeline, one slot per sub-tile: slot j issues the MFMAs of
// dV/dK for sub-tile j - 1 and of S/dP for sub-tile j + 1, and the vector
// work of sub-tile j (SSA transform, P, dS', dn/db sums).  The two streams are
// independent inside a slot; in the steady state they are interleaved in 32
// fenced ticks (one MFMA with its operand reads and a slice of a three-stage
// element pipeline per tick), so the wave keeps the matrix unit busy while it
// issues vector work.  Sub-tiles (Q, dO, M, Delta) live in four LDS buffers:
// sub-tile t is loaded in slot t - 2 (its buffer last held t - 4, read for
// the last time in slot t - 3) and complete at the start of slot t - 1.
// The step order and walk: DkdvPlan / StepWalk (ssa_plan.hpp).

// Store one wave's 32 keys x D block of dK or dV: the lane holds d = 32 db +
// l32 of key rows k0w + crow(r, hh).  The block goes through the wave's own
// LDS tile `tile` ([d][key], 72-byte rows) so that every lane stores 8 bytes
// (4 consecutive d of one key) per instruction.  Write: lane (l32, hh), keys
// 8 a + 4 hh .. + 3 of row d.  Transposed read t: in 16-lane group g, lane
// 4 e + q supplies row 8 t + 4 (g >> 1) + e, keys 16 (g & 1) + 4 q .. + 3, so
// lane 16 g + i receives key 16 (g & 1) + i, d = 8 t + 4 (g >> 1) + (0..3).
// `rows` is row 0 of the (sequence, kv-head) slice, `ss` its row stride.
template <typename T, int D>
__device__ __forceinline__ void store_key_block(const f32x16* acc, float scale, T* rows, int64_t ss, int k0w, int N,
                                                uint32_t tile, int lane) {
  typedef T v4 __attribute__((ext_vector_type(4)));
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  constexpr int RS = 72, ND32 = D / 32;
  const int l32 = lane & 31, hh = lane >> 5;
  const uint32_t wr0 = tile + l32 * RS + hh * 8;
  const int g16 = lane >> 4, s16 = lane & 15;
  const uint32_t rd0 = tile + (4 * (g16 >> 1) + (s16 >> 2)) * RS + (16 * (g16 & 1) + 4 * (s16 & 3)) * 2;
  const int okey = k0w + 16 * (g16 & 1) + s16;
  const int od0 = 4 * (g16 >> 1);
#pragma unroll
  for (int db = 0; db < ND32; ++db) {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      v4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = static_cast<T>(acc[db][4 * a + e] * scale);
      *(__attribute__((address_space(3))) v4*)(uintptr_t)(wr0 + db * 32 * RS + a * 16) = w;
    }
  }
  T* row = rows + static_cast<int64_t>(min(okey, N - 1)) * ss + od0;
#pragma unroll
  for (int i = 0; i < D / 8; ++i) {
    const v4 r = __builtin_bit_cast(v4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                                            (__attribute__((address_space(3))) bf16x4_t*)(uintptr_t)(rd0 + i * 8 * RS)));
    if (okey < N) *reinterpret_cast<v4*>(row + 8 * i) = r;
  }
}
// Byte size of one wave's LDS scratch for its dK / dV rows: the [d][key]
// tile above, or 32 whole key rows (store_cols_via_lds, ssa_tile.hpp).
template <int D>
constexpr int key_block_tile_bytes() {
  return D * 72 > 32 * D * 2 ? D * 72 : 32 * D * 2;
}

// OFF32: every Q / dO row a workgroup reads lies below 2 GiB of its base
// (q-head hk G of the sequence), and so does its dS' range (checked on the
// host): the per-slot loads and stores then take 32-bit scalar offsets into
// loop-invariant buffer descriptors instead of 64-bit address arithmetic.
template <typename T, int D, bool CAUSAL, bool DS, bool OFF32>
__global__ __launch_bounds__(256, 1) void ssa_bwd_dkdv_kernel(BwdParams p) {
  typedef typename Vec8<T>::type v8;
  typedef T v4 __attribute__((ext_vector_type(4)));
  using Loads = DkdvLoads<D, CAUSAL, OFF32>;
  using Plan = typename Loads::Plan;
  constexpr int BMQ = Loads::BMQ;
  constexpr int ND16 = D / 16, ND32 = D / 32;
  constexpr int TILE = Loads::TILE;  // one Q (or dO) sub-tile
  __shared__ __attribute__((aligned(1024))) char smem[Loads::LDS_BYTES];
  __shared__ float red[2][4];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
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
  // n and b read once here: a read after the main loop would queue behind its
  // memory traffic and hold the workgroup's end for the round trip
  const float n = *p.n_ptr, bv = *p.b_ptr;
  const float c = p.scale * bv;
  const uint32_t lds0 = lds_addr(smem);
  const RowBase<D> rb(l32, hh);
  const TrBase<D> tb(lane);

  const int k0 = pl.k0;
  const int k0w = k0 + wave * 32;
  const int key = k0w + l32;
  const T* kg = static_cast<const T*>(p.k.ptr) + sv.off(p.k, b) + hk * p.k.sh;
  const T* vg = static_cast<const T*>(p.v.ptr) + sv.off(p.v, b) + hk * p.v.sh;

  const int qstart = pl.qstart, nsub = pl.nsub, nsteps = pl.nsteps, nlo = pl.nlo;
  const int per_m = pl.per_m, per_u = pl.per_u, nmasked = pl.nmasked;
  auto step_q0 = [&](int st, int& g) { return pl.step_q0(st, g); };
  // a masked step whose queries all precede this wave's keys (or no keys)
  auto skipped = [&](int st) { return pl.skipped(st, k0w); };
  auto bufof = [&](int st) { return Loads::buf(lds0, st); };

  // walkers at the next step to load (j + 2) and at the current step j
  StepWalk wi(nmasked), wc(nmasked);
  // Q / dO / M / Delta loads of a step (ssa_plan.hpp): per-workgroup address
  // bases (q-head hk * G), so a slot's loads add only the q-head and row
  // offsets (a fifth fewer instructions per fast slot).
  const Loads ld(p, pl, wave, lane);
  auto issue = [&](int st, const StepWalk& w, auto unmasked_tag) {
    ld.template issue<decltype(unmasked_tag)::value>(pl, st, w, lds0);
  };
  issue(0, wi, std::false_type{});
  wi.next(per_m, per_u, G);
  issue(1, wi, std::false_type{});
  wi.next(per_m, per_u, G);

  v8 kf[ND16], vf[ND16];
#pragma unroll
  for (int ds = 0; ds < ND16; ++ds) {
    kf[ds] = key < N ? load16<v8>(kg + key * p.k.ss + ds * 16 + 8 * hh) : zero8<v8>();
    // negated V: flip the sign bit of every 16-bit element
    vf[ds] = key < N ? __builtin_bit_cast(v8, __builtin_bit_cast(u32x4, load16<v8>(vg + key * p.v.ss + ds * 16 + 8 * hh)) ^
                                                  u32x4{0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u})
                     : zero8<v8>();
  }

  f32x16 dk[ND32], dv[ND32];  // accumulation registers: mfma32_acc / acc_fence only
#pragma unroll
  for (int i = 0; i < ND32; ++i) {
    dk[i] = f32x16{};
    dv[i] = f32x16{};
  }
  float dn_acc = 0.f, dn_c = 0.f, db_acc = 0.f, db_c = 0.f;
  // S, dP of sub-tiles j and j + 1.  Zero-initialised: a skipped step leaves
  // them as they were, and the masked fast slot multiplies their entries by a
  // zero P, which must stay zero (finite operands).
  // Two sets of each, used alternately by consecutive fast slots so that the
  // steady state moves nothing between registers; the generic slot and the
  // ends of the fast runs use set 0 as current (sc, dc, pa, sa) and set 1 as
  // next (sn, dn2, pa2, sa2), and rotate() copies next into current.
  f32x16 s_set[2] = {f32x16{}, f32x16{}}, d_set[2] = {f32x16{}, f32x16{}};
  v8 p_set[2][2], a_set[2][2];  // P^T, dS'^T operands of sub-tiles j - 1 and j
  f32x16 &sc = s_set[0], &sn = s_set[1], &dc = d_set[0], &dn2 = d_set[1];
  v8(&pa)[2] = p_set[0];
  v8(&pa2)[2] = p_set[1];
  v8(&sa)[2] = a_set[0];
  v8(&sa2)[2] = a_set[1];

  auto kahan = [&](float tdn, float tdb) {
    const float y = tdn - dn_c, t = dn_acc + y;
    dn_c = (t - dn_acc) - y;
    dn_acc = t;
    const float y2 = tdb - db_c, t2 = db_acc + y2;
    db_c = (t2 - db_acc) - y2;
    db_acc = t2;
  };

  // ---- generic pieces (masked steps, pipeline fill and drain) ----
  // Delta of the 16 query rows crow(r, hh) of sub-tile st, as a dP accumulator
  auto delta_rows = [&](int st) {
    const uint32_t ml = bufof(st) + 2 * TILE + 128;
    f32x4_t d4[4];
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) d4[g4] = lds_read_f4(ml + (8 * g4 + 4 * hh) * 4);
    f32x16 r;
#pragma unroll
    for (int e = 0; e < 16; ++e) r[e] = d4[e >> 2][e & 3];
    return r;
  };
  // S and Delta - dP of sub-tile st
  auto sdp = [&](int st, f32x16& s_out, f32x16& d_out) {
    const RowBase<D> rq = at_tile(rb, bufof(st)), rd = at_tile(rb, bufof(st) + TILE);
    s_out = f32x16{};
    d_out = delta_rows(st);
#pragma unroll
    for (int ds = 0; ds < ND16; ++ds) {
      s_out = mfma32(tile_read_row<D, v8>(rq, 0, ds), kf[ds], s_out);
      d_out = mfma32(tile_read_row<D, v8>(rd, 0, ds), vf[ds], d_out);
    }
  };
  auto dvdk = [&](int st, const v8* pp, const v8* ss) {
    const TrBase<D> tq = at_tile(tb, bufof(st)), td = at_tile(tb, bufof(st) + TILE);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int db = 0; db < ND32; ++db) {
        const v4 dlo = tile_read_tr<D, v4>(td, 0, ks, 0, db);
        const v4 dhi = tile_read_tr<D, v4>(td, 0, ks, 1, db);
        const v4 qlo = tile_read_tr<D, v4>(tq, 0, ks, 0, db);
        const v4 qhi = tile_read_tr<D, v4>(tq, 0, ks, 1, db);
        mfma32_acc(dv[db], pp[ks], __builtin_shufflevector(dlo, dhi, 0, 1, 2, 3, 4, 5, 6, 7));
        mfma32_acc(dk[db], ss[ks], __builtin_shufflevector(qlo, qhi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    }
  };
  auto elementwise = [&](int st, auto masked_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    int g;
    const int q0 = step_q0(st, g);
    const uint32_t ml = bufof(st) + 2 * TILE;
    float tdn = 0.f, tdb = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4_t mv = lds_read_f4(ml + (8 * j + 4 * hh) * 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * j + e;
        const float x = sc[r];
        const float u1 = fmaf(c, fabsf(x), 1.f);
        const float sl = copysignf(fast_log2(u1), x);
        float pv = fast_exp2(fmaf(n, sl, -mv[e]));
        if (MASKED) {
          const int qi = q0 + crow(r, hh);
          const bool valid = qi < N && key < N && (!CAUSAL || key <= qi);
          pv = valid ? pv : 0.f;
        }
        const float ndt = pv * dc[r];  // -dT (dc = Delta - dP)
        const float nds = ndt * fast_rcp(u1);
        tdn = fmaf(ndt, sl, tdn);
        tdb = fmaf(nds, x, tdb);
        pa2[r >> 3][r & 7] = static_cast<T>(pv);
        sa2[r >> 3][r & 7] = static_cast<T>(nds);
      }
    }
    kahan(tdn, tdb);
  };
  auto rotate = [&]() {
    sc = sn;
    dc = dn2;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      pa[ks] = pa2[ks];
      sa[ks] = sa2[ks];
    }
  };
  // -dS' of sub-tile st to the workspace (DS): this wave's 32 keys are key
  // tiles kj0 = k0w / 16 and kj0 + 1 of query tile q0 / 32 (both inside the
  // causal triangle when the sub-tile is not skipped).  Lane (l32, hh) holds
  // key l32 and, in sa2[ks], queries 16 ks + 4 hh + (0..3) (elements 0..3) and
  // 16 ks + 8 + 4 hh + (0..3) (elements 4..7): in the tile format (lane
  // 16 g + kl: key kl, queries 16 t + 4 g + (0..3) at elements 4 t ..) these
  // are four 8-byte pieces, g = hh or 2 + hh, t = ks; the two of one g are
  // adjacent, so the lane writes two 16-byte pieces.
  // workspace tile (32 x 16) of q-head hk * G + g, query tile qi, key tile k0w / 16:
  // head_tile(b, hk G) + g tiles_per_head + row_offset(qi) + k0w / 16, 512 elements each
  // Exactly two vector-memory instructions (the fast slot's load wait
  // counts them), addressed by DkdvDsStores (ssa_plan.hpp).
  const DkdvDsStores<CAUSAL, OFF32> dss(p, pl, k0w, lane);
  auto ds_store = [&](const StepWalk& w, const v8 (&s2)[2], auto unmasked_tag) {
    const int q0 = pl.template q0<decltype(unmasked_tag)::value>(w);
    dss.store(w.g, q0, __builtin_bit_cast(u32x4, s2[0]), __builtin_bit_cast(u32x4, s2[1]));
  };
  auto slot_generic = [&](int j) {
    wait_vm<0>();  // sub-tile j + 1
    __builtin_amdgcn_s_barrier();
    issue(j + 2, wi, std::false_type{});
    wi.next(per_m, per_u, G);
    if (j >= 1 && !skipped(j - 1)) dvdk(j - 1, pa, sa);
    if (j + 1 < nsteps && !skipped(j + 1)) sdp(j + 1, sn, dn2);
    if (j < nsteps && !skipped(j)) {
      if (j < nmasked)
        elementwise(j, std::true_type{});
      else
        elementwise(j, std::false_type{});
      if constexpr (DS) ds_store(wc, sa2, std::false_type{});
    } else {
      // the masked fast slot after this one runs dV/dK of step j
      // unconditionally: zero operands add nothing
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) pa2[ks] = sa2[ks] = zero8<v8>();
    }
    wc.next(per_m, per_u, G);
    rotate();
  };

  // ---- steady-state slot: sub-tiles j - 1, j, j + 1 unmasked ----
  // MASKED: the same slot over masked steps (the causal diagonal, a partial
  // last sub-tile, a key block at the sequence end): P is zeroed outside the
  // mask, every MFMA runs (a skipped step contributes zeros), and only a step
  // with a valid pair stores its dS' tile.
  // PH: which state set is current (set PH ^ 1 is next); the slot leaves the
  // next sets filled for slot j + 1, which runs with the phase flipped.
  auto slot_fast = [&](int j, auto masked_tag, auto phase_tag) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr int PH = decltype(phase_tag)::value;
    f32x16 &sc = s_set[PH], &sn = s_set[PH ^ 1], &dc = d_set[PH], &dn2 = d_set[PH ^ 1];
    v8(&pa)[2] = p_set[PH];
    v8(&pa2)[2] = p_set[PH ^ 1];
    v8(&sa)[2] = a_set[PH];
    v8(&sa2)[2] = a_set[PH ^ 1];
    constexpr int NG = 4 * ND32 + 2 * ND16;  // MFMAs per slot
    // Sub-tile j + 1 (issued in slot j - 1).  The vector-memory counter also
    // counts stores, in issue order: slot j - 1 ended with its two dS' stores
    // (an unmasked slot always stores; a masked one unless its step was
    // skipped), which may stay in flight.
    if constexpr (!DS) {
      wait_vm<0>();
    } else if constexpr (MASKED) {
      if (skipped(j - 1))
        wait_vm<0>();
      else
        wait_vm<2>();
    } else {
      wait_vm<2>();
    }
    __builtin_amdgcn_s_barrier();
    issue(j + 2, wi, std::integral_constant<bool, !MASKED>{});
    if constexpr (MASKED)
      wi.next(per_m, per_u, G);
    else
      wi.next_unmasked(per_u);
    // masked: query row of element e is qm + 8 (e >> 2) + (e & 3)
    const int qm = qstart + wc.sub(nlo, nsub) * BMQ + 4 * hh;
    const TrBase<D> tq = at_tile(tb, bufof(j - 1)), td = at_tile(tb, bufof(j - 1) + TILE);
    const RowBase<D> rq = at_tile(rb, bufof(j + 1)), rd = at_tile(rb, bufof(j + 1) + TILE);
    const uint32_t ml = bufof(j) + 2 * TILE;
    f32x4_t mq[4];
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) mq[g4] = lds_read_f4(ml + (8 * g4 + 4 * hh) * 4);
    const f32x16 dnext = delta_rows(j + 1);  // accumulator start of dP of sub-tile j + 1
    v8 ops[3];
    // MFMA g: g < 4 ND32 -> dV (even) / dK (odd) of sub-tile j - 1, pair (ks, db);
    // else S (even) / dP (odd) of sub-tile j + 1, contraction slice ds.
    auto read = [&](auto gc) {
      constexpr int Gi = decltype(gc)::value;
      if constexpr (Gi < 4 * ND32) {
        constexpr int idx = Gi / 2, ks = idx / ND32, db = idx % ND32;
        const TrBase<D>& t = (Gi % 2 == 0) ? td : tq;
        const v4 lo = tile_read_tr<D, v4>(t, 0, ks, 0, db);
        const v4 hi = tile_read_tr<D, v4>(t, 0, ks, 1, db);
        ops[Gi % 3] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      } else if constexpr (Gi < NG) {
        constexpr int h = Gi - 4 * ND32, ds = h / 2;
        ops[Gi % 3] = tile_read_row<D, v8>((h % 2 == 0) ? rq : rd, 0, ds);
      }
    };
    auto mfma = [&](auto gc) {
      constexpr int Gi = decltype(gc)::value;
      if constexpr (Gi < 4 * ND32) {
        constexpr int idx = Gi / 2, ks = idx / ND32, db = idx % ND32;
        if constexpr (Gi % 2 == 0)
          mfma32_acc(dv[db], pa[ks], ops[Gi % 3]);
        else
          mfma32_acc(dk[db], sa[ks], ops[Gi % 3]);
      } else {
        constexpr int h = Gi - 4 * ND32, ds = h / 2;
        if constexpr (h % 2 == 0)
          sn = mfma32(ops[Gi % 3], kf[ds], ds == 0 ? f32x16{} : sn);
        else
          dn2 = mfma32(ops[Gi % 3], vf[ds], ds == 0 ? dnext : dn2);
      }
    };
    // element pipeline over the 16 entries of S_j / (Delta - dP)_j
    //   A: u = 1 + c|x|, L = log2 u, 1/u
    //   B: sL = copysign(L, x), p = exp2(n sL - M)
    //   C1: -dT = p (Delta - dP), -dS' = -dT / u      C2: dn, db sums, bf16 operands
    // (the ticks below run the four stages on different elements)
    float Lv[16], rv[16], slv[16], pv[16], dtv[16], dsv[16];
    float tdn = 0.f, tdb = 0.f;
    auto A = [&](int e) {
      const float x = sc[e];
      const float u1 = fmaf(c, fabsf(x), 1.f);
      Lv[e] = fast_log2(u1);
      rv[e] = fast_rcp(u1);
      pin(Lv[e]);
      pin(rv[e]);
    };
    auto B = [&](int e) {
      const float x = sc[e];
      slv[e] = copysignf(Lv[e], x);
      pv[e] = fast_exp2(fmaf(n, slv[e], -mq[e >> 2][e & 3]));
      if constexpr (MASKED) {
        const int qi = qm + 8 * (e >> 2) + (e & 3);
        const bool valid = qi < N && key < N && (!CAUSAL || key <= qi);
        pv[e] = valid ? pv[e] : 0.f;
      }
      pin(pv[e]);
    };
    auto C1 = [&](int e) {
      dtv[e] = pv[e] * dc[e];
      dsv[e] = dtv[e] * rv[e];
      pin(dtv[e]);
      pin(dsv[e]);
    };
    auto C2 = [&](int e) {
      tdn = fmaf(dtv[e], slv[e], tdn);
      tdb = fmaf(dsv[e], sc[e], tdb);
      pin(tdn);
      pin(tdb);
      if (e & 1) {
        pa2[e >> 3][(e & 7) - 1] = static_cast<T>(pv[e - 1]);
        pa2[e >> 3][e & 7] = static_cast<T>(pv[e]);
        sa2[e >> 3][(e & 7) - 1] = static_cast<T>(dsv[e - 1]);
        sa2[e >> 3][e & 7] = static_cast<T>(dsv[e]);
      }
    };
    // TK ticks per slot; tick t issues the MFMAs G in [t NG / TK, (t + 1) NG /
    // TK), each after the operand read two MFMAs ahead, beside four
    // independent stages on EPT elements each: A(t + 2), B(t + 1), C1(t),
    // C2(t - 1) in units of EPT elements.  Sixteen ticks at D >= 64 (two
    // MFMAs per tick at D = 128, one at D = 64: at D = 64 the shorter live
    // ranges of one element per stage keep every causal instance within 256
    // registers, two waves per SIMD), eight at D = 32.
    constexpr int TK = D >= 64 ? 16 : 8, EPT = 16 / TK;
    auto tick = [&](auto tc) {
      constexpr int t = decltype(tc)::value;
      constexpr int G0 = t * NG / TK, G1 = (t + 1) * NG / TK;
      [&]<int... g>(std::integer_sequence<int, g...>) {
        ((read(std::integral_constant<int, G0 + g + 2>{}), mfma(std::integral_constant<int, G0 + g>{})), ...);
      }(std::make_integer_sequence<int, G1 - G0>{});
#pragma unroll
      for (int k = 0; k < EPT; ++k)
        if (EPT * (t + 2) + k < 16) A(EPT * (t + 2) + k);
#pragma unroll
      for (int k = 0; k < EPT; ++k)
        if (EPT * (t + 1) + k < 16) B(EPT * (t + 1) + k);
#pragma unroll
      for (int k = 0; k < EPT; ++k) C1(EPT * t + k);
#pragma unroll
      for (int k = 0; k < EPT; ++k)
        if (t >= 1) C2(EPT * (t - 1) + k);
      __builtin_amdgcn_sched_barrier(0);
    };
    read(std::integral_constant<int, 0>{});
    read(std::integral_constant<int, 1>{});
#pragma unroll
    for (int e = 0; e < 2 * EPT; ++e) A(e);
#pragma unroll
    for (int e = 0; e < EPT; ++e) B(e);
    [&]<int... t>(std::integer_sequence<int, t...>) {
      (tick(std::integral_constant<int, t>{}), ...);
    }(std::make_integer_sequence<int, TK>{});
#pragma unroll
    for (int e = 16 - EPT; e < 16; ++e) C2(e);
    kahan(tdn, tdb);
    if constexpr (DS) {
      if (!MASKED || !skipped(j)) ds_store(wc, sa2, std::integral_constant<bool, !MASKED>{});
    }
    if constexpr (MASKED)
      wc.next(per_m, per_u, G);
    else
      wc.next_unmasked(per_u);
  };

  // prologue: sub-tiles 0 and 1 in flight, S/dP of sub-tile 0
  wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  if (!skipped(0)) sdp(0, sn, dn2);
  rotate();
  // generic slot 0 (no dV/dK yet), masked fast slots while steps j - 1 .. j + 1
  // exist up to the first unmasked step (which passes every mask and always
  // stores, so every unmasked fast slot follows a storing slot), generic if
  // that step ends the sequence, unmasked fast slots, generic drain
  slot_generic(0);
  int j = 1;
  // fast slots j < jend in pairs (phases 0, 1); an odd last one ends with the
  // copy that puts its next sets in place as set 0
  auto fast_run = [&](int jend, auto masked_tag) __attribute__((always_inline)) {
    for (; j + 1 < jend; j += 2) {
      slot_fast(j, masked_tag, std::integral_constant<int, 0>{});
      slot_fast(j + 1, masked_tag, std::integral_constant<int, 1>{});
    }
    if (j < jend) {
      slot_fast(j, masked_tag, std::integral_constant<int, 0>{});
      rotate();
      ++j;
    }
  };
  fast_run(min(nmasked + 1, nsteps - 1), std::true_type{});
  for (; j <= nmasked && j <= nsteps; ++j) slot_generic(j);
  fast_run(nsteps - 1, std::false_type{});
  for (; j <= nsteps; ++j) slot_generic(j);

  // Store dK (scaled by scale * n * b; the accumulator holds -dK_raw) and dV.
  __syncthreads();  // every wave is done with the sub-tile ring (no loads in flight)
  acc_fence(dk, dv);
  {
    const uint32_t tile = lds0 + wave * key_block_tile_bytes<D>();
    T* dkr = static_cast<T*>(const_cast<void*>(p.dk.ptr)) + sv.off(p.dk, b) + hk * p.dk.sh;
    T* dvr = static_cast<T*>(const_cast<void*>(p.dv.ptr)) + sv.off(p.dv, b) + hk * p.dv.sh;
    if constexpr (D >= 128) {
      // whole key rows per store instruction through the wave's scratch (at
      // D = 128 the kernel runs one wave per SIMD with registers to spare;
      // below, the staging code's registers would cost the second wave)
      auto slot = [&](int r) { return tile + r * (D * 2); };
      const int64_t k0r = static_cast<int64_t>(min(k0w, N - 1));
      store_cols_via_lds<T, D>(dk, -(p.scale * n * bv), slot, dkr + k0r * p.dk.ss, p.dk.ss, N - k0w, lane);
      store_cols_via_lds<T, D>(dv, 1.f, slot, dvr + k0r * p.dv.ss, p.dv.ss, N - k0w, lane);
    } else {
      store_key_block<T, D>(dk, -(p.scale * n * bv), dkr, p.dk.ss, k0w, N, tile, lane);
      store_key_block<T, D>(dv, 1.f, dvr, p.dv.ss, k0w, N, tile, lane);
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
    const float sdn = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    const float sdb = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    // the per-lane sums hold -dn and -db terms
    p.partials[static_cast<int64_t>(bhk) * nkb + kb] = -kLn2 * sdn;
    p.partials[P + static_cast<int64_t>(bhk) * nkb + kb] = -(n * p.scale) * sdb;
  }
}

// ---------------------------------------------------------------------------
// dQ for 128 query rows (32 per wave) of one (batch, q-head), laid out like
// the forward (query on the lane axis): S^T = K Q^T and dP^T = V dO^T with K/V
// rows read from double-buffered LDS tiles, dQ^T += K^T dS'^T with K^T from
// LDS transpose reads of the same K tile.  Q and dO stay in registers.
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void ssa_bwd_dq_kernel(BwdParams p) {
  typedef typename Vec8<T>::type v8;
  typedef T v4 __attribute__((ext_vector_type(4)));
  using Plan = DqPlan<D, CAUSAL>;
  constexpr int BM = Plan::BM, BN = Plan::BN;
  constexpr int ND16 = D / 16, ND32 = D / 32;
  constexpr int TILE_BYTES = Plan::TILE;
  __shared__ __attribute__((aligned(1024))) char smem[Plan::LDS_BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  // dispatch and K / V tile loads (ssa_plan.hpp)
  const Plan pl(p, blockIdx.x, gridDim.x);
  if (pl.empty()) return;  // packed: past the end of a shorter document
  const int qb = pl.qb, b = pl.b, h = pl.h, N = pl.N;
  const SeqView& sv = pl.sv;
  const uint32_t lds0 = lds_addr(smem);
  const RowBase<D> rb(l32, hh);
  const TrBase<D> tb(lane);
  const LoadLane llk(lane, wave, p.k.ss), llv(lane, wave, p.v.ss);

  const T* qg = static_cast<const T*>(p.q.ptr) + sv.off(p.q, b) + h * p.q.sh;
  const T* dog = static_cast<const T*>(p.dout.ptr) + sv.off(p.dout, b) + h * p.dout.sh;

  // n and b read once here: a read after the main loop would queue behind its
  // memory traffic and hold the workgroup's end for the round trip
  const float n = *p.n_ptr, bv = *p.b_ptr;
  const float c = p.scale * bv;
  const int q0 = qb * BM;
  const int wq0 = q0 + wave * 32;
  const int qrow = wq0 + l32;

  const int ntiles = pl.ntiles;
  const int nfull = CAUSAL ? min(q0 / BN, N / BN) : N / BN;

  pl.load_tile(0, lds0, wave, llk, llv);

  v8 qf[ND16], dof[ND16];
#pragma unroll
  for (int ds = 0; ds < ND16; ++ds) {
    qf[ds] = qrow < N ? load16<v8>(qg + qrow * p.q.ss + ds * 16 + 8 * hh) : zero8<v8>();
    dof[ds] = qrow < N ? load16<v8>(dog + qrow * p.dout.ss + ds * 16 + 8 * hh) : zero8<v8>();
  }
  const int64_t rowbase = sv.mrow(b, h, p.Hq, p.T, p.N);
  const float mq = qrow < N ? p.m[rowbase + qrow] : 0.f;
  const float dlq = qrow < N ? p.delta[rowbase + qrow] : 0.f;

  f32x16 dq[ND32];
#pragma unroll
  for (int i = 0; i < ND32; ++i) dq[i] = f32x16{};

  auto tile = [&](int t, auto masked_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const uint32_t kl = Plan::buf(lds0, t);
    const uint32_t vl = kl + TILE_BYTES;
    if (t + 1 < ntiles) pl.load_tile(t + 1, lds0, wave, llk, llv);
    const RowBase<D> rk = at_tile(rb, kl), rv = at_tile(rb, vl);
    const TrBase<D> tk = at_tile(tb, kl);
    const int kbase = t * BN;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int kstart = kbase + kb * 32;
      if (MASKED && (kstart >= N || (CAUSAL && kstart > wq0 + 31))) continue;
      f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int ds = 0; ds < ND16; ++ds) {
        const v8 ka = tile_read_row<D, v8>(rk, kb, ds);
        const v8 va = tile_read_row<D, v8>(rv, kb, ds);
        s = mfma32(ka, qf[ds], s);
        dp = mfma32(va, dof[ds], dp);
      }
      v8 sb[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = s[r];
        const float u1 = fmaf(c, fabsf(x), 1.f);
        const float sl = copysignf(fast_log2(u1), x);
        float pv = fast_exp2(fmaf(n, sl, -mq));
        if (MASKED) {
          const int kk = kstart + crow(r, hh);
          const bool valid = qrow < N && kk < N && (!CAUSAL || kk <= qrow);
          pv = valid ? pv : 0.f;
        }
        const float dsp = pv * (dp[r] - dlq) * fast_rcp(u1);
        sb[r >> 3][r & 7] = static_cast<T>(dsp);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int db = 0; db < ND32; ++db) {
          const v4 lo = tile_read_tr<D, v4>(tk, kb, ks, 0, db);
          const v4 hi = tile_read_tr<D, v4>(tk, kb, ks, 1, db);
          dq[db] = mfma32(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), sb[ks], dq[db]);
        }
      }
    }
  };
  for (int t = 0; t < nfull; ++t) tile(t, std::false_type{});
  for (int t = nfull; t < ntiles; ++t) tile(t, std::true_type{});

  const float qscale = p.scale * n * bv;
  if (qrow < N) {
    T* dqg = static_cast<T*>(const_cast<void*>(p.dq.ptr)) + sv.off(p.dq, b) + h * p.dq.sh + qrow * p.dq.ss;
#pragma unroll
    for (int db = 0; db < ND32; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        v4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = static_cast<T>(dq[db][4 * g + e] * qscale);
        *reinterpret_cast<v4*>(dqg + db * 32 + g * 8 + 4 * hh) = o4;
      }
    }
  }
}

// The reduction as a launch of its own (one workgroup).
__global__ __launch_bounds__(256) void ssa_reduce_partials_kernel(const float* partials, int64_t count,
                                                                  float* dn, float* db) {
  __shared__ float sh[2][256];
  reduce_partials_body(partials, count, dn, db, sh, threadIdx.x);
}

// ---------------------------------------------------------------------------
template <typename T>
static hipError_t pre_dt(const BwdParams& p, int D, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.N;
  const int rpb = 256 / (D / 8);
  const int grid = static_cast<int>((rows + rpb - 1) / rpb);
  switch (D) {
    case 32: hipLaunchKernelGGL((ssa_bwd_preprocess_kernel<T, 32>), dim3(grid), dim3(256), 0, s, p); break;
    case 64: hipLaunchKernelGGL((ssa_bwd_preprocess_kernel<T, 64>), dim3(grid), dim3(256), 0, s, p); break;
    case 128: hipLaunchKernelGGL((ssa_bwd_preprocess_kernel<T, 128>), dim3(grid), dim3(256), 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_bwd_preprocess(const BwdParams& p, int dtype, int D, hipStream_t s) {
  if (use_f32(dtype, D)) return launch_bwd_preprocess_f32(p, dtype, D, s);
  return dtype == 0 ? pre_dt<__bf16>(p, D, s) : pre_dt<_Float16>(p, D, s);
}


// Which dK/dV kernel runs (bf16 / fp16): the two-waves-per-SIMD kernel
// (ssa_bwd_dkdv2w.hip) at head dim 128, where it measured 1.3-5 % faster than
// the single-wave kernel on every dense and packed configuration, and the
// single-wave kernel of this file at head dims 32 and 64 (at 64 the two-wave
// kernel measured 6-8 % slower).  SSA_DKDV2W=1 / =0 forces one of them at
// every head dim; the variable is read at every launch, so a caller can
// switch within one process.
static bool use_dkdv2w(int D) {
  const char* e = getenv("SSA_DKDV2W");
  if (e != nullptr && (e[0] == '0' || e[0] == '1')) return e[0] == '1';
  return D == 128;
}

template <typename T, int D, bool CAUSAL>
static hipError_t dkdv_t(const BwdParams& p, hipStream_t s) {
  const int grid = DkdvPlan<128, 32, CAUSAL>::grid(p);
  const bool o32 = dkdv_off32(p, D, CAUSAL);
  if (use_dkdv2w(D)) return launch_bwd_dkdv2w(p, std::is_same_v<T, __bf16> ? 0 : 1, D, CAUSAL, o32, s);
  if (p.ds != nullptr) {
    if (o32)
      hipLaunchKernelGGL((ssa_bwd_dkdv_kernel<T, D, CAUSAL, true, true>), dim3(grid), dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((ssa_bwd_dkdv_kernel<T, D, CAUSAL, true, false>), dim3(grid), dim3(256), 0, s, p);
  } else {
    if (o32)
      hipLaunchKernelGGL((ssa_bwd_dkdv_kernel<T, D, CAUSAL, false, true>), dim3(grid), dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((ssa_bwd_dkdv_kernel<T, D, CAUSAL, false, false>), dim3(grid), dim3(256), 0, s, p);
  }
  return hipGetLastError();
}

template <typename T, int D, bool CAUSAL>
static hipError_t dq_t(const BwdParams& p, hipStream_t s) {
  if (p.ds != nullptr) {
    return launch_bwd_dq_ds(p, std::is_same_v<T, __bf16> ? 0 : 1, D, CAUSAL, s);  // ssa_bwd_dq.hip
  } else {
    const int grid = DqPlan<D, CAUSAL>::grid(p);
    hipLaunchKernelGGL((ssa_bwd_dq_kernel<T, D, CAUSAL>), dim3(grid), dim3(256), 0, s, p);
  }
  return hipGetLastError();
}

#define SSA_DISPATCH(FN, T, D, CAUSAL, P, S)                        \
  switch (D) {                                                      \
    case 32: return CAUSAL ? FN<T, 32, true>(P, S) : FN<T, 32, false>(P, S);    \
    case 64: return CAUSAL ? FN<T, 64, true>(P, S) : FN<T, 64, false>(P, S);    \
    case 128: return CAUSAL ? FN<T, 128, true>(P, S) : FN<T, 128, false>(P, S); \
    default: return hipErrorInvalidValue;                           \
  }

hipError_t launch_bwd_dkdv(const BwdParams& p, int dtype, int D, bool causal, hipStream_t s) {
  if (use_f32(dtype, D)) return launch_bwd_dkdv_f32(p, dtype, D, causal, s);
  if (dtype == 0) {
    SSA_DISPATCH(dkdv_t, __bf16, D, causal, p, s)
  }
  SSA_DISPATCH(dkdv_t, _Float16, D, causal, p, s)
}

hipError_t launch_bwd_dq(const BwdParams& p, int dtype, int D, bool causal, hipStream_t s) {
  if (use_f32(dtype, D)) return launch_bwd_dq_f32(p, dtype, D, causal, s);
  if (dtype == 0) {
    SSA_DISPATCH(dq_t, __bf16, D, causal, p, s)
  }
  SSA_DISPATCH(dq_t, _Float16, D, causal, p, s)
}

hipError_t launch_reduce_partials(const BwdParams& p, hipStream_t s) {
  const int64_t count = static_cast<int64_t>(p.B) * p.Hkv * dkdv_key_blocks(p.N);
  hipLaunchKernelGGL(ssa_reduce_partials_kernel, dim3(1), dim3(256), 0, s,
                     static_cast<const float*>(p.partials), count, p.dn, p.db);
  return hipGetLastError();
}

}  // namespace ssa
