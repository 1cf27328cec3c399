// Global-memory plans of the kernels that stream tiles: for one workgroup,
// wave and lane, the dispatch (which sequence, head and block a workgroup
// takes), which rows of which tensor every direct-to-LDS load fetches, and
// where every dS' workspace store goes.  The kernels issue their loads and
// stores through these (with ssa_tile.hpp's DeviceMem); because the plans are
// __host__ __device__, a host program replays exactly this code over every
// workgroup, wave and lane of a problem with a policy that performs the
// accesses on host memory and checks them (tests/host_addr/addr_replay.cpp,
// built with AddressSanitizer and UndefinedBehaviorSanitizer by
// tests/test_host_addr.py).
#pragma once

#include "ssa_launch.hpp"
#include "ssa_tile.hpp"

namespace ssa {

__host__ __device__ constexpr int imin(int a, int b) { return a < b ? a : b; }

// Step st of a dK/dV workgroup -> (q-head g, query sub-tile i), walked one
// step at a time without divisions: masked sub-tiles of every q-head first
// (j < per_m: i = j for the nlo diagonal ones, then the partial last
// sub-tile), then the unmasked ones (i = nlo + j).  Scalar state.
struct StepWalk {
  int g, j;
  bool unmasked;
  __host__ __device__ __forceinline__ explicit StepWalk(int nmasked) : g(0), j(0), unmasked(nmasked == 0) {}
  __host__ __device__ __forceinline__ void next(int per_m, int per_u, int G) {
    ++j;
    if (j >= (unmasked ? per_u : per_m)) {
      j = 0;
      if (++g >= G) {
        g = 0;
        unmasked = true;
      }
    }
  }
  __host__ __device__ __forceinline__ int sub(int nlo, int nsub) const {
    return unmasked ? nlo + j : (j < nlo ? j : nsub - 1);
  }
  // The same two inside the unmasked steps (the fast slots walk only those;
  // past the last step g runs to G, which no step reads).
  __host__ __device__ __forceinline__ void next_unmasked(int per_u) {
    if (++j >= per_u) {
      j = 0;
      ++g;
    }
  }
  __host__ __device__ __forceinline__ int sub_unmasked(int nlo) const { return nlo + j; }
};

// ----------------------------------------------------------------------------
// Forward (ssa_fwd.hip): a workgroup of 8 waves on 256 queries of (b, h); K
// and V tiles of 64 rows in a ring of NB buffers (tile t: K at buf(t), V at
// buf(t) + TILE).
template <int D, bool CAUSAL>
struct FwdPlan {
  static constexpr int BM = 256, BN = 64, NW = 8, NB = 4;
  static constexpr int TILE = BN * D * 2;  // one K (or V) tile
  static constexpr int BUF = 2 * TILE;     // K_t then V_t
  static constexpr int LDS_BYTES = NB * BUF;
  __host__ __device__ static int grid(const FwdParams& p) { return (p.N + BM - 1) / BM * p.B * p.Hq; }

  int qb, b, h, hk, N, NT;
  SeqView sv;
  const char* kg;
  const char* vg;
  int64_t kss, vss;
  __host__ __device__ __forceinline__ FwdPlan(const FwdParams& p, int block, int grid) {
    const int nqb = (p.N + BM - 1) / BM;
    const int L = xcd_remap(block, grid);
    // Logical order (head, sequence): each XCD's contiguous range holds a slice
    // of heads of every sequence (balanced when packed sequences differ in
    // length); query blocks heaviest (last) first within pairs of heads.
    int hb, rank;
    dispatch_order(L, grid / nqb, nqb, p.cu_seqlens ? 1 : kOrderGroup, hb, rank);
    qb = nqb - 1 - rank;
    b = hb % p.B;
    h = hb / p.B;
    hk = h / (p.Hq / p.Hkv);
    sv = SeqView(p.cu_seqlens, p.T, p.N, b);
    N = sv.N;
    const int q0 = qb * BM;
    const int kv_end = CAUSAL ? imin(N, q0 + BM) : N;
    NT = (kv_end + BN - 1) / BN;  // tiles streamed by the workgroup
    kg = static_cast<const char*>(p.k.ptr) + (sv.off(p.k, b) + hk * p.k.sh) * 2;
    vg = static_cast<const char*>(p.v.ptr) + (sv.off(p.v, b) + hk * p.v.sh) * 2;
    kss = p.k.ss;
    vss = p.v.ss;
  }
  // packed: past the end of a shorter document
  __host__ __device__ __forceinline__ bool empty() const { return qb * BM >= N; }
  __host__ __device__ __forceinline__ static uint32_t buf(uint32_t lds0, int t) { return lds0 + (t & (NB - 1)) * BUF; }
  // this wave's loads of tile t (none past the last)
  template <typename Mem = DeviceMem>
  __host__ __device__ __forceinline__ void load_tile(int t, uint32_t lds0, int wave, const LoadLane& llk,
                                                     const LoadLane& llv, const Mem& mem = Mem()) const {
    if (t >= NT) return;
    const uint32_t kl = buf(lds0, t);
    const int r0 = t * BN;
    if (r0 + BN <= N) {
      tile_load_pieces<D, BN, NW, false>(kg, kss, r0, N, kl, wave, llk, mem);
      tile_load_pieces<D, BN, NW, false>(vg, vss, r0, N, kl + TILE, wave, llv, mem);
    } else {
      tile_load_pieces<D, BN, NW, true>(kg, kss, r0, N, kl, wave, llk, mem);
      tile_load_pieces<D, BN, NW, true>(vg, vss, r0, N, kl + TILE, wave, llv, mem);
    }
  }
};

// ----------------------------------------------------------------------------
// dK/dV dispatch and step order: a workgroup of BN keys of (sequence b,
// kv-head hk) walks nsteps = G nsub steps of BMQ queries (q-head g of the
// group, sub-tile i).
template <int BN, int BMQ, bool CAUSAL>
struct DkdvPlan {
  __host__ __device__ static int grid(const BwdParams& p) { return dkdv_key_blocks(p.N) * p.B * p.Hkv; }

  int nkb, bhk, kb, b, hk, G, N, k0, qstart, nsub, nsteps, nlo, ntail, per_m, per_u, nmasked;
  bool key_edge;
  SeqView sv;
  __host__ __device__ __forceinline__ DkdvPlan(const BwdParams& p, int block, int grid) {
    static_assert(BN == 128, "dkdv_key_blocks() counts 128-key blocks");
    nkb = dkdv_key_blocks(p.N);
    const int L = xcd_remap(block, grid);
    // Logical order (kv-head, sequence), key blocks as in the forward's
    // dispatch order (ascending = heaviest first under causal).
    dispatch_order(L, grid / nkb, nkb, p.cu_seqlens ? 1 : kOrderGroup, bhk, kb);
    b = bhk % p.B;
    hk = bhk / p.B;
    G = p.Hq / p.Hkv;
    sv = SeqView(p.cu_seqlens, p.T, p.N, b);
    N = sv.N;
    k0 = kb * BN;
    qstart = CAUSAL ? k0 : 0;
    nsub = (N - qstart + BMQ - 1) / BMQ;
    nsteps = G * nsub;
    key_edge = k0 + BN > N;
    // Step order: every sub-tile that needs masks first (the causal
    // diagonal, a partial last sub-tile, or all of them at the sequence
    // end), then the unmasked ones.
    nlo = key_edge ? nsub : (CAUSAL ? imin(BN / BMQ, nsub) : 0);
    ntail = (!key_edge && (N % BMQ) != 0 && nsub > nlo) ? 1 : 0;
    per_m = nlo + ntail;
    per_u = nsub - per_m;  // per q-head
    nmasked = G * per_m;
  }
  // packed: past the end of a shorter document (the workgroup only zeroes its partials)
  __host__ __device__ __forceinline__ bool empty() const { return k0 >= N; }
  // first query of the step a walker is at (UNMASKED: a walker of the unmasked steps)
  template <bool UNMASKED>
  __host__ __device__ __forceinline__ int q0(const StepWalk& w) const {
    return qstart + (UNMASKED ? w.sub_unmasked(nlo) : w.sub(nlo, nsub)) * BMQ;
  }
  // the same by division (q-head in g)
  __host__ __device__ __forceinline__ int step_q0(int st, int& g) const {
    int i;
    if (st < nmasked) {
      g = st / per_m;
      const int j = st - g * per_m;
      i = j < nlo ? j : nsub - 1;
    } else {
      const int su = st - nmasked;
      g = su / per_u;
      i = nlo + (su - g * per_u);
    }
    return qstart + i * BMQ;
  }
  // a masked step whose queries all precede the keys k0w .. (or no keys):
  // nothing to compute or store for a wave whose first key is k0w
  __host__ __device__ __forceinline__ bool skipped(int st, int k0w) const {
    int g;
    return st < nmasked && (k0w >= N || (CAUSAL && step_q0(st, g) + BMQ - 1 < k0w));
  }
};

// Whether every dK/dV workgroup's Q / dO rows (from q-head hk G of its
// sequence: G heads, N rows, D columns) and its dS' tiles (G triangles of
// the longest sequence) lie below 2 GiB of their bases; strides are
// non-negative (validated at the boundary).  The kernels then take 32-bit
// offsets into loop-invariant buffer descriptors (OFF32).
inline bool dkdv_off32(const BwdParams& p, int D, bool causal) {
  const int64_t G = p.Hq / p.Hkv, lim = (int64_t{1} << 31) - 4096;
  auto span = [&](const Tensor4& t) { return ((G - 1) * t.sh + static_cast<int64_t>(p.N - 1) * t.ss + D) * 2; };
  if (span(p.q) >= lim || span(p.dout) >= lim) return false;
  return p.ds == nullptr || G * ds_tiles_per_head(p.N, causal) * 1024 < lim;
}

// Q / dO / M / Delta addressing shared by both dK/dV kernels: bases at q-head
// hk G of the workgroup's sequence, so a step's loads add only the q-head and
// row offsets.
struct DkdvBases {
  const char* q_head0;
  const char* do_head0;
  const float* m;
  const float* delta;
  int64_t m_row0, m_hstride, qsh, dosh, qss, doss;
  i32x4_t q_rs, do_rs;
  int q_hs2, q_ss2, do_hs2, do_ss2;
  template <class Plan>
  __host__ __device__ __forceinline__ DkdvBases(const BwdParams& p, const Plan& pl) {
    q_head0 = static_cast<const char*>(p.q.ptr) +
              (pl.sv.off(p.q, pl.b) + static_cast<int64_t>(pl.hk) * pl.G * p.q.sh) * 2;
    do_head0 = static_cast<const char*>(p.dout.ptr) +
               (pl.sv.off(p.dout, pl.b) + static_cast<int64_t>(pl.hk) * pl.G * p.dout.sh) * 2;
    m = p.m;
    delta = p.delta;
    m_row0 = pl.sv.mrow(pl.b, pl.hk * pl.G, p.Hq, p.T, p.N);
    m_hstride = pl.sv.packed ? p.T : p.N;  // M / Delta rows of consecutive q-heads
    q_rs = raw_rsrc(q_head0);
    do_rs = raw_rsrc(do_head0);
    qsh = p.q.sh;
    dosh = p.dout.sh;
    qss = p.q.ss;
    doss = p.dout.ss;
    q_hs2 = static_cast<int>(p.q.sh * 2);
    q_ss2 = static_cast<int>(p.q.ss * 2);
    do_hs2 = static_cast<int>(p.dout.sh * 2);
    do_ss2 = static_cast<int>(p.dout.ss * 2);
  }
};

// Loads of the 4-wave dK/dV kernel (ssa_bwd.hip): per step a Q and a dO
// sub-tile of 32 queries (block pieces from all four waves) and M / Delta of
// those queries (wave 3), into ring buffer buf(st).
template <int D, bool CAUSAL, bool OFF32>
struct DkdvLoads : DkdvBases {
  static constexpr int BN = 128, BMQ = 32, NW = 4, NB = 4;
  static constexpr int TILE = BMQ * D * 2;    // one Q (or dO) sub-tile
  static constexpr int BUF = 2 * TILE + 256;  // Q, dO, M[32], Delta[32]
  static constexpr int LDS_BYTES = NB * BUF;
  using Plan = DkdvPlan<BN, BMQ, CAUSAL>;
  int wave, lane;
  LoadLane llq, lld;
  __host__ __device__ __forceinline__ DkdvLoads(const BwdParams& p, const Plan& pl, int wave_, int lane_)
      : DkdvBases(p, pl), wave(wave_), lane(lane_), llq(lane_, wave_, p.q.ss), lld(lane_, wave_, p.dout.ss) {}
  __host__ __device__ __forceinline__ static uint32_t buf(uint32_t lds0, int st) { return lds0 + (st & (NB - 1)) * BUF; }
  // step st, the walker w at it (none past the last step)
  template <bool UNMASKED, typename Mem = DeviceMem>
  __host__ __device__ __forceinline__ void issue(const Plan& pl, int st, const StepWalk& w, uint32_t lds0,
                                                 const Mem& mem = Mem()) const {
    if (st >= pl.nsteps) return;
    const int g = w.g;
    const int N = pl.N;
    const int q0 = pl.template q0<UNMASKED>(w);
    const uint32_t b = buf(lds0, st);
    const char* qg = q_head0 + g * qsh * 2;
    const char* dog = do_head0 + g * dosh * 2;
    if (q0 + BMQ <= N) {
      if constexpr (OFF32) {
        tile_load_pieces_off<D, BMQ, NW>(q_rs, g * q_hs2 + q0 * q_ss2, q_ss2, b, wave, llq, mem);
        tile_load_pieces_off<D, BMQ, NW>(do_rs, g * do_hs2 + q0 * do_ss2, do_ss2, b + TILE, wave, lld, mem);
      } else {
        tile_load_pieces<D, BMQ, NW, false>(qg, qss, q0, N, b, wave, llq, mem);
        tile_load_pieces<D, BMQ, NW, false>(dog, doss, q0, N, b + TILE, wave, lld, mem);
      }
    } else {
      tile_load_pieces<D, BMQ, NW, true>(qg, qss, q0, N, b, wave, llq, mem);
      tile_load_pieces<D, BMQ, NW, true>(dog, doss, q0, N, b + TILE, wave, lld, mem);
    }
    if (wave == 3) {
      const int64_t rw = m_row0 + g * m_hstride;
      pair32_load_async(m + rw, delta + rw, q0, N, b + 2 * TILE, lane, mem);
    }
  }
};

// -dS' stores of the 4-wave dK/dV kernel: this wave's 32 keys are key tiles
// kj0 = k0w / 16 and kj0 + 1 of query tile q0 / 32 (both inside the causal
// triangle when the step is not skipped).  Lane (l32, hh) holds key l32 and,
// in its two operand vectors, queries 16 ks + 4 hh + (0..3) and 16 ks + 8 +
// 4 hh + (0..3); in the tile format (lane 16 g + kl: key kl, queries
// 16 t + 4 g + (0..3) at elements 4 t ..) these are four 8-byte pieces,
// g = hh or 2 + hh, t = ks, the two of one g adjacent: two 16-byte stores,
// at byte 256 hh of the lane's key row of the tile (+0: g = hh) and +512
// (g = 2 + hh).  Exactly two vector-memory instructions, which the kernel's
// load waits count.
template <bool CAUSAL, bool OFF32>
struct DkdvDsStores {
  char* ds_head0;  // key tile k0w / 16 of query tile 0 of the workgroup's first q-head
  i32x4_t ds_rs;
  uint32_t ds_voff;
  int64_t ds_tph;
  int ds_tph1k, N;
  template <class Plan>
  __host__ __device__ __forceinline__ DkdvDsStores(const BwdParams& p, const Plan& pl, int k0w, int lane) {
    const int l32 = lane & 31, hh = lane >> 5;
    N = pl.N;
    ds_tph = ds_tiles_per_head(N, CAUSAL);
    ds_head0 = static_cast<char*>(p.ds) +
               (ds_head_tile(pl.sv.packed, pl.sv.tok0, pl.b, pl.hk * pl.G, p.Hq, N, p.N, CAUSAL) + (k0w >> 4)) * 1024;
    ds_rs = raw_rsrc(ds_head0);
    ds_voff = static_cast<uint32_t>(((l32 >> 4) * 512 + (l32 & 15) * 8 + 16 * hh * 8) * 2);
    ds_tph1k = static_cast<int>(ds_tph * 1024);
  }
  // q-head g, query tile q0 / 32; s0, s1: the lane's operand vectors ks = 0, 1
  template <typename Mem = DeviceMem>
  __host__ __device__ __forceinline__ void store(int g, int q0, u32x4 s0, u32x4 s1, const Mem& mem = Mem()) const {
    const u32x4 lo = u32x4{s0[0], s0[1], s1[0], s1[1]}, hi = u32x4{s0[2], s0[3], s1[2], s1[3]};
    if constexpr (OFF32) {
      const int qi = q0 >> 5;
      const int soff = mem.uniform(g * ds_tph1k + (CAUSAL ? qi * (qi + 1) : qi * 2 * ((N + 31) >> 5)) * 1024);
      mem.template store16_nt<0>(ds_rs, ds_voff, soff, lo);
      mem.template store16_nt<512>(ds_rs, ds_voff, soff, hi);
    } else {
      char* dst = ds_head0 + (g * ds_tph + ds_row_offset(q0 >> 5, N, CAUSAL)) * 1024 + ds_voff;
      mem.template store16_nt_global<0>(dst, lo);
      mem.template store16_nt_global<512>(dst, hi);
    }
  }
};

// ----------------------------------------------------------------------------
// Loads of the two-waves-per-SIMD dK/dV kernel (ssa_bwd_dkdv2w.hip): 8 waves
// of 16 keys, steps of 64 queries; Q / dO tiles in the Swz8 layout
// (LoadLane::Swz8) at buf(st) and + TILE, M and Delta at + 2 TILE and
// + 2 TILE + 256.  Every wave issues LPT loads per tile: its Q and dO pieces
// (head dim 32: one of the two) and, from the 8 lanes of its own eighth of
// the wave, the rows 8 wave .. 8 wave + 7 of M and of Delta.  With SPREAD
// the steady-state tiles (OFF32, full) are prepared by issue() and their
// loads issued one at a time by issue_piece<K>().
template <int D, bool CAUSAL, bool OFF32, bool SPREAD>
struct Dkdv2wLoads : DkdvBases {
  static constexpr int NW = 8, KW = 16, BN = NW * KW, BMQ = 64, NB = 4;
  static constexpr int TILE = 2 * 32 * D * 2;  // 64 rows (two 32-row blocks)
  static constexpr int BUF = 2 * TILE + 512;   // Q, dO, M[64], Delta[64]
  static constexpr int LDS_BYTES = NB * BUF;
  static constexpr int NPIECE = TILE / 1024;  // 1 KB loads per tile
  static constexpr int PQ = NPIECE >= NW ? NPIECE / NW : 1;
  static constexpr int NLD = 2 * PQ + 2;                                // load slots per wave and tile
  static constexpr int LPT = (NPIECE >= NW ? 2 * NPIECE / NW : 1) + 2;  // loads issued per wave and tile
  static_assert(NPIECE >= NW || 2 * NPIECE == NW, "every wave loads the same number of pieces");
  using Plan = DkdvPlan<BN, BMQ, CAUSAL>;
  int wave, wave_do, lane;
  LoadLane llq, lld;
  // a tile whose loads issue() deferred to issue_piece()
  struct Deferred {
    bool on;
    uint32_t buf;
    int qoff, doff, q0;
    int64_t rw;
  } dfr;
  __host__ __device__ __forceinline__ Dkdv2wLoads(const BwdParams& p, const Plan& pl, int wave_, int lane_)
      : DkdvBases(p, pl), wave(wave_), lane(lane_), llq(lane_, p.q.ss, LoadLane::Swz8{}),
        lld(lane_, p.dout.ss, LoadLane::Swz8{}), dfr{false, 0, 0, 0, 0, 0} {
    // dO pieces from the upper waves when a tile has fewer pieces than waves
    wave_do = NPIECE < NW ? (wave + NW / 2) % NW : wave;
  }
  __host__ __device__ __forceinline__ static uint32_t buf(uint32_t lds0, int st) { return lds0 + (st & (NB - 1)) * BUF; }
  // M (which = 0) or Delta rows q0 .. q0 + 63 (clamped to N - 1), from this wave's eighth of the lanes
  template <typename Mem>
  __host__ __device__ __forceinline__ void load_md(int which, int64_t rw, int q0, int N, uint32_t b,
                                                   const Mem& mem) const {
    if ((lane >> 3) != wave) return;
    int r = q0 + lane;
    r = r < N ? r : N - 1;
    if (which == 0)
      mem.load4_global(b + 2 * TILE, m + rw + r);
    else
      mem.load4_global(b + 2 * TILE + 256, delta + rw + r);
  }
  // step st, the walker w at it (none past the last step)
  template <typename Mem = DeviceMem>
  __host__ __device__ __forceinline__ void issue(const Plan& pl, int st, const StepWalk& w, uint32_t lds0,
                                                 const Mem& mem = Mem()) {
    dfr.on = false;
    if (st >= pl.nsteps) return;
    const int g = w.g;
    const int N = pl.N;
    const int q0 = pl.template q0<false>(w);
    const uint32_t b = buf(lds0, st);
    const char* qg = q_head0 + g * qsh * 2;
    const char* dog = do_head0 + g * dosh * 2;
    const int64_t rw = m_row0 + g * m_hstride;
    if (q0 + BMQ <= N) {
      if constexpr (OFF32 && SPREAD) {
        dfr = Deferred{true, b, mem.uniform(g * q_hs2 + q0 * q_ss2), mem.uniform(g * do_hs2 + q0 * do_ss2), q0, rw};
        return;
      } else if constexpr (OFF32) {
        tile_load_pieces_off<D, BMQ, NW>(q_rs, g * q_hs2 + q0 * q_ss2, q_ss2, b, wave, llq, mem);
        tile_load_pieces_off<D, BMQ, NW>(do_rs, g * do_hs2 + q0 * do_ss2, do_ss2, b + TILE, wave_do, lld, mem);
      } else {
        tile_load_pieces<D, BMQ, NW, false>(qg, qss, q0, N, b, wave, llq, mem);
        tile_load_pieces<D, BMQ, NW, false>(dog, doss, q0, N, b + TILE, wave_do, lld, mem);
      }
    } else {
      tile_load_pieces<D, BMQ, NW, true>(qg, qss, q0, N, b, wave, llq, mem);
      tile_load_pieces<D, BMQ, NW, true>(dog, doss, q0, N, b + TILE, wave_do, lld, mem);
    }
    load_md(0, rw, q0, N, b, mem);
    load_md(1, rw, q0, N, b, mem);
  }
  // Load K (0 .. NLD - 1) of a deferred tile: the Q / dO pieces alternating,
  // then M and Delta.  N: the sequence length.
  template <int K, typename Mem = DeviceMem>
  __host__ __device__ __forceinline__ void issue_piece(int N, const Mem& mem = Mem()) const {
    if (!dfr.on) return;
    if constexpr (K < 2 * PQ) {
      constexpr bool DO = K % 2 == 1;
      const int j = (DO ? wave_do : wave) + NW * (K / 2);
      if (NPIECE % NW != 0 && j >= NPIECE) return;
      constexpr int IPB = BlockLayout<D>::IPB;
      const int blk = j / IPB, cp = j % IPB;
      if constexpr (DO)
        mem.load16(dfr.buf + TILE + j * 1024, do_rs, lld.off, dfr.doff + blk * 32 * do_ss2 + cp * 32);
      else
        mem.load16(dfr.buf + j * 1024, q_rs, llq.off, dfr.qoff + blk * 32 * q_ss2 + cp * 32);
    } else {
      load_md(K - 2 * PQ, dfr.rw, dfr.q0, N, dfr.buf, mem);
    }
  }
};

// -dS' stores of the two-wave kernel: this wave's key tile k0w / 16 of the
// step's two 32-query tiles; lane 16 g + i writes its 16 bytes (key i,
// queries 16 t + 4 g + (0..3) in elements 4 t ..) at byte 16 lane of a tile.
template <bool CAUSAL, bool OFF32>
struct Dkdv2wDsStores {
  char* ds_head0;  // key tile k0w / 16 of query tile 0 of the workgroup's first q-head
  i32x4_t ds_rs;
  uint32_t ds_voff;
  int64_t ds_tph;
  int ds_tph1k, N, nq32, k0w;
  template <class Plan>
  __host__ __device__ __forceinline__ Dkdv2wDsStores(const BwdParams& p, const Plan& pl, int k0w_, int lane)
      : k0w(k0w_) {
    N = pl.N;
    ds_tph = ds_tiles_per_head(N, CAUSAL);
    ds_head0 = static_cast<char*>(p.ds) +
               (ds_head_tile(pl.sv.packed, pl.sv.tok0, pl.b, pl.hk * pl.G, p.Hq, N, p.N, CAUSAL) + (k0w >> 4)) * 1024;
    ds_rs = raw_rsrc(ds_head0);
    ds_voff = static_cast<uint32_t>(lane * 16);
    ds_tph1k = static_cast<int>(ds_tph * 1024);
    nq32 = (N + 31) >> 5;
  }
  // Which of the two 32-query tiles of a masked step this wave stores: tiles
  // inside the sequence whose queries reach this wave's keys (exactly the
  // tiles of the causal triangle the dQ pass reads).  Unmasked steps store both.
  __host__ __device__ __forceinline__ int which(int q0) const {
    if (k0w >= N) return 0;
    int w = 0;
#pragma unroll
    for (int hq = 0; hq < 2; ++hq) {
      const int qt0 = q0 + 32 * hq;
      if (qt0 < N && (!CAUSAL || qt0 + 31 >= k0w)) w |= 1 << hq;
    }
    return w;
  }
  // tile hq (0, 1) of step (q-head g, queries q0 ..): one vector-memory instruction
  template <typename Mem = DeviceMem>
  __host__ __device__ __forceinline__ void store(int g, int q0, int hq, u32x4 v, const Mem& mem = Mem()) const {
    const int qt = (q0 >> 5) + hq;
    if constexpr (OFF32) {
      const int soff = mem.uniform(g * ds_tph1k + (CAUSAL ? qt * (qt + 1) : qt * 2 * nq32) * 1024);
      mem.template store16_nt<0>(ds_rs, ds_voff, soff, v);
    } else {
      char* dst = ds_head0 + (g * ds_tph + ds_row_offset(qt, N, CAUSAL)) * 1024 + ds_voff;
      mem.template store16_nt_global<0>(dst, v);
    }
  }
};

// ----------------------------------------------------------------------------
// The dS' K pass (ssa_bwd.hip, ssa_bwd_dq_ds_kernel): 32 NW queries of (b, h)
// per workgroup, K tiles of 64 rows (row-swizzled at head dim 128) in a ring
// of NK, and each wave's row of 1 KB dS' tiles, four per step in a ring of
// NDS stages, loads clamped to its last tile.  Step t issues K(t + PFK) and
// dS'(t + PFD): K(0 .. ntiles + PFK - 1) and dS'(0 .. ntiles + PFD - 1) in all.

// 8 waves (256 queries per workgroup; 128 KB of LDS at head dim 128, 112 KB
// at 64) at head dims 64 and 128, so each K tile is read once per 256
// queries (measured 4 % faster than 4-wave workgroups at both); 4 waves at
// head dim 32.
template <int D>
constexpr int dq_ds_waves() {
  return D >= 64 ? 8 : 4;
}

// Ring depths: NK K buffers loaded PFK steps ahead, NDS dS' stages loaded
// PFD steps ahead.
template <int D, bool CAUSAL, int NW, int NK_ = 2, int PFK_ = 1, int NDS_ = 3, int PFD_ = 2>
struct DqDsLoads {
  static constexpr int BM = 32 * NW, BN = 64;
  static constexpr int NK = NK_, PFK = PFK_, NDS = NDS_, PFD = PFD_;
  static constexpr int KTILE = BN * D * 2;
  static constexpr int DSTAGE = NW * 4096;  // NW waves x 4 dS' tiles
  static constexpr int LDS_BYTES = NK * KTILE + NDS * DSTAGE;
  static constexpr bool ROWSWZ = D == 128;
  static constexpr int KP = (BN / 32) * BlockLayout<D>::IPB / NW;  // K load pieces per wave and tile
  static_assert(KP >= 1, "K tile split");
  static_assert(PFD > PFK && PFK >= 1 && PFK < NK && PFD < NDS, "ring depths");
  __host__ __device__ static int grid(const BwdParams& p) { return (p.N + BM - 1) / BM * p.B * p.Hq; }

  int qb, b, h, hk, N, wq0, ntiles, nkj, kj_max, wave;
  SeqView sv;
  const char* kg;
  int64_t kss;
  i32x4_t ds_rsrc;
  uint32_t ds_src;
  LoadLane llk;
  RowSwzLoad rlk;
  __host__ __device__ __forceinline__ DqDsLoads(const BwdParams& p, int block, int grid, int wave_, int lane)
      : wave(wave_), llk(lane, wave_, p.k.ss), rlk(lane, p.k.ss) {
    const int nqb = (p.N + BM - 1) / BM;
    const int L = xcd_remap(block, grid);
    int hb, rank;
    dispatch_order(L, grid / nqb, nqb, p.cu_seqlens ? 1 : kOrderGroup, hb, rank);
    qb = CAUSAL ? nqb - 1 - rank : rank;
    b = hb % p.B;
    h = hb / p.B;
    hk = h / (p.Hq / p.Hkv);
    sv = SeqView(p.cu_seqlens, p.T, p.N, b);
    N = sv.N;
    const int q0 = qb * BM;
    wq0 = q0 + wave * 32;
    const int kv_end = CAUSAL ? imin(N, q0 + BM) : N;
    ntiles = (kv_end + BN - 1) / BN;
    // dS' tiles of this wave's query rows: kj < nkj (loads clamped to kj_max)
    const int nk16 = (N + 15) / 16;
    nkj = wq0 >= N ? 0 : (CAUSAL ? imin(2 * (wq0 >> 5) + 2, nk16) : nk16);
    kj_max = nkj > 0 ? nkj - 1 : 0;
    // the wave's row of workspace tiles (at most 2 nq32 KB: 32-bit offsets)
    ds_rsrc = raw_rsrc(static_cast<const char*>(p.ds) + (ds_head_tile(sv.packed, sv.tok0, b, h, p.Hq, N, p.N, CAUSAL) +
                                                         ds_row_offset(imin(wq0, N - 1) >> 5, N, CAUSAL)) * 1024);
    kg = static_cast<const char*>(p.k.ptr) + (sv.off(p.k, b) + hk * p.k.sh) * 2;
    kss = p.k.ss;
    // A stored tile holds, in lane s = 16 g + kl, key kl and queries 16 t +
    // 4 g + (0..3) (elements 4 t ..).  LDS slot 16 g + m receives stored lane
    // 16 g + (m ^ 4 g).
    ds_src = static_cast<uint32_t>((16 * (lane >> 4) + ((lane & 15) ^ (4 * (lane >> 4)))) * 16);
  }
  // packed: past the end of a shorter document
  __host__ __device__ __forceinline__ bool empty() const { return qb * BM >= N; }
  __host__ __device__ __forceinline__ static uint32_t ktile(uint32_t lds0, int t) { return lds0 + (t % NK) * KTILE; }
  __host__ __device__ __forceinline__ uint32_t dstage(uint32_t lds0, int t) const {
    return lds0 + NK * KTILE + (t % NDS) * DSTAGE + wave * 4096;
  }
  template <typename Mem = DeviceMem>
  __host__ __device__ __forceinline__ void issue_k(int t, uint32_t lds0, const Mem& mem = Mem()) const {
    if constexpr (ROWSWZ)
      rowswz_load<BN, NW>(kg, kss, t * BN, N, ktile(lds0, t), wave, rlk, mem);
    else
      tile_load_async<D, BN, NW>(kg, kss, t * BN, N, ktile(lds0, t), wave, llk, mem);
  }
  template <typename Mem = DeviceMem>
  __host__ __device__ __forceinline__ void issue_ds(int t, uint32_t lds0, const Mem& mem = Mem()) const {
    const uint32_t dst = dstage(lds0, t);
    // dS' is read exactly once: streaming cache policy
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) mem.load16_nt(dst + s4 * 1024, ds_rsrc, ds_src, imin(4 * t + s4, kj_max) * 1024);
  }
};

// ----------------------------------------------------------------------------
// The recompute dQ pass (ssa_bwd.hip, ssa_bwd_dq_kernel; backwards without a
// dS' workspace): 128 queries of (b, h) per workgroup of 4 waves, K and V
// tiles of 64 rows double-buffered (tile t: K at buf(t), V at buf(t) + TILE).
template <int D, bool CAUSAL>
struct DqPlan {
  static constexpr int BM = 128, BN = 64, NW = 4;
  static constexpr int TILE = BN * D * 2;
  static constexpr int LDS_BYTES = 2 * 2 * TILE;
  __host__ __device__ static int grid(const BwdParams& p) { return (p.N + BM - 1) / BM * p.B * p.Hq; }

  int qb, b, h, hk, N, ntiles;
  SeqView sv;
  const char* kg;
  const char* vg;
  int64_t kss, vss;
  __host__ __device__ __forceinline__ DqPlan(const BwdParams& p, int block, int grid) {
    const int nqb = (p.N + BM - 1) / BM;
    const int L = xcd_remap(block, grid);
    // Logical order (head, sequence, query block), as in the forward.
    int hb, rank;
    dispatch_order(L, grid / nqb, nqb, p.cu_seqlens ? 1 : kOrderGroup, hb, rank);
    qb = nqb - 1 - rank;
    b = hb % p.B;
    h = hb / p.B;
    hk = h / (p.Hq / p.Hkv);
    sv = SeqView(p.cu_seqlens, p.T, p.N, b);
    N = sv.N;
    const int q0 = qb * BM;
    const int kv_end = CAUSAL ? imin(N, q0 + BM) : N;
    ntiles = (kv_end + BN - 1) / BN;
    kg = static_cast<const char*>(p.k.ptr) + (sv.off(p.k, b) + hk * p.k.sh) * 2;
    vg = static_cast<const char*>(p.v.ptr) + (sv.off(p.v, b) + hk * p.v.sh) * 2;
    kss = p.k.ss;
    vss = p.v.ss;
  }
  // packed: past the end of a shorter document
  __host__ __device__ __forceinline__ bool empty() const { return qb * BM >= N; }
  __host__ __device__ __forceinline__ static uint32_t buf(uint32_t lds0, int t) { return lds0 + (t & 1) * 2 * TILE; }
  // this wave's loads of tile t (< ntiles)
  template <typename Mem = DeviceMem>
  __host__ __device__ __forceinline__ void load_tile(int t, uint32_t lds0, int wave, const LoadLane& llk,
                                                     const LoadLane& llv, const Mem& mem = Mem()) const {
    const uint32_t kl = buf(lds0, t);
    tile_load_async<D, BN, NW>(kg, kss, t * BN, N, kl, wave, llk, mem);
    tile_load_async<D, BN, NW>(vg, vss, t * BN, N, kl + TILE, wave, llv, mem);
  }
};

// ----------------------------------------------------------------------------
// Decode against a KV cache (ssa_decode.hip): a workgroup per (sequence b,
// kv-head hk, group qg of up to 32 q-heads, key split); each wave streams
// its own tiles of 32 keys (tile i of wave w: keys kbeg + 32 (w + NW i) ..)
// through a private ring of NB buffers (K block, then V block).
template <int D>
struct DecodeCfg {
  static constexpr int NW = D == 128 ? 4 : 8;           // waves per workgroup
  static constexpr int BLOCK = BlockLayout<D>::BLOCK;  // one 32-row K or V block
  static constexpr int TB = 2 * BLOCK;                 // K block, then V block
  static constexpr int NB = 131072 / (NW * TB);        // ring depth per wave
  static constexpr int LPT = 2 * BlockLayout<D>::IPB;  // loads per tile
  static constexpr int SMEM = NW * NB * TB;            // 128 KB
  static constexpr int ACC_LD = D + 1;                 // merge row stride (floats)
  static constexpr int ML_BYTES = NW * 2 * 32 * 4;     // merge (m, l) per wave and q-head
  static_assert(NB >= 2 && (NB - 1) * LPT < 64, "ring depth");
  static_assert(ML_BYTES + NW * 32 * ACC_LD * 4 <= SMEM, "merge area");
};

// Rows row0 .. row0 + 31 (clamped to nrows - 1) of a [*, D] matrix with row
// stride `ss` elements into one LDS block at `dst`, in the tile layout of
// ssa_tile.hpp, issued by a single wave: piece j (1 KB) holds chunks 2 j and
// 2 j + 1, whose swizzle parity is j & 1, hence the two LoadLane variants.
template <int D, typename Mem = DeviceMem>
__host__ __device__ __forceinline__ void block_load_wave(const char* g, int64_t ss, int row0, int nrows, uint32_t dst,
                                                         const LoadLane& ll0, const LoadLane& ll1,
                                                         const Mem& mem = Mem()) {
#pragma unroll
  for (int j = 0; j < BlockLayout<D>::IPB; ++j) {
    const LoadLane& ll = (j & 1) ? ll1 : ll0;
    int row = row0 + ll.r;
    row = row < nrows ? row : nrows - 1;
    mem.load16_global(dst + j * 1024, g + (static_cast<int64_t>(row) * ss + j * 16) * 2 + ll.hoff);
  }
}

template <int D>
struct DecodePlan {
  using C = DecodeCfg<D>;
  __host__ __device__ static int grid(const DecodeParams& p) {
    return p.B * p.Hkv * ((p.Hq / p.Hkv + 31) / 32) * p.splits;
  }
  int b, hk, qg, split, kbeg, kend, ntile;
  const char* kg;
  const char* vg;
  int64_t kss, vss;
  __host__ __device__ __forceinline__ DecodePlan(const DecodeParams& p, int block) {
    const int nqg = (p.Hq / p.Hkv + 31) / 32;
    int u = block;
    split = u % p.splits;
    u /= p.splits;
    qg = u % nqg;
    u /= nqg;
    hk = u % p.Hkv;
    b = u / p.Hkv;
    int L = load_table_entry(p.seqlens, b);
    L = L < 0 ? 0 : (L > p.cap ? p.cap : L);
    kbeg = split * p.split_keys;
    kend = imin(L, kbeg + p.split_keys);
    ntile = kend > kbeg ? (kend - kbeg + 31) / 32 : 0;
    kg = static_cast<const char*>(p.k.ptr) + (b * p.k.sb + hk * p.k.sh) * 2;
    vg = static_cast<const char*>(p.v.ptr) + (b * p.v.sb + hk * p.v.sh) * 2;
    kss = p.k.ss;
    vss = p.v.ss;
  }
  // tiles of wave w
  __host__ __device__ __forceinline__ int tiles_of(int w) const {
    return ntile > w ? (ntile - w + C::NW - 1) / C::NW : 0;
  }
  // The i-th tile of wave w into its ring at `ring`; past the wave's last
  // tile the rows clamp to kend - 1 (loads into a free buffer, never read),
  // so every iteration issues the same number of loads.  Only for a wave
  // with at least one tile (kend > kbeg).
  template <typename Mem = DeviceMem>
  __host__ __device__ __forceinline__ void issue(int i, int w, uint32_t ring, const LoadLane& lk0, const LoadLane& lk1,
                                                 const LoadLane& lv0, const LoadLane& lv1, const Mem& mem = Mem()) const {
    const int row0 = kbeg + 32 * (w + C::NW * i);
    const uint32_t dst = ring + (i % C::NB) * C::TB;
    block_load_wave<D>(kg, kss, row0, kend, dst, lk0, lk1, mem);
    block_load_wave<D>(vg, vss, row0, kend, dst + C::BLOCK, lv0, lv1, mem);
  }
};

}  // namespace ssa
