// Host replay of the kernels' global-memory plans (luciole-1b_amd/csrc/ssa_plan.hpp).
//
// The plans hold the dispatch and per-lane address arithmetic of every
// tile-streaming kernel, as __host__ __device__ code that the kernels call
// with DeviceMem.  This program calls the same code on the CPU, for every
// workgroup, wave and lane of a problem, in the order the kernels issue it,
// with HostMem: each direct-to-LDS load and each dS' store is performed on
// host memory (exact-size allocations, so AddressSanitizer sees any stray
// byte; UndefinedBehaviorSanitizer sees any signed overflow in the offset
// arithmetic) and checked:
//
//  * dispatch: the grid's workgroups cover every (sequence, head, block) unit
//    exactly once;
//  * every 16-byte (4-byte for M / Delta) load reads one row of the tensor
//    and head the workgroup works on, at a row inside the tile being loaded
//    (rows past the sequence end clamped to its last row) and inside the
//    sequence: no byte of padding, of another head or of another document;
//  * each tile's LDS bytes are written exactly once, and the set of
//    (row, 16-byte chunk) pairs loaded is exactly the tile's;
//  * buffer-descriptor offsets stay in [0, 2^31 - 1) (the descriptors'
//    range), and values the kernels declare wave-uniform are equal in all
//    64 lanes;
//  * dS' workspace: every store lies inside the size the library reports
//    for the problem and no byte is written twice; every tile the dS' K
//    pass multiplies was written, and after its load each LDS slot holds the
//    (query, key) pairs the pass reads there.  For the last check the replay
//    stores tags (query, key and tile identity per element) in the layout
//    each dK/dV kernel states for its operand lanes.
//
// Cases: dense, GQA, Megatron-strided, ragged lengths, packed (including
// malformed document tables) and the benchmark sizes (a sample of their
// workgroups, on address-only buffers).  Exit status 0 and "0 failures" when
// every check holds.
#include <cinttypes>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "ssa_plan.hpp"

using namespace ssa;

namespace {

long g_checks = 0;
long g_fail = 0;
std::string g_ctx;

void failf(const char* fmt, ...) {
  if (g_fail++ < 25) {
    va_list ap;
    va_start(ap, fmt);
    fprintf(stderr, "FAIL [%s] ", g_ctx.c_str());
    vfprintf(stderr, fmt, ap);
    fputc('\n', stderr);
    va_end(ap);
  }
}
#define CHECK(cond, ...)          \
  do {                            \
    ++g_checks;                   \
    if (!(cond)) failf(__VA_ARGS__); \
  } while (0)

std::string fmt(const char* f, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, f);
  vsnprintf(buf, sizeof buf, f, ap);
  va_end(ap);
  return buf;
}

// ---------------------------------------------------------------------------
// Tensors.  Layouts: 0 = [B, H, N, D] contiguous, 1 = [N, B, H, D] memory
// viewed as [B, H, N, D] (Megatron), 2 = packed [T, H, D], 3 = fp32 rows
// [B H, N] (M / Delta, dense), 4 = fp32 rows [H, T] (packed), 5 = the dS'
// workspace (bytes).  Virtual tensors have no memory (benchmark sizes):
// their accesses are checked, not performed.
struct Tensor {
  std::string name;
  int layout = 0, B = 0, H = 0, N = 0, D = 0, T = 0, esize = 2;
  int64_t sb = 0, sh = 0, ss = 0;
  size_t bytes = 0;
  char* base = nullptr;
  std::unique_ptr<char[]> mem;
  bool is_virtual = false;
  std::vector<uint8_t> written;  // workspace: bytes stored so far
};

std::vector<Tensor*> g_tensors;
uint64_t g_next_virtual = 0x100000000000ull;

void alloc(Tensor& t, bool virt) {
  t.is_virtual = virt;
  if (virt) {
    t.base = reinterpret_cast<char*>(g_next_virtual);
    g_next_virtual += (t.bytes + (1ull << 32)) & ~((1ull << 32) - 1);
  } else {
    t.mem.reset(new char[t.bytes ? t.bytes : 1]);
    memset(t.mem.get(), 0, t.bytes ? t.bytes : 1);
    t.base = t.mem.get();
  }
  g_tensors.push_back(&t);
}

Tensor make_rows(const char* name, int layout, int B, int H, int N, int D, int T) {
  Tensor t;
  t.name = name;
  t.layout = layout;
  t.B = B;
  t.H = H;
  t.N = N;
  t.D = D;
  t.T = T;
  if (layout == 0) {
    t.ss = D, t.sh = static_cast<int64_t>(N) * D, t.sb = static_cast<int64_t>(H) * N * D;
    t.bytes = static_cast<size_t>(B) * H * N * D * 2;
  } else if (layout == 1) {
    t.sh = D, t.sb = static_cast<int64_t>(H) * D, t.ss = static_cast<int64_t>(B) * H * D;
    t.bytes = static_cast<size_t>(N) * B * H * D * 2;
  } else {
    t.sh = D, t.ss = static_cast<int64_t>(H) * D, t.sb = 0;
    t.bytes = static_cast<size_t>(T) * H * D * 2;
  }
  return t;
}

Tensor make_md(const char* name, bool packed, int B, int H, int N, int T) {
  Tensor t;
  t.name = name;
  t.layout = packed ? 4 : 3;
  t.B = B, t.H = H, t.N = N, t.T = T, t.D = 1, t.esize = 4;
  t.bytes = packed ? static_cast<size_t>(H) * T * 4 : static_cast<size_t>(B) * H * N * 4;
  return t;
}

// Where an element lies: sequence (dense) or -1 (packed), head, row (token
// for packed), column; ok = false for bytes outside every element.
struct Owner {
  int64_t b = -1, row = -1;
  int h = -1, c = -1;
  bool ok = false;
};

Owner owner_of(const Tensor& t, int64_t e) {
  Owner o;
  if (e < 0) return o;
  switch (t.layout) {
    case 0: {
      o.b = e / t.sb;
      const int64_t r = e % t.sb;
      o.h = static_cast<int>(r / t.sh);
      o.row = (r % t.sh) / t.ss;
      o.c = static_cast<int>(r % t.ss);
      o.ok = o.b < t.B && o.h < t.H && o.row < t.N && o.c < t.D;
      break;
    }
    case 1: {
      o.row = e / t.ss;
      const int64_t r = e % t.ss;
      o.b = r / t.sb;
      o.h = static_cast<int>((r % t.sb) / t.sh);
      o.c = static_cast<int>(r % t.sh);
      o.ok = o.row < t.N && o.b < t.B && o.h < t.H && o.c < t.D;
      break;
    }
    case 2: {
      o.row = e / t.ss;  // token
      o.h = static_cast<int>((e % t.ss) / t.sh);
      o.c = static_cast<int>(e % t.sh);
      o.ok = o.row < t.T && o.h < t.H && o.c < t.D;
      break;
    }
    case 3: {
      o.b = e / (static_cast<int64_t>(t.H) * t.N);
      o.h = static_cast<int>((e / t.N) % t.H);
      o.row = e % t.N;
      o.c = 0;
      o.ok = o.b < t.B;
      break;
    }
    case 4: {
      o.h = static_cast<int>(e / t.T);
      o.row = e % t.T;
      o.c = 0;
      o.ok = o.h < t.H;
      break;
    }
    default:
      break;
  }
  return o;
}

// ---------------------------------------------------------------------------
// One replayed workgroup: its LDS image and the accesses logged since the
// last check.
struct Access {
  Tensor* t;
  int64_t off;  // bytes from the tensor base
  int bytes;
  uint32_t lds;  // LDS byte written (loads)
};

struct Replay {
  std::unique_ptr<uint8_t[]> lds;
  std::vector<uint16_t> lds_count;  // writes per LDS byte since the last check
  size_t lds_bytes = 0;
  int lane = 0;
  bool lane0 = true;
  std::vector<int> uni;
  size_t uni_pos = 0;
  std::vector<Access> log;

  void reset_lds(size_t n) {
    lds_bytes = n;
    lds.reset(new uint8_t[n]);
    memset(lds.get(), 0, n);
    lds_count.assign(n, 0);
  }
  void start_lane(int l) {
    lane = l;
    lane0 = l == 0;
    if (lane0) uni.clear();
    uni_pos = 0;
  }
  int uniform(int x) {
    if (lane0) {
      uni.push_back(x);
    } else {
      CHECK(uni_pos < uni.size(), "wave-uniform value %d: lane %d makes more uniform() calls than lane 0", x, lane);
      if (uni_pos < uni.size())
        CHECK(uni[uni_pos] == x, "wave-uniform value differs: lane 0 %d, lane %d %d", uni[uni_pos], lane, x);
      ++uni_pos;
    }
    return x;
  }
  Tensor* find(const char* p, int bytes, int64_t& off) {
    for (Tensor* t : g_tensors) {
      const char* b = t->base;
      if (p >= b && p + bytes <= b + t->bytes) {
        off = p - b;
        return t;
      }
    }
    return nullptr;
  }
  // a load of `bytes` from p into LDS byte `l`
  void load(const char* p, int bytes, uint32_t l) {
    int64_t off = 0;
    Tensor* t = find(p, bytes, off);
    CHECK(t != nullptr, "load of %d bytes at %p lies in no tensor", bytes, static_cast<const void*>(p));
    CHECK(static_cast<size_t>(l) + bytes <= lds_bytes, "LDS destination %u + %d past the %zu-byte allocation", l, bytes,
          lds_bytes);
    if (t == nullptr || static_cast<size_t>(l) + bytes > lds_bytes) return;
    if (!t->is_virtual) memcpy(lds.get() + l, p, bytes);
    for (int i = 0; i < bytes; ++i) ++lds_count[l + i];
    log.push_back(Access{t, off, bytes, l});
  }
  static const char* desc_base(const i32x4_t& rs) {
    CHECK(rs[2] == 0x7fffffff && rs[3] == 0x00020000, "buffer descriptor words 2, 3: %#x %#x", rs[2], rs[3]);
    const uint64_t a = static_cast<uint64_t>(static_cast<uint32_t>(rs[0])) |
                       (static_cast<uint64_t>(static_cast<uint32_t>(rs[1]) & 0xffffu) << 32);
    return reinterpret_cast<const char*>(a);
  }
  // buffer addressing: base + voffset + soffset + instruction offset; the
  // whole access must lie below the descriptor's num_records (2^31 - 1)
  const char* buffer_addr(const i32x4_t& rs, uint32_t voff, int soff, int imm, int bytes) {
    CHECK(soff >= 0, "negative scalar offset %d", soff);
    const uint64_t off = static_cast<uint64_t>(voff) + static_cast<uint64_t>(static_cast<uint32_t>(soff)) + imm;
    CHECK(off + bytes <= 0x7fffffffull, "buffer offset %" PRIu64 " past the descriptor range", off);
    return desc_base(rs) + off;
  }
  void store(char* p, const u32x4& v) {
    int64_t off = 0;
    Tensor* t = find(p, 16, off);
    CHECK(t != nullptr && t->layout == 5, "dS' store at %p outside the workspace", static_cast<void*>(p));
    if (t == nullptr || t->layout != 5) return;
    if (!t->written.empty())
      for (int i = 0; i < 16; ++i) {
        CHECK(!t->written[off + i], "dS' workspace byte %" PRId64 " written twice", off + i);
        t->written[off + i] = 1;
      }
    if (!t->is_virtual) memcpy(p, &v, 16);
  }
};

Replay* g_r = nullptr;

// The plans' memory policy on the host.
struct HostMem {
  void load16(uint32_t lds, const i32x4_t& rs, uint32_t voff, int soff) const {
    g_r->load(g_r->buffer_addr(rs, voff, soff, 0, 16), 16, lds + 16 * g_r->lane);
  }
  void load16_nt(uint32_t lds, const i32x4_t& rs, uint32_t voff, int soff) const { load16(lds, rs, voff, soff); }
  void load16_global(uint32_t lds, const void* src) const {
    g_r->load(static_cast<const char*>(src), 16, lds + 16 * g_r->lane);
  }
  void load4_global(uint32_t lds, const void* src) const {
    g_r->load(static_cast<const char*>(src), 4, lds + 4 * g_r->lane);
  }
  template <int OFF>
  void store16_nt(const i32x4_t& rs, uint32_t voff, int soff, u32x4 v) const {
    g_r->store(const_cast<char*>(g_r->buffer_addr(rs, voff, soff, OFF, 16)), v);
  }
  template <int OFF>
  void store16_nt_global(void* p, u32x4 v) const {
    g_r->store(static_cast<char*>(p) + OFF, v);
  }
  int uniform(int x) const { return g_r->uniform(x); }
};

// ---------------------------------------------------------------------------
// Tile checks.  A region: `rows` rows from row0 of tensor t, head h, of
// sequence b (dense) or of the document at token tok0 (packed), rows at or
// past N clamped to N - 1, loaded to LDS [lds, lds + rows * row bytes).
struct Region {
  Tensor* t;
  int64_t b, tok0;
  bool packed;
  int h, row0, rows, N;
  uint32_t lds;
};

int64_t row_bytes(const Tensor& t) { return static_cast<int64_t>(t.D) * t.esize; }

// Every logged access lies in one region and reads its own rows; every
// region byte of LDS is written exactly once; the (row, chunk) pairs read
// are exactly the region's.  Clears the log and the LDS write counts.
void check_regions(Replay& R, const std::vector<Region>& regs) {
  std::vector<std::set<std::pair<int64_t, int64_t>>> got(regs.size());
  for (const Access& a : R.log) {
    int k = -1;
    for (size_t i = 0; i < regs.size(); ++i) {
      const Region& g = regs[i];
      const uint32_t len = static_cast<uint32_t>(g.rows * row_bytes(*g.t));
      if (a.lds >= g.lds && a.lds < g.lds + len) k = static_cast<int>(i);
    }
    CHECK(k >= 0, "%s load to LDS %u outside every tile of this issue", a.t->name.c_str(), a.lds);
    if (k < 0) continue;
    const Region& g = regs[k];
    CHECK(a.t == g.t, "LDS %u of the %s tile loaded from %s", a.lds, g.t->name.c_str(), a.t->name.c_str());
    if (a.t != g.t) continue;
    CHECK(a.off % a.bytes == 0, "%s: unaligned %d-byte load at byte %" PRId64, a.t->name.c_str(), a.bytes, a.off);
    const Owner o0 = owner_of(*a.t, a.off / a.t->esize);
    const Owner o1 = owner_of(*a.t, (a.off + a.bytes) / a.t->esize - 1);
    CHECK(o0.ok && o1.ok, "%s: load at byte %" PRId64 " reads outside every element", a.t->name.c_str(), a.off);
    if (!(o0.ok && o1.ok)) continue;
    CHECK(o0.row == o1.row && o0.h == o1.h && o0.b == o1.b, "%s: load at byte %" PRId64 " spans two rows",
          a.t->name.c_str(), a.off);
    CHECK(o0.h == g.h, "%s: head %d read by a workgroup of head %d", a.t->name.c_str(), o0.h, g.h);
    if (!g.packed) CHECK(o0.b == g.b, "%s: sequence %" PRId64 " read for sequence %" PRId64, a.t->name.c_str(), o0.b, g.b);
    const int64_t row = g.packed ? o0.row - g.tok0 : o0.row;
    CHECK(row >= 0 && row < g.N, "%s: row %" PRId64 " outside the sequence [0, %d)", a.t->name.c_str(), row, g.N);
    const int64_t hi = g.row0 + g.rows - 1 < g.N - 1 ? g.row0 + g.rows - 1 : g.N - 1;
    const int64_t lo = g.row0 < hi ? g.row0 : hi;
    CHECK(row >= lo && row <= hi, "%s: row %" PRId64 " outside the tile rows [%" PRId64 ", %" PRId64 "]",
          a.t->name.c_str(), row, lo, hi);
    got[k].insert({row, static_cast<int64_t>(o0.c) * a.t->esize / a.bytes});
  }
  for (size_t i = 0; i < regs.size(); ++i) {
    const Region& g = regs[i];
    const int64_t rb = row_bytes(*g.t);
    const int64_t chunk = g.t->esize == 4 ? 4 : 16;
    std::set<std::pair<int64_t, int64_t>> want;
    for (int r = 0; r < g.rows; ++r) {
      const int64_t row = g.row0 + r < g.N ? g.row0 + r : g.N - 1;
      for (int64_t c = 0; c < rb / chunk; ++c) want.insert({row, c});
    }
    CHECK(got[i] == want, "%s tile (head %d, rows %d + %d of %d): loaded %zu (row, chunk) pairs, want %zu",
          g.t->name.c_str(), g.h, g.row0, g.rows, g.N, got[i].size(), want.size());
    const uint32_t len = static_cast<uint32_t>(g.rows * rb);
    int bad = 0;
    for (uint32_t x = 0; x < len; ++x) bad += R.lds_count[g.lds + x] != 1;
    CHECK(bad == 0, "%s tile at LDS %u: %d of %u bytes not written exactly once", g.t->name.c_str(), g.lds, bad, len);
  }
  for (const Access& a : R.log)
    for (int i = 0; i < a.bytes; ++i) R.lds_count[a.lds + i] = 0;
  R.log.clear();
}

// ---------------------------------------------------------------------------
// dS' tags: element (query qq of the 32-query tile, key kk of the 16-key
// tile) of tile (b, h, qi, kj), 16 bits.
uint16_t ds_tag(int64_t b, int h, int qi, int kj, int qq, int kk) {
  const int id = static_cast<int>((b * 131 + h * 31 + qi * 7 + kj) & 0x7f);
  return static_cast<uint16_t>((qq << 11) | (kk << 7) | id);
}
u32x4 pack8(const uint16_t (&e)[8]) {
  u32x4 v;
  for (int i = 0; i < 4; ++i) v[i] = static_cast<uint32_t>(e[2 * i]) | (static_cast<uint32_t>(e[2 * i + 1]) << 16);
  return v;
}

// ---------------------------------------------------------------------------
struct Case {
  std::string name;
  int B, Hq, Hkv, N, D;
  bool causal;
  int layout;           // 0 contiguous, 1 Megatron-strided, 2 packed
  std::vector<int> cu;  // packed: document table (B + 1 entries, may be malformed)
  int T;
  int sample;  // 0: every workgroup on real memory; s > 0: every s-th workgroup and the last 8, address-only
};

struct Problem {
  Case c;
  Tensor q, k, v, dout, m, delta, ws;
  BwdParams bp{};
  FwdParams fp{};
  bool packed = false;
};

Tensor make_ws(const Case& c, bool virt) {
  Tensor t;
  t.name = "dS'";
  t.layout = 5;
  t.esize = 1;
  const bool packed = c.layout == 2;
  const int64_t tiles = packed ? ds_packed_tiles(c.B, c.Hq, c.T, c.N, c.causal)
                               : static_cast<int64_t>(c.B) * c.Hq * ds_tiles_per_head(c.N, c.causal);
  t.bytes = static_cast<size_t>(tiles) * 1024;
  return t;
}

void setup(Problem& P) {
  const Case& c = P.c;
  g_tensors.clear();
  const bool virt = c.sample > 0;
  P.packed = c.layout == 2;
  const int lay = c.layout;
  P.q = make_rows("Q", lay, c.B, c.Hq, c.N, c.D, c.T);
  P.dout = make_rows("dO", lay, c.B, c.Hq, c.N, c.D, c.T);
  P.k = make_rows("K", lay, c.B, c.Hkv, c.N, c.D, c.T);
  P.v = make_rows("V", lay, c.B, c.Hkv, c.N, c.D, c.T);
  P.m = make_md("M", P.packed, c.B, c.Hq, c.N, c.T);
  P.delta = make_md("Delta", P.packed, c.B, c.Hq, c.N, c.T);
  for (Tensor* t : {&P.q, &P.dout, &P.k, &P.v, &P.m, &P.delta}) alloc(*t, virt);
  P.ws = make_ws(c, virt);
  alloc(P.ws, virt);
  // written map: address-only runs (the benchmark sizes) keep none
  if (!virt) P.ws.written.assign(P.ws.bytes, 0);
  auto t4 = [](const Tensor& t) { return Tensor4{t.base, t.sb, t.sh, t.ss}; };
  BwdParams& p = P.bp;
  p = BwdParams{};
  p.q = t4(P.q), p.k = t4(P.k), p.v = t4(P.v), p.dout = t4(P.dout);
  p.m = reinterpret_cast<const float*>(P.m.base);
  p.delta = reinterpret_cast<float*>(P.delta.base);
  p.B = c.B, p.Hq = c.Hq, p.Hkv = c.Hkv, p.N = c.N, p.T = c.T;
  p.cu_seqlens = P.packed ? P.c.cu.data() : nullptr;
  p.ds = P.ws.base;
  FwdParams& f = P.fp;
  f = FwdParams{};
  f.q = t4(P.q), f.k = t4(P.k), f.v = t4(P.v);
  f.B = c.B, f.Hq = c.Hq, f.Hkv = c.Hkv, f.N = c.N, f.T = c.T;
  f.cu_seqlens = p.cu_seqlens;
}

bool replay_block(const Case& c, int block, int grid) {
  if (c.sample <= 0) return true;
  return block % c.sample == 0 || block >= grid - 8;
}

// ---------------------------------------------------------------------------
template <int D, bool CAUSAL>
void run_fwd(Problem& P) {
  using Plan = FwdPlan<D, CAUSAL>;
  const FwdParams& p = P.fp;
  const int grid = Plan::grid(p);
  Replay R;
  g_r = &R;
  std::set<std::tuple<int, int, int>> units;
  for (int blk = 0; blk < grid; ++blk) {
    const Plan pl(p, blk, grid);
    CHECK(units.insert({pl.b, pl.h, pl.qb}).second, "forward: unit (b %d, h %d, qb %d) dispatched twice", pl.b, pl.h,
          pl.qb);
    if (pl.empty() || !replay_block(P.c, blk, grid)) continue;
    g_ctx = fmt("%s fwd D=%d causal=%d block %d (b %d h %d qb %d)", P.c.name.c_str(), D, CAUSAL, blk, pl.b, pl.h, pl.qb);
    R.reset_lds(Plan::LDS_BYTES);
    for (int t = 0; t < pl.NT + 2; ++t) {
      for (int w = 0; w < Plan::NW; ++w)
        for (int l = 0; l < 64; ++l) {
          R.start_lane(l);
          const LoadLane llk(l, w, p.k.ss), llv(l, w, p.v.ss);
          pl.load_tile(t, 0u, w, llk, llv, HostMem());
        }
      if (t >= pl.NT) {
        CHECK(R.log.empty(), "forward issues loads for tile %d past the last (%d)", t, pl.NT);
        continue;
      }
      check_regions(R, {Region{&P.k, pl.b, pl.sv.tok0, pl.sv.packed, pl.hk, t * Plan::BN, Plan::BN, pl.N, Plan::buf(0, t)},
                        Region{&P.v, pl.b, pl.sv.tok0, pl.sv.packed, pl.hk, t * Plan::BN, Plan::BN, pl.N,
                               Plan::buf(0, t) + Plan::TILE}});
    }
  }
  CHECK(static_cast<int64_t>(units.size()) == grid, "forward: %zu units for %d workgroups", units.size(), grid);
}

// M / Delta tiles of a dK/dV step
void md_regions(std::vector<Region>& regs, Problem& P, int64_t b, const SeqView& sv, int h, int q0, int rows, int N,
                uint32_t lds) {
  regs.push_back(Region{&P.m, b, sv.tok0, sv.packed, h, q0, rows, N, lds});
  regs.push_back(Region{&P.delta, b, sv.tok0, sv.packed, h, q0, rows, N, lds + 4u * rows});
}

// 4-wave dK/dV kernel (ssa_bwd.hip): step loads, dS' stores with tags
template <int D, bool CAUSAL, bool OFF32>
void run_dkdv(Problem& P) {
  using Loads = DkdvLoads<D, CAUSAL, OFF32>;
  using Plan = typename Loads::Plan;
  const BwdParams& p = P.bp;
  const int grid = Plan::grid(p);
  Replay R;
  g_r = &R;
  std::set<std::tuple<int, int, int>> units;
  for (int blk = 0; blk < grid; ++blk) {
    const Plan pl(p, blk, grid);
    CHECK(units.insert({pl.b, pl.hk, pl.kb}).second, "dK/dV: unit dispatched twice");
    if (pl.empty() || !replay_block(P.c, blk, grid)) continue;
    g_ctx = fmt("%s dkdv D=%d causal=%d off32=%d block %d (b %d hk %d kb %d)", P.c.name.c_str(), D, CAUSAL, OFF32, blk,
                pl.b, pl.hk, pl.kb);
    R.reset_lds(Loads::LDS_BYTES);
    // loads: steps 0 .. nsteps + 1 (the last two issue nothing); the
    // unmasked slots walk with next_unmasked / sub_unmasked, which must
    // agree with the general walker
    StepWalk wi(pl.nmasked), wu(pl.nmasked);
    bool wu_live = false;
    for (int st = 0; st < pl.nsteps + 2; ++st) {
      const bool unm = st >= pl.nmasked && st < pl.nsteps;
      if (unm && !wu_live) {
        wu = wi;
        wu_live = true;
      }
      if (unm) CHECK(wu.g == wi.g && pl.template q0<true>(wu) == pl.template q0<false>(wi),
                     "step %d: unmasked walker at (g %d, q0 %d), general walker at (g %d, q0 %d)", st, wu.g,
                     pl.template q0<true>(wu), wi.g, pl.template q0<false>(wi));
      int gd = -1;
      if (st < pl.nsteps)
        CHECK(pl.step_q0(st, gd) == pl.template q0<false>(wi) && gd == wi.g, "step %d: walker and division disagree", st);
      for (int w = 0; w < Loads::NW; ++w)
        for (int l = 0; l < 64; ++l) {
          R.start_lane(l);
          const Loads ld(p, pl, w, l);
          if (unm)
            ld.template issue<true>(pl, st, wu, 0u, HostMem());
          else
            ld.template issue<false>(pl, st, wi, 0u, HostMem());
        }
      if (st >= pl.nsteps) {
        CHECK(R.log.empty(), "dK/dV issues loads for step %d past the last (%d)", st, pl.nsteps);
      } else {
        const int q0 = pl.template q0<false>(wi), h = pl.hk * pl.G + wi.g;
        const uint32_t b0 = Loads::buf(0, st);
        std::vector<Region> regs{Region{&P.q, pl.b, pl.sv.tok0, pl.sv.packed, h, q0, Loads::BMQ, pl.N, b0},
                                 Region{&P.dout, pl.b, pl.sv.tok0, pl.sv.packed, h, q0, Loads::BMQ, pl.N, b0 + Loads::TILE}};
        md_regions(regs, P, pl.b, pl.sv, h, q0, Loads::BMQ, pl.N, b0 + 2 * Loads::TILE);
        check_regions(R, regs);
      }
      wi.next(pl.per_m, pl.per_u, pl.G);
      if (wu_live) wu.next_unmasked(pl.per_u);
    }
    // dS' stores: every step a wave does not skip; lane (l32, hh) holds key
    // k0w + l32 and, in its operand vector ks, queries 16 ks + 4 hh + (0..3)
    // (elements 0..3) and 16 ks + 8 + 4 hh + (0..3) (elements 4..7)
    StepWalk wc(pl.nmasked);
    for (int st = 0; st < pl.nsteps; ++st) {
      const int q0 = pl.template q0<false>(wc);
      const int h = pl.hk * pl.G + wc.g;
      for (int w = 0; w < Loads::NW; ++w) {
        const int k0w = pl.k0 + 32 * w;
        if (pl.skipped(st, k0w)) continue;
        for (int l = 0; l < 64; ++l) {
          R.start_lane(l);
          const int l32 = l & 31, hh = l >> 5;
          const int key = k0w + l32;
          uint16_t e0[8], e1[8];
          for (int e = 0; e < 8; ++e) {
            const int qa = 4 * hh + (e < 4 ? e : 8 + e - 4);
            e0[e] = ds_tag(pl.b, h, q0 >> 5, key >> 4, qa, key & 15);
            e1[e] = ds_tag(pl.b, h, q0 >> 5, key >> 4, 16 + qa, key & 15);
          }
          const DkdvDsStores<CAUSAL, OFF32> dss(p, pl, k0w, l);
          dss.store(wc.g, q0, pack8(e0), pack8(e1), HostMem());
        }
      }
      wc.next(pl.per_m, pl.per_u, pl.G);
    }
  }
  CHECK(static_cast<int64_t>(units.size()) == grid, "dK/dV: %zu units for %d workgroups", units.size(), grid);
}

// two-waves-per-SIMD dK/dV kernel (ssa_bwd_dkdv2w.hip)
template <int D, bool CAUSAL, bool OFF32, bool SPREAD>
void run_dkdv2w(Problem& P) {
  using Loads = Dkdv2wLoads<D, CAUSAL, OFF32, SPREAD>;
  using Plan = typename Loads::Plan;
  const BwdParams& p = P.bp;
  const int grid = Plan::grid(p);
  Replay R;
  g_r = &R;
  std::set<std::tuple<int, int, int>> units;
  for (int blk = 0; blk < grid; ++blk) {
    const Plan pl(p, blk, grid);
    CHECK(units.insert({pl.b, pl.hk, pl.kb}).second, "dK/dV (2w): unit dispatched twice");
    if (pl.empty() || !replay_block(P.c, blk, grid)) continue;
    g_ctx = fmt("%s dkdv2w D=%d causal=%d off32=%d spread=%d block %d (b %d hk %d kb %d)", P.c.name.c_str(), D, CAUSAL,
                OFF32, SPREAD, blk, pl.b, pl.hk, pl.kb);
    R.reset_lds(Loads::LDS_BYTES);
    StepWalk wi(pl.nmasked);
    for (int st = 0; st < pl.nsteps + 2; ++st) {
      for (int w = 0; w < Loads::NW; ++w)
        for (int l = 0; l < 64; ++l) {
          R.start_lane(l);
          Loads ld(p, pl, w, l);
          ld.issue(pl, st, wi, 0u, HostMem());
          [&]<int... K>(std::integer_sequence<int, K...>) {
            (ld.template issue_piece<K>(pl.N, HostMem()), ...);
          }(std::make_integer_sequence<int, Loads::NLD>{});
        }
      if (st >= pl.nsteps) {
        CHECK(R.log.empty(), "dK/dV (2w) issues loads for step %d past the last (%d)", st, pl.nsteps);
      } else {
        const int q0 = pl.template q0<false>(wi), h = pl.hk * pl.G + wi.g;
        const uint32_t b0 = Loads::buf(0, st);
        std::vector<Region> regs{Region{&P.q, pl.b, pl.sv.tok0, pl.sv.packed, h, q0, Loads::BMQ, pl.N, b0},
                                 Region{&P.dout, pl.b, pl.sv.tok0, pl.sv.packed, h, q0, Loads::BMQ, pl.N, b0 + Loads::TILE}};
        md_regions(regs, P, pl.b, pl.sv, h, q0, Loads::BMQ, pl.N, b0 + 2 * Loads::TILE);
        check_regions(R, regs);
      }
      wi.next(pl.per_m, pl.per_u, pl.G);
    }
    // stores: masked steps store the tiles which() names, unmasked ones both;
    // lane 16 g + i holds key k0w + i, queries 16 t + 4 g + (0..3) of the
    // 32-query half hq in elements 4 t ..
    StepWalk wc(pl.nmasked);
    for (int st = 0; st < pl.nsteps; ++st) {
      const int q0 = pl.template q0<false>(wc);
      const int h = pl.hk * pl.G + wc.g;
      for (int w = 0; w < Loads::NW; ++w) {
        const int k0w = pl.k0 + 16 * w;
        for (int l = 0; l < 64; ++l) {
          R.start_lane(l);
          const Dkdv2wDsStores<CAUSAL, OFF32> dss(p, pl, k0w, l);
          const int which = st < pl.nmasked ? dss.which(q0) : 3;
          for (int hq = 0; hq < 2; ++hq) {
            if (!(which & (1 << hq))) continue;
            const int g4 = l >> 4, i = l & 15, qt = (q0 >> 5) + hq, key = k0w + i;
            uint16_t e8[8];
            for (int e = 0; e < 8; ++e) e8[e] = ds_tag(pl.b, h, qt, key >> 4, 16 * (e >> 2) + 4 * g4 + (e & 3), key & 15);
            dss.store(wc.g, q0, hq, pack8(e8), HostMem());
          }
        }
      }
      wc.next(pl.per_m, pl.per_u, pl.G);
    }
  }
  CHECK(static_cast<int64_t>(units.size()) == grid, "dK/dV (2w): %zu units for %d workgroups", units.size(), grid);
}

// The dS' K pass: K tiles, and each wave's dS' tiles with their tags
template <int D, bool CAUSAL>
void run_dq_ds(Problem& P, bool check_written) {
  constexpr int NW = dq_ds_waves<D>();
  using Loads = DqDsLoads<D, CAUSAL, NW>;
  const BwdParams& p = P.bp;
  const int grid = Loads::grid(p);
  Replay R;
  g_r = &R;
  std::set<std::tuple<int, int, int>> units;
  for (int blk = 0; blk < grid; ++blk) {
    const Loads l0(p, blk, grid, 0, 0);
    CHECK(units.insert({l0.b, l0.h, l0.qb}).second, "dS' K pass: unit dispatched twice");
    if (l0.empty() || !replay_block(P.c, blk, grid)) continue;
    g_ctx = fmt("%s dq_ds D=%d causal=%d block %d (b %d h %d qb %d)", P.c.name.c_str(), D, CAUSAL, blk, l0.b, l0.h, l0.qb);
    R.reset_lds(Loads::LDS_BYTES);
    for (int t = 0; t <= l0.ntiles; ++t) {  // K(t + PFK), t < ntiles
      for (int w = 0; w < NW; ++w)
        for (int l = 0; l < 64; ++l) {
          R.start_lane(l);
          const Loads ld(p, blk, grid, w, l);
          ld.issue_k(t, 0u, HostMem());
        }
      check_regions(R, {Region{&P.k, l0.b, l0.sv.tok0, l0.sv.packed, l0.hk, t * Loads::BN, Loads::BN, l0.N,
                               Loads::ktile(0, t)}});
    }
    for (int t = 0; t < l0.ntiles + Loads::PFD; ++t) {
      for (int w = 0; w < NW; ++w) {
        for (int l = 0; l < 64; ++l) {
          R.start_lane(l);
          const Loads ld(p, blk, grid, w, l);
          ld.issue_ds(t, 0u, HostMem());
        }
        const Loads lw(p, blk, grid, w, 0);
        const uint32_t st0 = lw.dstage(0, t);
        for (const Access& a : R.log) {
          CHECK(a.t == &P.ws && a.bytes == 16, "dS' K pass: a dS' load reads %s", a.t->name.c_str());
          CHECK(a.lds >= st0 && a.lds < st0 + 4096, "dS' load to LDS %u outside the wave's stage", a.lds);
        }
        // tiles the pass multiplies (t < ntiles, kj < nkj): written, and
        // LDS slot 16 g + m holds key m ^ 4 g, queries 16 t' + 4 g + (0..3)
        const int qi = (lw.wq0 < lw.N ? lw.wq0 : lw.N - 1) >> 5;
        for (int s4 = 0; s4 < 4; ++s4) {
          const int kj = 4 * t + s4;
          if (t >= l0.ntiles || kj >= lw.nkj) continue;
          for (const Access& a : R.log) {
            if (a.lds < st0 + s4 * 1024u || a.lds >= st0 + (s4 + 1) * 1024u) continue;
            if (check_written) {
              bool all = true;
              for (int i = 0; i < 16; ++i) all = all && P.ws.written[a.off + i];
              CHECK(all, "dS' tile (qi %d, kj %d) read before any store wrote it", qi, kj);
            }
            if (P.ws.is_virtual) continue;
            const int slot = static_cast<int>((a.lds - st0 - s4 * 1024u) / 16), g = slot >> 4, m = slot & 15;
            uint16_t e8[8];
            memcpy(e8, R.lds.get() + a.lds, 16);
            for (int e = 0; e < 8; ++e) {
              const uint16_t want = ds_tag(l0.b, l0.h, qi, kj, 16 * (e >> 2) + 4 * g + (e & 3), m ^ (4 * g));
              CHECK(e8[e] == want, "dS' (qi %d, kj %d) LDS slot %d element %d: tag %#x, want %#x", qi, kj, slot, e,
                    e8[e], want);
            }
          }
        }
        R.log.clear();
      }
    }
  }
  CHECK(static_cast<int64_t>(units.size()) == grid, "dS' K pass: %zu units for %d workgroups", units.size(), grid);
}

// The recompute dQ pass
template <int D, bool CAUSAL>
void run_dq(Problem& P) {
  using Plan = DqPlan<D, CAUSAL>;
  const BwdParams& p = P.bp;
  const int grid = Plan::grid(p);
  Replay R;
  g_r = &R;
  std::set<std::tuple<int, int, int>> units;
  for (int blk = 0; blk < grid; ++blk) {
    const Plan pl(p, blk, grid);
    CHECK(units.insert({pl.b, pl.h, pl.qb}).second, "dQ: unit dispatched twice");
    if (pl.empty() || !replay_block(P.c, blk, grid)) continue;
    g_ctx = fmt("%s dq D=%d causal=%d block %d (b %d h %d qb %d)", P.c.name.c_str(), D, CAUSAL, blk, pl.b, pl.h, pl.qb);
    R.reset_lds(Plan::LDS_BYTES);
    for (int t = 0; t < pl.ntiles; ++t) {
      for (int w = 0; w < Plan::NW; ++w)
        for (int l = 0; l < 64; ++l) {
          R.start_lane(l);
          const LoadLane llk(l, w, p.k.ss), llv(l, w, p.v.ss);
          pl.load_tile(t, 0u, w, llk, llv, HostMem());
        }
      check_regions(R, {Region{&P.k, pl.b, pl.sv.tok0, pl.sv.packed, pl.hk, t * Plan::BN, Plan::BN, pl.N, Plan::buf(0, t)},
                        Region{&P.v, pl.b, pl.sv.tok0, pl.sv.packed, pl.hk, t * Plan::BN, Plan::BN, pl.N,
                               Plan::buf(0, t) + Plan::TILE}});
    }
  }
  CHECK(static_cast<int64_t>(units.size()) == grid, "dQ: %zu units for %d workgroups", units.size(), grid);
}

// ---------------------------------------------------------------------------
// Decode: a KV cache [B, Hkv, cap, D] and per-sequence lengths.
template <int D>
void run_decode(int B, int Hq, int Hkv, int cap, int splits_req, const std::vector<int>& lens) {
  using C = DecodeCfg<D>;
  using Plan = DecodePlan<D>;
  g_tensors.clear();
  Tensor k = make_rows("Kcache", 0, B, Hkv, cap, D, 0), v = make_rows("Vcache", 0, B, Hkv, cap, D, 0);
  alloc(k, false);
  alloc(v, false);
  DecodeParams p{};
  p.k = Tensor4{k.base, k.sb, k.sh, k.ss};
  p.v = Tensor4{v.base, v.sb, v.sh, v.ss};
  p.seqlens = lens.data();
  p.B = B, p.Hq = Hq, p.Hkv = Hkv, p.cap = cap;
  p.splits = decode_splits(B, Hq, Hkv, cap, splits_req);
  p.split_keys = decode_split_keys(cap, p.splits);
  const int grid = Plan::grid(p);
  Replay R;
  g_r = &R;
  std::set<std::tuple<int, int, int, int>> units;
  for (int blk = 0; blk < grid; ++blk) {
    const Plan pl(p, blk);
    CHECK(units.insert({pl.b, pl.hk, pl.qg, pl.split}).second, "decode: unit dispatched twice");
    g_ctx = fmt("decode D=%d B=%d Hq=%d Hkv=%d cap=%d splits=%d block %d (b %d hk %d split %d)", D, B, Hq, Hkv, cap,
                p.splits, blk, pl.b, pl.hk, pl.split);
    R.reset_lds(C::SMEM);
    for (int w = 0; w < C::NW; ++w) {
      const int ntw = pl.tiles_of(w);
      if (ntw == 0) continue;
      const uint32_t ring = static_cast<uint32_t>(w * C::NB * C::TB);
      for (int i = 0; i < ntw + C::NB - 1; ++i) {
        for (int l = 0; l < 64; ++l) {
          R.start_lane(l);
          const LoadLane lk0(l, 0, p.k.ss), lk1(l, 1, p.k.ss), lv0(l, 0, p.v.ss), lv1(l, 1, p.v.ss);
          pl.issue(i, w, ring, lk0, lk1, lv0, lv1, HostMem());
        }
        const int row0 = pl.kbeg + 32 * (w + C::NW * i);
        const uint32_t dst = ring + (i % C::NB) * C::TB;
        // rows past the split's end clamp to kend - 1 (loaded, never read)
        check_regions(R, {Region{&k, pl.b, 0, false, pl.hk, row0 < pl.kend ? row0 : pl.kend - 1, 32, pl.kend, dst},
                          Region{&v, pl.b, 0, false, pl.hk, row0 < pl.kend ? row0 : pl.kend - 1, 32, pl.kend,
                                 dst + C::BLOCK}});
      }
    }
  }
  CHECK(static_cast<int64_t>(units.size()) == grid, "decode: %zu units for %d workgroups", units.size(), grid);
}

// ---------------------------------------------------------------------------
template <int D, bool CAUSAL>
void run_case_dc(Problem& P) {
  const bool sampled = P.c.sample > 0;
  run_fwd<D, CAUSAL>(P);
  run_dq<D, CAUSAL>(P);
  // dK/dV in both address forms (the launcher picks OFF32 when dkdv_off32
  // holds), each followed by the dS' K pass on its workspace
  const bool off32 = dkdv_off32(P.bp, D, CAUSAL);
  auto fresh_ws = [&]() {
    if (!P.ws.is_virtual) {
      std::fill(P.ws.written.begin(), P.ws.written.end(), 0);
      memset(P.ws.mem.get(), 0, P.ws.bytes);
    }
  };
  if (off32) {
    fresh_ws();
    run_dkdv<D, CAUSAL, true>(P);
    run_dq_ds<D, CAUSAL>(P, !sampled);
  }
  if (!sampled || !off32) {
    fresh_ws();
    run_dkdv<D, CAUSAL, false>(P);
    run_dq_ds<D, CAUSAL>(P, !sampled);
  }
  if (off32) {
    fresh_ws();
    run_dkdv2w<D, CAUSAL, true, true>(P);
    run_dq_ds<D, CAUSAL>(P, !sampled);
    if (!sampled) {
      fresh_ws();
      run_dkdv2w<D, CAUSAL, true, false>(P);
      run_dq_ds<D, CAUSAL>(P, true);
    }
  }
  if (!sampled || !off32) {
    fresh_ws();
    run_dkdv2w<D, CAUSAL, false, true>(P);
    run_dq_ds<D, CAUSAL>(P, !sampled);
  }
}

void run_case(const Case& c) {
  Problem P;
  P.c = c;
  setup(P);
  const long f0 = g_fail;
  switch (c.D * 2 + c.causal) {
    case 64: run_case_dc<32, false>(P); break;
    case 65: run_case_dc<32, true>(P); break;
    case 128: run_case_dc<64, false>(P); break;
    case 129: run_case_dc<64, true>(P); break;
    case 256: run_case_dc<128, false>(P); break;
    case 257: run_case_dc<128, true>(P); break;
    default: failf("head dim %d not built", c.D);
  }
  printf("case %-34s %s\n", c.name.c_str(), g_fail == f0 ? "ok" : "FAILED");
  fflush(stdout);
}

Case dense(const char* name, int B, int Hq, int Hkv, int N, int D, bool causal, int layout) {
  return Case{name, B, Hq, Hkv, N, D, causal, layout, {}, 0, 0};
}
Case packed(const char* name, std::vector<int> cu, int T, int Nmax, int Hq, int Hkv, int D, bool causal) {
  const int B = static_cast<int>(cu.size()) - 1;
  return Case{name, B, Hq, Hkv, Nmax, D, causal, 2, std::move(cu), T, 0};
}

}  // namespace

int main(int argc, char** argv) {
  const bool quick = argc > 1 && strcmp(argv[1], "--quick") == 0;
  std::vector<Case> cases = {
      dense("mha s256 d128 causal", 1, 4, 4, 256, 128, true, 0),
      dense("gqa s200 d128 causal", 2, 4, 2, 200, 128, true, 0),
      dense("gqa s129 d64", 1, 2, 1, 129, 64, false, 0),
      dense("gqa s511 d64 causal strided", 2, 8, 2, 511, 64, true, 1),
      dense("gqa s33 d32 causal", 1, 3, 1, 33, 32, true, 0),
      dense("mha s7 d128 strided", 2, 2, 2, 7, 128, false, 1),
      dense("mha s1 d64 causal", 1, 2, 2, 1, 64, true, 0),
      dense("gqa s300 d32", 1, 6, 2, 300, 32, false, 0),
      dense("mha s320 d32 causal strided", 1, 4, 4, 320, 32, true, 1),
      dense("gqa s384 d128 strided", 2, 4, 2, 384, 128, false, 1),
      packed("packed d64 causal", {0, 37, 157, 160}, 160, 120, 4, 2, 64, true),
      packed("packed d128 causal", {0, 300, 813}, 813, 513, 2, 1, 128, true),
      packed("packed d128", {0, 129, 160, 360}, 360, 200, 4, 2, 128, false),
      packed("packed malformed d64 causal", {-5, 40, 250}, 100, 100, 2, 2, 64, true),
      packed("packed uncovered tail d64", {0, 37, 120}, 200, 60, 4, 2, 64, true),
      packed("packed six docs d128 causal", {0, 5, 105, 138, 398, 399}, 399, 260, 4, 2, 128, true),
      packed("packed d32 causal", {0, 70, 71, 199}, 199, 128, 4, 4, 32, true),
  };
  if (!quick) {
    // the benchmark sizes, address-only, a sample of workgroups
    Case a = dense("bench b4 h16 s4096 d128 causal", 4, 16, 16, 4096, 128, true, 0);
    a.sample = 97;
    Case b = dense("bench gqa b4 h32/8 s4096 d64 causal", 4, 32, 8, 4096, 64, true, 0);
    b.sample = 89;
    Case c = dense("long b1 h16 s16384 d128 causal", 1, 16, 16, 16384, 128, true, 0);
    c.sample = 61;
    cases.push_back(a);
    cases.push_back(b);
    cases.push_back(c);
  }
  for (const Case& c : cases) run_case(c);
  // decode against a KV cache: ragged lengths, lengths beyond the capacity
  // and below zero (clamped), one and several splits, q-head groups past 32
  g_ctx = "decode";
  run_decode<128>(3, 8, 2, 700, 0, {700, 1, 333});
  run_decode<64>(2, 64, 1, 300, 3, {-4, 1000});
  run_decode<32>(4, 4, 4, 129, 1, {0, 129, 64, 65});
  printf("decode cases %s\n", g_fail == 0 ? "ok" : "FAILED");
  printf("%ld checks, %ld failures\n", g_checks, g_fail);
  return g_fail == 0 ? 0 : 1;
}
