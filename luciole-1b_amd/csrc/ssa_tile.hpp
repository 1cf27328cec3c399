// LDS tile staging shared by the kernels that stream K/V (or Q/dO) tiles.
//
// Layout.  A tile is a stack of 32-row blocks of D bf16/fp16 columns.  Inside
// a block the 16-byte chunks are stored chunk-major: chunk c (columns 8c..8c+7)
// of all 32 rows occupies 512 contiguous bytes, and row r sits at position
//   pos(r, c) = r ^ (4 * (c & 3))
// in it.  So
//   off(r, c) = (r / 32) * BLOCK + c * 512 + ((r % 32) ^ 4 (c & 3)) * 16.
// MFMA operand fetches then hit no LDS bank conflicts:
//   * ds_read_b128 of one chunk for 16 consecutive rows (one row per lane, 16
//     lanes per LDS cycle) reads 256 contiguous bytes;
//   * a ds_read_b64_tr_b16 transpose read (32 lanes per LDS cycle) takes 4
//     aligned rows from 4 aligned chunks, whose positions differ in bits 2-3
//     and so fall in 4 disjoint 64-byte bank groups,
// and every operand address is one of two per-lane base offsets plus a
// compile-time immediate (the row XOR depends only on the lane and on one bit
// of the step index), which keeps address arithmetic out of the inner loops.
//
// Tiles are filled with global_load_lds_dwordx4: each instruction moves 1 KB
// (two chunk columns of one block), lane L writing LDS bytes [16 L, 16 L + 16)
// of that KB; the layout is applied on the global side (which 16 bytes each
// lane fetches).  Rows past the end of the sequence are clamped to the last
// valid row; callers mask them.
#pragma once

#include "ssa_common.hpp"

namespace ssa {

template <int D>
struct BlockLayout {
  static constexpr int CPR = D / 8;          // 16-byte chunks per row
  static constexpr int BLOCK = 32 * D * 2;   // bytes per 32-row block
  static constexpr int IPB = BLOCK / 1024;   // 1 KB load instructions per block
};

// Per-lane constants of the direct loads issued by one wave.  Wave w issues
// the 1 KB pieces j = w, w + NW, ... of a tile; piece j covers chunks
// c = 2 (j % IPB) + half (half = lane / 32) of block j / IPB.  With NW and IPB
// even, c & 3 = 2 (w & 1) + half for all of them, so the row a lane fetches
// inside a block, pos ^ 4 (c & 3), is fixed per lane.  Row strides below
// 2^24 elements (checked on the host) keep every offset under 2^31.
//
// The row swizzle 4 (c & 3) fits the gfx950 LDS as measured: a read is served
// one half-wave (32 lanes) at a time; a 16-byte read runs at full rate when
// the two 16-lane groups of a half-wave apply the same permutation to their
// 256-byte windows (RowBase: both groups read one chunk), and an 8-byte
// transpose read when the chunks its lanes touch land on different banks
// (TrBase: four chunks, four swizzles).
struct LoadLane {
  uint32_t off;   // r * row stride + half * 16, bytes
  uint32_t hoff;  // half * 16, bytes
  int r;          // row within the block
  __host__ __device__ __forceinline__ LoadLane(int lane, int wave, int64_t ss) {
    const int pos = lane & 31, half = lane >> 5;
    r = pos ^ (4 * (2 * (wave & 1) + half));
    hoff = static_cast<uint32_t>(half * 16);
    off = static_cast<uint32_t>(r * ss * 2) + hoff;
  }
  // The Swz8 layout (Swz8Tile below): row r of chunk c at position
  // r ^ 8 (c & 1).  A 1 KB piece covers chunks 2 cp and 2 cp + 1, so the
  // row a lane fetches depends on its half only, not on the wave.
  struct Swz8 {};
  __host__ __device__ __forceinline__ LoadLane(int lane, int64_t ss, Swz8) {
    const int pos = lane & 31, half = lane >> 5;
    r = pos ^ (8 * half);
    hoff = static_cast<uint32_t>(half * 16);
    off = static_cast<uint32_t>(r * ss * 2) + hoff;
  }
};

// Issue the loads of one ROWS x D tile (rows row0.. of a [*, D] matrix with
// row stride `ss` elements) into `lds` (byte address).  Called by all NW waves
// of the workgroup with `wave` wave-uniform (an SGPR); a wave may issue none
// when the tile has fewer 1 KB pieces than there are waves.  Rows at or past
// `nrows` are clamped to nrows - 1.
// Direct-to-LDS loads, written as inline assembly.  The compiler's wait-count
// insertion, when it sees an LDS DMA builtin in flight, puts a full vmcnt(0)
// wait in front of later LDS transpose reads, which would drain the tile
// prefetch; issued from assembly the loads are invisible to it, and the
// kernels order them explicitly (wait_vm<N>() + barrier before a tile is
// read).  M0 holds the LDS destination (wave-uniform).  It is an input operand
// of each statement ("{m0}" constraint), so the compiler writes M0 itself and
// knows it is live there.
//
// Wait states.  The compiler inserts the NOPs that hardware hazards need only
// around instructions it can see: for an inline-assembly statement it checks
// the registers the statement writes, not the ones it reads.  A vector-memory
// instruction that reads an SGPR written by a VALU instruction (v_readfirstlane
// of an offset, v_readlane reloading a spilled descriptor word) needs 5 wait
// states in between, and one that reads M0 after an SALU write of M0 needs 1;
// without them it can take the SGPR's previous value, i.e. a wrong address.
// Every statement below that issues a vector-memory instruction with SGPR
// operands therefore starts with s_nop 4 (5 wait states) itself.
typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Raw buffer descriptor: base address, stride 0, no bounds check in practice.
__host__ __device__ __forceinline__ i32x4_t raw_rsrc(const void* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return i32x4_t{static_cast<int>(static_cast<uint32_t>(a)), static_cast<int>((a >> 32) & 0xffff), 0x7fffffff,
                 0x00020000};
}

// 16 bytes per lane from rsrc.base + voff + soff to LDS [m0 + 16 lane].
// NT: non-temporal (streaming) cache policy, for data read exactly once.
template <bool NT = false>
__device__ __forceinline__ void dma_buffer16(uint32_t lds, const i32x4_t& rsrc, uint32_t voff, int soff) {
  if constexpr (NT)
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
                 :
                 : "{m0}"(lds), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory");
  else
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "{m0}"(lds), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory");
}

// 16 bytes per lane from a per-lane global address to LDS [m0 + 16 lane].
__device__ __forceinline__ void dma_global16(uint32_t lds, const void* src) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "{m0}"(lds), "v"(reinterpret_cast<uint64_t>(src))
               : "memory");
}

// 4 bytes per lane from a per-lane global address to LDS [m0 + 4 lane].
__device__ __forceinline__ void dma_global4(uint32_t lds, const void* src) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dword %1, off"
               :
               : "{m0}"(lds), "v"(reinterpret_cast<uint64_t>(src))
               : "memory");
}

// 8 bytes to global memory at p + OFF bytes: exactly one vector-memory
// instruction, never merged with a neighbour, so a kernel can count its
// stores for a vmcnt wait.  8-byte data has no store-data hazard.
template <int OFF>
__device__ __forceinline__ void store_b64(void* p, u32x2 v) {
  asm volatile("global_store_dwordx2 %0, %1, off offset:%2" : : "v"(reinterpret_cast<uint64_t>(p)), "v"(v), "i"(OFF)
               : "memory");
}

// 8 bytes to rs.base + voff + soff + OFF: one vector-memory instruction.
template <int OFF>
__device__ __forceinline__ void buffer_store_b64(const i32x4_t& rs, uint32_t voff, int soff, u32x2 v) {
  asm volatile("s_nop 4\n\tbuffer_store_dwordx2 %0, %1, %2, %3 offen offset:%4"
               :
               : "v"(v), "v"(voff), "s"(rs), "s"(soff), "i"(OFF)
               : "memory");
}

// 16 bytes per lane with the non-temporal (streaming) cache policy, one
// vector-memory instruction each (as store_b64 / buffer_store_b64): for data
// written once and read back once by a later kernel, so that it does not
// evict reused tiles from L2.  On gfx940 and later a store of more than 8
// bytes needs 2 wait states before a VALU instruction overwrites its data
// registers (the compiler pads only the stores it sees): the trailing s_nop 1
// keeps them inside the statement, and the build's assembly scan
// (SSA/_hazards.py) rejects any store whose data is overwritten sooner.
template <int OFF>
__device__ __forceinline__ void store_b128_nt(void* p, u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off offset:%2 nt\n\ts_nop 1" : : "v"(reinterpret_cast<uint64_t>(p)),
               "v"(v), "i"(OFF)
               : "memory");
}
template <int OFF>
__device__ __forceinline__ void buffer_store_b128_nt(const i32x4_t& rs, uint32_t voff, int soff, u32x4 v) {
  asm volatile("s_nop 4\n\tbuffer_store_dwordx4 %0, %1, %2, %3 offen offset:%4 nt\n\ts_nop 1"
               :
               : "v"(v), "v"(voff), "s"(rs), "s"(soff), "i"(OFF)
               : "memory");
}

// The global-memory operations of the tile helpers below and of the kernels'
// load / store plans (ssa_plan.hpp), as a policy: DeviceMem issues them with
// the statements above.  The helpers and plans are __host__ __device__, so a
// host program can replay them with a policy that records every address
// instead (tests/host_addr: every workgroup, wave and lane of a problem).
// `uniform` states that a value is wave-uniform (an SGPR on the device).
struct DeviceMem {
  __device__ __forceinline__ void load16(uint32_t lds, const i32x4_t& rs, uint32_t voff, int soff) const {
    dma_buffer16<false>(lds, rs, voff, soff);
  }
  __device__ __forceinline__ void load16_nt(uint32_t lds, const i32x4_t& rs, uint32_t voff, int soff) const {
    dma_buffer16<true>(lds, rs, voff, soff);
  }
  __device__ __forceinline__ void load16_global(uint32_t lds, const void* src) const { dma_global16(lds, src); }
  __device__ __forceinline__ void load4_global(uint32_t lds, const void* src) const { dma_global4(lds, src); }
  template <int OFF>
  __device__ __forceinline__ void store16_nt(const i32x4_t& rs, uint32_t voff, int soff, u32x4 v) const {
    buffer_store_b128_nt<OFF>(rs, voff, soff, v);
  }
  template <int OFF>
  __device__ __forceinline__ void store16_nt_global(void* p, u32x4 v) const {
    store_b128_nt<OFF>(p, v);
  }
  __device__ __forceinline__ int uniform(int x) const { return __builtin_amdgcn_readfirstlane(x); }
};

template <int D, int ROWS, int NW, bool CLAMP, typename Mem = DeviceMem>
__host__ __device__ __forceinline__ void tile_load_pieces(const char* g, int64_t ss, int row0, int nrows, uint32_t lds,
                                                          int wave, const LoadLane& ll, const Mem& mem = Mem()) {
  using BL = BlockLayout<D>;
  constexpr int NINST = ROWS / 32 * BL::IPB;
  constexpr int PER = (NINST + NW - 1) / NW;
  const i32x4_t rs = raw_rsrc(g + static_cast<int64_t>(row0) * ss * 2);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int j = wave + NW * i;
    if (NINST % NW != 0 && j >= NINST) break;
    const int blk = j / BL::IPB, cp = j % BL::IPB;
    if (!CLAMP) {
      // descriptor base at row0 (scalar), per-lane row offset fixed for the
      // kernel (VGPR), block/chunk offset in soffset
      mem.load16(lds + j * 1024, rs, ll.off, static_cast<int>(blk * 32 * ss * 2 + cp * 32));
    } else {
      int grow = row0 + blk * 32 + ll.r;
      grow = grow < nrows ? grow : nrows - 1;
      mem.load16_global(lds + j * 1024, g + (static_cast<int64_t>(grow) * ss + cp * 16) * 2 + ll.hoff);
    }
  }
}

// tile_load_pieces for a tile of full rows at byte soff0 of the buffer rs,
// with 32-bit offsets (the caller keeps every byte of the tile below 2 GiB of
// the descriptor base): one scalar add per piece, no 64-bit address math.
template <int D, int ROWS, int NW, typename Mem = DeviceMem>
__host__ __device__ __forceinline__ void tile_load_pieces_off(const i32x4_t& rs, int soff0, int ss2, uint32_t lds,
                                                              int wave, const LoadLane& ll, const Mem& mem = Mem()) {
  using BL = BlockLayout<D>;
  constexpr int NINST = ROWS / 32 * BL::IPB;
  constexpr int PER = (NINST + NW - 1) / NW;
  // wave-uniform by construction; stated so that the offset is an SGPR
  const int base = mem.uniform(soff0);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int j = wave + NW * i;
    if (NINST % NW != 0 && j >= NINST) break;
    const int blk = j / BL::IPB, cp = j % BL::IPB;
    mem.load16(lds + j * 1024, rs, ll.off, base + blk * 32 * ss2 + cp * 32);
  }
}

template <int D, int ROWS, int NW, typename Mem = DeviceMem>
__host__ __device__ __forceinline__ void tile_load_async(const void* gbase, int64_t ss, int row0, int nrows,
                                                         uint32_t lds, int wave, const LoadLane& ll,
                                                         const Mem& mem = Mem()) {
  static_assert(NW % 2 == 0 && BlockLayout<D>::IPB % 2 == 0, "chunk parity must be fixed per wave");
  const char* g = static_cast<const char*>(gbase);
  if (row0 + ROWS <= nrows)
    tile_load_pieces<D, ROWS, NW, false>(g, ss, row0, nrows, lds, wave, ll, mem);
  else
    tile_load_pieces<D, ROWS, NW, true>(g, ss, row0, nrows, lds, wave, ll, mem);
}

// Wait until at most N vector-memory instructions of this wave (direct tile
// loads included) are outstanding.  gfx9 s_waitcnt: vmcnt in bits 3:0 and
// 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima (no wait).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 31]; larger n wait for all.
__device__ __forceinline__ void wait_vm_dyn(int n) {
  switch (n) {
    case 1: wait_vm<1>(); break;
    case 2: wait_vm<2>(); break;
    case 3: wait_vm<3>(); break;
    case 4: wait_vm<4>(); break;
    case 5: wait_vm<5>(); break;
    case 6: wait_vm<6>(); break;
    case 7: wait_vm<7>(); break;
    case 8: wait_vm<8>(); break;
    case 9: wait_vm<9>(); break;
    case 10: wait_vm<10>(); break;
    case 11: wait_vm<11>(); break;
    case 12: wait_vm<12>(); break;
    case 13: wait_vm<13>(); break;
    case 14: wait_vm<14>(); break;
    case 15: wait_vm<15>(); break;
    case 16: wait_vm<16>(); break;
    case 17: wait_vm<17>(); break;
    case 18: wait_vm<18>(); break;
    case 19: wait_vm<19>(); break;
    case 20: wait_vm<20>(); break;
    case 21: wait_vm<21>(); break;
    case 22: wait_vm<22>(); break;
    case 23: wait_vm<23>(); break;
    case 24: wait_vm<24>(); break;
    case 25: wait_vm<25>(); break;
    case 26: wait_vm<26>(); break;
    case 27: wait_vm<27>(); break;
    case 28: wait_vm<28>(); break;
    case 29: wait_vm<29>(); break;
    case 30: wait_vm<30>(); break;
    case 31: wait_vm<31>(); break;
    default: wait_vm<0>(); break;
  }
}

// A VGPR copy of x that the compiler cannot re-associate with later
// arithmetic: per-tile base addresses stay in registers and the operand
// fetches use their immediate offset fields.
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Per-lane base offsets for the row-wise operand fetch "row 32*blk + l32,
// chunk 2*ds + hh": index by the parity of ds.
template <int D>
struct RowBase {
  uint32_t b[2];
  __device__ __forceinline__ RowBase(int l32, int hh) {
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int c = 2 * par + hh;  // c & 3 for chunk 2*ds + hh with ds & 1 == par
      b[par] = static_cast<uint32_t>(hh * 512 + ((l32 ^ (4 * c)) << 4));
    }
  }
};

// The same bases moved to a tile at LDS byte address `lds`.
template <int D>
__device__ __forceinline__ RowBase<D> at_tile(const RowBase<D>& rb, uint32_t lds) {
  RowBase<D> r = rb;
  r.b[0] = opaque(rb.b[0] + lds);
  r.b[1] = opaque(rb.b[1] + lds);
  return r;
}

// 16-byte fetch of chunk 2*ds + hh of row 32*blk + l32 (an MFMA operand of 8
// consecutive elements) of the tile whose bases are `rb` (see at_tile).  ds
// and blk are compile-time at the call sites.
template <int D, typename V>
__device__ __forceinline__ V tile_read_row(const RowBase<D>& rb, int blk, int ds) {
  const uint32_t imm = blk * BlockLayout<D>::BLOCK + ds * 2 * 512;
  return *(const __attribute__((address_space(3))) V*)(uintptr_t)(rb.b[ds & 1] + imm);
}

// Per-lane base offsets for transpose fetches: within each 16-lane group g,
// lane i supplies row rbase + i/4 (rbase = 16 ks + 8 hi + 4 hh inside a block)
// and the 8 bytes at columns dgrp + 4 (i%4) with dgrp = 32 db + 16 (g&1);
// indexed by hi.
template <int D>
struct TrBase {
  uint32_t b[2];
  __device__ __forceinline__ TrBase(int lane) {
    const int g = lane >> 4, i = lane & 15, hh = lane >> 5;
    const int cl = (g & 1) * 2 + ((i & 3) >> 1);  // chunk within the 32-column group (= c & 3)
#pragma unroll
    for (int hi = 0; hi < 2; ++hi) {
      const int rl = 8 * hi + 4 * hh + (i >> 2);
      b[hi] = static_cast<uint32_t>(cl * 512 + ((rl ^ (4 * cl)) << 4) + ((i & 1) << 3));
    }
  }
};

template <int D>
__device__ __forceinline__ TrBase<D> at_tile(const TrBase<D>& tb, uint32_t lds) {
  TrBase<D> r = tb;
  r.b[0] = opaque(tb.b[0] + lds);
  r.b[1] = opaque(tb.b[1] + lds);
  return r;
}

// Transposed fetch: column 32*db + l32 of rows 32*blk + 16*ks + 8*hi + 4*hh + (0..3)
// of the tile whose bases are `tb`, as 4 elements (k-slots 4*hi .. 4*hi+3 of
// an MFMA operand whose contraction index runs over the rows).
template <int D, typename V4>
__device__ __forceinline__ V4 tile_read_tr(const TrBase<D>& tb, int blk, int ks, int hi, int db) {
  const uint32_t imm = blk * BlockLayout<D>::BLOCK + db * 4 * 512 + ks * 16 * 16;
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  const bf16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
      (__attribute__((address_space(3))) bf16x4_t*)(uintptr_t)(tb.b[hi] + imm));
  return __builtin_bit_cast(V4, v);
}

// Row-major tile of D = 128 (256-byte rows) with the 64-byte quarters of
// row r permuted q -> q ^ (r & 3): chunk c (16 bytes) of row r sits at
// r * 256 + (c ^ 4 (r & 3)) * 16.  A 1 KB direct load then covers four whole
// rows with every 4-lane group reading 64 contiguous bytes in lane order
// (measured on the dS' K pass: 7% faster than the block-chunk-major pieces,
// which touch 32 rows each; a 16-byte-chunk permutation of the same four
// rows, which breaks the lane order inside 4-lane groups, gained nothing), and
// the transpose read of a 16-lane group (4 rows x 32 bytes) lands on four
// distinct 32-byte bank groups.  For operands read only by transpose reads:
// 16 rows of one chunk (a row-wise MFMA operand fetch) share 4 bank slots.
struct RowSwzLoad {
  uint32_t voff;  // lane's byte offset from a piece's first row
  int rsub;       // row within the piece (lane / 16)
  int chunk;      // chunk of that row the lane fetches
  __host__ __device__ __forceinline__ RowSwzLoad(int lane, int64_t ss) {
    rsub = lane >> 4;
    chunk = (lane & 15) ^ (4 * rsub);  // rows of a piece start at a multiple of 4: r & 3 = rsub
    voff = static_cast<uint32_t>(rsub * ss * 2 + chunk * 16);
  }
};

// Rows row0 .. row0 + ROWS - 1 (clamped to nrows - 1) of a [*, 128] matrix
// with row stride `ss` elements into a RowSwz tile at `lds`: piece j (rows
// 4 j .. 4 j + 3) from wave j % NW.
template <int ROWS, int NW, typename Mem = DeviceMem>
__host__ __device__ __forceinline__ void rowswz_load(const char* g, int64_t ss, int row0, int nrows, uint32_t lds,
                                                     int wave, const RowSwzLoad& rl, const Mem& mem = Mem()) {
  static_assert(ROWS % (4 * NW) == 0, "whole pieces per wave");
  constexpr int PER = ROWS / 4 / NW;
  if (row0 + ROWS <= nrows) {
    const i32x4_t rs = raw_rsrc(g + static_cast<int64_t>(row0) * ss * 2);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int j = wave + NW * i;
      mem.load16(lds + j * 1024, rs, rl.voff, static_cast<int>(4 * j * ss * 2));
    }
  } else {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int j = wave + NW * i;
      int row = row0 + 4 * j + rl.rsub;
      row = row < nrows ? row : nrows - 1;
      mem.load16_global(lds + j * 1024, g + (static_cast<int64_t>(row) * ss + rl.chunk * 8) * 2);
    }
  }
}

// Transpose-read bases of a RowSwz tile, one per 32-column block db: lane i
// of 16-lane group g supplies row 4 hh + i / 4 (+ the immediate rows, a
// multiple of 8) and the 8 bytes at columns 32 db + 16 (g & 1) + 4 (i % 4).
struct RowSwzTr {
  uint32_t b[4];
  __device__ __forceinline__ explicit RowSwzTr(int lane) {
    const int g = lane >> 4, i = lane & 15, hh = lane >> 5;
    const int r8 = 4 * hh + (i >> 2);  // row & 7; row & 3 = i / 4
#pragma unroll
    for (int db = 0; db < 4; ++db)
      b[db] = static_cast<uint32_t>(r8 * 256 + (((4 * db + 2 * (g & 1) + ((i & 3) >> 1)) ^ (4 * (i >> 2))) * 16) +
                                    8 * (i & 1));
  }
};

__device__ __forceinline__ RowSwzTr at_tile(const RowSwzTr& t, uint32_t lds) {
  RowSwzTr r = t;
#pragma unroll
  for (int db = 0; db < 4; ++db) r.b[db] = opaque(t.b[db] + lds);
  return r;
}

// Column 32 db + l32 of rows 32 blk + 16 ks + 8 hi + 4 hh + (0..3), as
// tile_read_tr returns it from the block-chunk-major layout.
template <typename V4>
__device__ __forceinline__ V4 rowswz_read_tr(const RowSwzTr& t, int blk, int ks, int hi, int db) {
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  const uint32_t imm = (32 * blk + 16 * ks + 8 * hi) * 256;
  const bf16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
      (__attribute__((address_space(3))) bf16x4_t*)(uintptr_t)(t.b[db] + imm));
  return __builtin_bit_cast(V4, v);
}

// Wait until at most N LDS (and scalar-memory) operations of this wave are
// outstanding; vmcnt and expcnt left at their maxima.
template <int N>
__device__ __forceinline__ void wait_lgkm() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (N << 8) | (3 << 14));
}

// 32 consecutive fp32 values of each of two vectors (rows row0.. of `a` and of
// `b`, clamped to nrows - 1) into 256 bytes of LDS at `lds`: a first, then b.
// One global_load_lds_dword issued by the calling wave.
template <typename Mem = DeviceMem>
__host__ __device__ __forceinline__ void pair32_load_async(const float* a, const float* b, int row0, int nrows,
                                                           uint32_t lds, int lane, const Mem& mem = Mem()) {
  int r = row0 + (lane & 31);
  r = r < nrows ? r : nrows - 1;
  const float* src = (lane < 32 ? a : b) + r;
  mem.load4_global(lds, src);
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t lds_read_f4(uint32_t addr) {
  return *(const __attribute__((address_space(3))) f32x4_t*)(uintptr_t)(addr);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(p)));
}

// A wave's 32 x D output block (rows row0 .. row0 + 31 of a [*, D] bf16/fp16
// matrix, row stride ss elements, rows >= nrows skipped) leaves the matrix
// core in a transposed register layout, so a direct store instruction would
// touch 32 rows with 8-16 bytes each.  These helpers stage the block in the
// wave's own LDS scratch (`slot(r)`: byte address of row r, 2 D bytes per row,
// used by no other wave meanwhile) and store it as whole rows: 16 lanes per
// row, 16 bytes per lane.  Within a row the 16-byte chunks are XOR-swizzled by
// the row index, which spreads the staging writes over the banks.  The wave
// writes and reads its scratch itself, and LDS serves one wave in order.

// LDS byte offset of element d within row r of the staging layout.
template <int D>
__device__ __forceinline__ uint32_t stage_off(int r, int d) {
  constexpr int CH = D * 2 / 16;  // 16-byte chunks per row
  return static_cast<uint32_t>((((d >> 3) ^ (r & (CH - 1))) << 4) + ((d & 7) << 1));
}

// Staged rows (ROWS of them) to global memory, whole rows per store instruction.
template <typename T, int D, int ROWS = 32, typename SlotFn>
__device__ __forceinline__ void stage_to_rows(SlotFn slot, T* row0, int64_t ss, int nrows, int lane) {
  constexpr int CH = D * 2 / 16;
  static_assert(ROWS * CH % 64 == 0, "whole store instructions");
#pragma unroll
  for (int k = 0; k < ROWS * CH / 64; ++k) {
    const int q = 64 * k + lane, r = q / CH, c = q % CH;
    const u32x4 v = *(__attribute__((address_space(3))) u32x4*)(uintptr_t)(slot(r) + stage_off<D>(r, 8 * c));
    if (r < nrows) *reinterpret_cast<u32x4*>(row0 + static_cast<int64_t>(r) * ss + c * 8) = v;
  }
}

// Row-per-lane accumulators: lane (l32, hh) holds row l32, elements
// 32 db + 8 g + 4 hh + (0..3) in acc[db][4 g ..] (the forward's O, dQ).
template <typename T, int D, typename SlotFn>
__device__ __forceinline__ void store_rows_via_lds(const f32x16* acc, float scale, SlotFn slot, T* row0, int64_t ss,
                                                   int nrows, int lane) {
  typedef T v4 __attribute__((ext_vector_type(4)));
  const int l32 = lane & 31, hh = lane >> 5;
  const uint32_t wr = slot(l32);
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      v4 o4;
#pragma unroll
      for (int e = 0; e < 4; ++e) o4[e] = static_cast<T>(acc[db][4 * g + e] * scale);
      *(__attribute__((address_space(3))) v4*)(uintptr_t)(wr + stage_off<D>(l32, 32 * db + 8 * g + 4 * hh)) = o4;
    }
  }
  stage_to_rows<T, D>(slot, row0, ss, nrows, lane);
}

// Column-per-lane accumulators: lane (l32, hh) holds element 32 db + l32 of
// rows crow(r, hh), r = 0..15, in acc[db][r] (dK, dV).
template <typename T, int D, typename SlotFn>
__device__ __forceinline__ void store_cols_via_lds(const f32x16* acc, float scale, SlotFn slot, T* row0, int64_t ss,
                                                   int nrows, int lane) {
  const int l32 = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = crow(r, hh);
      *(__attribute__((address_space(3))) T*)(uintptr_t)(slot(row) + stage_off<D>(row, 32 * db + l32)) =
          static_cast<T>(acc[db][r] * scale);
    }
  }
  stage_to_rows<T, D>(slot, row0, ss, nrows, lane);
}

}  // namespace ssa
