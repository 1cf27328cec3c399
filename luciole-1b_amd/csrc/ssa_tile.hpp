// LDS tile staging shared by the kernels that stream K/V (or Q/dO) tiles.
//
// A tile is ROWS rows of D bf16/fp16 elements, row-major, 2*D bytes per row,
// with no padding.  Bank conflicts are avoided by permuting the 16-byte chunks
// of each row: logical chunk c of row r lives in slot c ^ swz(r).  With RP
// rows per 256-byte bank window (RP = 256 / (2 D)),
//   swz(r) = (((r / RP) % 4) << 2 | (r / 4) % 4) & (chunks per row - 1)
// is a bijection on the slots of a row such that
//   * 16 consecutive rows read at one logical chunk (ds_read_b128 operand
//     fetches, one row per lane, 16 lanes per LDS cycle) hit 16 distinct
//     16-byte bank groups, and
//   * 4 aligned consecutive rows read at 4 aligned chunks (the 32 lanes of a
//     ds_read_b64_tr_b16 transpose read that the LDS serves together) hit
//     disjoint 64-byte bank groups.
// Measured on MI355X: ~215 B/clk/CU for the b128 pattern and ~150 B/clk/CU
// for the transpose pattern, the same as fully contiguous reads; plain rows
// give 16 and 61 B/clk/CU, and no row padding is conflict-free for both.
//
// Tiles are filled with global_load_lds_dwordx4: each instruction moves 1 KB,
// lane L writing LDS bytes [16 L, 16 L + 16) of that KB, so the swizzle is
// applied on the global side (which chunk each lane fetches).  Rows past the
// end of the sequence are clamped to the last valid row; callers mask them.
#pragma once

#include "ssa_common.hpp"

namespace ssa {

template <int D>
struct TileLayout {
  static constexpr int CPR = D / 8;               // 16-byte chunks per row
  static constexpr int ROW_BYTES = D * 2;
  static constexpr int RPI = 1024 / ROW_BYTES;    // rows per 1 KB load instruction
  static constexpr int RP = 256 / ROW_BYTES;      // rows per 256-byte bank window
  __device__ static __forceinline__ int swz(int r) {
    return ((((r / RP) & 3) << 2) | ((r >> 2) & 3)) & (CPR - 1);
  }
  // Byte offset of logical chunk c of row r.
  __device__ static __forceinline__ int chunk_off(int r, int c) { return r * ROW_BYTES + ((c ^ swz(r)) << 4); }
};

// Issue the loads of one ROWS x D tile (rows row0.. of a [*, D] matrix with
// row stride `ss` elements) into `lds` (byte address).  Called by all NW waves
// of the workgroup; wave w issues instructions w, w + NW, ... (a wave may
// issue none when the tile has fewer 1 KB pieces than there are waves).
template <int D, int ROWS, int NW>
__device__ __forceinline__ void tile_load_async(const void* gbase, int64_t ss, int row0, int nrows, uint32_t lds,
                                                int wave, int lane) {
  using TL = TileLayout<D>;
  constexpr int NINST = ROWS * TL::ROW_BYTES / 1024;
  static_assert(NINST * 1024 == ROWS * TL::ROW_BYTES, "tile must be a whole number of 1 KB pieces");
  const int rl = lane / TL::CPR, slot = lane % TL::CPR;
#pragma unroll
  for (int j = wave; j < NINST; j += NW) {
    const int r = j * TL::RPI + rl;
    int grow = row0 + r;
    grow = grow < nrows ? grow : nrows - 1;
    const int c = slot ^ TL::swz(r);
    const char* src = static_cast<const char*>(gbase) + (static_cast<int64_t>(grow) * ss + c * 8) * 2;
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src),
                                     (__attribute__((address_space(3))) void*)(uintptr_t)(lds + j * 1024), 16, 0, 0);
  }
}

// 16-byte fetch of logical chunk c of row r (an MFMA operand: 8 consecutive elements).
template <int D, typename V>
__device__ __forceinline__ V tile_read16(uint32_t lds, int r, int c) {
  return *(const __attribute__((address_space(3))) V*)(uintptr_t)(lds + TileLayout<D>::chunk_off(r, c));
}

// Transposed fetch for an MFMA operand that needs column d of rows rbase..rbase+3:
// within each 16-lane group, lane i supplies row rbase + i/4, columns
// dgrp + 4 (i%4) .. +3 (8 bytes), and receives column dgrp + i of the 4 rows.
// dgrp = 16-column group of this lane's 16-lane group.
template <int D, typename V4>
__device__ __forceinline__ V4 tile_read_tr(uint32_t lds, int rbase, int dgrp, int i) {
  const int r = rbase + (i >> 2);
  const int col = dgrp + 4 * (i & 3);
  const uint32_t off = TileLayout<D>::chunk_off(r, col >> 3) + ((col & 4) << 1);
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  const bf16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4_t*)(uintptr_t)(lds + off));
  return __builtin_bit_cast(V4, v);
}

// 32 consecutive fp32 values of each of two vectors (rows row0.. of `a` and of
// `b`, clamped to nrows - 1) into 256 bytes of LDS at `lds`: a first, then b.
// One global_load_lds_dword issued by the calling wave.
__device__ __forceinline__ void pair32_load_async(const float* a, const float* b, int row0, int nrows, uint32_t lds,
                                                  int lane) {
  int r = row0 + (lane & 31);
  r = r < nrows ? r : nrows - 1;
  const float* src = (lane < 32 ? a : b) + r;
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src),
                                   (__attribute__((address_space(3))) void*)(uintptr_t)(lds), 4, 0, 0);
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t lds_read_f4(uint32_t addr) {
  return *(const __attribute__((address_space(3))) f32x4_t*)(uintptr_t)(addr);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(p)));
}

}  // namespace ssa
