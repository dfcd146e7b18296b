// Tiles and MFMA operands of the head_dim 256 kernels (nq_prefill_wide.hip,
// nq_backward_wide.hip).
//
// A tile is 32 rows (keys or query rows) x 256 bf16 = 32 rows of 512 B in
// LDS.  512-byte rows, like 256-byte ones, alias the 256-byte bank line, so
// the chunks of row r are XOR-swizzled by r, in one of two layouts:
//   row layout:  16-byte chunk c at c ^ (r & 15); a ds_read_b128 of one chunk
//                from 16 consecutive rows hits 16 distinct bank groups;
//   tr layout:   chunk c at c ^ 2 (r & 7); a transpose read of 8 consecutive
//                rows hits 8 distinct 32-byte bank groups.
// A tile read both ways is stored twice.  The products run on
// v_mfma_f32_16x16x32_bf16 (lane l: row/col l % 16, k group l / 16).
#pragma once

#include "nq_common.hpp"

namespace nq {

constexpr int PW_D = 256;
constexpr int PW_TILE = 32;                           // rows per tile
constexpr int PW_RB = PW_D * 2;                       // bytes per row
constexpr int PW_TILE_BYTES = PW_TILE * PW_RB;        // 16 KiB
constexpr int PW_PIECES = PW_TILE_BYTES / 16 / 256;   // 16-byte pieces per thread (256 threads)

__device__ __forceinline__ int pw_kswz(int row) { return row & 15; }
__device__ __forceinline__ int pw_vswz(int row) { return (row & 7) * 2; }

// Piece pc (row pc / 32, chunk pc % 32) of a tile, in the row and tr layouts.
__device__ __forceinline__ void pw_store_row(unsigned char* t, int pc, bf16x8 v) {
  const int r = pc >> 5, c = pc & 31;
  *reinterpret_cast<bf16x8*>(t + r * PW_RB + ((c ^ pw_kswz(r)) << 4)) = v;
}
__device__ __forceinline__ void pw_store_tr(unsigned char* t, int pc, bf16x8 v) {
  const int r = pc >> 5, c = pc & 31;
  *reinterpret_cast<bf16x8*>(t + r * PW_RB + ((c ^ pw_vswz(r)) << 4)) = v;
}

// Rows row0 .. row0+15 as an MFMA operand with rows on the M (or N) side:
// lane l holds row row0 + l % 16, dims 32 dq + 8 (l / 16) .. +8 (row layout).
__device__ __forceinline__ bf16x8 pw_row_operand(const unsigned char* t, int row0, int dq, int lane) {
  const int r = row0 + (lane & 15), c = 4 * dq + (lane >> 4);
  return *reinterpret_cast<const bf16x8*>(t + r * PW_RB + ((c ^ pw_kswz(r)) << 4));
}

// Dims 16 dd .. 16 dd + 15 (lane l: dim 16 dd + l % 16) of the tile's 32 rows
// as the A operand, with the k index running over rows in the order
// 4g, 4g+1, 4g+2, 4g+3, 16+4g, .., 16+4g+3 for lane group g = l / 16: the
// order in which a lane holds the two 16-row halves of a 16x16 MFMA result
// (rows 4g + i of each half), so that result, packed to bf16, is the matching
// B operand (tr layout).
__device__ __forceinline__ bf16x8 pw_tr_operand(const unsigned char* t, int dd, int lane) {
  const int jj = lane & 15, g = lane >> 4;
  const int vrow = 4 * g + (jj >> 2);
  const int off = vrow * PW_RB + ((pw_vswz(vrow) >> 1) << 5) + (jj & 3) * 8;
  const unsigned char* src = t + (off ^ (dd << 5));
  return lds_read_tr8(reinterpret_cast<const bf16*>(src), reinterpret_cast<const bf16*>(src + 16 * PW_RB));
}

}  // namespace nq
