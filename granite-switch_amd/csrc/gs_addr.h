// Address arithmetic of the switched-LoRA kernels, shared by the kernels and
// by the host-side address model that replays their memory accesses on the
// CPU (gs_check_segment_addresses / gs_check_small_addresses).
//
// Every hot loop issues its loads unconditionally from clamped addresses and
// masks the values afterwards (so the compiler can count the loads in
// flight); a wrong clamp is an out-of-bounds access.  Each clamp and index
// formula lives here, in one function that the kernel calls and the address
// model calls, so the model checks the very arithmetic the kernel runs.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define GS_HD __host__ __device__ __forceinline__
#else
#define GS_HD inline
#endif

namespace gs {
namespace addr {

GS_HD int imin(int a, int b) { return a < b ? a : b; }
GS_HD int64_t lmin(int64_t a, int64_t b) { return a < b ? a : b; }

// Row r of a tile of nrows rows: rows past the tile re-read its first row
// (their results are never stored).
GS_HD int tile_row(int r, int nrows) { return r < nrows ? r : 0; }

// ---- shrink, ring form (shrink_dma_kernel) ---------------------------------
// 64-k stages [s_lo, s_lo + nst) of k-chunk ks of KS over the H / 64 stages.
GS_HD void dma_kchunk(int H, int ks, int KS, int& s_lo, int& nst) {
  const int all = H / 64;
  s_lo = (ks * all) / KS;
  nst = ((ks + 1) * all) / KS - s_lo;
}
// A wave transfer moves 8 rows of 128 bytes: lane l takes row l / 8 of them
// and, within it, the 16-byte piece that lands swizzled at LDS position l % 8.
GS_HD int dma_trow(int l) { return l >> 3; }
GS_HD int dma_gpiece_bytes(int l) { return ((l & 7) ^ (l >> 3)) * 16; }
// Tile row (x) of transfer t of a wave: 16 rows per wave.
GS_HD int dma_x_row(int wave, int t, int trow) { return 16 * wave + 8 * t + trow; }
// lora_A row (of the adapter's S*r) of transfer t of a wave: arw rows per
// wave from col0, clamped to the adapter's last row.
GS_HD int dma_a_row(int col0, int arw, int wave, int t, int trow, int ncols) {
  return imin(col0 + arw * wave + 8 * t + trow, ncols - 1);
}
// Result piece pc of the store phase: row pc / ppr4, columns c4 .. c4 + 3.
GS_HD int dma_res_row(int pc, int ppr4) { return pc / ppr4; }
GS_HD int dma_res_col(int pc, int ppr4) { return (pc % ppr4) * 4; }

// ---- shrink, register form (shrink_kernel) ---------------------------------
// Element offset, within the lane's lora_A base row, of piece j at k kp
// (rows past the adapter and k past the chunk read the base row at k_lo).
GS_HD int64_t reg_a_elem(bool ok, int j, int64_t astep_elems, int64_t kp, int64_t k_lo) {
  return ok ? j * astep_elems + kp : k_lo;
}
// Element offset, within the lane's x row, of the piece at k kp.
GS_HD int64_t reg_x_elem(bool ok, int64_t kp, int64_t k_lo) { return ok ? kp : k_lo; }

// ---- expand (expand_kernel, expand_sparse_kernel) --------------------------
// First output column of the lane's 16-byte y piece in sub-tile sub of NT
// columns (the last piece of a partial sub-tile re-reads the row's last one).
GS_HD int64_t y_col(int sub, int nt, int cx, int out_total, int epl) {
  return lmin(static_cast<int64_t>(sub) * nt + cx, static_cast<int64_t>(out_total) - epl);
}
// Output column (lora_B row) whose k-groups a lane loads, clamped to the last.
GS_HD int b_col(int n, int out_total) { return imin(n, out_total - 1); }
// k of a lora_B / shrink piece: k-groups past the rank read k = 0 and are masked.
GS_HD int k_or_zero(int k0, int r) { return k0 < r ? k0 : 0; }

// Shrink values staged per tile: item it of per_row 4-element items per row.
GS_HD int stage_row(int it, int per_row) { return it / per_row; }
GS_HD int stage_col(int it, int row, int per_row, int col_base) { return col_base + (it - row * per_row) * 4; }

}  // namespace addr
}  // namespace gs
