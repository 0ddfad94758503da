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
// LDS rows of 128 bytes hold their 16-byte pieces XOR-swizzled: piece p of
// row r sits at position p ^ lds_swz(r).  A 128-bit LDS read is served 16
// lanes at a time; an operand read has those lanes on 16 consecutive rows
// (from a multiple of 16) at one piece, and with this swizzle the 16 rows
// give 16 distinct (row parity, position) pairs -- all 64 banks once.
// (r & 7) would put rows r and r + 8 on the same banks.
GS_HD int lds_swz(int r) { return (r >> 1) & 7; }
// A wave transfer moves 8 rows of 128 bytes: lane l takes row l / 8 of them
// and, within it, the 16-byte piece that lands at LDS position l % 8 of LDS
// row lds_row.
GS_HD int dma_trow(int l) { return l >> 3; }
GS_HD int dma_gpiece_bytes(int l, int lds_row) { return ((l & 7) ^ lds_swz(lds_row)) * 16; }
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

// ---- reference-semantics ops over x_ext (gs_xext.hip) ----------------------
// Tier of kernel-local id kid (ids are numbered 1.. across the six tiers in
// ascending-rank order; tier t holds na[t] adapters of rank 16 << t): its
// tier t, the tier's first id and the tier's offset in the packed lora_B
// ([na[t]][N][r] per tier).  False for an id past the last tier.
GS_HD bool xext_tier(const int* na, int N, int kid, int& t, int& first, int64_t& lb_off) {
  t = 0;
  first = 1;
  lb_off = 0;
  while (t < 6 && kid >= first + na[t]) {
    first += na[t];
    lb_off += static_cast<int64_t>(na[t]) * N * (16 << t);
    ++t;
  }
  return t < 6;
}
// First x_ext column of the shrink values of the idx-th adapter of its tier
// for one slice, from that slice's tier base scr_st (slice_col_r[s][t]).
GS_HD int64_t xext_zcol(int scr_st, int idx, int S, int r) {
  return static_cast<int64_t>(scr_st) + static_cast<int64_t>(idx) * S * r;
}
// Element of lora_B row n (output column) of the idx-th adapter of a tier.
GS_HD int64_t xext_brow(int64_t lb_off, int idx, int N, int r, int64_t n) {
  return lb_off + static_cast<int64_t>(idx) * N * r + n * r;
}
// The x_ext row a lane reads: a row past the batch reads row 0.
GS_HD int64_t xext_row(bool row_ok, int64_t m) { return row_ok ? m : 0; }
// Read-modify-write piece q of thread tid of a 32 x 128 tile: row
// (tid + 256 q) / 16, columns 8 ((tid + 256 q) % 16) on.
GS_HD int xext_piece_row(int tid, int q) { return (tid + 256 * q) >> 4; }
GS_HD int xext_piece_col(int tid, int q) { return ((tid + 256 * q) & 15) * 8; }
// Column block of the column-block kernel: piece pc of an adapter's staged
// lora_B block (r / 8 16-byte pieces per column) lands at column pc >> sh,
// piece pc & (2^sh - 1) of it (sh = log2(r / 8)).
GS_HD int xext_stage_colof(int pc, int sh) { return pc >> sh; }
GS_HD int xext_stage_kof(int pc, int sh) { return pc & ((1 << sh) - 1); }

// ---- one-launch small-batch kernel (gs_small.hip) --------------------------
// Entry a thread loads for routing slot u (tokens / sequences u * 256 + tid),
// clamped to the last of n (n >= 1).
GS_HD int small_route_index(int u, int tid, int n) { return imin(u * 256 + tid, n - 1); }
// Producer workgroup bid: its (k-chunk, adapter) pair q, column block cb and
// row split rs (the NCB * RS siblings of a pair get ids 8 apart).
GS_HD void small_producer(int bid, int NCB, int RS, int& q, int& cb, int& rs) {
  const int inner = (bid >> 3) % (NCB * RS);
  cb = inner % NCB;
  rs = inner / NCB;
  q = ((bid >> 3) / (NCB * RS)) * 8 + (bid & 7);
}
// Consumer cid: its (tile group, adapter) item and row split rs.
GS_HD void small_consumer(int cid, int RS, int& item, int& rs) {
  item = ((cid >> 3) / RS) * 8 + (cid & 7);
  rs = (cid >> 3) % RS;
}
// A token slot of a row chunk: slots past the adapter's n_g tokens re-read
// the chunk's first (rt0 < n_g).
GS_HD int small_slot(int slot, int n_g, int rt0) { return slot < n_g ? slot : rt0; }
// ---- GEMM (gs_gemm.hip) -----------------------------------------------------
// Tile (tm, tn) of workgroup bid: tiles are ordered in groups of `group` tile
// rows (column by column inside a group) and XCD x = bid % 8 takes the
// contiguous range [x * per, (x + 1) * per) of that order.  False for an id
// past the last tile.
GS_HD bool gemm_tile(int bid, int tiles_m, int tiles_n, int group, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int per = (total + 7) >> 3;
  const int t = (bid & 7) * per + (bid >> 3);
  if (t >= total) return false;
  const int grp = t / (group * tiles_n);
  const int first_m = grp * group;
  const int gm = imin(group, tiles_m - first_m);
  const int rr = t - grp * group * tiles_n;
  tm = first_m + rr % gm;
  tn = rr / gm;
  return true;
}
// An operand row a thread moves: rows past the matrix re-read its last.
GS_HD int gemm_row(int r, int rows) { return imin(r, rows - 1); }
// The global 16-byte piece a lane moves into LDS position l % 8 of row r.
GS_HD int gemm_piece(int l, int r) { return (l & 7) ^ lds_swz(r); }

// Tagged partial (g, ks, slot, col) in the workspace: adapter g's region,
// [KS][cap][zw] 8-byte elements.
GS_HD int64_t small_part(int64_t region, int g, int ks, int cap, int slot, int zw, int col) {
  return static_cast<int64_t>(g - 1) * region + (static_cast<int64_t>(ks) * cap + slot) * zw + col;
}

}  // namespace addr
}  // namespace gs
