// The reference's expand ops over x_ext = x . w_ext^T, with the reference's
// argument lists and semantics (bitmask skip, tier layout of the packed
// lora_B, kernel-local ids), on gfx950 bf16 MFMA: the in-place expand, the
// fused gate/up expand + SwiGLU, and the W-less expand into a fresh output.
//
// A workgroup owns 32 rows x 128 columns (4 waves x one 32-column block).  Each
// wave loops over the adapters that are both set in the tile bitmask and
// present in its rows, and accumulates a 32x32 MFMA product per adapter with
// the rows of other adapters fed as zeros, so a row only ever receives its own
// adapter's delta.  The delta goes through LDS to a row-major tile and is
// added to x_ext in one bf16 read-modify-write per element.
#include <stdarg.h>

#include <algorithm>
#include <array>
#include <type_traits>
#include <vector>

#include "gs_addr.h"
#include "gs_common.h"

namespace gs {

namespace {

constexpr int kRanks[6] = {16, 32, 64, 128, 256, 512};

struct XextArgs {
  const void* x_ext;         // read: shrink columns (and base columns for swiglu)
  int64_t stride_m;
  int64_t M;
  const void* ids;
  int idx_bytes;
  const int64_t* bitmask;
  int64_t stride_bm;
  const uint16_t* lb;
  const int32_t* slice_col_r;
  int na[6];
  int S;
  int N;
};

// silu(g) * u = g / (1 + e^-g) * u in fp32 through the hardware's exp2 and
// reciprocal (v_exp_f32, v_rcp_f32; each within 1 ulp), a handful of VALU
// operations instead of a library exp and an IEEE division.  The result is
// rounded to bf16 (2^-8 relative), far above the few fp32 ulps this adds.
// Large |g| behaves: e^-g overflowing to +inf gives a reciprocal of 0 (silu
// -> -0), underflowing to 0 gives 1 (silu -> g); NaN propagates.
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

__device__ __forceinline__ int load_id(const void* p, int bytes, int64_t i) {
  return bytes == 8 ? static_cast<int>(static_cast<const int64_t*>(p)[i]) : static_cast<const int32_t*>(p)[i];
}

// Delta of one 32x32 block: rows m0..m0+31, columns n0..n0+31 (lane i owns
// row m0+i for the A operand and column n0+i for the B operand), slice s.
// scr is the slice_col_r table staged in LDS.
__device__ f32x16 xext_block_delta(const XextArgs& a, const int* scr, int64_t m0, int n0, int s, int id, bool row_ok,
                                   uint64_t bm) {
  const int l = __lane_id();
  const int i = l & 31;
  const int h = l >> 5;
  f32x16 acc = f32x16{};
  // adapters present in these rows and set in the tile mask
  uint64_t mine = (row_ok && id >= 1 && id <= 64) ? (1ull << (id - 1)) : 0ull;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) mine |= __shfl_xor(mine, d, 64);
  uint64_t todo = mine & bm;
  const uint16_t* xrow = static_cast<const uint16_t*>(a.x_ext) + (m0 + i) * a.stride_m;   // read only when sel
  while (todo) {
    const int b = __builtin_amdgcn_readfirstlane(__ffsll(static_cast<long long>(todo)) - 1);   // uniform
    todo &= todo - 1;
    const int kid = b + 1;   // kernel-local id
    int t, first;
    int64_t lb_off;
    if (!addr::xext_tier(a.na, a.N, kid, t, first, lb_off)) break;   // cannot happen: only valid bits are followed
    const int r = 16 << t;
    const int idx = kid - first;
    const int64_t c0 = addr::xext_zcol(scr[s * 6 + t], idx, a.S, r);
    const uint16_t* brow = a.lb + addr::xext_brow(lb_off, idx, a.N, r, n0 + i);
    const bool sel = row_ok && id == kid;
    for (int kb = 0; kb < r; kb += 16) {
      const int k0 = kb + 8 * h;
      const u32x4 za = sel ? *reinterpret_cast<const u32x4*>(xrow + c0 + k0) : u32x4{0u, 0u, 0u, 0u};
      const u32x4 bb = *reinterpret_cast<const u32x4*>(brow + k0);
      acc = mfma32_bf16(za, bb, acc);
    }
  }
  return acc;
}

// Tier of kernel-local id kid (ids are numbered 1.. across the tiers in
// ascending-rank order): tier t holds rank 16 << t; first = the tier's first
// id; lb_off = the tier's offset in the packed lora_B.  Returns false for an
// id past the last tier.
__device__ __forceinline__ bool xext_tier(const XextArgs& a, int kid, int& t, int& first, int64_t& lb_off) {
  return addr::xext_tier(a.na, a.N, kid, t, first, lb_off);
}

// Fast path for modules whose tiers all have rank <= 16 KK.  A row only ever
// receives its own adapter's delta, so each lane loads its row's shrink
// values once (KK 16-byte pieces of slice s, zero when the row's adapter is
// not followed), and the lora_B blocks of up to BA followed adapters are
// loaded together, so a tile with several adapters costs one memory trip per
// BA adapters instead of one per adapter.  The MFMA per adapter feeds the
// rows of other adapters as zeros, as in the general path.
// lora_B pieces one lane holds in flight per batch of adapters (registers)
#ifndef GS_XEXT_SLOTS
#define GS_XEXT_SLOTS 16
#endif
constexpr int kXextSlots = GS_XEXT_SLOTS;
#ifndef GS_XEXT_RT8
#define GS_XEXT_RT8 1
#endif
// The column-block expand and the SwiGLU form read and write the output
// columns' pieces of x_ext (and the SwiGLU output) once per launch: they are
// streamed, so the lora_B blocks and the rows' shrink values, which several
// workgroups read, stay in L2 (decode QKV 7.77 -> 7.33 us, SwiGLU at the
// step shape 104 -> 92 us).  The per-tile expand measured slower with it
// (multiswitch down 28.3 -> 30.5 us) and keeps the default policy.
__device__ __forceinline__ u32x4 ld_row(const void* p) { return ld16_nt(p); }
__device__ __forceinline__ void st_row(void* p, const u32x4& v) { st16_nt(p, v); }
#ifndef GS_XEXT_COLS
#define GS_XEXT_COLS 1
#endif
#ifndef GS_XEXT_GATE_UP_ONE_TRIP
#define GS_XEXT_GATE_UP_ONE_TRIP 1
#endif


template <int KK>
__device__ __forceinline__ void xext_own_z(const XextArgs& a, const int* scr, int64_t m0, int s, int id, bool row_ok,
                                           uint64_t todo, u32x4 (&z)[KK]) {
  const int l = __lane_id();
  const int i = l & 31;
  const int h = l >> 5;
  bool ok = row_ok && id >= 1 && id <= 64 && ((todo >> (id - 1)) & 1ull);
  int t = 0, first = 1;
  int64_t lb_off = 0;
  ok = xext_tier(a, ok ? id : 1, t, first, lb_off) && ok;
  const int r = 16 << t;
  const int64_t c0 = addr::xext_zcol(scr[s * 6 + t], (ok ? id : first) - first, a.S, r);
  // a row past the batch (row_ok false: also the idle waves of a column-block
  // workgroup, whose whole tile lies past it) reads row 0
  const uint16_t* xrow = static_cast<const uint16_t*>(a.x_ext) + addr::xext_row(row_ok, m0 + i) * a.stride_m;
  // unmasked (a clamped address when the row's adapter is not followed):
  // a value is only used by the MFMA of the row's own adapter, k-step by
  // k-step within its rank, so the loads need no wait before that
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    const bool kin = ok && kk * 16 < r;
    z[kk] = *reinterpret_cast<const u32x4*>(xrow + (kin ? c0 + kk * 16 + 8 * h : 0));
  }
}

// NS column blocks at once (the SwiGLU form computes the gate and the up
// block of the same rows): n0[j] is block j's first column, z[j] the rows'
// shrink values of its slice.
template <int KK, int BA, int NS>
__device__ void xext_block_delta_fast(const XextArgs& a, const int (&n0)[NS], int id, uint64_t todo,
                                      const u32x4 (&z)[NS][KK], f32x16 (&acc)[NS]) {
  const int l = __lane_id();
  const int i = l & 31;
  const int h = l >> 5;
#pragma unroll
  for (int j = 0; j < NS; ++j) acc[j] = f32x16{};
  while (todo) {
    int kid[BA], rk[BA];
    const uint16_t* bp[BA];
#pragma unroll
    for (int b = 0; b < BA; ++b) {
      kid[b] = 0;
      rk[b] = 0;
      bp[b] = a.lb;
      if (todo) {   // uniform
        const int bit = __builtin_amdgcn_readfirstlane(__ffsll(static_cast<long long>(todo)) - 1);
        todo &= todo - 1;
        int t, first;
        int64_t lb_off;
        if (xext_tier(a, bit + 1, t, first, lb_off)) {
          kid[b] = bit + 1;
          rk[b] = 16 << t;
          bp[b] = a.lb + addr::xext_brow(lb_off, bit + 1 - first, a.N, rk[b], i) + 8 * h;
        }
      }
    }
    // every followed adapter's lora_B pieces in flight at once (unconditional
    // loads; pieces past an adapter's rank read the packed array's first line)
    u32x4 bb[NS][BA][KK];
#pragma unroll
    for (int j = 0; j < NS; ++j)
#pragma unroll
      for (int b = 0; b < BA; ++b)
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          bb[j][b][kk] = *reinterpret_cast<const u32x4*>(
              kk * 16 < rk[b] ? bp[b] + static_cast<int64_t>(n0[j]) * rk[b] + kk * 16 : a.lb);
#pragma unroll
    for (int b = 0; b < BA; ++b) {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        if (kk * 16 < rk[b]) {   // uniform
#pragma unroll
          for (int j = 0; j < NS; ++j) acc[j] = mfma32_bf16(sel16(id == kid[b], z[j][kk]), bb[j][b][kk], acc[j]);
        }
      }
    }
  }
}

// Only bits for kernel-local ids that exist (1..sum(na)) may be followed.
__device__ __forceinline__ uint64_t valid_bits(const int na[6]) {
  int tot = 0;
  for (int t = 0; t < 6; ++t) tot += na[t];
  return tot >= 64 ? ~0ull : ((1ull << tot) - 1ull);
}

// KK = 0: the general path (one memory trip per adapter present in the
// tile); KK > 0: the fast path above (every tier of rank <= 16 KK).
template <int KK>
__device__ __forceinline__ f32x16 xext_delta(const XextArgs& a, const int* scr, int64_t m0, int n0, int s, int id,
                                             bool row_ok, uint64_t bm) {
  if constexpr (KK == 0) {
    return xext_block_delta(a, scr, m0, n0, s, id, row_ok, bm);
  } else {
    constexpr int BA = kXextSlots / KK;
    uint64_t mine = (row_ok && id >= 1 && id <= 64) ? (1ull << (id - 1)) : 0ull;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) mine |= __shfl_xor(mine, d, 64);
    const uint64_t todo = mine & bm;
    u32x4 z[1][KK];
    xext_own_z<KK>(a, scr, m0, s, id, row_ok, todo, z[0]);
    const int n0s[1] = {n0};
    f32x16 acc[1];
    xext_block_delta_fast<KK, BA, 1>(a, n0s, id, todo, z, acc);
    return acc[0];
  }
}

// Gate and up deltas of the SwiGLU form (columns h0 of slice 0 and H + h0 of
// slice 1).
// General path of the SwiGLU form: per followed adapter, the gate block's and
// the up block's shrink values and lora_B for two k-steps are loaded in one
// memory trip (eight 16-byte pieces per lane), then the four MFMAs run; a
// rank of 32 costs one trip per adapter instead of one per k-step and slice.
__device__ __forceinline__ void xext_gate_up_general(const XextArgs& a, const int* scr, int64_t m0, int h0, int H,
                                                     int id, bool row_ok, uint64_t bm, f32x16& ag, f32x16& au) {
  const int l = __lane_id();
  const int i = l & 31;
  const int h = l >> 5;
  ag = f32x16{};
  au = f32x16{};
  uint64_t mine = (row_ok && id >= 1 && id <= 64) ? (1ull << (id - 1)) : 0ull;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) mine |= __shfl_xor(mine, d, 64);
  uint64_t todo = mine & bm;
  const uint16_t* xrow = static_cast<const uint16_t*>(a.x_ext) + addr::xext_row(row_ok, m0 + i) * a.stride_m;
  while (todo) {
    const int kid = __builtin_amdgcn_readfirstlane(__ffsll(static_cast<long long>(todo)));   // uniform
    todo &= todo - 1;
    int t, first;
    int64_t lb_off;
    if (!xext_tier(a, kid, t, first, lb_off)) break;   // cannot happen: only valid bits are followed
    const int r = 16 << t;
    const int idx = kid - first;
    const int64_t cg = addr::xext_zcol(scr[t], idx, a.S, r);
    const int64_t cu = addr::xext_zcol(scr[6 + t], idx, a.S, r);
    const uint16_t* bg = a.lb + addr::xext_brow(lb_off, idx, a.N, r, h0 + i);
    const uint16_t* bu = a.lb + addr::xext_brow(lb_off, idx, a.N, r, H + h0 + i);
    const bool sel = row_ok && id == kid;
    for (int kb = 0; kb < r; kb += 32) {
      // all eight pieces load unconditionally (clamped addresses), so that
      // none is deferred behind a branch; the second k-step exists unless
      // the rank is 16, and a missing step feeds zeros
      const bool two = kb + 16 < r;
      const int k0 = kb + 8 * h;
      const int k1 = two ? k0 + 16 : k0;
      const int64_t og = sel ? cg : 0, ou = sel ? cu : 0;
      const u32x4 zg0 = ld16(xrow + og + k0);
      const u32x4 zu0 = ld16(xrow + ou + k0);
      const u32x4 zg1 = ld16(xrow + og + k1);
      const u32x4 zu1 = ld16(xrow + ou + k1);
      const u32x4 bg0 = ld16(bg + k0);
      const u32x4 bu0 = ld16(bu + k0);
      const u32x4 bg1 = ld16(bg + k1);
      const u32x4 bu1 = ld16(bu + k1);
      ag = mfma32_bf16(sel16(sel, zg0), bg0, ag);
      au = mfma32_bf16(sel16(sel, zu0), bu0, au);
      ag = mfma32_bf16(sel16(sel && two, zg1), bg1, ag);
      au = mfma32_bf16(sel16(sel && two, zu1), bu1, au);
    }
  }
}

template <int KK>
__device__ __forceinline__ void xext_delta_gate_up(const XextArgs& a, const int* scr, int64_t m0, int h0, int H, int id,
                                                   bool row_ok, uint64_t bm, f32x16& ag, f32x16& au) {
  if constexpr (KK == 0) {
#if GS_XEXT_GATE_UP_ONE_TRIP
    xext_gate_up_general(a, scr, m0, h0, H, id, row_ok, bm, ag, au);
#else
    ag = xext_block_delta(a, scr, m0, h0, 0, id, row_ok, bm);
    au = xext_block_delta(a, scr, m0, H + h0, 1, id, row_ok, bm);
#endif
  } else {
    constexpr int BA = kXextSlots / 2 / KK;
    uint64_t mine = (row_ok && id >= 1 && id <= 64) ? (1ull << (id - 1)) : 0ull;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) mine |= __shfl_xor(mine, d, 64);
    const uint64_t todo = mine & bm;
    u32x4 z[2][KK];
    xext_own_z<KK>(a, scr, m0, 0, id, row_ok, todo, z[0]);
    xext_own_z<KK>(a, scr, m0, 1, id, row_ok, todo, z[1]);
    const int n0s[2] = {h0, H + h0};
    f32x16 acc[2];
    xext_block_delta_fast<KK, BA, 2>(a, n0s, id, todo, z, acc);
    ag = acc[0];
    au = acc[1];
  }
}

template <int KK>
__global__ __launch_bounds__(256) void xext_expand_kernel(XextArgs a, uint16_t* x_out, const int32_t* __restrict__ tile_slice,
                                                          int block_n) {
  __shared__ float dtile[32][128 + 4];
  __shared__ int scr[GS_MAX_SLICES * 6];
  const int64_t pm = blockIdx.y;
  const int n_tile0 = blockIdx.x * 128;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int i = l & 31;
  const int64_t m0 = pm * 32;
  // everything that depends on no earlier load goes out first: the tile
  // mask, the rows' ids, the slice tables and this thread's read-modify-write
  // piece (row tid / 8, 16 columns, from a clamped in-bounds address)
  const int64_t bm_raw = a.bitmask[pm * a.stride_bm];
  const bool row_ok = (m0 + i) < a.M;
  const int id = row_ok ? load_id(a.ids, a.idx_bytes, m0 + i) : 0;
  if (tid < a.S * 6) scr[tid] = a.slice_col_r[tid];
  const int n0 = n_tile0 + 32 * wave;
  const int s = tile_slice[(n0 < a.N ? n0 : n_tile0) / block_n];
  // piece q of this thread: row (tid + 256 q) / 16, columns 8 ((tid + 256 q)
  // % 16) on, so every wave access covers whole 256-byte row segments
  int prow[2], pc[2], out_id[2];
  bool out_ok[2];
  uint16_t* p[2];
  u32x4 in[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    prow[q] = addr::xext_piece_row(tid, q);
    pc[q] = addr::xext_piece_col(tid, q);
    const int64_t m = m0 + prow[q];
    out_ok[q] = m < a.M && n_tile0 + pc[q] < a.N;
    p[q] = x_out + (out_ok[q] ? m : m0) * a.stride_m + (out_ok[q] ? n_tile0 + pc[q] : n_tile0);
    out_id[q] = out_ok[q] ? load_id(a.ids, a.idx_bytes, m) : 0;
    in[q] = ld16(p[q]);
  }
  if (bm_raw == 0) return;
  const uint64_t bm = static_cast<uint64_t>(bm_raw) & valid_bits(a.na);
  lds_barrier();
  f32x16 acc = f32x16{};
  if (n0 < a.N) acc = xext_delta<KK>(a, scr, m0, n0, s, id, row_ok, bm);
#pragma unroll
  for (int v = 0; v < 16; ++v) dtile[mfma32_row(v, l)][32 * wave + i] = acc[v];
  lds_barrier();

#pragma unroll
  for (int q = 0; q < 2; ++q) {
    if (!out_ok[q] || out_id[q] == 0) continue;   // base rows are never written
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = bf16_bits_to_f32(static_cast<uint16_t>(in[q][e] & 0xffffu)) + dtile[prow[q]][pc[q] + 2 * e];
      const float hi = bf16_bits_to_f32(static_cast<uint16_t>(in[q][e] >> 16)) + dtile[prow[q]][pc[q] + 2 * e + 1];
      o[e] = static_cast<uint32_t>(f32_to_bf16_bits(lo)) | (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
    }
    st16(p[q], u32x4{o[0], o[1], o[2], o[3]});
  }
}

// ----------------------------------------------------------------------------
// Column-block form of the in-place expand, for modules whose tiers all have
// rank <= 16 KK.  A workgroup owns 32 CB columns over RT = 4 or 8
// consecutive 32-row tiles, one wave per row tile.  The lora_B blocks of the
// adapters followed in any of its tiles are staged in LDS once per workgroup
// (an adapter's block for 32 CB consecutive columns is one contiguous run of
// the packed array), so a column's lora_B is read once per RT row tiles
// instead of once per tile -- in a decode batch every tile holds most
// adapters, and the per-tile form moved ~7x the unique lora_B bytes.  Each
// lane loads its own row's shrink values once (a row only receives its own
// adapter's delta); the per-adapter MFMA feeds the rows of other adapters as
// zeros, as in the per-tile form.  At most kColsChunk(KK) adapters are staged
// at a time.  Results go through LDS to row-major pieces for the
// read-modify-write, whose loads are issued first.
// ----------------------------------------------------------------------------

// The id of row i: int64 ids are read as their low 32-bit word (little
// endian), which is exactly static_cast<int> of the value, so no load leaves
// a dead high half whose register reuse would force a wait.
template <bool I64>
__device__ __forceinline__ int load_id_t(const void* p, int64_t i) {
  return static_cast<const int32_t*>(p)[I64 ? 2 * i : i];
}

template <int KK, int CB, int RT, bool I64>
__global__ __launch_bounds__(64 * RT) void xext_cols_kernel(XextArgs a, uint16_t* x_out,
                                                            const int32_t* __restrict__ tile_slice, int block_n) {
  constexpr int NC = 32 * CB;                  // columns of the workgroup
  constexpr int RMAX = 16 * KK;                // largest rank of the module
  constexpr int CST = RMAX * 2 + 16;           // LDS bytes per column of a staged block (padded)
  constexpr int ABLK = NC * CST;               // LDS bytes per staged adapter
  constexpr int CA = CB == 1 ? 16 : 8;         // adapters staged at a time
  constexpr int CAW = CA / RT;                 // adapters each wave stages
  constexpr int QP = NC * RMAX / 8 / 64;       // 16-byte pieces per lane of one block at rank RMAX
  constexpr int DLD = NC + 4;                  // fp32 row stride of the transposed delta
  constexpr int LPR = NC / 16;                 // lanes per row in the read-modify-write
  constexpr int PASSES = 32 * LPR / 64;        // rows per lane
  static_assert(RT * 32 * DLD * 4 <= CA * ABLK, "the delta tile must fit the staging buffer");
  __shared__ __align__(16) char bs[CA * ABLK + 64 * 16];   // + a sink for masked-off pieces
  __shared__ int scr[GS_MAX_SLICES * 6];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63;
  const int i = l & 31;
  const int h = l >> 5;
  const int n_blk0 = blockIdx.x * NC;
  const int64_t pm0 = static_cast<int64_t>(blockIdx.y) * RT;
  const int64_t pm = pm0 + wave;               // this wave's row tile
  const int64_t m0 = pm * 32;
  const int64_t n_tiles = (a.M + 31) / 32;
  const int ncols = min(NC, a.N - n_blk0);

  // The tile masks (uniform) name the adapters the reference's loop follows
  // in each tile; their union over the workgroup's tiles is staged.
  int64_t bmt[RT];
#pragma unroll
  for (int w = 0; w < RT; ++w) bmt[w] = pm0 + w < n_tiles ? a.bitmask[(pm0 + w) * a.stride_bm] : 0;
  // loads that depend on nothing: ids, slice tables, this lane's
  // read-modify-write pieces (clamped in-bounds addresses, masked afterwards)
  const bool row_ok = (m0 + i) < a.M;
  const int id_raw = load_id_t<I64>(a.ids, addr::xext_row(row_ok, m0 + i));
  const int scr_v = a.slice_col_r[tid < a.S * 6 ? tid : 0];
  int sc[CB];
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    const int n0 = n_blk0 + 32 * c;
    sc[c] = tile_slice[(n0 < a.N ? n0 : n_blk0) / block_n];
  }
  const int cx = (l % LPR) * 16;
  int64_t orow[PASSES];
  bool ook[PASSES];
  int oid[PASSES];
  u32x4 in[PASSES][2];
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int64_t m = m0 + ps * (64 / LPR) + l / LPR;
    ook[ps] = m < a.M && n_blk0 + cx < a.N;
    orow[ps] = addr::xext_row(ook[ps], m);
    const uint16_t* src = x_out + orow[ps] * a.stride_m + (ook[ps] ? n_blk0 + cx : 0);
    in[ps][0] = ld_row(src);
    in[ps][1] = ld_row(src + 8);
    oid[ps] = load_id_t<I64>(a.ids, orow[ps]);
  }
  __builtin_amdgcn_sched_barrier(0);   // all of the above in flight before any of it is used

  const uint64_t valid = valid_bits(a.na);
  int64_t bm_tile = 0;
  uint64_t all = 0;
#pragma unroll
  for (int w = 0; w < RT; ++w) {
    bm_tile = wave == w ? bmt[w] : bm_tile;   // uniform
    all |= static_cast<uint64_t>(bmt[w]);
  }
  const uint64_t todo = static_cast<uint64_t>(bm_tile) & valid;
  all &= valid;

  f32x16 acc[2][CB];
#pragma unroll
  for (int c = 0; c < CB; ++c) acc[0][c] = acc[1][c] = f32x16{};
  u32x4 z[CB][KK];
  int id = 0;
  // one chunk of up to CA adapters; the first is straight-line code (its
  // staging loads go out right behind the first loads, before the ids are
  // used), later chunks run in a loop
  auto chunk = [&](auto first_tag) {
    constexpr bool FIRST = decltype(first_tag)::value;
    // lane j < CA describes the chunk's j-th adapter: kernel-local id, rank
    // and the offset of its block for this workgroup's columns
    int my_kid = 0, my_r = 0;
    int64_t my_off = 0;
    if (l < CA) {
      uint64_t mm = all;
      for (int k = 0; k < l; ++k) mm &= mm - 1;
      if (mm) {
        const int bit = __ffsll(static_cast<long long>(mm)) - 1;
        int t, first;
        int64_t lb_off;
        if (xext_tier(a, bit + 1, t, first, lb_off)) {
          my_kid = bit + 1;
          my_r = 16 << t;
          my_off = addr::xext_brow(lb_off, bit + 1 - first, a.N, my_r, n_blk0);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < CA; ++k) all &= all - 1;
    // wave w stages adapters w, w + RT, ...: lane l moves pieces l + 64 q of
    // each block (pieces past the adapter's ncols * r / 8 read the first line)
    u32x4 v[CAW][QP];
#pragma unroll
    for (int jw = 0; jw < CAW; ++jw) {
      const int j = RT * jw + wave;
      const int r = __builtin_amdgcn_readlane(my_r, j);
      const int64_t off = static_cast<int64_t>(
          (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(my_off >> 32), j))) << 32) |
          static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(my_off & 0xffffffff), j)));
      const uint16_t* base = a.lb + off;
#pragma unroll
      for (int q = 0; q < QP; ++q) {
        const int pc = l + 64 * q;
        v[jw][q] = *reinterpret_cast<const u32x4*>(pc < ncols * r / 8 ? base + 8 * pc : a.lb);
      }
    }
    if constexpr (FIRST) {
      // the rows' own shrink values: they need the ids and the slice table,
      // whose loads were issued before the staging loads
      if (tid < a.S * 6) scr[tid] = scr_v;
      id = row_ok && pm < n_tiles ? id_raw : 0;
      lds_barrier();   // scr
#pragma unroll
      for (int c = 0; c < CB; ++c) xext_own_z<KK>(a, scr, m0, sc[c], id, row_ok, todo, z[c]);
    }
    // every lane stores every piece: masked-off ones go to the sink, so no
    // store sits under a branch (r / 8 = 2 << tier pieces per column)
#pragma unroll
    for (int jw = 0; jw < CAW; ++jw) {
      const int j = RT * jw + wave;
      const int r = __builtin_amdgcn_readlane(my_r, j);
      const int sh = 31 - __builtin_clz(r > 0 ? r / 8 : 1);
#pragma unroll
      for (int q = 0; q < QP; ++q) {
        const int pc = l + 64 * q;
        char* dst = pc < ncols * r / 8
                        ? bs + j * ABLK + addr::xext_stage_colof(pc, sh) * CST + addr::xext_stage_kof(pc, sh) * 16
                        : bs + CA * ABLK + l * 16;
        *reinterpret_cast<u32x4*>(dst) = v[jw][q];
      }
    }
    lds_barrier();
    // adapters this wave's tile follows, two accumulation chains; each
    // adapter's operands are read from LDS one adapter ahead
    u32x4 bn[CB][KK];
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        bn[c][kk] = *reinterpret_cast<const u32x4*>(bs + (32 * c + i) * CST + (kk * 16 + 8 * h) * 2);
#pragma unroll
    for (int j = 0; j < CA; ++j) {
      u32x4 bc[CB][KK];
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) bc[c][kk] = bn[c][kk];
      if (j + 1 < CA) {
#pragma unroll
        for (int c = 0; c < CB; ++c)
#pragma unroll
          for (int kk = 0; kk < KK; ++kk)
            bn[c][kk] = *reinterpret_cast<const u32x4*>(bs + (j + 1) * ABLK + (32 * c + i) * CST + (kk * 16 + 8 * h) * 2);
      }
      const int kid = __builtin_amdgcn_readlane(my_kid, j);
      const int r = __builtin_amdgcn_readlane(my_r, j);
      if (kid == 0 || !((todo >> (kid - 1)) & 1ull)) continue;   // uniform
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        if (kk * 16 >= r) break;
#pragma unroll
        for (int c = 0; c < CB; ++c)
          acc[j & 1][c] = mfma32_bf16(sel16(id == kid, z[c][kk]), bc[c][kk], acc[j & 1][c]);
      }
    }
    lds_barrier();   // the staging buffer is refilled (or becomes the delta tile)
  };
  if (all) {
    chunk(std::true_type{});
    while (all) chunk(std::false_type{});
  }

  if (bm_tile == 0) return;   // the reference skips a tile whose mask is 0
  float* dt = reinterpret_cast<float*>(bs) + wave * 32 * DLD;
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) dt[mfma32_row(e, l) * DLD + 32 * c + i] = acc[0][c][e] + acc[1][c][e];
  __builtin_amdgcn_wave_barrier();
  // rows with an adapter get x + delta rounded once (a zero delta stores x
  // back, as the reference's read-modify-write does); base rows are untouched
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    if (!ook[ps] || oid[ps] == 0) continue;
    const int row = ps * (64 / LPR) + l / LPR;
    uint16_t* dst = x_out + orow[ps] * a.stride_m + n_blk0 + cx;
    st_row(dst, add_y16<true>(in[ps][0], dt + row * DLD + cx));
    st_row(dst + 8, add_y16<true>(in[ps][1], dt + row * DLD + cx + 8));
  }
}

// W-less expand (the reference's switch_lora_shrink_expand): x_ext holds only
// shrink columns, and out[M, N] receives the delta itself.  The reference
// zeroes out and then stores the delta of every tile with a nonzero bitmask;
// here every workgroup stores its whole 32 x 128 tile -- the delta, exactly
// zero for base rows (they select no adapter), and zeros for a tile whose
// bitmask is 0 -- so out is written once and no zeroing pass is needed.
template <bool F32OUT, int KK>
__global__ __launch_bounds__(256) void xext_shrink_expand_kernel(XextArgs a, void* out, int64_t stride_om,
                                                                 const int32_t* __restrict__ tile_slice,
                                                                 int block_n) {
  __shared__ float dtile[32][128 + 4];
  __shared__ int scr[GS_MAX_SLICES * 6];
  const int64_t pm = blockIdx.y;
  const int64_t bm_raw = a.bitmask[pm * a.stride_bm];
  const uint64_t bm = static_cast<uint64_t>(bm_raw) & valid_bits(a.na);
  const int n_tile0 = blockIdx.x * 128;
  const int tid = threadIdx.x;
  const int64_t m0 = pm * 32;
  if (bm_raw != 0) {   // uniform over the workgroup
    const int wave = tid >> 6;
    const int l = tid & 63;
    const int i = l & 31;
    if (tid < a.S * 6) scr[tid] = a.slice_col_r[tid];
    const bool row_ok = (m0 + i) < a.M;
    const int id = row_ok ? load_id(a.ids, a.idx_bytes, m0 + i) : 0;
    const int n0 = n_tile0 + 32 * wave;
    const int s = tile_slice[(n0 < a.N ? n0 : n_tile0) / block_n];
    lds_barrier();
    f32x16 acc = f32x16{};
    if (n0 < a.N) acc = xext_delta<KK>(a, scr, m0, n0, s, id, row_ok, bm);
#pragma unroll
    for (int v = 0; v < 16; ++v) dtile[mfma32_row(v, l)][32 * wave + i] = acc[v];
    lds_barrier();
  }
  const int row = tid >> 3;
  const int cx = (tid & 7) * 16;
  const int64_t m = m0 + row;
  if (m >= a.M || n_tile0 + cx >= a.N) return;
  float d[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) d[c] = bm_raw != 0 ? dtile[row][cx + c] : 0.f;
  if constexpr (F32OUT) {
    float* p = static_cast<float*>(out) + m * stride_om + n_tile0 + cx;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<u32x4*>(p + 4 * q) = u32x4{__float_as_uint(d[4 * q]), __float_as_uint(d[4 * q + 1]),
                                                   __float_as_uint(d[4 * q + 2]), __float_as_uint(d[4 * q + 3])};
  } else {
    uint16_t* p = static_cast<uint16_t*>(out) + m * stride_om + n_tile0 + cx;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = static_cast<uint32_t>(f32_to_bf16_bits(d[half * 8 + 2 * e])) |
               (static_cast<uint32_t>(f32_to_bf16_bits(d[half * 8 + 2 * e + 1])) << 16);
      *reinterpret_cast<u32x4*>(p + half * 8) = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
}

template <int KK>
__global__ __launch_bounds__(256) void xext_swiglu_kernel(XextArgs a, uint16_t* out, int64_t stride_om, int H) {
  __shared__ float dg[32][128 + 4];
  __shared__ float du[32][128 + 4];
  __shared__ int scr[GS_MAX_SLICES * 6];
  const int64_t pm = blockIdx.y;
  const int h_tile0 = blockIdx.x * 128;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int i = l & 31;
  const int64_t m0 = pm * 32;
  const bool row_ok = (m0 + i) < a.M;
  // this thread's two 8-column pieces of gate and up do not depend on the
  // delta: they go out early, from clamped in-bounds addresses.  Piece q is
  // row (tid + 256 q) / 16, columns 8 ((tid + 256 q) % 16) on, so that every
  // wave access covers whole 256-byte row segments.
  int prow[2], pc[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    prow[q] = addr::xext_piece_row(tid, q);
    pc[q] = addr::xext_piece_col(tid, q);
  }
  // the ids and the slice table go out first, then the gate and up pieces,
  // then the tile mask (a scalar load: the wait for the kernel arguments
  // before the first vector loads must not include it), so the delta's
  // inputs are one trip away
  const int id = load_id(a.ids, a.idx_bytes, addr::xext_row(row_ok, m0 + i));
  const int scr_v = a.slice_col_r[tid < a.S * 6 ? tid : 0];
  __builtin_amdgcn_sched_barrier(0);
  u32x4 gi[2], ui[2];
  bool pok[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int64_t m = m0 + prow[q];
    pok[q] = m < a.M && h_tile0 + pc[q] < H;
    const uint16_t* src = static_cast<const uint16_t*>(a.x_ext) + (pok[q] ? m : m0) * a.stride_m +
                          (pok[q] ? h_tile0 + pc[q] : h_tile0);
    gi[q] = ld_row(src);
    ui[q] = ld_row(src + H);
  }
  __builtin_amdgcn_sched_barrier(0);
  const int64_t bm_raw = a.bitmask[pm * a.stride_bm];
  const uint64_t bm = static_cast<uint64_t>(bm_raw) & valid_bits(a.na);

  // the deltas through LDS to this thread's pieces (held as fp32)
  float gadd[2][8], uadd[2][8];
#pragma unroll
  for (int q = 0; q < 2; ++q)
#pragma unroll
    for (int c = 0; c < 8; ++c) gadd[q][c] = uadd[q][c] = 0.f;
  if (bm_raw != 0) {
    if (tid < a.S * 6) scr[tid] = scr_v;
    lds_barrier();
    const int h0 = h_tile0 + 32 * wave;
    f32x16 ag = f32x16{}, au = f32x16{};
    if (h0 < H) xext_delta_gate_up<KK>(a, scr, m0, h0, H, id, row_ok, bm, ag, au);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      dg[mfma32_row(v, l)][32 * wave + i] = ag[v];
      du[mfma32_row(v, l)][32 * wave + i] = au[v];
    }
    lds_barrier();
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        gadd[q][c] = dg[prow[q]][pc[q] + c];
        uadd[q][c] = du[prow[q]][pc[q] + c];
      }
  }

#pragma unroll
  for (int q = 0; q < 2; ++q) {
    if (!pok[q]) continue;
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float r2[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = 2 * e + j;
        const float g = bf16_bits_to_f32(static_cast<uint16_t>((gi[q][e] >> (16 * j)) & 0xffffu)) + gadd[q][c];
        const float u = bf16_bits_to_f32(static_cast<uint16_t>((ui[q][e] >> (16 * j)) & 0xffffu)) + uadd[q][c];
        r2[j] = silu_mul(g, u);
      }
      o[e] = static_cast<uint32_t>(f32_to_bf16_bits(r2[0])) | (static_cast<uint32_t>(f32_to_bf16_bits(r2[1])) << 16);
    }
    st_row(out + (m0 + prow[q]) * stride_om + h_tile0 + pc[q], u32x4{o[0], o[1], o[2], o[3]});
  }
}

// Fast-path width for the module's tiers: 2 pieces (rank <= 32), 4 (<= 64),
// or 0 (a tier of rank 128 or more is used: the general path).
// Only decode-sized batches take it: with many tokens a 32-row tile holds one
// or two adapters, the per-adapter trips are few, and the general kernels'
// higher occupancy wins.
constexpr int64_t kFastMaxRows = 1024;
int xext_kk(const int32_t* na, int64_t M) {
  if (M > kFastMaxRows) return 0;
  int top = -1;
  for (int t = 0; t < 6; ++t)
    if (na[t] > 0) top = t;
  return top <= 1 ? 2 : (top == 2 ? 4 : 0);
}

// Launch form of gs_switch_lora_expand (shared by the launch and the address
// model): the column-block kernel with CB 32-column blocks over RT row tiles
// per workgroup, or the per-tile kernel; KK as xext_kk.  The column-block
// kernel takes 64-column blocks (whole 128-byte row pieces) once they give
// two workgroups per CU; 32-column blocks otherwise, over eight row tiles
// when four would take more than one round of workgroups (each column's
// lora_B is then staged half as often, and no CU runs two workgroups' worth
// of staging where one would do).
struct XextForm {
  int kk;
  bool cols;
  int CB, RT;
  unsigned gx, gy;
};
XextForm xext_expand_form(const int32_t* na, int64_t M, int32_t N, int64_t cus) {
  XextForm f{xext_kk(na, M), false, 0, 0, static_cast<unsigned>((N + 127) / 128), static_cast<unsigned>((M + 31) / 32)};
  if (f.kk > 0 && GS_XEXT_COLS) {
    const int64_t tiles = (M + 31) / 32;
    const unsigned rg4 = static_cast<unsigned>((tiles + 3) / 4), rg8 = static_cast<unsigned>((tiles + 7) / 8);
    const bool wide = int64_t(N / 64) * rg4 >= 2 * cus;
    const bool eight = !wide && GS_XEXT_RT8 && int64_t(N / 32) * rg4 > cus;
    f.cols = true;
    f.CB = wide ? 2 : 1;
    f.RT = eight ? 8 : 4;
    f.gx = static_cast<unsigned>(wide ? (N + 63) / 64 : N / 32);
    f.gy = eight ? rg8 : rg4;
  }
  return f;
}

int check_xext(const char* who, const void* x_ext, int64_t stride_n, int64_t stride_m, int64_t M, int32_t idx_bytes,
               const int32_t* na, int32_t S, int32_t block_n, int32_t N, const void* lb) {
  GS_CHECK_ARG(idx_bytes == 4 || idx_bytes == 8, "%s: idx_bytes=%d", who, idx_bytes);
  GS_CHECK_ARG(stride_n == 1, "%s: x_ext must have unit column stride (got %lld)", who, (long long)stride_n);
  GS_CHECK_ARG(stride_m % 8 == 0 && aligned16(x_ext) && aligned16(lb), "%s: x_ext rows and lb_packed must be 16-byte aligned", who);
  GS_CHECK_ARG(M >= 0 && M < (int64_t(1) << 31) && (M + 31) / 32 <= 65535, "%s: M=%lld out of range", who, (long long)M);
  GS_CHECK_ARG(S >= 1 && S <= GS_MAX_SLICES, "%s: S=%d", who, S);
  GS_CHECK_ARG(block_n > 0 && block_n % 32 == 0, "%s: block_n=%d must be a multiple of 32", who, block_n);
  GS_CHECK_ARG(N > 0 && N % 32 == 0, "%s: N=%d must be a multiple of 32", who, N);
  int tot = 0;
  for (int t = 0; t < 6; ++t) {
    GS_CHECK_ARG(na[t] >= 0, "%s: NA_%d < 0", who, kRanks[t]);
    tot += na[t];
  }
  GS_CHECK_ARG(tot <= 64, "%s: %d kernel-local adapters exceed the 64-bit tile mask", who, tot);
  return GS_OK;
}

// ----------------------------------------------------------------------------
// Address model (test support): replays on the host every global and LDS
// access the x_ext kernels make for one call -- every workgroup, wave, lane
// and loop step, with the launch form the call would choose and the addr::
// formulas the kernels use -- and checks each access against its buffer.
// It follows the values that steer the kernels (the tile masks, the rows'
// kernel-local ids, the slice tables), so the caller passes host copies of
// them.  No HIP call is made.
// ----------------------------------------------------------------------------
struct XextModel {
  // the call
  int64_t M, stride_m, x_cols;      // x_ext: M rows of x_cols valid elements, stride_m apart
  const int64_t* ids;               // kernel-local ids [M]
  int idx_bytes;
  const int64_t* bm;                // tile masks
  int64_t stride_bm, bm_elems;
  int64_t lb_elems;
  const int32_t* tile_slice;
  int64_t ts_len;
  const int32_t* scr;               // slice_col_r [S * 6]
  int na[6];
  int S, block_n, N, H;
  int64_t cus;
  // outcome
  int64_t checked = 0, bad = 0;
  char msg[512] = {0};

  void fail(const char* fmt, ...) {
    if (++bad > 1) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof msg, fmt, ap);
    va_end(ap);
  }
  bool in(const char* what, int64_t lo, int64_t len, int64_t size) {
    ++checked;
    if (lo < 0 || len < 0 || lo + len > size) {
      fail("%s: [%lld, %lld) outside [0, %lld)", what, (long long)lo, (long long)(lo + len), (long long)size);
      return false;
    }
    return true;
  }
  // an access of n elements at column col of x_ext row `row`
  void x_at(const char* what, int64_t row, int64_t col, int n) {
    if (in(what, row, 1, M)) in(what, col, n, x_cols);
  }
  void lb_at(const char* what, int64_t elem) { in(what, elem, 8, lb_elems); }
  // the id of row m as the kernel loads it (an int64 id as its low word)
  int id_at(int64_t m, bool low_word_form) {
    if (low_word_form && idx_bytes == 8) in("ids (low words)", 2 * m, 1, 2 * M);
    else in("ids", m, 1, M);
    return m >= 0 && m < M ? static_cast<int>(ids[m]) : 0;
  }
  int64_t mask_at(int64_t pm) {
    in("bitmask", pm * stride_bm, 1, bm_elems);
    const int64_t e = pm * stride_bm;
    return e >= 0 && e < bm_elems ? bm[e] : 0;
  }
  int slice_at(int64_t idx) {
    in("tile_slice", idx, 1, ts_len);
    const int v = idx >= 0 && idx < ts_len ? tile_slice[idx] : 0;
    in("tile_slice value (slice)", v, 1, S);
    return v >= 0 && v < S ? v : 0;
  }
  int scr_at(int idx) {
    in("slice_col_r (staged)", idx, 1, GS_MAX_SLICES * 6);
    in("slice_col_r (written part)", idx, 1, S * 6);
    return idx >= 0 && idx < S * 6 ? scr[idx] : 0;
  }
  uint64_t valid() const {
    int tot = 0;
    for (int t = 0; t < 6; ++t) tot += na[t];
    return tot >= 64 ? ~0ull : ((1ull << tot) - 1ull);
  }
  static int lowest(uint64_t v) { return __builtin_ctzll(v); }

  // The ids of a 32-row tile's rows as a wave's lanes hold them (0 past the
  // batch) and the mask of the adapters present in them.
  uint64_t rows_mask(int64_t m0, int (&id)[32], bool low_word_form, bool conditional) {
    uint64_t mine = 0;
    for (int i = 0; i < 32; ++i) {
      const bool ok = m0 + i < M;
      id[i] = ok || !conditional ? id_at(addr::xext_row(ok, m0 + i), low_word_form) : 0;
      if (!ok) id[i] = 0;
      if (ok && id[i] >= 1 && id[i] <= 64) mine |= 1ull << (id[i] - 1);
    }
    return mine;
  }

  // xext_block_delta: one memory trip per followed adapter
  void block_delta(int64_t m0, int n0, int s, const int (&id)[32], uint64_t todo) {
    while (todo) {
      const int kid = lowest(todo) + 1;
      todo &= todo - 1;
      int t, first;
      int64_t lb_off;
      if (!addr::xext_tier(na, N, kid, t, first, lb_off)) break;
      const int r = 16 << t, idx = kid - first;
      const int64_t c0 = addr::xext_zcol(scr_at(s * 6 + t), idx, S, r);
      for (int l = 0; l < 64; ++l) {
        const int i = l & 31, h = l >> 5;
        const bool sel = m0 + i < M && id[i] == kid;
        for (int kb = 0; kb < r; kb += 16) {
          const int k0 = kb + 8 * h;
          if (sel) x_at("x_ext shrink values (general)", m0 + i, c0 + k0, 8);
          lb_at("lora_B (general)", addr::xext_brow(lb_off, idx, N, r, n0 + i) + k0);
        }
      }
    }
  }
  // xext_own_z: each lane's own row's shrink values of slice s
  void own_z(int KK, int64_t m0, int s, const int (&id)[32], uint64_t todo) {
    for (int l = 0; l < 64; ++l) {
      const int i = l & 31, h = l >> 5;
      const bool row_ok = m0 + i < M;
      bool ok = row_ok && id[i] >= 1 && id[i] <= 64 && ((todo >> (id[i] - 1)) & 1ull);
      int t, first;
      int64_t lb_off;
      ok = addr::xext_tier(na, N, ok ? id[i] : 1, t, first, lb_off) && ok;
      const int r = 16 << t;
      const int64_t c0 = addr::xext_zcol(scr_at(s * 6 + t), (ok ? id[i] : first) - first, S, r);
      for (int kk = 0; kk < KK; ++kk) {
        const bool kin = ok && kk * 16 < r;
        x_at("x_ext own shrink values", addr::xext_row(row_ok, m0 + i), kin ? c0 + kk * 16 + 8 * h : 0, 8);
      }
    }
  }
  // xext_block_delta_fast: the lora_B of BA followed adapters per trip
  void block_delta_fast(int KK, int BA, int NS, const int* n0, uint64_t todo) {
    while (todo) {
      std::vector<int> rk(BA, 0);
      std::vector<int64_t> boff(BA, -1);   // -1: reads the packed array's first line
      std::vector<int> bidx(BA, 0);
      std::vector<int64_t> blb(BA, 0);
      for (int b = 0; b < BA; ++b) {
        if (!todo) continue;
        const int bit = lowest(todo);
        todo &= todo - 1;
        int t, first;
        int64_t lb_off;
        if (addr::xext_tier(na, N, bit + 1, t, first, lb_off)) {
          rk[b] = 16 << t;
          bidx[b] = bit + 1 - first;
          blb[b] = lb_off;
          boff[b] = 0;
        }
      }
      for (int l = 0; l < 64; ++l) {
        const int i = l & 31, h = l >> 5;
        for (int j = 0; j < NS; ++j)
          for (int b = 0; b < BA; ++b)
            for (int kk = 0; kk < KK; ++kk) {
              if (kk * 16 < rk[b])
                lb_at("lora_B (fast)", addr::xext_brow(blb[b], bidx[b], N, rk[b], i) + 8 * h +
                                           static_cast<int64_t>(n0[j]) * rk[b] + kk * 16);
              else
                lb_at("lora_B (fast, clamped)", 0);
            }
      }
    }
  }
  // xext_delta<KK> of one wave (the caller checked n0 < N)
  void delta(int KK, int64_t m0, int n0, int s, const int (&id)[32], uint64_t bm) {
    uint64_t mine = 0;
    for (int i = 0; i < 32; ++i)
      if (m0 + i < M && id[i] >= 1 && id[i] <= 64) mine |= 1ull << (id[i] - 1);
    const uint64_t todo = mine & bm;
    if (KK == 0) {
      block_delta(m0, n0, s, id, todo);
      return;
    }
    own_z(KK, m0, s, id, todo);
    block_delta_fast(KK, kXextSlots / KK, 1, &n0, todo);
  }

  // ---- xext_expand_kernel / xext_shrink_expand_kernel ----------------------
  // wless: the W-less form (the delta stored into out [M, >= N], stride_om)
  void tile_kernel(int KK, bool wless, int64_t stride_om, int out_es) {
    const int64_t gy = (M + 31) / 32, gx = (N + 127) / 128;
    for (int64_t pm = 0; pm < gy; ++pm) {
      const int64_t m0 = pm * 32;
      const int64_t bm_raw = mask_at(pm);
      int id[32];
      // the rows' ids: loaded by the lanes whose row is in the batch
      rows_mask(m0, id, false, true);
      for (int64_t bx = 0; bx < gx; ++bx) {
        const int n_tile0 = static_cast<int>(bx * 128);
        if (!wless) {
          // the read-modify-write pieces (clamped loads) and their rows' ids
          for (int tid = 0; tid < 256; ++tid)
            for (int q = 0; q < 2; ++q) {
              const int prow = addr::xext_piece_row(tid, q), pc = addr::xext_piece_col(tid, q);
              const int64_t m = m0 + prow;
              const bool ok = m < M && n_tile0 + pc < N;
              x_at("x_ext read-modify-write", ok ? m : m0, ok ? n_tile0 + pc : n_tile0, 8);
              in("delta tile (LDS)", prow * (128 + 4) + pc, 8, 32 * (128 + 4));
              if (ok && id_at(m, false) != 0) x_at("x_ext store", m, n_tile0 + pc, 8);
            }
        }
        // the slice tables (the in-place form loads them before its tile
        // mask test, the W-less form after it)
        int s_of[4];
        if (bm_raw != 0 || !wless) {
          for (int tid = 0; tid < S * 6; ++tid) scr_at(tid);
          for (int wave = 0; wave < 4; ++wave) {
            const int n0 = n_tile0 + 32 * wave;
            s_of[wave] = slice_at((n0 < N ? n0 : n_tile0) / block_n);
          }
        }
        const uint64_t bm = static_cast<uint64_t>(bm_raw) & valid();
        if (bm_raw != 0) {
          for (int wave = 0; wave < 4; ++wave) {
            const int n0 = n_tile0 + 32 * wave;
            if (n0 < N) delta(KK, m0, n0, s_of[wave], id, bm);
          }
        }
        if (wless) {
          for (int tid = 0; tid < 256; ++tid) {
            const int row = tid >> 3, cx = (tid & 7) * 16;
            const int64_t m = m0 + row;
            if (m >= M || n_tile0 + cx >= N) continue;
            in("delta tile (LDS)", row * (128 + 4) + cx, 16, 32 * (128 + 4));
            if (in("out row", m, 1, M)) in("out store", m * stride_om + n_tile0 + cx, 16, (M - 1) * stride_om + N);
            (void)out_es;
          }
        }
      }
    }
  }

  // ---- xext_swiglu_kernel ----------------------------------------------------
  void swiglu(int KK, int64_t stride_om) {
    const int64_t gy = (M + 31) / 32, gx = (H + 127) / 128;
    for (int64_t pm = 0; pm < gy; ++pm) {
      const int64_t m0 = pm * 32;
      int id[32];
      rows_mask(m0, id, false, false);   // every lane loads (a row past the batch reads row 0)
      const int64_t bm_raw = mask_at(pm);
      for (int64_t bx = 0; bx < gx; ++bx) {
        const int h_tile0 = static_cast<int>(bx * 128);
        for (int tid = 0; tid < 256; ++tid) {
          scr_at(tid < S * 6 ? tid : 0);
          for (int q = 0; q < 2; ++q) {
            const int prow = addr::xext_piece_row(tid, q), pc = addr::xext_piece_col(tid, q);
            const int64_t m = m0 + prow;
            const bool pok = m < M && h_tile0 + pc < H;
            x_at("x_ext gate", pok ? m : m0, pok ? h_tile0 + pc : h_tile0, 8);
            x_at("x_ext up", pok ? m : m0, (pok ? h_tile0 + pc : h_tile0) + H, 8);
            in("gate / up delta (LDS)", prow * (128 + 4) + pc, 8, 32 * (128 + 4));
            if (pok && in("out row", m, 1, M)) in("out store", m * stride_om + h_tile0 + pc, 8, (M - 1) * stride_om + H);
          }
        }
        if (bm_raw == 0) continue;
        const uint64_t bm = static_cast<uint64_t>(bm_raw) & valid();
        uint64_t mine = 0;
        for (int i = 0; i < 32; ++i)
          if (m0 + i < M && id[i] >= 1 && id[i] <= 64) mine |= 1ull << (id[i] - 1);
        const uint64_t todo0 = mine & bm;
        for (int wave = 0; wave < 4; ++wave) {
          const int h0 = h_tile0 + 32 * wave;
          if (h0 >= H) continue;
          if (KK == 0) {
            uint64_t todo = todo0;
            while (todo) {
              const int kid = lowest(todo) + 1;
              todo &= todo - 1;
              int t, first;
              int64_t lb_off;
              if (!addr::xext_tier(na, N, kid, t, first, lb_off)) break;
              const int r = 16 << t, idx = kid - first;
              const int64_t cg = addr::xext_zcol(scr_at(t), idx, S, r), cu = addr::xext_zcol(scr_at(6 + t), idx, S, r);
              for (int l = 0; l < 64; ++l) {
                const int i = l & 31, h = l >> 5;
                const bool row_ok = m0 + i < M, sel = row_ok && id[i] == kid;
                const int64_t xr = addr::xext_row(row_ok, m0 + i);
                for (int kb = 0; kb < r; kb += 32) {
                  const bool two = kb + 16 < r;
                  const int k0 = kb + 8 * h, k1 = two ? k0 + 16 : k0;
                  for (int k : {k0, k1}) {
                    x_at("x_ext gate shrink values", xr, (sel ? cg : 0) + k, 8);
                    x_at("x_ext up shrink values", xr, (sel ? cu : 0) + k, 8);
                    lb_at("gate lora_B", addr::xext_brow(lb_off, idx, N, r, h0 + i) + k);
                    lb_at("up lora_B", addr::xext_brow(lb_off, idx, N, r, H + h0 + i) + k);
                  }
                }
              }
            }
          } else {
            own_z(KK, m0, 0, id, todo0);
            own_z(KK, m0, 1, id, todo0);
            const int n0s[2] = {h0, H + h0};
            block_delta_fast(KK, kXextSlots / 2 / KK, 2, n0s, todo0);
          }
        }
      }
    }
  }

  // ---- xext_cols_kernel ------------------------------------------------------
  void cols(int KK, int CB, int RT, unsigned gx, unsigned gy) {
    const int NC = 32 * CB, RMAX = 16 * KK, CST = RMAX * 2 + 16, ABLK = NC * CST, CA = CB == 1 ? 16 : 8;
    const int CAW = CA / RT, QP = NC * RMAX / 8 / 64, DLD = NC + 4, LPR = NC / 16, PASSES = 32 * LPR / 64;
    const int64_t bs_bytes = static_cast<int64_t>(CA) * ABLK + 64 * 16;
    const int64_t n_tiles = (M + 31) / 32;
    const uint64_t vb = valid();
    for (unsigned by = 0; by < gy; ++by)
      for (unsigned bx = 0; bx < gx; ++bx) {
        const int n_blk0 = static_cast<int>(bx) * NC;
        const int64_t pm0 = static_cast<int64_t>(by) * RT;
        const int ncols = std::min(NC, N - n_blk0);
        std::vector<int64_t> bmt(RT, 0);
        uint64_t all = 0;
        for (int w = 0; w < RT; ++w) {
          bmt[w] = pm0 + w < n_tiles ? mask_at(pm0 + w) : 0;
          all |= static_cast<uint64_t>(bmt[w]);
        }
        all &= vb;
        std::vector<std::array<int, 32>> wid(RT);
        std::vector<int> wsc(RT * CB);
        for (int wave = 0; wave < RT; ++wave) {
          const int64_t m0 = (pm0 + wave) * 32;
          for (int l = 0; l < 64; ++l) {
            const int tid = 64 * wave + l;
            scr_at(tid < S * 6 ? tid : 0);
            const int cx = (l % LPR) * 16;
            for (int ps = 0; ps < PASSES; ++ps) {
              const int row = ps * (64 / LPR) + l / LPR;
              const int64_t m = m0 + row;
              const bool ook = m < M && n_blk0 + cx < N;
              const int64_t orow = addr::xext_row(ook, m);
              x_at("x_ext read-modify-write", orow, ook ? n_blk0 + cx : 0, 16);
              const int oid = id_at(orow, true);
              in("delta tile (LDS)", (static_cast<int64_t>(wave) * 32 * DLD + row * DLD + cx) * 4, 16 * 4, bs_bytes);
              if (ook && oid != 0) x_at("x_ext store", orow, n_blk0 + cx, 16);
            }
          }
          for (int i = 0; i < 32; ++i) {
            const bool row_ok = m0 + i < M;
            const int v = id_at(addr::xext_row(row_ok, m0 + i), true);
            wid[wave][i] = row_ok && pm0 + wave < n_tiles ? v : 0;
          }
          for (int c = 0; c < CB; ++c) {
            const int n0 = n_blk0 + 32 * c;
            wsc[wave * CB + c] = slice_at((n0 < N ? n0 : n_blk0) / block_n);
          }
        }
        bool first_chunk = true;
        while (all) {
          // the chunk's adapters (lane j < CA describes the j-th)
          std::vector<int> my_r(CA, 0);
          std::vector<int64_t> my_off(CA, 0);
          uint64_t mm = all;
          for (int j = 0; j < CA; ++j) {
            if (mm) {
              const int bit = lowest(mm);
              int t, first;
              int64_t lb_off;
              if (addr::xext_tier(na, N, bit + 1, t, first, lb_off)) {
                my_r[j] = 16 << t;
                my_off[j] = addr::xext_brow(lb_off, bit + 1 - first, N, my_r[j], n_blk0);
              }
              mm &= mm - 1;
            }
          }
          for (int k = 0; k < CA; ++k) all &= all - 1;
          for (int wave = 0; wave < RT; ++wave)
            for (int jw = 0; jw < CAW; ++jw) {
              const int j = RT * jw + wave, r = my_r[j];
              const int sh = 31 - __builtin_clz(r > 0 ? r / 8 : 1);
              for (int l = 0; l < 64; ++l)
                for (int q = 0; q < QP; ++q) {
                  const int pc = l + 64 * q;
                  const bool real = pc < ncols * r / 8;
                  lb_at("lora_B block (staged)", real ? my_off[j] + 8 * pc : 0);
                  if (real) {
                    const int col = addr::xext_stage_colof(pc, sh), kq = addr::xext_stage_kof(pc, sh);
                    in("staged block column", col, 1, NC);
                    in("staged block piece", kq * 16, 16, CST);
                    in("staging buffer (LDS)", static_cast<int64_t>(j) * ABLK + col * CST + kq * 16, 16, bs_bytes);
                  } else {
                    in("staging sink (LDS)", static_cast<int64_t>(CA) * ABLK + l * 16, 16, bs_bytes);
                  }
                }
            }
          if (first_chunk) {
            for (int wave = 0; wave < RT; ++wave) {
              const int64_t m0 = (pm0 + wave) * 32;
              const uint64_t todo = static_cast<uint64_t>(bmt[wave]) & vb;
              int id[32];
              for (int i = 0; i < 32; ++i) id[i] = wid[wave][i];
              for (int c = 0; c < CB; ++c) own_z(KK, m0, wsc[wave * CB + c], id, todo);
            }
            first_chunk = false;
          }
          for (int j = 0; j < CA; ++j)
            for (int l = 0; l < 64; ++l)
              for (int c = 0; c < CB; ++c)
                for (int kk = 0; kk < KK; ++kk)
                  in("staged operand read (LDS)",
                     static_cast<int64_t>(j) * ABLK + (32 * c + (l & 31)) * CST + (kk * 16 + 8 * (l >> 5)) * 2, 16,
                     bs_bytes);
        }
      }
  }
};
}  // namespace

}  // namespace gs

using namespace gs;

extern "C" {

int gs_switch_lora_expand(void* x_ext, int64_t stride_m, int64_t stride_n, int64_t M, const void* adapter_indices,
                          int32_t idx_bytes, const int64_t* bitmask, int64_t stride_bm, const void* lb_packed,
                          const int32_t* tile_slice, const int32_t* slice_col_r, const int32_t* na, int32_t S,
                          int32_t block_n, int32_t N, void* stream) {
  int rc = check_xext("gs_switch_lora_expand", x_ext, stride_n, stride_m, M, idx_bytes, na, S, block_n, N, lb_packed);
  if (rc != GS_OK) return rc;
  if (M == 0) return GS_OK;
  XextArgs a{};
  a.x_ext = x_ext;
  a.stride_m = stride_m;
  a.M = M;
  a.ids = adapter_indices;
  a.idx_bytes = idx_bytes;
  a.bitmask = bitmask;
  a.stride_bm = stride_bm;
  a.lb = static_cast<const uint16_t*>(lb_packed);
  a.slice_col_r = slice_col_r;
  for (int t = 0; t < 6; ++t) a.na[t] = na[t];
  a.S = S;
  a.N = N;
  dim3 grid((N + 127) / 128, static_cast<unsigned>((M + 31) / 32));
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint16_t* xo = static_cast<uint16_t*>(x_ext);
  const XextForm f = xext_expand_form(na, M, N, device_cus());
  const int kk = f.kk;
  if (f.cols) {
    const dim3 g(f.gx, f.gy);
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, g, dim3(64 * f.RT), 0, st, a, xo, tile_slice, block_n); };
    auto pick = [&](auto i64) {
      constexpr bool I64 = decltype(i64)::value;
      if (kk == 2) {
        if (f.CB == 2) go(xext_cols_kernel<2, 2, 4, I64>);
        else if (f.RT == 8) go(xext_cols_kernel<2, 1, 8, I64>);
        else go(xext_cols_kernel<2, 1, 4, I64>);
      } else {
        if (f.CB == 2) go(xext_cols_kernel<4, 2, 4, I64>);
        else if (f.RT == 8) go(xext_cols_kernel<4, 1, 8, I64>);
        else go(xext_cols_kernel<4, 1, 4, I64>);
      }
    };
    if (idx_bytes == 8) pick(std::true_type{});
    else pick(std::false_type{});
    GS_CHECK_LAUNCH("gs_switch_lora_expand");
    return GS_OK;
  }
  switch (kk) {
    case 2: hipLaunchKernelGGL(xext_expand_kernel<2>, grid, dim3(256), 0, st, a, xo, tile_slice, block_n); break;
    case 4: hipLaunchKernelGGL(xext_expand_kernel<4>, grid, dim3(256), 0, st, a, xo, tile_slice, block_n); break;
    default: hipLaunchKernelGGL(xext_expand_kernel<0>, grid, dim3(256), 0, st, a, xo, tile_slice, block_n); break;
  }
  GS_CHECK_LAUNCH("gs_switch_lora_expand");
  return GS_OK;
}

int gs_switch_lora_shrink_expand(void* out, int32_t out_dtype, int64_t stride_om, int64_t stride_on,
                                 const void* x_ext, int64_t stride_m, int64_t stride_n, int64_t M,
                                 const void* adapter_indices, int32_t idx_bytes, const int64_t* bitmask,
                                 int64_t stride_bm, const void* lb_packed, const int32_t* tile_slice,
                                 const int32_t* slice_col_r, const int32_t* na, int32_t S, int32_t block_n, int32_t N,
                                 void* stream) {
  const char* who = "gs_switch_lora_shrink_expand";
  int rc = check_xext(who, x_ext, stride_n, stride_m, M, idx_bytes, na, S, block_n, N, lb_packed);
  if (rc != GS_OK) return rc;
  GS_CHECK_ARG(out_dtype == GS_DTYPE_BF16 || out_dtype == GS_DTYPE_FP32, "%s: out_dtype=%d", who, out_dtype);
  const int vec = out_dtype == GS_DTYPE_BF16 ? 8 : 4;
  GS_CHECK_ARG(stride_on == 1 && stride_om >= N && stride_om % vec == 0 && aligned16(out),
               "%s: out must be row-contiguous [M, >= N] with 16-byte aligned rows", who);
  if (M == 0) return GS_OK;
  XextArgs a{};
  a.x_ext = x_ext;
  a.stride_m = stride_m;
  a.M = M;
  a.ids = adapter_indices;
  a.idx_bytes = idx_bytes;
  a.bitmask = bitmask;
  a.stride_bm = stride_bm;
  a.lb = static_cast<const uint16_t*>(lb_packed);
  a.slice_col_r = slice_col_r;
  for (int t = 0; t < 6; ++t) a.na[t] = na[t];
  a.S = S;
  a.N = N;
  dim3 grid((N + 127) / 128, static_cast<unsigned>((M + 31) / 32));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int kk = xext_kk(na, M);
  if (out_dtype == GS_DTYPE_FP32) {
    if (kk == 2) hipLaunchKernelGGL((xext_shrink_expand_kernel<true, 2>), grid, dim3(256), 0, st, a, out, stride_om, tile_slice, block_n);
    else if (kk == 4) hipLaunchKernelGGL((xext_shrink_expand_kernel<true, 4>), grid, dim3(256), 0, st, a, out, stride_om, tile_slice, block_n);
    else hipLaunchKernelGGL((xext_shrink_expand_kernel<true, 0>), grid, dim3(256), 0, st, a, out, stride_om, tile_slice, block_n);
  } else {
    if (kk == 2) hipLaunchKernelGGL((xext_shrink_expand_kernel<false, 2>), grid, dim3(256), 0, st, a, out, stride_om, tile_slice, block_n);
    else if (kk == 4) hipLaunchKernelGGL((xext_shrink_expand_kernel<false, 4>), grid, dim3(256), 0, st, a, out, stride_om, tile_slice, block_n);
    else hipLaunchKernelGGL((xext_shrink_expand_kernel<false, 0>), grid, dim3(256), 0, st, a, out, stride_om, tile_slice, block_n);
  }
  GS_CHECK_LAUNCH(who);
  return GS_OK;
}

int gs_switch_lora_expand_swiglu(void* out, int64_t stride_om, int64_t stride_on, const void* x_ext,
                                 int64_t stride_m, int64_t stride_n, int64_t M, const void* adapter_indices,
                                 int32_t idx_bytes, const int64_t* bitmask, int64_t stride_bm,
                                 const void* lb_packed, const int32_t* slice_col_r, const int32_t* na, int32_t S,
                                 int32_t block_n, int32_t H, int32_t N, void* stream) {
  int rc = check_xext("gs_switch_lora_expand_swiglu", x_ext, stride_n, stride_m, M, idx_bytes, na, S, block_n, N,
                      lb_packed);
  if (rc != GS_OK) return rc;
  GS_CHECK_ARG(S == 2 && N == 2 * H && H % 32 == 0, "gs_switch_lora_expand_swiglu: need S == 2, N == 2H, H %% 32 == 0");
  GS_CHECK_ARG(stride_on == 1 && stride_om % 8 == 0 && aligned16(out), "gs_switch_lora_expand_swiglu: out must be row-contiguous and 16-byte aligned");
  if (M == 0) return GS_OK;
  XextArgs a{};
  a.x_ext = x_ext;
  a.stride_m = stride_m;
  a.M = M;
  a.ids = adapter_indices;
  a.idx_bytes = idx_bytes;
  a.bitmask = bitmask;
  a.stride_bm = stride_bm;
  a.lb = static_cast<const uint16_t*>(lb_packed);
  a.slice_col_r = slice_col_r;
  for (int t = 0; t < 6; ++t) a.na[t] = na[t];
  a.S = S;
  a.N = N;
  dim3 grid((H + 127) / 128, static_cast<unsigned>((M + 31) / 32));
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint16_t* o = static_cast<uint16_t*>(out);
  switch (xext_kk(na, M)) {
    case 2: hipLaunchKernelGGL(xext_swiglu_kernel<2>, grid, dim3(256), 0, st, a, o, stride_om, H); break;
    case 4: hipLaunchKernelGGL(xext_swiglu_kernel<4>, grid, dim3(256), 0, st, a, o, stride_om, H); break;
    default: hipLaunchKernelGGL(xext_swiglu_kernel<0>, grid, dim3(256), 0, st, a, o, stride_om, H); break;
  }
  GS_CHECK_LAUNCH("gs_switch_lora_expand_swiglu");
  return GS_OK;
}

int64_t gs_check_xext_addresses(int32_t op, int64_t M, int64_t stride_m, int64_t x_cols, const int64_t* ids,
                                int32_t idx_bytes, const int64_t* bitmask, int64_t stride_bm, int64_t bitmask_elems,
                                int64_t lb_elems, const int32_t* tile_slice, int64_t tile_slice_len,
                                const int32_t* slice_col_r, const int32_t* na, int32_t S, int32_t block_n, int32_t N,
                                int32_t H, int64_t stride_om, int32_t out_dtype, char* msg, int64_t msg_len,
                                int64_t* checked) {
  const char* who = "gs_check_xext_addresses";
  GS_CHECK_ARG(op >= 0 && op <= 2, "%s: op=%d", who, op);
  GS_CHECK_ARG(M >= 0 && stride_m >= x_cols && x_cols > 0 && (ids || M == 0) && (bitmask || M == 0) && slice_col_r &&
                   na && (tile_slice || op == 2),
               "%s: bad arguments", who);
  GS_CHECK_ARG(idx_bytes == 4 || idx_bytes == 8, "%s: idx_bytes=%d", who, idx_bytes);
  GS_CHECK_ARG(S >= 1 && S <= GS_MAX_SLICES && block_n > 0 && N > 0, "%s: S / block_n / N", who);
  XextModel m{};
  m.M = M;
  m.stride_m = stride_m;
  m.x_cols = x_cols;
  m.ids = ids;
  m.idx_bytes = idx_bytes;
  m.bm = bitmask;
  m.stride_bm = stride_bm;
  m.bm_elems = bitmask_elems;
  m.lb_elems = lb_elems;
  m.tile_slice = tile_slice;
  m.ts_len = tile_slice_len;
  m.scr = slice_col_r;
  for (int t = 0; t < 6; ++t) m.na[t] = na[t];
  m.S = S;
  m.block_n = block_n;
  m.N = N;
  m.H = H;
  m.cus = device_cus();
  if (M > 0) {
    const int kk = xext_kk(na, M);
    if (op == 0) {
      // the form the launch would take on this device, and every other
      // column-block shape (they depend on the CU count)
      const XextForm f = xext_expand_form(na, M, N, m.cus);
      if (f.cols) {
        m.cols(f.kk, f.CB, f.RT, f.gx, f.gy);
        const int64_t tiles = (M + 31) / 32;
        const unsigned rg4 = static_cast<unsigned>((tiles + 3) / 4), rg8 = static_cast<unsigned>((tiles + 7) / 8);
        if (!(f.CB == 2)) m.cols(f.kk, 2, 4, static_cast<unsigned>((N + 63) / 64), rg4);
        if (!(f.CB == 1 && f.RT == 8)) m.cols(f.kk, 1, 8, static_cast<unsigned>(N / 32), rg8);
        if (!(f.CB == 1 && f.RT == 4)) m.cols(f.kk, 1, 4, static_cast<unsigned>(N / 32), rg4);
      }
      m.tile_kernel(kk, false, 0, 2);   // the per-tile form (taken past 1024 rows, or without the fast path)
      if (kk > 0) m.tile_kernel(0, false, 0, 2);
    } else if (op == 1) {
      GS_CHECK_ARG(stride_om >= N, "%s: stride_om", who);
      m.tile_kernel(kk, true, stride_om, out_dtype == GS_DTYPE_FP32 ? 4 : 2);
      if (kk > 0) m.tile_kernel(0, true, stride_om, out_dtype == GS_DTYPE_FP32 ? 4 : 2);
    } else {
      GS_CHECK_ARG(S == 2 && N == 2 * H && stride_om >= H, "%s: the SwiGLU form needs S == 2, N == 2H", who);
      m.swiglu(kk, stride_om);
      if (kk > 0) m.swiglu(0, stride_om);
    }
  }
  if (checked) *checked = m.checked;
  if (msg && msg_len > 0) snprintf(msg, static_cast<size_t>(msg_len), "%s", m.msg);
  return m.bad;
}

}  // extern "C"
