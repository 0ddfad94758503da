// Shared device and host helpers for the gfx950 switched-LoRA kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>

#include "../../include/granite_switch_amd.h"

namespace gs {

// ---------------------------------------------------------------------------
// Host-side error reporting: every entry point returns a GS_* status and leaves
// a human-readable message retrievable with gs_last_error().
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);

#define GS_CHECK_ARG(cond, ...)                 \
  do {                                          \
    if (!(cond)) {                              \
      ::gs::set_error(__VA_ARGS__);             \
      return GS_ERR_INVALID;                    \
    }                                           \
  } while (0)

#define GS_CHECK_LAUNCH(what)                                                   \
  do {                                                                          \
    hipError_t e_ = hipGetLastError();                                          \
    if (e_ != hipSuccess) {                                                     \
      ::gs::set_error("%s: launch failed: %s", what, hipGetErrorString(e_));    \
      return GS_ERR_HIP;                                                        \
    }                                                                           \
  } while (0)

// Compute units of the current device, cached per device (one cache for the
// whole library; concurrent first calls store the same value); 256 when no
// device answers.
inline int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even float -> bf16 bits: gfx950's v_cvt_pk_bf16_f32 (one
// instruction for two values; NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Exclusive lane mask: bits of lanes below the calling lane (wave64).
__device__ __forceinline__ uint64_t lanemask_lt() {
  int l = __lane_id();
  return l == 0 ? 0ull : (~0ull >> (64 - l));
}

// 32x32 output tile, K=16 bf16 per step: D[i][j] += sum_k A[i][k] B[k][j].
// Lane l supplies A[l%32][8*(l/32) .. +8) and B[8*(l/32) .. +8)[l%32].
__device__ __forceinline__ f32x16 mfma32_bf16(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// 32x32 output tile, K=2 fp32 per step. Lane l supplies A[l%32][l/32] and B[l/32][l%32].
__device__ __forceinline__ f32x16 mfma32_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also
// orders global memory, which on gfx9 waits for every outstanding global load
// and store of the wave -- including prefetches meant to stay in flight across
// the barrier.  Use this one where the barrier protects LDS data only.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Row of the 32x32 MFMA accumulator element v (0..15) held by lane l; the
// column is l % 32.
__device__ __forceinline__ int mfma32_row(int v, int l) { return ((v >> 2) << 3) + ((l >> 5) << 2) + (v & 3); }

// ----------------------------------------------------------------------------
// Element traits.  A "batch" is the k-span one lane pair covers with four
// 16-byte loads per row: 64 bf16 or 32 fp32 (each lane half loads 64 bytes).
// ----------------------------------------------------------------------------
template <bool BF16>
struct Elt;
template <>
struct Elt<true> {
  static constexpr int kBatch = 64;       // k per batch
  static constexpr int kPerPiece = 8;     // elements per 16-byte piece
  static constexpr int kSize = 2;
};
template <>
struct Elt<false> {
  static constexpr int kBatch = 32;
  static constexpr int kPerPiece = 4;
  static constexpr int kSize = 4;
};

// ---- direct global -> LDS transfers -----------------------------------------
// s_waitcnt immediate for "vmcnt <= n" (expcnt and lgkmcnt not waited on)
constexpr int wait_vm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// One wave-wide global_load_lds_dwordx4: lane i moves the 16 bytes at its src
// to LDS at M0 + 16 i, where M0 holds the wave's (uniform) destination.  The
// transfer counts in vmcnt until the bytes are in LDS; it is written as
// assembly, so the compiler neither waits for it nor orders LDS reads
// against it -- wait with s_waitcnt(wait_vm(n)) and a barrier.
__device__ __forceinline__ void dma16(const char* src, char* lds_dst) {
  const uint32_t dst =
      __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr_t)(lds_dst))));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(dst) : "memory", "m0");
}

// As dma16 for data read once (streamed: the nt policy keeps it from
// displacing data that other workgroups re-read from L2).
__device__ __forceinline__ void dma16_nt(const char* src, char* lds_dst) {
  const uint32_t dst =
      __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr_t)(lds_dst))));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(dst) : "memory", "m0");
}

__device__ __forceinline__ void mem_fence_compiler() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }
// 16-byte load and store with the streaming (nt) cache policy, for data a
// launch touches once: it does not displace what other workgroups re-read
// from L2.
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16_nt(void* p, const u32x4& v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}
__device__ __forceinline__ u32x4 sel16(bool keep, const u32x4& v) {
  return keep ? v : u32x4{0u, 0u, 0u, 0u};
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// y piece (16 bytes = 8 bf16 / 4 fp32) + delta, rounded once, stored back.
template <bool BF16, bool NT = false>
__device__ __forceinline__ void add_store_y(void* y, int64_t off, const u32x4& in, const float* d) {
  u32x4* p = reinterpret_cast<u32x4*>(static_cast<char*>(y) + off * Elt<BF16>::kSize);
  if constexpr (BF16) {
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t w = in[e];
      const float lo = bf16_bits_to_f32(static_cast<uint16_t>(w & 0xffffu)) + d[2 * e];
      const float hi = bf16_bits_to_f32(static_cast<uint16_t>(w >> 16)) + d[2 * e + 1];
      o[e] = pack_bf16x2(lo, hi);
    }
    const u32x4 v = u32x4{o[0], o[1], o[2], o[3]};
    if constexpr (NT) st16_nt(p, v);
    else *p = v;
  } else {
    const f32x4 f = __builtin_bit_cast(f32x4, in);
    const u32x4 v = __builtin_bit_cast(u32x4, f32x4{f.x + d[0], f.y + d[1], f.z + d[2], f.w + d[3]});
    if constexpr (NT) st16_nt(p, v);
    else *p = v;
  }
}

// y piece (16 bytes = 8 bf16 / 4 fp32) + delta, rounded once; returns the bits.
template <bool BF16>
__device__ __forceinline__ u32x4 add_y16(const u32x4& in, const float* d) {
  if constexpr (BF16) {
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t w = in[e];
      const float lo = bf16_bits_to_f32(static_cast<uint16_t>(w & 0xffffu)) + d[2 * e];
      const float hi = bf16_bits_to_f32(static_cast<uint16_t>(w >> 16)) + d[2 * e + 1];
      o[e] = pack_bf16x2(lo, hi);
    }
    return u32x4{o[0], o[1], o[2], o[3]};
  } else {
    const f32x4 f = __builtin_bit_cast(f32x4, in);
    return __builtin_bit_cast(u32x4, f32x4{f.x + d[0], f.y + d[1], f.z + d[2], f.w + d[3]});
  }
}

// acc += one 16-byte piece of each operand (bf16: K=16 over both lane halves;
// fp32: four K=2 steps).  Both operands pair their elements by (lane half,
// element), so any fixed assignment of k to pieces is a correct contraction.
template <bool BF16>
__device__ __forceinline__ f32x16 mfma_piece(const u32x4& a, const u32x4& b, f32x16 acc) {
  if constexpr (BF16) {
    return mfma32_bf16(a, b, acc);
  } else {
    const f32x4 x = __builtin_bit_cast(f32x4, a);
    const f32x4 w = __builtin_bit_cast(f32x4, b);
    acc = mfma32_f32(x.x, w.x, acc);
    acc = mfma32_f32(x.y, w.y, acc);
    acc = mfma32_f32(x.z, w.z, acc);
    return mfma32_f32(x.w, w.w, acc);
  }
}

// Output slices of a projection: slice s covers columns [bounds[s], bounds[s+1]).
struct SliceInfo {
  int S;
  int bounds[GS_MAX_SLICES + 1];
};

// ---------------------------------------------------------------------------
// Segment work lists. Adapter g (1..NA) owns slots [seg[g-1], seg[g]) of the
// adapter-sorted token permutation. A launch covers the adapters whose rank in
// this module lies in its rank window [rw.lo, rw.hi] (lo >= 1, so adapters of
// rank 0 -- not applicable here -- are always skipped): a module whose ranks
// differ widely runs one launch per rank class, each sized for its own ranks.
// Tiles are TM consecutive slots of one adapter. Every wave computes the same
// answer, so no LDS or barrier is needed.
// ---------------------------------------------------------------------------
struct RankWindow {
  int lo;
  int hi;
};

__host__ __device__ __forceinline__ bool in_window(const RankWindow& rw, int r) { return r >= rw.lo && r <= rw.hi; }

struct TileRef {
  int g;        // global adapter id (0 = no tile: the workgroup exits)
  int slot0;    // first slot of the tile
  int nrows;    // rows in the tile (1..TM)
  int rank;     // the adapter's rank in this module
  int64_t off;  // offs[g] (the adapter's weight offset), fetched in the same pass
};

// Number of tiles of TM slots over all applicable adapters (every wave
// computes the same value).
template <int TM>
__device__ __forceinline__ int count_tiles(const int32_t* __restrict__ seg, const int32_t* __restrict__ ranks,
                                           int num_adapters, RankWindow rw) {
  const int l = __lane_id();
  int total = 0;
  for (int g0 = 1; g0 <= num_adapters; g0 += 64) {
    const int g = g0 + l;
    int ntiles = 0;
    if (g <= num_adapters && in_window(rw, ranks[g])) ntiles = (seg[g] - seg[g - 1] + TM - 1) / TM;
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) ntiles += __shfl_xor(ntiles, d, 64);
    total += ntiles;
  }
  return total;
}

// Work item `lin` of a 1-D launch over (tile, sub) pairs, sub < nsub.
// Workgroups are dealt to the 8 XCDs round-robin by id, so XCD x runs ids
// x, x+8, ...; each XCD gets a contiguous range of the batch's tiles, so the
// tiles of one adapter -- which read the same weights -- share an XCD's L2.
// The launch has 8 * ceil(max_tiles / 8) * nsub workgroups; ids past the
// batch's tiles get tile = -1.
struct XcdItem {
  int tile;
  int sub;
};
__host__ __device__ __forceinline__ XcdItem xcd_item(int lin, int total_tiles, int nsub) {
  const int tpx = (total_tiles + 7) >> 3;
  XcdItem it{-1, 0};
  if (tpx == 0) return it;
  const int j = lin >> 3;
  const int tt = j % tpx;
  const int sub = j / tpx;
  const int tile = (lin & 7) * tpx + tt;
  if (sub < nsub && tile < total_tiles) {
    it.tile = tile;
    it.sub = sub;
  }
  return it;
}

// Item layout of a launch over (tile, sub) pairs.  The XCD form (xcd_item)
// gives each XCD a contiguous range of tiles, so an adapter's tiles share one
// L2: for launches of many tiles.  The flat form makes item lin the pair
// (lin / nsub, lin % nsub), so consecutive items -- and workgroups, which are
// dealt to the XCDs round-robin -- fall on different XCDs: for a launch of a
// few tiles with many subs each (a rank class of one large adapter), which
// the XCD form would leave to one XCD.
__host__ __device__ __forceinline__ XcdItem work_item(int lin, int total_tiles, int nsub, bool flat) {
  if (!flat) return xcd_item(lin, total_tiles, nsub);
  XcdItem it{-1, 0};
  if (lin >= 0 && lin < total_tiles * nsub) {
    it.tile = lin / nsub;
    it.sub = lin - it.tile * nsub;
  }
  return it;
}

// Items a launch over `total_tiles` tiles must cover (ids at or past it have
// no work in either form).
__host__ __device__ __forceinline__ int work_items(int total_tiles, int nsub, bool flat) {
  return flat ? total_tiles * nsub : 8 * ((total_tiles + 7) >> 3) * nsub;
}

// Tile jj of an adapter whose slots are [lo, hi): TM consecutive slots (the
// last tile shorter), or, with BAL, one of ceil(n / TM) tiles of near-equal
// size (rows spread evenly, at most TM each).
template <int TM, bool BAL>
__host__ __device__ __forceinline__ void tile_span(int lo, int hi, int jj, int& slot0, int& nrows) {
  if constexpr (BAL) {
    const int n = hi - lo;
    const int nt = (n + TM - 1) / TM;
    static_assert(TM >= 32, "the 32-bit products below assume at most n / 32 + 1 tiles");
    if (n < (1 << 18)) {                   // (jj + 1) * n < 2^13 * 2^18: 32-bit products
      slot0 = lo + (jj * n) / nt;
      nrows = lo + ((jj + 1) * n) / nt - slot0;
    } else {                               // an adapter with 2^18 or more slots
      slot0 = lo + static_cast<int>((static_cast<int64_t>(jj) * n) / nt);
      nrows = lo + static_cast<int>((static_cast<int64_t>(jj + 1) * n) / nt) - slot0;
    }
  } else {
    slot0 = lo + jj * TM;
    nrows = min(TM, hi - slot0);
  }
}

template <int TM, bool BAL = false>
__device__ __forceinline__ TileRef find_tile(const int32_t* __restrict__ seg, const int32_t* __restrict__ ranks,
                                             const int64_t* __restrict__ offs, int num_adapters, RankWindow rw,
                                             int tile_id) {
  TileRef ref{0, 0, 0, 0, 0};
  const int l = __lane_id();
  int carry = 0;
  for (int g0 = 1; g0 <= num_adapters; g0 += 64) {
    const int g = g0 + l;
    int ntiles = 0;
    int lo = 0, hi = 0, rk = 0;
    int64_t of = 0;
    if (g <= num_adapters) {
      lo = seg[g - 1];
      hi = seg[g];
      rk = ranks[g];
      of = offs[g];
      ntiles = in_window(rw, rk) ? (hi - lo + TM - 1) / TM : 0;
    }
    // inclusive scan over the wave
    int incl = ntiles;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      int v = __shfl_up(incl, d, 64);
      if (l >= d) incl += v;
    }
    const int excl = incl - ntiles;
    const int total = __shfl(incl, 63, 64);
    const bool mine = (ntiles > 0) && (tile_id >= carry + excl) && (tile_id < carry + incl);
    const uint64_t bal = __ballot(mine);
    if (bal) {
      const int src = __ffsll(static_cast<long long>(bal)) - 1;
      const int jj = tile_id - carry - __shfl(excl, src, 64);
      const int slo = __shfl(lo, src, 64);
      const int shi = __shfl(hi, src, 64);
      ref.g = g0 + src;
      tile_span<TM, BAL>(slo, shi, jj, ref.slot0, ref.nrows);
      ref.rank = __shfl(rk, src, 64);
      ref.off = __shfl(of, src, 64);
      return ref;
    }
    carry += total;
  }
  return ref;
}

// The tile of work item `lin` of a 1-D launch over (tile, sub) pairs (see
// work_item), in one pass over the adapter table when it fits one wave
// (<= 64 adapters): the tile count and the tile's lookup share the same
// loads.  nsub_of(total tiles) gives the number of subs per tile (every wave
// computes the same value); the tile count is returned in `total_out` (a
// workgroup that loops over items finds its later tiles with tile_at).
// Returns g = 0 when the item has no tile.
template <int TM, bool BAL = false, typename NsubOf>
__device__ __forceinline__ TileRef locate_tile_by(const int32_t* __restrict__ seg, const int32_t* __restrict__ ranks,
                                                  const int64_t* __restrict__ offs, int num_adapters, RankWindow rw,
                                                  int lin, bool flat, NsubOf nsub_of, int& sub, int& total_out) {
  TileRef ref{0, 0, 0, 0, 0};
  if (num_adapters > 64) {
    const int total = count_tiles<TM>(seg, ranks, num_adapters, rw);
    total_out = total;
    const XcdItem it = work_item(lin, total, nsub_of(total), flat);
    sub = it.sub;
    return it.tile < 0 ? ref : find_tile<TM, BAL>(seg, ranks, offs, num_adapters, rw, it.tile);
  }
  const int l = __lane_id();
  const int g = 1 + l;
  int ntiles = 0, lo = 0, hi = 0, rk = 0;
  int64_t of = 0;
  if (g <= num_adapters) {
    lo = seg[g - 1];
    hi = seg[g];
    rk = ranks[g];
    of = offs[g];
    ntiles = in_window(rw, rk) ? (hi - lo + TM - 1) / TM : 0;
  }
  int incl = ntiles;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int v = __shfl_up(incl, d, 64);
    if (l >= d) incl += v;
  }
  const int total = __shfl(incl, 63, 64);
  total_out = total;
  const XcdItem it = work_item(lin, total, nsub_of(total), flat);
  sub = it.sub;
  if (it.tile < 0) return ref;
  const int excl = incl - ntiles;
  const uint64_t bal = __ballot(ntiles > 0 && it.tile >= excl && it.tile < incl);
  if (bal == 0) return ref;
  const int src = __ffsll(static_cast<long long>(bal)) - 1;
  const int jj = it.tile - __shfl(excl, src, 64);
  const int slo = __shfl(lo, src, 64);
  const int shi = __shfl(hi, src, 64);
  ref.g = 1 + src;
  tile_span<TM, BAL>(slo, shi, jj, ref.slot0, ref.nrows);
  ref.rank = __shfl(rk, src, 64);
  ref.off = __shfl(of, src, 64);
  return ref;
}

// As locate_tile_by with a fixed number of subs per tile.
template <int TM>
__device__ __forceinline__ TileRef locate_tile(const int32_t* __restrict__ seg, const int32_t* __restrict__ ranks,
                                               const int64_t* __restrict__ offs, int num_adapters, RankWindow rw,
                                               int lin, bool flat, int nsub, int& sub, int& total) {
  return locate_tile_by<TM>(seg, ranks, offs, num_adapters, rw, lin, flat, [nsub](int) { return nsub; }, sub, total);
}

// The tile of a later item `lin` of a workgroup that loops over items, the
// batch's tile count already known.
template <int TM, bool BAL = false>
__device__ __forceinline__ TileRef tile_at(const int32_t* __restrict__ seg, const int32_t* __restrict__ ranks,
                                           const int64_t* __restrict__ offs, int num_adapters, RankWindow rw, int lin,
                                           bool flat, int total, int nsub, int& sub) {
  const XcdItem it = work_item(lin, total, nsub, flat);
  sub = it.sub;
  if (it.tile < 0) return TileRef{0, 0, 0, 0, 0};
  return find_tile<TM, BAL>(seg, ranks, offs, num_adapters, rw, it.tile);
}

}  // namespace gs
