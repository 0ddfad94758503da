// Switched-LoRA shrink (x . A_g^T) and expand (y += z . B_g^T) for gfx950.
//
// Both kernels walk adapter-sorted segments (gs_build_segments): a workgroup
// owns a tile of up to 32 consecutive slots of ONE adapter, so every MFMA is a
// dense product with one adapter's weights -- no per-row adapter masks and no
// repeated passes over the adapters present in a tile.
#include "gs_common.h"

namespace gs {

constexpr int kTM = 32;            // slots (tokens) per tile
constexpr int kThreads = 256;      // 4 waves

__host__ __device__ inline int max_tiles_for(int64_t T, int NA) {
  return static_cast<int>((T + kTM - 1) / kTM + (NA < T ? NA : T));
}

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

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }

// 4 pieces of 16 bytes starting at element k of a row, zero where piece start >= kend.
template <bool BF16>
__device__ __forceinline__ void load_row4(const void* row, int64_t k, int64_t kend, bool valid, u32x4 out[4]) {
  constexpr int P = Elt<BF16>::kPerPiece;
  const char* base = static_cast<const char*>(row);
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int64_t kp = k + p * P;
    if (valid && kp < kend) out[p] = ld16(base + kp * Elt<BF16>::kSize);
    else out[p] = u32x4{0u, 0u, 0u, 0u};
  }
}

// acc += (lane's 4 pieces of x) x (lane's 4 pieces of A) over one batch.
template <bool BF16>
__device__ __forceinline__ f32x16 mfma_batch(const u32x4 xa[4], const u32x4 wb[4], f32x16 acc) {
  if constexpr (BF16) {
#pragma unroll
    for (int t = 0; t < 4; ++t) acc = mfma32_bf16(xa[t], wb[t], acc);
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float* a = reinterpret_cast<const float*>(&xa[t]);
      const float* b = reinterpret_cast<const float*>(&wb[t]);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = mfma32_f32(a[e], b[e], acc);
    }
  }
  return acc;
}

// ----------------------------------------------------------------------------
// Shrink.  Grid (max_tiles, n_chunks, KS).  A workgroup computes the partial
// product of one tile (32 slots) x 128 output columns (4 n-blocks of 32) over
// the k-chunk [ks*KC, ks*KC+KC); its 4 waves split that chunk in 4 and are
// reduced through LDS in a fixed order.  With KS > 1 the partial tile goes to
// the workspace; the last workgroup of the tile (a self-resetting counter
// decides) sums the KS partials in ks order and writes z, so the result does
// not depend on scheduling.
// ----------------------------------------------------------------------------
constexpr int kShrinkNB = 4;
constexpr int kShrinkCols = 32 * kShrinkNB;            // 128
constexpr int kTileFloats = kTM * kShrinkCols;         // 4096
constexpr int kOutPad = 4;

struct ShrinkParams {
  const void* x;
  int64_t ldx;
  int H;
  const void* a_pack;
  const int64_t* a_off;
  const int32_t* ranks;
  int S;
  int NA;
  const int32_t* seg;
  const int32_t* perm;
  void* z;
  int64_t ldz;
  float* part;
  int* counters;
  int KS;
  int KC;
  int n_chunks;
};

template <bool BF16>
__device__ __forceinline__ void store_z16(void* z, int64_t ldz, int slot, int col, int ncols, const float* v) {
  // 16 consecutive columns of one z row; ncols is a multiple of 8.
  if constexpr (BF16) {
    uint16_t* zr = static_cast<uint16_t*>(z) + static_cast<int64_t>(slot) * ldz + col;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      if (col + half * 8 < ncols) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[e] = static_cast<uint32_t>(f32_to_bf16_bits(v[half * 8 + 2 * e])) |
                 (static_cast<uint32_t>(f32_to_bf16_bits(v[half * 8 + 2 * e + 1])) << 16);
        st16(zr + half * 8, u32x4{w[0], w[1], w[2], w[3]});
      }
    }
  } else {
    float* zr = static_cast<float*>(z) + static_cast<int64_t>(slot) * ldz + col;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (col + q * 4 < ncols) *reinterpret_cast<f32x4*>(zr + q * 4) = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
    }
  }
}

template <bool BF16>
__global__ __launch_bounds__(kThreads) void shrink_kernel(ShrinkParams p) {
  __shared__ float red[2][kShrinkNB][16][64];           // 32 KB: cross-wave reduction
  __shared__ int s_last;
  float(*tile_s)[kShrinkCols + kOutPad] = reinterpret_cast<float(*)[kShrinkCols + kOutPad]>(&red[0][0][0][0]);

  const TileRef tr = find_tile<kTM>(p.seg, p.ranks, p.NA, blockIdx.x);
  if (tr.g == 0) return;
  const int r = p.ranks[tr.g];
  const int ncols = p.S * r;
  const int col0 = blockIdx.y * kShrinkCols;
  if (col0 >= ncols) return;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int i = l & 31;
  const int h = l >> 5;

  const int64_t k_lo = static_cast<int64_t>(blockIdx.z) * p.KC;
  const int64_t k_hi = min(static_cast<int64_t>(p.H), k_lo + p.KC);
  const int wk = p.KC / 4;
  const int64_t wk_lo = k_lo + static_cast<int64_t>(wave) * wk;
  const int64_t wk_hi = min(k_hi, wk_lo + wk);

  const bool row_ok = i < tr.nrows;
  const int token = row_ok ? p.perm[tr.slot0 + i] : 0;
  const char* xrow = static_cast<const char*>(p.x) + (static_cast<int64_t>(token) * p.ldx) * Elt<BF16>::kSize;
  const char* arow[kShrinkNB];
  bool n_ok[kShrinkNB];
  const int64_t a_base = p.a_off[tr.g];
#pragma unroll
  for (int nb = 0; nb < kShrinkNB; ++nb) {
    const int n = col0 + 32 * nb + i;
    n_ok[nb] = n < ncols;
    arow[nb] = static_cast<const char*>(p.a_pack) + (a_base + static_cast<int64_t>(n_ok[nb] ? n : 0) * p.H) * Elt<BF16>::kSize;
  }
  int nblk = (ncols - col0 + 31) / 32;
  if (nblk > kShrinkNB) nblk = kShrinkNB;

  f32x16 acc[kShrinkNB];
#pragma unroll
  for (int nb = 0; nb < kShrinkNB; ++nb) acc[nb] = f32x16{};

  constexpr int B = Elt<BF16>::kBatch;
  for (int64_t kb = wk_lo; kb < wk_hi; kb += B) {
    const int64_t kk = kb + h * (B / 2);
    u32x4 xv[4];
    load_row4<BF16>(xrow, kk, wk_hi, row_ok, xv);
#pragma unroll
    for (int nb = 0; nb < kShrinkNB; ++nb) {
      if (nb < nblk) {
        u32x4 av[4];
        load_row4<BF16>(arow[nb], kk, wk_hi, n_ok[nb], av);
        acc[nb] = mfma_batch<BF16>(xv, av, acc[nb]);
      }
    }
  }

  // Fixed-order cross-wave reduction: (w0 + w2) + (w1 + w3).
  if (wave >= 2) {
#pragma unroll
    for (int nb = 0; nb < kShrinkNB; ++nb)
#pragma unroll
      for (int v = 0; v < 16; ++v) red[wave - 2][nb][v][l] = acc[nb][v];
  }
  __syncthreads();
  if (wave < 2) {
#pragma unroll
    for (int nb = 0; nb < kShrinkNB; ++nb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[nb][v] += red[wave][nb][v][l];
  }
  __syncthreads();
  if (wave == 1) {
#pragma unroll
    for (int nb = 0; nb < kShrinkNB; ++nb)
#pragma unroll
      for (int v = 0; v < 16; ++v) red[0][nb][v][l] = acc[nb][v];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int nb = 0; nb < kShrinkNB; ++nb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[nb][v] += red[0][nb][v][l];
  }
  __syncthreads();
  // wave 0 scatters the MFMA layout into a row-major [32][128] tile
  if (wave == 0) {
#pragma unroll
    for (int nb = 0; nb < kShrinkNB; ++nb)
#pragma unroll
      for (int v = 0; v < 16; ++v) tile_s[mfma32_row(v, l)][32 * nb + i] = acc[nb][v];
  }
  __syncthreads();

  // each thread owns 16 consecutive columns of one row
  const int row = tid >> 3;
  const int cx = (tid & 7) * 16;
  float vals[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) vals[e] = tile_s[row][cx + e];

  if (p.KS == 1) {
    if (row < tr.nrows) store_z16<BF16>(p.z, p.ldz, tr.slot0 + row, col0 + cx, ncols, vals);
    return;
  }

  const int64_t pair = static_cast<int64_t>(blockIdx.x) * p.n_chunks + blockIdx.y;
  float* part_base = p.part + pair * p.KS * kTileFloats;
  {
    f32x4* dst = reinterpret_cast<f32x4*>(part_base + static_cast<int64_t>(blockIdx.z) * kTileFloats + tid * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = f32x4{vals[4 * q], vals[4 * q + 1], vals[4 * q + 2], vals[4 * q + 3]};
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const int prev = atomicAdd(&p.counters[pair], 1);
    s_last = (prev == p.KS - 1) ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  float sum[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) sum[e] = 0.f;
  for (int ks = 0; ks < p.KS; ++ks) {
    const f32x4* src = reinterpret_cast<const f32x4*>(part_base + static_cast<int64_t>(ks) * kTileFloats + tid * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 v = __builtin_nontemporal_load(src + q);
      sum[4 * q] += v.x;
      sum[4 * q + 1] += v.y;
      sum[4 * q + 2] += v.z;
      sum[4 * q + 3] += v.w;
    }
  }
  if (row < tr.nrows) store_z16<BF16>(p.z, p.ldz, tr.slot0 + row, col0 + cx, ncols, sum);
  if (tid == 0) atomicExch(&p.counters[pair], 0);
}

// ----------------------------------------------------------------------------
// Expand.  Grid (n_tiles, max_tiles).  A workgroup owns one tile (32 slots of
// one adapter) x NT output columns; each wave computes NBW 32x32 blocks of the
// delta with MFMA over the adapter's rank, the blocks go through LDS to a
// row-major tile, and every thread read-modify-writes 16 consecutive y columns
// of one token row (loaded before the MFMA work to hide the latency).  Only the
// tile's token rows are touched.
// ----------------------------------------------------------------------------
struct SliceInfo {
  int S;
  int bounds[GS_MAX_SLICES + 1];
};

struct ExpandParams {
  void* y;
  int64_t ldy;
  int out_total;
  SliceInfo si;
  const void* z;
  int64_t ldz;
  int z_by_token;
  const int32_t* z_off;
  const void* b_pack;
  const int64_t* b_off;
  const int32_t* ranks;
  int NA;
  const int32_t* seg;
  const int32_t* perm;
};

template <bool BF16>
__device__ __forceinline__ void load_y16(const void* y, int64_t off, u32x4 out[4]) {
  const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const char*>(y) + off * Elt<BF16>::kSize);
  if constexpr (BF16) {
    out[0] = __builtin_nontemporal_load(p);
    out[1] = __builtin_nontemporal_load(p + 1);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) out[q] = __builtin_nontemporal_load(p + q);
  }
}

template <bool BF16>
__device__ __forceinline__ void add_store_y16(void* y, int64_t off, const u32x4 in[4], const float* d) {
  u32x4* p = reinterpret_cast<u32x4*>(static_cast<char*>(y) + off * Elt<BF16>::kSize);
  if constexpr (BF16) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const uint32_t* w = reinterpret_cast<const uint32_t*>(&in[half]);
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = bf16_bits_to_f32(static_cast<uint16_t>(w[e] & 0xffffu)) + d[half * 8 + 2 * e];
        const float hi = bf16_bits_to_f32(static_cast<uint16_t>(w[e] >> 16)) + d[half * 8 + 2 * e + 1];
        o[e] = static_cast<uint32_t>(f32_to_bf16_bits(lo)) | (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
      }
      __builtin_nontemporal_store(u32x4{o[0], o[1], o[2], o[3]}, p + half);
    }
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float* f = reinterpret_cast<const float*>(&in[q]);
      const f32x4 o = f32x4{f[0] + d[4 * q], f[1] + d[4 * q + 1], f[2] + d[4 * q + 2], f[3] + d[4 * q + 3]};
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o), p + q);
    }
  }
}

template <bool BF16, int NBW>
__global__ __launch_bounds__(kThreads) void expand_kernel(ExpandParams p) {
  constexpr int NT = 4 * NBW * 32;           // columns per workgroup
  constexpr int TPR = NT / 16;               // threads per row in the RMW
  constexpr int RPP = kThreads / TPR;        // rows per RMW pass
  constexpr int PASSES = kTM / RPP;
  __shared__ float dtile[kTM][NT + kOutPad];

  const TileRef tr = find_tile<kTM>(p.seg, p.ranks, p.NA, blockIdx.y);
  if (tr.g == 0) return;
  const int r = p.ranks[tr.g];
  const int n_tile0 = blockIdx.x * NT;
  if (n_tile0 >= p.out_total) return;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int i = l & 31;
  const int h = l >> 5;

  // 1. issue the y loads of this thread's RMW rows
  u32x4 yv[PASSES][4];
  int64_t yoff[PASSES];
  bool yok[PASSES];
  const int cx = (tid % TPR) * 16;
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int row = ps * RPP + tid / TPR;
    yok[ps] = row < tr.nrows && (n_tile0 + cx) < p.out_total;
    const int tok = yok[ps] ? p.perm[tr.slot0 + row] : 0;
    yoff[ps] = static_cast<int64_t>(tok) * p.ldy + n_tile0 + cx;
    if (yok[ps]) load_y16<BF16>(p.y, yoff[ps], yv[ps]);
  }

  // 2. delta blocks with MFMA
  const bool row_ok = i < tr.nrows;
  const int slot = tr.slot0 + (row_ok ? i : 0);
  const int64_t zrow = p.z_by_token ? static_cast<int64_t>(p.perm[slot]) : static_cast<int64_t>(slot);
  const int zo = (p.z_off != nullptr) ? p.z_off[tr.g] : 0;
  const int64_t b_base = p.b_off[tr.g];
#pragma unroll
  for (int q = 0; q < NBW; ++q) {
    const int nbl = wave * NBW + q;
    const int n0 = n_tile0 + 32 * nbl;
    f32x16 acc = f32x16{};
    if (n0 < p.out_total) {
      int s = 0;
      while (s + 1 < p.si.S && n0 >= p.si.bounds[s + 1]) ++s;
      const int n = n0 + i;
      const char* zr = static_cast<const char*>(p.z) + (zrow * p.ldz + zo + s * r) * Elt<BF16>::kSize;
      const char* br = static_cast<const char*>(p.b_pack) + (b_base + static_cast<int64_t>(n) * r) * Elt<BF16>::kSize;
      // The k loops are uniform across the wave (MFMA is a whole-wave
      // instruction); a lane half whose k range passed r feeds zeros.
      if constexpr (BF16) {
        for (int kb = 0; kb < r; kb += 16) {
          const int k0 = kb + 8 * h;
          const bool kin = k0 < r;
          const u32x4 za = (row_ok && kin) ? ld16(zr + k0 * 2) : u32x4{0u, 0u, 0u, 0u};
          const u32x4 bb = kin ? ld16(br + k0 * 2) : u32x4{0u, 0u, 0u, 0u};
          acc = mfma32_bf16(za, bb, acc);
        }
      } else {
        for (int kb = 0; kb < r; kb += 8) {
          const int k0 = kb + 4 * h;
          const bool kin = k0 < r;
          f32x4 za = f32x4{0.f, 0.f, 0.f, 0.f}, bb = f32x4{0.f, 0.f, 0.f, 0.f};
          if (kin) {
            if (row_ok) za = *reinterpret_cast<const f32x4*>(zr + k0 * 4);
            bb = *reinterpret_cast<const f32x4*>(br + k0 * 4);
          }
          acc = mfma32_f32(za.x, bb.x, acc);
          acc = mfma32_f32(za.y, bb.y, acc);
          acc = mfma32_f32(za.z, bb.z, acc);
          acc = mfma32_f32(za.w, bb.w, acc);
        }
      }
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) dtile[mfma32_row(v, l)][32 * nbl + i] = acc[v];
  }
  __syncthreads();

  // 3. read-modify-write y
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    if (!yok[ps]) continue;
    const int row = ps * RPP + tid / TPR;
    float d[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) d[e] = dtile[row][cx + e];
    add_store_y16<BF16>(p.y, yoff[ps], yv[ps], d);
  }
}

// ----------------------------------------------------------------------------
// Host-side planning (shared by the workspace query and the launch).
// ----------------------------------------------------------------------------
struct ShrinkPlan {
  int max_tiles, n_chunks, KS, KC;
  int64_t counter_bytes, part_bytes;
};

static ShrinkPlan plan_shrink(int64_t T, int H, int S, int NA, int max_rank, bool bf16) {
  ShrinkPlan pl{};
  pl.max_tiles = max_tiles_for(T, NA);
  pl.n_chunks = (S * max_rank + kShrinkCols - 1) / kShrinkCols;
  const int unit = 4 * (bf16 ? Elt<true>::kBatch : Elt<false>::kBatch);   // k per workgroup step
  const int units = (H + unit - 1) / unit;
  const int64_t wgs = static_cast<int64_t>(pl.max_tiles) * pl.n_chunks;
  int ks = static_cast<int>((1024 + wgs - 1) / (wgs > 0 ? wgs : 1));
  if (ks < 1) ks = 1;
  if (ks > units) ks = units;
  const int per = (units + ks - 1) / ks;
  pl.KC = per * unit;
  pl.KS = (H + pl.KC - 1) / pl.KC;
  if (pl.KS < 1) pl.KS = 1;
  pl.counter_bytes = ((static_cast<int64_t>(pl.max_tiles) * pl.n_chunks * 4 + 255) / 256) * 256;
  pl.part_bytes = pl.KS > 1 ? static_cast<int64_t>(pl.max_tiles) * pl.n_chunks * pl.KS * kTileFloats * 4 : 0;
  return pl;
}

}  // namespace gs

using namespace gs;

extern "C" {

int64_t gs_shrink_workspace_bytes(int64_t num_tokens, int32_t hidden, int32_t num_slices, int32_t num_adapters,
                                  int32_t max_rank) {
  if (num_tokens <= 0 || hidden <= 0) return 256;
  const ShrinkPlan pl = plan_shrink(num_tokens, hidden, num_slices, num_adapters, max_rank, true);
  const ShrinkPlan pf = plan_shrink(num_tokens, hidden, num_slices, num_adapters, max_rank, false);
  const int64_t a = pl.counter_bytes + pl.part_bytes, b = pf.counter_bytes + pf.part_bytes;
  return a > b ? a : b;
}

int64_t gs_shrink_counter_bytes(int64_t num_tokens, int32_t num_slices, int32_t num_adapters, int32_t max_rank) {
  if (num_tokens <= 0) return 256;
  const ShrinkPlan pl = plan_shrink(num_tokens, 256, num_slices, num_adapters, max_rank, true);
  return pl.counter_bytes;
}

static int check_common(const char* who, int32_t dtype, int64_t T, int32_t num_slices, int32_t num_adapters,
                        int32_t max_rank) {
  GS_CHECK_ARG(dtype == GS_DTYPE_BF16 || dtype == GS_DTYPE_FP32, "%s: dtype=%d", who, dtype);
  GS_CHECK_ARG(T >= 0 && T < (int64_t(1) << 31), "%s: num_tokens out of range", who);
  GS_CHECK_ARG(num_slices >= 1 && num_slices <= GS_MAX_SLICES, "%s: num_slices=%d", who, num_slices);
  GS_CHECK_ARG(num_adapters >= 1 && num_adapters <= GS_MAX_ADAPTERS, "%s: num_adapters=%d", who, num_adapters);
  GS_CHECK_ARG(max_rank >= 8 && max_rank <= GS_MAX_RANK && max_rank % 8 == 0,
               "%s: max_rank=%d must be a multiple of 8 in [8,%d]", who, max_rank, GS_MAX_RANK);
  return GS_OK;
}

int gs_shrink(int32_t dtype, const void* x, int64_t ldx, int64_t num_tokens, int32_t hidden, const void* a_pack,
              const int64_t* a_off, const int32_t* ranks, int32_t num_slices, int32_t num_adapters,
              int32_t max_rank, const int32_t* seg_offsets, const int32_t* perm, void* z, int64_t ldz,
              void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_common("gs_shrink", dtype, num_tokens, num_slices, num_adapters, max_rank);
  if (rc != GS_OK) return rc;
  const bool bf16 = dtype == GS_DTYPE_BF16;
  const int vec = bf16 ? 8 : 4;
  GS_CHECK_ARG(hidden > 0 && hidden % 8 == 0, "gs_shrink: hidden=%d must be a positive multiple of 8", hidden);
  GS_CHECK_ARG(ldx >= hidden && ldx % vec == 0, "gs_shrink: ldx=%lld", (long long)ldx);
  GS_CHECK_ARG(ldz >= int64_t(num_slices) * max_rank && ldz % vec == 0, "gs_shrink: ldz=%lld", (long long)ldz);
  GS_CHECK_ARG(aligned16(x) && aligned16(a_pack) && aligned16(z), "gs_shrink: x, a_pack and z must be 16-byte aligned");
  if (num_tokens == 0) return GS_OK;
  const ShrinkPlan pl = plan_shrink(num_tokens, hidden, num_slices, num_adapters, max_rank, bf16);
  GS_CHECK_ARG(pl.max_tiles <= 65535 * 64, "gs_shrink: too many tiles");
  if (pl.KS > 1) {
    if (workspace == nullptr || workspace_bytes < pl.counter_bytes + pl.part_bytes || !aligned16(workspace)) {
      set_error("gs_shrink: workspace of %lld bytes needed (got %lld)", (long long)(pl.counter_bytes + pl.part_bytes),
                (long long)workspace_bytes);
      return GS_ERR_WORKSPACE;
    }
  }
  ShrinkParams p{};
  p.x = x;
  p.ldx = ldx;
  p.H = hidden;
  p.a_pack = a_pack;
  p.a_off = a_off;
  p.ranks = ranks;
  p.S = num_slices;
  p.NA = num_adapters;
  p.seg = seg_offsets;
  p.perm = perm;
  p.z = z;
  p.ldz = ldz;
  p.counters = static_cast<int*>(workspace);
  p.part = pl.KS > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + pl.counter_bytes) : nullptr;
  p.KS = pl.KS;
  p.KC = pl.KC;
  p.n_chunks = pl.n_chunks;
  dim3 grid(pl.max_tiles, pl.n_chunks, pl.KS);
  if (bf16) hipLaunchKernelGGL(shrink_kernel<true>, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream), p);
  else hipLaunchKernelGGL(shrink_kernel<false>, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream), p);
  GS_CHECK_LAUNCH("gs_shrink");
  return GS_OK;
}

int gs_expand_add(int32_t dtype, void* y, int64_t ldy, int64_t num_tokens, int32_t out_total,
                  const int32_t* slice_bounds, int32_t num_slices, const void* z, int64_t ldz, int32_t z_by_token,
                  const int32_t* z_off, const void* b_pack, const int64_t* b_off, const int32_t* ranks,
                  int32_t num_adapters, int32_t max_rank, const int32_t* seg_offsets, const int32_t* perm,
                  void* stream) {
  int rc = check_common("gs_expand_add", dtype, num_tokens, num_slices, num_adapters, max_rank);
  if (rc != GS_OK) return rc;
  const bool bf16 = dtype == GS_DTYPE_BF16;
  const int vec = bf16 ? 8 : 4;
  GS_CHECK_ARG(out_total > 0 && out_total % 32 == 0, "gs_expand_add: out_total=%d must be a multiple of 32", out_total);
  GS_CHECK_ARG(slice_bounds != nullptr, "gs_expand_add: slice_bounds is NULL");
  GS_CHECK_ARG(slice_bounds[0] == 0 && slice_bounds[num_slices] == out_total, "gs_expand_add: slice_bounds must span [0,out_total]");
  for (int s = 0; s < num_slices; ++s)
    GS_CHECK_ARG(slice_bounds[s + 1] > slice_bounds[s] && (slice_bounds[s + 1] - slice_bounds[s]) % 32 == 0,
                 "gs_expand_add: slice %d width must be a positive multiple of 32", s);
  GS_CHECK_ARG(ldy >= out_total && ldy % vec == 0, "gs_expand_add: ldy=%lld", (long long)ldy);
  GS_CHECK_ARG(ldz % vec == 0, "gs_expand_add: ldz=%lld", (long long)ldz);
  GS_CHECK_ARG(aligned16(y) && aligned16(z) && aligned16(b_pack), "gs_expand_add: y, z and b_pack must be 16-byte aligned");
  if (num_tokens == 0) return GS_OK;
  ExpandParams p{};
  p.y = y;
  p.ldy = ldy;
  p.out_total = out_total;
  p.si.S = num_slices;
  for (int s = 0; s <= num_slices; ++s) p.si.bounds[s] = slice_bounds[s];
  p.z = z;
  p.ldz = ldz;
  p.z_by_token = z_by_token;
  p.z_off = z_off;
  p.b_pack = b_pack;
  p.b_off = b_off;
  p.ranks = ranks;
  p.NA = num_adapters;
  p.seg = seg_offsets;
  p.perm = perm;
  const int max_tiles = max_tiles_for(num_tokens, num_adapters);
  GS_CHECK_ARG(max_tiles <= 65535, "gs_expand_add: num_tokens too large for one launch");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool wide = num_tokens >= 2048;
  const int NT = wide ? 256 : 128;
  dim3 grid((out_total + NT - 1) / NT, max_tiles);
  if (bf16) {
    if (wide) hipLaunchKernelGGL((expand_kernel<true, 2>), grid, dim3(kThreads), 0, st, p);
    else hipLaunchKernelGGL((expand_kernel<true, 1>), grid, dim3(kThreads), 0, st, p);
  } else {
    if (wide) hipLaunchKernelGGL((expand_kernel<false, 2>), grid, dim3(kThreads), 0, st, p);
    else hipLaunchKernelGGL((expand_kernel<false, 1>), grid, dim3(kThreads), 0, st, p);
  }
  GS_CHECK_LAUNCH("gs_expand_add");
  return GS_OK;
}

int gs_switched_lora(int32_t dtype, const void* x, int64_t ldx, void* y, int64_t ldy, int64_t num_tokens,
                     int32_t hidden, int32_t out_total, const int32_t* slice_bounds, int32_t num_slices,
                     const void* a_pack, const int64_t* a_off, const void* b_pack, const int64_t* b_off,
                     const int32_t* ranks, int32_t num_adapters, int32_t max_rank, const int32_t* seg_offsets,
                     const int32_t* perm, void* z, void* workspace, int64_t workspace_bytes, void* stream) {
  const int64_t ldz = static_cast<int64_t>(num_slices) * max_rank;
  int rc = gs_shrink(dtype, x, ldx, num_tokens, hidden, a_pack, a_off, ranks, num_slices, num_adapters, max_rank,
                     seg_offsets, perm, z, ldz, workspace, workspace_bytes, stream);
  if (rc != GS_OK) return rc;
  return gs_expand_add(dtype, y, ldy, num_tokens, out_total, slice_bounds, num_slices, z, ldz, 0, nullptr, b_pack,
                       b_off, ranks, num_adapters, max_rank, seg_offsets, perm, stream);
}

}  // extern "C"
