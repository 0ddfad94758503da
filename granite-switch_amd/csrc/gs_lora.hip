// Switched-LoRA shrink (x . A_g^T) and expand (y += z . B_g^T) for gfx950.
//
// Both kernels walk adapter-sorted segments (gs_build_segments): a workgroup
// owns a tile of up to 32 consecutive slots of ONE adapter, so every MFMA is a
// dense product with one adapter's weights -- no per-row adapter masks and no
// repeated passes over the adapters present in a tile.
//
// No workgroup ever waits for or reads data produced by another workgroup of
// the same launch.  When the shrink splits the hidden dimension over several
// workgroups (split-K, needed to spread a decode-sized A over all CUs) it
// writes fp32 partial sums; the consumer -- the expand kernel, or a small
// reduce kernel when z itself is asked for -- adds the partials in a fixed
// order, so results are deterministic and need no cross-XCD fences.
#include <stdarg.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <vector>

#include "gs_addr.h"
#include "gs_common.h"

namespace gs {

constexpr int kTM = 32;            // slots (tokens) per tile
constexpr int kThreads = 256;      // 4 waves

__host__ __device__ inline int max_tiles_for(int64_t T, int NA) {
  return static_cast<int>((T + kTM - 1) / kTM + (NA < T ? NA : T));
}

// Loads below are issued unconditionally from clamped, in-bounds addresses and
// masked afterwards with a select: with no branches around memory
// instructions the compiler can count the loads in flight, so a prefetch
// really overlaps the work on the previous batch instead of being drained by
// a conservative wait.

// ----------------------------------------------------------------------------
// Shrink.  1-D grid over (tile, column chunk, k-chunk) items, tiles spread
// over the XCDs in contiguous ranges (xcd_item).  A workgroup computes one
// tile of kTMS = 64 slots of one adapter x COLS = 32*NB output columns over
// the k-chunk [ks*KC, ks*KC + KC).  Each wave owns 16 of the slots and the
// whole column range, so no cross-wave reduction is needed.  The chunk is
// streamed in batches of BK k: the workgroup stages the batch's lora_A tile
// (COLS rows, 512 contiguous bytes per row) in LDS once, each wave keeps its
// 16 x rows in registers (64 contiguous bytes per row and load), and 16x16
// MFMAs (x rows x lora_A rows) accumulate.  The next batch's loads are issued
// before the current batch is computed.  KS == 1 writes z in the element
// type; KS > 1 writes the fp32 partial of chunk ks to part[ks][slot][col].
// ----------------------------------------------------------------------------
constexpr int kTMS = 64;           // slots per shrink tile
#ifndef GS_SHRINK_TARGET_WGS
#define GS_SHRINK_TARGET_WGS 640
#endif
constexpr int kShrinkTargetWgs = GS_SHRINK_TARGET_WGS;   // workgroups the k-split aims for
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
  void* z;                // KS == 1
  int64_t ldz;
  float* part;            // KS > 1: [KS][T][zw]
  int64_t part_stride;    // T * zw
  int zw;
  int KS;
  int KC;
  int n_chunks;
  RankWindow rw;          // adapters of this launch's rank class
  int flat;               // flat item layout (work_item) instead of tile ranges per XCD
  int ks_target;          // > 0: the k-split is chosen on the device (dyn_ksplit), KS is its maximum
};

// The k-split of a launch whose workgroups loop (a large-rank class): chosen
// on the device from the batch's real tile count, as the host chooses it from
// an estimate -- about `target` items, 1..KS_max -- so that a class holding
// fewer tokens than expected still spreads over the GPU.  The expand of the
// class computes the same value from the same count.
__host__ __device__ __forceinline__ int dyn_ksplit(int tiles, int n_chunks, int target, int ks_max) {
  const int w = tiles * n_chunks;
  int ks = w > 0 ? (target + w / 2) / w : ks_max;
  return ks < 1 ? 1 : (ks > ks_max ? ks_max : ks);
}

// 16x16 MFMA over one 16-byte piece of each operand (K = 32 bf16, or four
// K = 4 fp32 steps).  Lane l supplies row l % 16 of each operand and elements
// of lane group l / 16; both operands pair elements the same way, so any
// fixed assignment of k to pieces is a correct contraction.  Result: lane l
// holds D[4*(l/16) + e][l % 16].
template <bool BF16>
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, f32x4 acc) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc,
                                                   0, 0, 0);
  } else {
    const f32x4 x = __builtin_bit_cast(f32x4, a);
    const f32x4 w = __builtin_bit_cast(f32x4, b);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.x, w.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.y, w.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.z, w.z, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x4f32(x.w, w.w, acc, 0, 0, 0);
  }
}

// NB <= 2 fits 3 workgroups per CU (<= 168 registers, no spills), so a grid
// of ~640 runs in one round on 256 CUs; wider tiles would spill.
template <bool BF16, int NB>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(NB <= 2 ? 3 : 1))) void shrink_kernel(
    ShrinkParams p) {
  constexpr int P = Elt<BF16>::kPerPiece;        // elements per 16-byte piece
  constexpr int ES = Elt<BF16>::kSize;
  constexpr int KSTEP = 4 * P;                   // k of one piece over the 4 lane groups
  constexpr int NPB = 8;                         // pieces per batch and lane
  constexpr int BK = NPB * KSTEP;                // k per batch (256 bf16, 128 fp32)
  constexpr int COLS = 32 * NB;
  constexpr int NC16 = COLS / 16;
  constexpr int ROWB = BK * ES;                  // bytes of one lora_A row per batch
  constexpr int ALD = ROWB + 16;                 // LDS row stride (padded against bank conflicts)
  constexpr int PPR = ROWB / 16;                 // 16-byte pieces per row and batch
  constexpr int APT = COLS * PPR / kThreads;     // lora_A pieces per thread and batch
  static_assert(COLS * PPR % kThreads == 0, "lora_A pieces must split evenly over the workgroup");
  __shared__ __align__(16) char a_s[COLS * ALD];

  int sub = 0, total = 0;
  const TileRef tr = locate_tile<kTMS>(p.seg, p.ranks, p.a_off, p.NA, p.rw, static_cast<int>(blockIdx.x), p.flat != 0,
                                       p.n_chunks * p.KS, sub, total);
  if (tr.g == 0) return;
  const int chunk = sub % p.n_chunks;
  const int ks = sub / p.n_chunks;
  const int ncols = p.S * tr.rank;
  const int col0 = chunk * COLS;
  if (col0 >= ncols) return;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int i16 = l & 15;
  const int q4 = l >> 4;
  const int64_t k_lo = static_cast<int64_t>(ks) * p.KC;
  const int64_t k_hi = min(static_cast<int64_t>(p.H), k_lo + p.KC);
  const int nbat = static_cast<int>((k_hi - k_lo + BK - 1) / BK);

  // this lane's x row (slots past the tile re-read the tile's first token)
  const int srow = 16 * wave + i16;
  const bool row_ok = srow < tr.nrows;
  const int token = p.perm[tr.slot0 + addr::tile_row(srow, tr.nrows)];
  // this thread's lora_A pieces: flat piece f = tid + 256*j of the COLS x PPR
  // batch tile is row tid/PPR + j*(256/PPR), piece tid % PPR of the row, so
  // PPR consecutive threads read one row's 512 contiguous bytes
  constexpr int RSTEP = kThreads / PPR;          // rows between a thread's pieces
  const int ar0 = tid / PPR;
  const int apc = tid % PPR;
  const char* abase = static_cast<const char*>(p.a_pack) + (tr.off + static_cast<int64_t>(col0 + ar0) * p.H) * ES;
  const int64_t astep = static_cast<int64_t>(RSTEP) * p.H * ES;
  const int arows = ncols - col0 - ar0;          // this thread's pieces j with j*RSTEP < arows are real rows

  // Straight-line loads from clamped in-bounds addresses, masked afterwards,
  // so the compiler counts the loads in flight exactly.
  auto load_a = [&](int b, u32x4 (&av)[APT]) {
    const int64_t kp = k_lo + static_cast<int64_t>(b) * BK + apc * P;
#pragma unroll
    for (int j = 0; j < APT; ++j) {
      const bool ok = j * RSTEP < arows && kp < k_hi;
      av[j] = sel16(ok, ld16(abase + addr::reg_a_elem(ok, j, astep / ES, kp, k_lo) * ES));
    }
  };
  // lora_A of the first batch goes out before the wait for the token index
  u32x4 xc[NPB], xn[NPB], an[APT];
  load_a(0, an);
  const char* xrow = static_cast<const char*>(p.x) + static_cast<int64_t>(token) * p.ldx * ES;
  auto load_x = [&](int b, u32x4 (&xv)[NPB]) {
    const int64_t kb = k_lo + static_cast<int64_t>(b) * BK;
#pragma unroll
    for (int pp = 0; pp < NPB; ++pp) {
      const int64_t kp = kb + pp * KSTEP + q4 * P;
      const bool ok = row_ok && kp < k_hi;
      xv[pp] = sel16(ok, ld16(xrow + addr::reg_x_elem(ok, kp, k_lo) * ES));
    }
  };
  auto stage_a = [&](const u32x4 (&av)[APT]) {
#pragma unroll
    for (int j = 0; j < APT; ++j) st16(a_s + (ar0 + j * RSTEP) * ALD + apc * 16, av[j]);
  };

  f32x4 acc[NC16];
#pragma unroll
  for (int c = 0; c < NC16; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  load_x(0, xc);
  stage_a(an);
  lds_barrier();
  for (int b = 0; b < nbat; ++b) {
    load_x(b + 1, xn);                 // past the chunk every piece is masked
    load_a(b + 1, an);
#pragma unroll
    for (int pp = 0; pp < NPB; ++pp) {
#pragma unroll
      for (int c = 0; c < NC16; ++c) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(a_s + (16 * c + i16) * ALD + (pp * KSTEP + q4 * P) * ES);
        acc[c] = mfma16<BF16>(xc[pp], a, acc[c]);
      }
    }
    lds_barrier();                     // every wave is done with this batch's tile
    stage_a(an);
    lds_barrier();
#pragma unroll
    for (int pp = 0; pp < NPB; ++pp) xc[pp] = xn[pp];
  }

  // lane (i16, q4) holds slots 16*wave + 4*q4 + e, column col0 + 16*c + i16
#pragma unroll
  for (int c = 0; c < NC16; ++c) {
    const int col = col0 + 16 * c + i16;
    if (col >= ncols) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 16 * wave + 4 * q4 + e;
      if (row >= tr.nrows) continue;
      const int64_t slot = tr.slot0 + row;
      if (p.KS == 1) {
        if constexpr (BF16) static_cast<uint16_t*>(p.z)[slot * p.ldz + col] = f32_to_bf16_bits(acc[c][e]);
        else static_cast<float*>(p.z)[slot * p.ldz + col] = acc[c][e];
      } else {
        p.part[static_cast<int64_t>(ks) * p.part_stride + slot * p.zw + col] = acc[c][e];
      }
    }
  }
}

// ----------------------------------------------------------------------------
// Shrink, bf16 with H % 64 == 0: the same work items, tile placement,
// k-split and outputs as shrink_kernel, but the operands travel through a
// ring of LDS stages filled by direct global -> LDS transfers, so several
// stages are in flight per workgroup without staging registers.  A stage is
// 64 k of the tile's 64 x rows and its COLS lora_A rows, one 128-byte line per
// row (whole-line requests); a wave moves 16 x rows and COLS/4 lora_A rows of
// every stage (1 KB per transfer: 8 rows, lane l row l/8 position l%8).
// Pieces are XOR-swizzled (piece p of row r at position p ^ addr::lds_swz(r))
// so the 16 rows an MFMA operand read touches fall in distinct banks.  NST stages
// form a ring with NST - 1 in flight: iteration s waits for its own stage
// (vmcnt), passes one barrier -- after which every wave is done with stage
// s - 1, whose slot then receives stage s + NST - 1 -- and runs its MFMAs
// from LDS.  The waiting in the old kernel was one memory round trip per
// batch: the next batch's lora_A had to be in registers before it could be
// staged.  Rows past the tile (x) or past the adapter's S*r (lora_A) re-read
// a valid row; their results are never stored.
// ----------------------------------------------------------------------------
constexpr int kDmaBK = 64;                 // k per stage
constexpr int kDmaRow = kDmaBK * 2;        // bytes of a bf16 row per stage (one cache line)


// ring depth per column width: about 72 KB of LDS, two workgroups per CU
#ifndef GS_DMA_NST1
#define GS_DMA_NST1 6
#endif
#ifndef GS_DMA_NST2
#define GS_DMA_NST2 4
#endif
#ifndef GS_DMA_NST3
#define GS_DMA_NST3 3
#endif
#ifndef GS_DMA_NST4
#define GS_DMA_NST4 3
#endif
template <int NB>
struct DmaRing {
  static constexpr int NST = NB == 1 ? GS_DMA_NST1 : (NB == 2 ? GS_DMA_NST2 : (NB == 3 ? GS_DMA_NST3 : GS_DMA_NST4));
};

// s_waitcnt until at most `after` stages (TPW transfers each) are outstanding
template <int TPW, int N>
__device__ __forceinline__ void wait_stages(int after) {
  if constexpr (N >= 0) {
    if (after >= N) {
      __builtin_amdgcn_s_waitcnt(wait_vm(N * TPW));
      return;
    }
    wait_stages<TPW, N - 1>(after);
  }
}

// One work item of shrink_dma_kernel: tile tr, sub = (k-chunk, column chunk).
template <int NB>
__device__ __forceinline__ void shrink_dma_item(const ShrinkParams& p, const TileRef& tr, int sub, int KS,
                                                char* ring) {
  constexpr int COLS = 32 * NB;
  constexpr int NC16 = COLS / 16;
  constexpr int ROWS = kTMS + COLS;        // LDS rows of a stage: x rows, then lora_A rows
  constexpr int STAGE = ROWS * kDmaRow;
  constexpr int NST = DmaRing<NB>::NST;
  constexpr int XT = kTMS / 4 / 8;         // x transfers per wave and stage
  constexpr int ARW = COLS / 4;            // lora_A rows per wave and stage
  constexpr int AT = ARW / 8;              // lora_A transfers per wave and stage
  constexpr int TPW = XT + AT;
  static_assert(TPW * (NST - 2) <= 63, "vmcnt counts at most 63 outstanding transfers");

  const int chunk = sub % p.n_chunks;
  const int ks = sub / p.n_chunks;
  const int ncols = p.S * tr.rank;
  const int col0 = chunk * COLS;
  if (col0 >= ncols) return;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int i16 = l & 15;
  const int q4 = l >> 4;
  // k-chunk ks: stages [ks * all / KS, (ks + 1) * all / KS) of the all = H / 64
  // stages, so the chunks differ by at most one stage
  int s_lo = 0, nst = 0;
  addr::dma_kchunk(p.H, ks, KS, s_lo, nst);
  const int64_t k_lo = static_cast<int64_t>(s_lo) * kDmaBK;

  // this lane's source in each transfer: row 8t + l/8 of the wave's rows, the
  // global piece that LDS position l % 8 of its LDS row holds swizzled
  const int trow = addr::dma_trow(l);
  const char* xsrc[XT];
#pragma unroll
  for (int t = 0; t < XT; ++t) {
    const int xrow = addr::dma_x_row(wave, t, trow);    // also its LDS row
    const int token = p.perm[tr.slot0 + addr::tile_row(xrow, tr.nrows)];
    xsrc[t] = static_cast<const char*>(p.x) + (static_cast<int64_t>(token) * p.ldx + k_lo) * 2 +
              addr::dma_gpiece_bytes(l, xrow);
  }
  const char* asrc[AT];
#pragma unroll
  for (int t = 0; t < AT; ++t) {
    const int arow = addr::dma_a_row(col0, ARW, wave, t, trow, ncols);
    asrc[t] = static_cast<const char*>(p.a_pack) + (tr.off + static_cast<int64_t>(arow) * p.H + k_lo) * 2 +
              addr::dma_gpiece_bytes(l, kTMS + ARW * wave + 8 * t + trow);
  }
  auto issue = [&](int st) {
    char* slot = ring + (st % NST) * STAGE;
    const int64_t off = static_cast<int64_t>(st) * kDmaRow;
#pragma unroll
    for (int t = 0; t < XT; ++t)   // x is read once per launch: streamed, so lora_A stays in L2
      dma16_nt(xsrc[t] + off, slot + (16 * wave + 8 * t) * kDmaRow);
#pragma unroll
    for (int t = 0; t < AT; ++t) dma16(asrc[t] + off, slot + (kTMS + ARW * wave + 8 * t) * kDmaRow);
  };

  f32x4 acc[NC16];
#pragma unroll
  for (int c = 0; c < NC16; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int sw = addr::lds_swz(i16);      // swizzle of every row this lane reads (blocks start at multiples of 16)
  for (int st = 0; st < NST - 1 && st < nst; ++st) issue(st);
  for (int st = 0; st < nst; ++st) {
    wait_stages<TPW, NST - 2>(min(NST - 2, nst - 1 - st));
    mem_fence_compiler();
    __builtin_amdgcn_s_barrier();
    mem_fence_compiler();
    if (st + NST - 1 < nst) issue(st + NST - 1);
    const char* slot = ring + (st % NST) * STAGE;
    const char* xs = slot + (16 * wave + i16) * kDmaRow;
    const char* as = slot + (kTMS + i16) * kDmaRow;
#pragma unroll
    for (int kk = 0; kk < kDmaBK / 32; ++kk) {
      const int pos = ((4 * kk + q4) ^ sw) * 16;
      const u32x4 xa = *reinterpret_cast<const u32x4*>(xs + pos);
#pragma unroll
      for (int c = 0; c < NC16; ++c)
        acc[c] = mfma16<true>(xa, *reinterpret_cast<const u32x4*>(as + 16 * c * kDmaRow + pos), acc[c]);
    }
  }

  // Results go through LDS (the ring is free once every wave is past its last
  // stage) so that each thread stores whole 16-byte pieces of output rows:
  // lane (i16, q4) holds slots 16*wave + 4*q4 + e, column 16*c + i16.
  constexpr int OLD = COLS + 4;            // fp32 row stride of the staged results
  static_assert(kTMS * OLD * 4 <= NST * STAGE, "staged results must fit the ring");
  float* res = reinterpret_cast<float*>(ring);
  lds_barrier();
#pragma unroll
  for (int c = 0; c < NC16; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) res[(16 * wave + 4 * q4 + e) * OLD + 16 * c + i16] = acc[c][e];
  lds_barrier();
  constexpr int PPR4 = COLS / 4;           // 4-column pieces per row
  const int wcols = min(COLS, ncols - col0);
#pragma unroll
  for (int it = 0; it < kTMS * PPR4 / kThreads; ++it) {
    const int pc = tid + it * kThreads;
    const int row = addr::dma_res_row(pc, PPR4);
    const int c4 = addr::dma_res_col(pc, PPR4);
    if (row >= tr.nrows || c4 >= wcols) continue;
    const f32x4 v = *reinterpret_cast<const f32x4*>(res + row * OLD + c4);
    const int64_t slot = tr.slot0 + row;
    if (KS == 1) {
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.z) + slot * p.ldz + col0 + c4) =
          make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
    } else {
      *reinterpret_cast<f32x4*>(p.part + static_cast<int64_t>(ks) * p.part_stride + slot * p.zw + col0 + c4) = v;
    }
  }
}

// LOOP = false: one item per workgroup (the launch is sized for every tile
// the batch can have).  LOOP = true (a rank class expected to hold far fewer
// tiles than it could, whose grid the host caps): a workgroup takes items
// blockIdx.x, + gridDim.x, ... while they lie in the batch's item range.  The
// loop is a separate instantiation: its live state would cost the one-item
// form registers.
template <int NB, bool LOOP>
__global__ __launch_bounds__(kThreads) void shrink_dma_kernel(ShrinkParams p) {
  __shared__ __align__(16) char ring[DmaRing<NB>::NST * (kTMS + 32 * NB) * kDmaRow];
  const bool flat = LOOP && p.flat != 0;       // the one-item form is never flat
  int lin = static_cast<int>(blockIdx.x);
  int sub = 0, total = 0;
  if constexpr (!LOOP) {
    const TileRef tr =
        locate_tile<kTMS>(p.seg, p.ranks, p.a_off, p.NA, p.rw, lin, false, p.n_chunks * p.KS, sub, total);
    if (tr.g != 0) shrink_dma_item<NB>(p, tr, sub, p.KS, ring);
    return;
  }
  int KS = p.KS;
  TileRef tr = locate_tile_by<kTMS>(p.seg, p.ranks, p.a_off, p.NA, p.rw, lin, flat,
                                    [&](int tot) {
                                      if (p.ks_target > 0) KS = dyn_ksplit(tot, p.n_chunks, p.ks_target, p.KS);
                                      return p.n_chunks * KS;
                                    }, sub, total);
  const int nsub = p.n_chunks * KS;
  const int items = work_items(total, nsub, flat);
  for (;;) {
    if (tr.g != 0) shrink_dma_item<NB>(p, tr, sub, KS, ring);
    lin += static_cast<int>(gridDim.x);
    if (lin >= items) break;
    lds_barrier();                         // every wave is done with the ring before the next item's transfers
    tr = tile_at<kTMS>(p.seg, p.ranks, p.a_off, p.NA, p.rw, lin, flat, total, nsub, sub);
  }
}

// z[slot][col] = sum_ks part[ks][slot][col] (fixed order), for the active
// slots of the adapters in the launch's rank window (the other classes' slots
// are written by their own launches).
template <bool BF16>
__global__ __launch_bounds__(kThreads) void reduce_parts_kernel(const float* __restrict__ part, int64_t part_stride,
                                                               int KS, int zw, const int32_t* __restrict__ seg,
                                                               const int32_t* __restrict__ ranks, RankWindow rw,
                                                               int NA, void* z, int64_t ldz) {
  const int64_t e8 = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * 8;   // 8 elements
  const int64_t slot = e8 / zw;
  const int col = static_cast<int>(e8 % zw);
  if (slot >= seg[NA]) return;
  // the slot's adapter: the smallest g with seg[g] > slot
  int glo = 1, ghi = NA;
  while (glo < ghi) {
    const int mid = (glo + ghi) >> 1;
    if (seg[mid] > slot) ghi = mid;
    else glo = mid + 1;
  }
  if (!in_window(rw, ranks[glo])) return;
  // all partial loads in flight at once (KS <= 16), summed in ks order
  f32x4 a[16], b[16];
#pragma unroll
  for (int ks = 0; ks < 16; ++ks) {
    if (ks < KS) {
      const f32x4* src = reinterpret_cast<const f32x4*>(part + ks * part_stride + slot * zw + col);
      a[ks] = src[0];
      b[ks] = src[1];
    }
  }
  float s[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) s[e] = 0.f;
#pragma unroll
  for (int ks = 0; ks < 16; ++ks) {
    if (ks < KS) {
      s[0] += a[ks].x; s[1] += a[ks].y; s[2] += a[ks].z; s[3] += a[ks].w;
      s[4] += b[ks].x; s[5] += b[ks].y; s[6] += b[ks].z; s[7] += b[ks].w;
    }
  }
  if constexpr (BF16) {
    uint16_t* zr = static_cast<uint16_t*>(z) + slot * ldz + col;
    st16(zr, u32x4{pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3]), pack_bf16x2(s[4], s[5]), pack_bf16x2(s[6], s[7])});
  } else {
    float* zr = static_cast<float*>(z) + slot * ldz + col;
    *reinterpret_cast<f32x4*>(zr) = f32x4{s[0], s[1], s[2], s[3]};
    *reinterpret_cast<f32x4*>(zr + 4) = f32x4{s[4], s[5], s[6], s[7]};
  }
}

// ----------------------------------------------------------------------------
// Expand.  1-D grid over (tile, group of column sub-tiles) items, tiles
// spread over the XCDs in contiguous ranges (xcd_item).  A workgroup owns one
// tile (32 slots of one adapter) and walks its group's consecutive column
// sub-tiles of NT columns.  The number of groups per tile is chosen on the
// device from the batch's tile count so that the items about fill the GPU
// once (wt workgroups): each workgroup's start -- the tile lookup and the
// staging of its shrink values -- is paid once per group, and a group long
// enough to hide it beats a second round of workgroups.  The tile's shrink values for every slice (z rows, or the sum of
// the split-K partials rounded to the element type exactly like a
// materialised z) are staged in LDS once.  Per sub-tile each wave computes NBW
// 32x32 delta blocks with MFMA over the adapter's rank (all KSTEP k-groups of
// B held in registers, PRE of them), the blocks go through LDS to a row-major
// tile, and every thread read-modify-writes 16 consecutive y columns of one
// token row.  The next sub-tile's B and y loads are issued before the current
// one is computed.  Only the tile's token rows are written.
// ----------------------------------------------------------------------------
struct ExpandParams {
  void* y;
  int64_t ldy;
  int out_total;
  SliceInfo si;
  const void* z;          // nparts == 0
  int64_t ldz;
  int z_by_token;
  const int32_t* z_off;
  const float* part;      // nparts > 0: [nparts][T][zw] fp32
  int64_t part_stride;
  int zw;
  int nparts;
  const void* b_pack;
  const int64_t* b_off;
  const int32_t* ranks;
  int NA;
  int max_rank;
  int wt;                 // workgroups that fill the GPU once
  const int32_t* seg;
  const int32_t* perm;
  RankWindow rw;          // adapters of this launch's rank class
  int flat;               // flat item layout, one sub-tile per item (work_item)
  int ks_target;          // > 0: the shrink chose its k-split on the device (dyn_ksplit over
  int ks_chunks;          //   its 64-slot tiles, ks_chunks column chunks, at most nparts)
};

// Shrink values of the tile for slices s_lo..s_hi (the ones the workgroup's
// output columns lie in), 4 elements per item: item it covers row
// it / (width/4) and columns c4 .. c4+3 of the row's S*r values (slice c4 / r).
// Split-K partials are loaded kPartGroup at a time and summed in ks order;
// values are rounded to the element type when stored to LDS, exactly as a
// materialised z would have been.
constexpr int kPartGroup = 8;

template <bool BF16>
__device__ __forceinline__ void z_stage(const ExpandParams& p, const TileRef& tr, int r, int zo, char* zs, int zs_ld,
                                        int s_lo, int s_hi, int nparts) {
  const int per_row = ((s_hi - s_lo + 1) * r) >> 2;
  const int items = kTM * per_row;
  for (int it = threadIdx.x; it < items; it += kThreads) {
    const int row = addr::stage_row(it, per_row);
    const int c4 = addr::stage_col(it, row, per_row, s_lo * r);
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (row < tr.nrows) {
      const int slot = tr.slot0 + row;
      if (nparts > 0) {
        const float* src = p.part + static_cast<int64_t>(slot) * p.zw + c4;
        for (int ks0 = 0; ks0 < nparts; ks0 += kPartGroup) {
          f32x4 a[kPartGroup];
#pragma unroll
          for (int u = 0; u < kPartGroup; ++u)
            if (ks0 + u < nparts) a[u] = *reinterpret_cast<const f32x4*>(src + (ks0 + u) * p.part_stride);
#pragma unroll
          for (int u = 0; u < kPartGroup; ++u) {
            if (ks0 + u < nparts) {
              v[0] += a[u].x;
              v[1] += a[u].y;
              v[2] += a[u].z;
              v[3] += a[u].w;
            }
          }
        }
      } else {
        const int64_t zrow = p.z_by_token ? static_cast<int64_t>(p.perm[slot]) : static_cast<int64_t>(slot);
        const char* zr = static_cast<const char*>(p.z) + (zrow * p.ldz + zo + c4) * Elt<BF16>::kSize;
        if constexpr (BF16) {
          const uint2 w = *reinterpret_cast<const uint2*>(zr);
          v[0] = bf16_bits_to_f32(static_cast<uint16_t>(w.x & 0xffffu));
          v[1] = bf16_bits_to_f32(static_cast<uint16_t>(w.x >> 16));
          v[2] = bf16_bits_to_f32(static_cast<uint16_t>(w.y & 0xffffu));
          v[3] = bf16_bits_to_f32(static_cast<uint16_t>(w.y >> 16));
        } else {
          const f32x4 a = *reinterpret_cast<const f32x4*>(zr);
          v[0] = a.x;
          v[1] = a.y;
          v[2] = a.z;
          v[3] = a.w;
        }
      }
    }
    char* dst = zs + (static_cast<int64_t>(row) * zs_ld + c4) * Elt<BF16>::kSize;
    if constexpr (BF16) {
      *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    } else {
      *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
    }
  }
}

// Column groups per tile: as many as keep 8*ceil(tiles/8) * groups within wt
// (the launch holds max(wt, 8*ceil(max_tiles/8)) workgroups), 1..n_sub.
__host__ __device__ inline int expand_groups(int tiles, int n_sub, int wt) {
  const int t8 = 8 * ((tiles + 7) / 8);
  int g = t8 > 0 ? wt / t8 : n_sub;
  if (g > n_sub) g = n_sub;
  if (g < 1) g = 1;
  return g;
}

// An adapter's slots are cut into 32-slot tiles of near-equal size (the
// short last tile of a plain cut left the CUs holding one with less work
// than the rest, and the launch waited for the others).
#ifndef GS_EXPAND_BALANCED
#define GS_EXPAND_BALANCED 1
#endif
constexpr bool kExpandBalanced = GS_EXPAND_BALANCED;

// One work item of expand_kernel: tile tr, sub-tiles [sub0, sub0 + nsub).
// PIPE: ranks above PRE k-groups load lora_B chunk kc + 1 before chunk kc is
// multiplied (the looping form for large ranks); otherwise each later chunk
// is loaded where it is used, which keeps the one-item forms' registers.
// before_last() runs before the last sub-tile's products (the pair expand
// issues its claim there).
struct NoHook {
  __device__ void operator()() const {}
};
template <bool BF16, int NBW, int PRE, bool PIPE, typename Hook = NoHook>
__device__ __forceinline__ void expand_item(const ExpandParams& p, const TileRef& tr, int sub0, int nsub,
                                            int nparts, float (&dtile)[kTM][4 * NBW * 32 + kOutPad], char* zs,
                                            Hook before_last = Hook{}) {
  constexpr int NT = 4 * NBW * 32;           // columns per sub-tile
  // read-modify-write mapping: each lane owns one 16-byte piece per row it
  // touches, consecutive lanes consecutive pieces, so every wave access
  // covers whole row segments
  constexpr int EPL = 16 / Elt<BF16>::kSize;  // elements per 16-byte piece
  constexpr int LPR = NT / EPL;               // lanes per row
  constexpr int RPI = kThreads / LPR;         // rows per workgroup-wide access
  constexpr int PASSES = kTM / RPI;           // rows per thread
  constexpr int KSTEP = BF16 ? 16 : 8;       // k per MFMA group (both lane halves)
  constexpr int KHALF = KSTEP / 2;
  // y rows with the streaming policy in the 256-column form: the lora_B
  // blocks and partials that the workgroups share stay in L2 (decoder step
  // 7 000 -> 6 544 us).  The 128-column form (ranks above 32) measured
  // slower with it (multiswitch down expand 16.3 -> 18.8 us).
  constexpr bool YNT = NBW == 2;

  const int r = tr.rank;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int i = l & 31;
  const int h = l >> 5;
  const int zs_ld = p.si.S * p.max_rank + 8;
  const int zo = (p.z_off != nullptr) ? p.z_off[tr.g] : 0;
  const int cx = (tid % LPR) * EPL;
  const int nchunk = (r + PRE * KSTEP - 1) / (PRE * KSTEP);   // 1 unless the rank exceeds PRE k-groups

  // token rows of this thread's read-modify-write (rows past the tile re-read
  // the tile's first token; their stores are masked)
  int64_t yrow[PASSES];
  bool rok[PASSES];
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int row = ps * RPI + tid / LPR;
    rok[ps] = row < tr.nrows;
    yrow[ps] = static_cast<int64_t>(p.perm[tr.slot0 + addr::tile_row(row, tr.nrows)]) * p.ldy;
  }

  auto load_y = [&](int sub, u32x4 (&yv)[PASSES]) {
    const int64_t col = addr::y_col(sub, NT, cx, p.out_total, EPL);
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      const char* src = static_cast<const char*>(p.y) + (yrow[ps] + col) * Elt<BF16>::kSize;
      yv[ps] = YNT ? ld16_nt(src) : ld16(src);
    }
  };
  // B k-groups [kc*PRE, kc*PRE + PRE) of this wave's n-blocks in sub-tile sub
  auto load_b = [&](int sub, int kc, u32x4 (&bp)[NBW][PRE]) {
#pragma unroll
    for (int q = 0; q < NBW; ++q) {
      const int n = addr::b_col(sub * NT + 32 * (wave * NBW + q) + i, p.out_total);
      const char* br = static_cast<const char*>(p.b_pack) + (tr.off + static_cast<int64_t>(n) * r) * Elt<BF16>::kSize;
#pragma unroll
      for (int st = 0; st < PRE; ++st) {
        const int k0 = (kc * PRE + st) * KSTEP + KHALF * h;
        bp[q][st] = sel16(k0 < r, ld16(br + addr::k_or_zero(k0, r) * Elt<BF16>::kSize));
      }
    }
  };

  u32x4 yc[PASSES], bc[NBW][PRE];
  load_b(sub0, 0, bc);
  load_y(sub0, yc);
  // the slices of the group's first and last output column
  int s_lo = 0, s_hi = 0;
  {
    const int c_first = sub0 * NT;
    const int c_last = min((sub0 + nsub) * NT, p.out_total) - 1;
    while (s_lo + 1 < p.si.S && c_first >= p.si.bounds[s_lo + 1]) ++s_lo;
    s_hi = s_lo;
    while (s_hi + 1 < p.si.S && c_last >= p.si.bounds[s_hi + 1]) ++s_hi;
  }
  z_stage<BF16>(p, tr, r, zo, zs, zs_ld, s_lo, s_hi, nparts);
  lds_barrier();

  auto compute = [&](int sub, u32x4 (&bcur)[NBW][PRE], u32x4 (&ycur)[PASSES]) {
    const int n_tile0 = sub * NT;
    f32x16 acc[NBW];
#pragma unroll
    for (int q = 0; q < NBW; ++q) {
      const int n0 = n_tile0 + 32 * (wave * NBW + q);
      int s = 0;
      while (s + 1 < p.si.S && n0 >= p.si.bounds[s + 1]) ++s;
      const char* zrow_s = zs + (static_cast<int64_t>(i) * zs_ld + s * r) * Elt<BF16>::kSize;
      acc[q] = f32x16{};
      // k-groups [kc*PRE, kc*PRE + PRE) of the rank against the staged shrink values
      auto mma = [&](int kc, const u32x4 (&bx)[PRE]) {
#pragma unroll
        for (int st = 0; st < PRE; ++st) {
          const int k0 = (kc * PRE + st) * KSTEP + KHALF * h;
          const bool kin = k0 < r;
          const u32x4 za = sel16(kin, *reinterpret_cast<const u32x4*>(zrow_s + (kin ? k0 : 0) * Elt<BF16>::kSize));
          if constexpr (BF16) {
            acc[q] = mfma32_bf16(za, bx[st], acc[q]);
          } else {
            const f32x4 zf = __builtin_bit_cast(f32x4, za);
            const f32x4 bf = __builtin_bit_cast(f32x4, bx[st]);
            acc[q] = mfma32_f32(zf.x, bf.x, acc[q]);
            acc[q] = mfma32_f32(zf.y, bf.y, acc[q]);
            acc[q] = mfma32_f32(zf.z, bf.z, acc[q]);
            acc[q] = mfma32_f32(zf.w, bf.w, acc[q]);
          }
        }
      };
      if constexpr (!PIPE) {
        for (int kc = 0; kc < nchunk; ++kc) {
          u32x4 bx[PRE];
          if (kc == 0) {
#pragma unroll
            for (int st = 0; st < PRE; ++st) bx[st] = bcur[q][st];
          } else {
            // ranks above PRE k-groups: the later groups are loaded here
            const int n = addr::b_col(n0 + i, p.out_total);
            const char* br =
                static_cast<const char*>(p.b_pack) + (tr.off + static_cast<int64_t>(n) * r) * Elt<BF16>::kSize;
#pragma unroll
            for (int st = 0; st < PRE; ++st) {
              const int k0 = (kc * PRE + st) * KSTEP + KHALF * h;
              bx[st] = sel16(k0 < r, ld16(br + addr::k_or_zero(k0, r) * Elt<BF16>::kSize));
            }
          }
#pragma unroll
          for (int st = 0; st < PRE; ++st) {
            const int k0 = (kc * PRE + st) * KSTEP + KHALF * h;
            const bool kin = k0 < r;
            const u32x4 za = sel16(kin, *reinterpret_cast<const u32x4*>(zrow_s + (kin ? k0 : 0) * Elt<BF16>::kSize));
            if constexpr (BF16) {
              acc[q] = mfma32_bf16(za, bx[st], acc[q]);
            } else {
              const f32x4 zf = __builtin_bit_cast(f32x4, za);
              const f32x4 bf = __builtin_bit_cast(f32x4, bx[st]);
              acc[q] = mfma32_f32(zf.x, bf.x, acc[q]);
              acc[q] = mfma32_f32(zf.y, bf.y, acc[q]);
              acc[q] = mfma32_f32(zf.z, bf.z, acc[q]);
              acc[q] = mfma32_f32(zf.w, bf.w, acc[q]);
            }
          }
        }
      } else if (nchunk == 1) {
        mma(0, bcur[q]);
      } else {
        // ranks above PRE k-groups: chunk kc + 1 of lora_B is loaded before
        // chunk kc is multiplied, so two chunks are in flight (the last
        // iteration re-reads its own chunk: no branch around the loads)
        const int n = addr::b_col(n0 + i, p.out_total);
        const char* br = static_cast<const char*>(p.b_pack) + (tr.off + static_cast<int64_t>(n) * r) * Elt<BF16>::kSize;
        u32x4 bx[PRE];
#pragma unroll
        for (int st = 0; st < PRE; ++st) bx[st] = bcur[q][st];
        for (int kc = 0; kc < nchunk; ++kc) {
          const int kn = min(kc + 1, nchunk - 1);
          u32x4 bnx[PRE];
#pragma unroll
          for (int st = 0; st < PRE; ++st) {
            const int k0 = (kn * PRE + st) * KSTEP + KHALF * h;
            bnx[st] = sel16(k0 < r, ld16(br + addr::k_or_zero(k0, r) * Elt<BF16>::kSize));
          }
          mma(kc, bx);
#pragma unroll
          for (int st = 0; st < PRE; ++st) bx[st] = bnx[st];
        }
      }
    }
#pragma unroll
    for (int q = 0; q < NBW; ++q)
#pragma unroll
      for (int v = 0; v < 16; ++v) dtile[mfma32_row(v, l)][32 * (wave * NBW + q) + i] = acc[q][v];
    lds_barrier();
    const int64_t col = static_cast<int64_t>(n_tile0) + cx;
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      const int row = ps * RPI + tid / LPR;
      float d[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) d[e] = dtile[row][cx + e];
      if (rok[ps] && col < p.out_total) add_store_y<BF16, YNT>(p.y, yrow[ps] + col, ycur[ps], d);
    }
    lds_barrier();                          // dtile is rewritten by the next sub-tile
  };

  for (int it = 0; it + 1 < nsub; ++it) {
    u32x4 yn[PASSES], bn[NBW][PRE];
    load_b(sub0 + it + 1, 0, bn);
    load_y(sub0 + it + 1, yn);
    compute(sub0 + it, bc, yc);
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) yc[ps] = yn[ps];
#pragma unroll
    for (int q = 0; q < NBW; ++q)
#pragma unroll
      for (int st = 0; st < PRE; ++st) bc[q][st] = bn[q][st];
  }
  before_last();
  compute(sub0 + nsub - 1, bc, yc);
}

// LOOP = false: one item per workgroup (the grid covers the items).  LOOP =
// true (a rank class expected to hold few tiles, laid out flat with one
// sub-tile per item, grid capped at one round): a workgroup takes items
// blockIdx.x, + gridDim.x, ... while they lie in the batch's item range.  A
// separate instantiation, so the one-item form keeps its registers.
// The narrow bf16 forms up to rank 64 hold 4 workgroups per CU (<= 128
// registers per lane; the rank-64 multiswitch projection measured faster at
// 4 than at 3).
template <bool BF16, int NBW, int PRE, bool LOOP>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(BF16 && NBW == 1 && PRE <= 4 && !LOOP ? 4 : 1)))
void expand_kernel(ExpandParams p) {
  constexpr int NT = 4 * NBW * 32;
  __shared__ float dtile[kTM][NT + kOutPad];
  extern __shared__ __align__(16) char zs[];   // [32][S*max_rank + 8] element type
  const int n_sub = (p.out_total + NT - 1) / NT;
  const bool flat = LOOP;                      // the looping form is the flat one
  int lin = static_cast<int>(blockIdx.x);
  int sub = 0, groups = 1, total = 0;
  TileRef tr = locate_tile_by<kTM, kExpandBalanced>(p.seg, p.ranks, p.b_off, p.NA, p.rw, lin, flat,
                                                    [&](int tot) {
                                                      groups = flat ? n_sub : expand_groups(tot, n_sub, p.wt);
                                                      return groups;
                                                    }, sub, total);
  if constexpr (!LOOP) {
    if (tr.g == 0) return;
    // group sub of `groups` covers sub-tiles [sub*n_sub/groups, (sub+1)*n_sub/groups)
    const int sub0 = (sub * n_sub) / groups;
    const int nsub = ((sub + 1) * n_sub) / groups - sub0;
    if (nsub > 0) expand_item<BF16, NBW, PRE, false>(p, tr, sub0, nsub, p.nparts, dtile, zs);
    return;
  }
  // the shrink's k-split when it chose it on the device: the same function of
  // the same 64-slot tile count
  int nparts = p.nparts;
  if (p.ks_target > 0) {
    const int ks = dyn_ksplit(count_tiles<kTMS>(p.seg, p.ranks, p.NA, p.rw), p.ks_chunks, p.ks_target, p.nparts);
    nparts = ks > 1 ? ks : 0;
  }
  const int items = work_items(total, groups, flat);
  for (;;) {
    if (tr.g != 0) {
      const int sub0 = (sub * n_sub) / groups;
      const int nsub = ((sub + 1) * n_sub) / groups - sub0;
      if (nsub > 0) expand_item<BF16, NBW, PRE, true>(p, tr, sub0, nsub, nparts, dtile, zs);
    }
    lin += static_cast<int>(gridDim.x);
    if (lin >= items) break;
    lds_barrier();                         // every wave is done with zs and dtile before the next item
    tr = tile_at<kTM, kExpandBalanced>(p.seg, p.ranks, p.b_off, p.NA, p.rw, lin, flat, total, groups, sub);
  }
}

// ----------------------------------------------------------------------------
// Expand of a sparse large-rank class (bf16; a few tiles of an adapter of rank
// 72..512, e.g. one rank-512 adapter among rank-32 ones at decode).  One item
// is (tile, 128-column sub-tile), laid out flat over a looping grid of one
// round.  The 4 waves split the RANK instead of the columns: wave w takes
// k-groups [w*KG, (w+1)*KG) of all 128 columns, so the item's whole lora_B
// block (128 x r) is in flight in one memory trip (the column-split kernel
// streams a large rank in dependent chunks).  The waves' partial deltas are
// summed through LDS in a fixed order, (w0 + w2) + (w1 + w3), then every
// thread read-modify-writes 16-byte pieces of its token rows.  Sub-tiles lie
// inside one slice (slice widths are multiples of 128), so only that slice's
// shrink values are staged.
// ----------------------------------------------------------------------------
constexpr int kSpNT = 128;                   // columns per item of expand_sparse_kernel

// One item of the rank-split expand: tile tr, sub-tile `sub` of 32 * QB
// columns (inside one slice).  red: the waves' partial deltas.  Each output
// element is the same sum in the same order whatever QB: wave w's k-groups
// [w*KG, (w+1)*KG) in order, then (w0 + w2) + (w1 + w3).
template <int KG, int QB>
__device__ __forceinline__ void expand_sparse_item(const ExpandParams& p, const TileRef& tr, int sub, int nparts,
                                                   float (&red)[2][kTM][32 * QB + kOutPad], char* zs) {
  constexpr int NTC = 32 * QB;               // columns per item
  constexpr int KSTEP = 16;                  // bf16 k per MFMA group (both lane halves)
  constexpr int KHALF = 8;
  constexpr int EPL = 8;                     // bf16 elements per 16-byte piece
  constexpr int LPR = NTC / EPL;             // lanes per row
  constexpr int RPI = kThreads / LPR;        // rows per workgroup-wide access
  constexpr int PASSES = kTM / RPI;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int i = l & 31;
  const int h = l >> 5;
  const int zs_ld = p.max_rank + 8;
  const int cx = (tid % LPR) * EPL;
    const int r = tr.rank;
    const int n_tile0 = sub * NTC;
    int s = 0;
    while (s + 1 < p.si.S && n_tile0 >= p.si.bounds[s + 1]) ++s;
    // the token rows of the item's y pieces (rows past the tile re-read its
    // first token) and, when z is read by token, of its z pieces: the only
    // loads the others wait for, so they go first
    const int zo = (p.z_off != nullptr) ? p.z_off[tr.g] : 0;
    const int per_row = r >> 2;
    constexpr int ZIT = kTM * (4 * KG * KSTEP) / 4 / kThreads;   // z pieces per thread at the largest rank
    int64_t yrow[PASSES];
    bool rok[PASSES];
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      const int row = ps * RPI + tid / LPR;
      rok[ps] = row < tr.nrows;
      yrow[ps] = static_cast<int64_t>(p.perm[tr.slot0 + addr::tile_row(row, tr.nrows)]) * p.ldy;
    }
    int32_t zrow[ZIT];                     // slot, or token, indices (widened where they address z)
#pragma unroll
    for (int j = 0; j < ZIT; ++j)
      zrow[j] = tr.slot0 + addr::tile_row(addr::stage_row(tid + j * kThreads, per_row), tr.nrows);
    if (nparts == 0 && p.z_by_token) {   // uniform
#pragma unroll
      for (int j = 0; j < ZIT; ++j) zrow[j] = p.perm[zrow[j]];
    }
    __builtin_amdgcn_sched_barrier(0);
    // then, all in flight together: the slice's z pieces of the tile's rows
    // (when z is given; the oldest, so staging them waits for nothing
    // else; pieces past the rank read clamped addresses and are not
    // stored), this wave's k-groups of lora_B for the 4 column blocks
    // (pieces past the rank read the row's first piece and are masked) and
    // the y pieces
    uint2 w[ZIT];
    if (nparts == 0) {
      const uint16_t* zp = static_cast<const uint16_t*>(p.z) + zo + s * r;
#pragma unroll
      for (int j = 0; j < ZIT; ++j) {
        const int it = tid + j * kThreads;
        const int c4 = it < kTM * per_row ? addr::stage_col(it, addr::stage_row(it, per_row), per_row, 0) : 0;
        w[j] = *reinterpret_cast<const uint2*>(zp + static_cast<int64_t>(zrow[j]) * p.ldz + c4);
      }
    }
    u32x4 bv[QB][KG];
#pragma unroll
    for (int q = 0; q < QB; ++q) {
      const int n = n_tile0 + 32 * q + i;
      const char* br = static_cast<const char*>(p.b_pack) + (tr.off + static_cast<int64_t>(n) * r) * 2;
#pragma unroll
      for (int kg = 0; kg < KG; ++kg) {
        const int k0 = (wave * KG + kg) * KSTEP + KHALF * h;
        bv[q][kg] = sel16(k0 < r, ld16(br + addr::k_or_zero(k0, r) * 2));
      }
    }
    u32x4 yv[PASSES];
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) yv[ps] = ld16(static_cast<const char*>(p.y) + (yrow[ps] + n_tile0 + cx) * 2);
    // the slice's shrink values of the tile's rows in LDS: the z pieces
    // loaded above, or split-K partials summed in ks order (kPartGroup at a
    // time) and rounded to bf16 as a stored z would be
    if (nparts == 0) {
#pragma unroll
      for (int j = 0; j < ZIT; ++j) {
        const int it = tid + j * kThreads;
        const int row = addr::stage_row(it, per_row);
        if (it < kTM * per_row) {
          const int c4 = addr::stage_col(it, row, per_row, 0);
          *reinterpret_cast<uint2*>(zs + (static_cast<int64_t>(row) * zs_ld + c4) * 2) =
              row < tr.nrows ? w[j] : make_uint2(0u, 0u);
        }
      }
    }
    // partials: the tile's real rows only (the products of the rows past
    // them are never stored), UNR passes' pieces in flight per trip (two
    // for 128-column items at rank > 256, where the kernel holds one wave
    // per SIMD anyway; one otherwise, which keeps the registers of the
    // narrower items that share a launch with the small class)
    constexpr int UNR = KG >= 8 && QB == 4 ? 2 : 1;
    const int npieces = nparts == 0 ? 0 : tr.nrows * per_row;
    for (int it0 = tid; it0 < npieces; it0 += UNR * kThreads) {
      float v[UNR][4];
      const float* src[UNR];
#pragma unroll
      for (int w2 = 0; w2 < UNR; ++w2) {
        const int it = it0 + w2 * kThreads < npieces ? it0 + w2 * kThreads : it0;
        const int row = addr::stage_row(it, per_row);
        src[w2] = p.part + static_cast<int64_t>(tr.slot0 + row) * p.zw + s * r +
                  addr::stage_col(it, row, per_row, 0);
        v[w2][0] = v[w2][1] = v[w2][2] = v[w2][3] = 0.f;
      }
      for (int ks0 = 0; ks0 < nparts; ks0 += kPartGroup) {
        f32x4 a[UNR][kPartGroup];
#pragma unroll
        for (int w2 = 0; w2 < UNR; ++w2)
#pragma unroll
          for (int u = 0; u < kPartGroup; ++u)
            if (ks0 + u < nparts) a[w2][u] = *reinterpret_cast<const f32x4*>(src[w2] + (ks0 + u) * p.part_stride);
#pragma unroll
        for (int w2 = 0; w2 < UNR; ++w2)
#pragma unroll
          for (int u = 0; u < kPartGroup; ++u) {
            if (ks0 + u < nparts) {
              v[w2][0] += a[w2][u].x;
              v[w2][1] += a[w2][u].y;
              v[w2][2] += a[w2][u].z;
              v[w2][3] += a[w2][u].w;
            }
          }
      }
#pragma unroll
      for (int w2 = 0; w2 < UNR; ++w2) {
        const int it = it0 + w2 * kThreads;
        if (it < npieces) {
          const int row = addr::stage_row(it, per_row);
          const int c4 = addr::stage_col(it, row, per_row, 0);
          *reinterpret_cast<uint2*>(zs + (static_cast<int64_t>(row) * zs_ld + c4) * 2) =
              make_uint2(pack_bf16x2(v[w2][0], v[w2][1]), pack_bf16x2(v[w2][2], v[w2][3]));
        }
      }
    }
    lds_barrier();
    f32x16 acc[QB];
#pragma unroll
    for (int q = 0; q < QB; ++q) acc[q] = f32x16{};
    const char* zrow_l = zs + static_cast<int64_t>(i) * zs_ld * 2;
#pragma unroll
    for (int kg = 0; kg < KG; ++kg) {
      const int k0 = (wave * KG + kg) * KSTEP + KHALF * h;
      const bool kin = k0 < r;
      const u32x4 za = sel16(kin, *reinterpret_cast<const u32x4*>(zrow_l + (kin ? k0 : 0) * 2));
#pragma unroll
      for (int q = 0; q < QB; ++q) acc[q] = mfma32_bf16(za, bv[q][kg], acc[q]);
    }
    // fixed-order sum of the waves' partial deltas
    if (wave < 2) {
#pragma unroll
      for (int q = 0; q < QB; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) red[wave][mfma32_row(v, l)][32 * q + i] = acc[q][v];
    }
    lds_barrier();
    if (wave >= 2) {
#pragma unroll
      for (int q = 0; q < QB; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) red[wave - 2][mfma32_row(v, l)][32 * q + i] += acc[q][v];
    }
    lds_barrier();
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      const int row = ps * RPI + tid / LPR;
      float d[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) d[e] = red[0][row][cx + e] + red[1][row][cx + e];
      if (rok[ps]) add_store_y<true>(p.y, yrow[ps] + n_tile0 + cx, yv[ps], d);
    }
}

// The k-split of a sparse class's partial sums: the shrink's, which it chose
// on the device from the class's 64-slot tile count when ks_target > 0.
__device__ __forceinline__ int sparse_nparts(const ExpandParams& p) {
  if (p.ks_target <= 0) return p.nparts;
  const int ks = dyn_ksplit(count_tiles<kTMS>(p.seg, p.ranks, p.NA, p.rw), p.ks_chunks, p.ks_target, p.nparts);
  return ks > 1 ? ks : 0;
}

template <int KG>
__global__ __launch_bounds__(kThreads) void expand_sparse_kernel(ExpandParams p) {
  __shared__ float red[2][kTM][kSpNT + kOutPad];
  extern __shared__ __align__(16) char zs[];   // [32][max_rank + 8] bf16: one slice's shrink values
  const int n_sub = p.out_total / kSpNT;
  int lin = static_cast<int>(blockIdx.x);
  int sub = 0, total = 0;
  TileRef tr = locate_tile_by<kTM, kExpandBalanced>(p.seg, p.ranks, p.b_off, p.NA, p.rw, lin, true,
                                                    [&](int) { return n_sub; }, sub, total);
  const int nparts = sparse_nparts(p);
  const int items = work_items(total, n_sub, true);
  for (;;) {
    if (tr.g != 0) expand_sparse_item<KG, kSpNT / 32>(p, tr, sub, nparts, red, zs);
    lin += static_cast<int>(gridDim.x);
    if (lin >= items) break;
    lds_barrier();                         // every wave is done with zs and red before the next item
    tr = tile_at<kTM, kExpandBalanced>(p.seg, p.ranks, p.b_off, p.NA, p.rw, lin, true, total, n_sub, sub);
  }
}

// ----------------------------------------------------------------------------
// Both rank classes of a module in the same two launches (bf16, a small class
// of the one-item forms and a sparse large class).  Run on their own, the
// large class's few items were a chain of two launches of dependent memory
// trips (~20 us per projection at the decoder step whatever its bytes) that a
// second stream hid only in part.  Here the small class's grid carries them:
//   shrink_dma_pair_kernel: workgroup b shrinks its small-class item, then
//     the large class's items b, b + grid, ... (its looping form, 32-column
//     chunks, k-split chosen on the device); workgroup 0 also zeroes the
//     expand's item counter.
//   expand_pair_kernel: workgroup b expands its small-class item, then takes
//     large-class items (64-column sub-tiles of the rank-split form) from that
//     counter until none are left, so the workgroups that finish first take
//     them and they fill the launch's end.
// Every output element is computed as by the separate launches (the same
// item functions, the same sums in the same order).
// ----------------------------------------------------------------------------
constexpr int kPairQB = 2;                     // 32-column blocks per large-class expand item

// Takes the next item number of the pair expand (agent scope, the counter's
// old value).  A wrapping increment, which the compiler's atomic combining
// leaves alone: combined, the returned value is read with a wait right
// behind the atomic, while here the wait sits where the value is used.
__device__ __forceinline__ int claim_next(int* counter) {
  return static_cast<int>(__builtin_amdgcn_atomic_inc32(reinterpret_cast<uint32_t*>(counter), 0xffffffffu,
                                                        __ATOMIC_RELAXED, "agent"));
}

template <int NB0>
__global__ __launch_bounds__(kThreads) void shrink_dma_pair_kernel(ShrinkParams p0, ShrinkParams p1, int* claim) {
  constexpr int R0 = DmaRing<NB0>::NST * (kTMS + 32 * NB0) * kDmaRow;
  constexpr int R1 = DmaRing<1>::NST * (kTMS + 32) * kDmaRow;
  __shared__ __align__(16) char ring[R0 > R1 ? R0 : R1];
  if (blockIdx.x == 0 && threadIdx.x == 0) *claim = 0;   // ordered before the expand launch by the launch boundary
  // the large class's first item is looked up before the small item, so its
  // memory trip overlaps that item
  int lin = static_cast<int>(blockIdx.x);
  int KS = p1.KS, sub1 = 0, total = 0;
  TileRef tr = locate_tile_by<kTMS>(p1.seg, p1.ranks, p1.a_off, p1.NA, p1.rw, lin, true,
                                    [&](int tot) {
                                      if (p1.ks_target > 0) KS = dyn_ksplit(tot, p1.n_chunks, p1.ks_target, p1.KS);
                                      return p1.n_chunks * KS;
                                    }, sub1, total);
  {
    int sub = 0, total0 = 0;
    const TileRef tr0 = locate_tile<kTMS>(p0.seg, p0.ranks, p0.a_off, p0.NA, p0.rw, static_cast<int>(blockIdx.x),
                                          false, p0.n_chunks * p0.KS, sub, total0);
    if (tr0.g != 0) shrink_dma_item<NB0>(p0, tr0, sub, p0.KS, ring);
  }
  int sub = sub1;
  const int items = work_items(total, p1.n_chunks * KS, true);
  while (lin < items) {
    lds_barrier();                         // every wave is done with the ring before the item's transfers
    if (tr.g != 0) shrink_dma_item<1>(p1, tr, sub, KS, ring);
    lin += static_cast<int>(gridDim.x);
    if (lin >= items) break;
    tr = tile_at<kTMS>(p1.seg, p1.ranks, p1.a_off, p1.NA, p1.rw, lin, true, total, p1.n_chunks * KS, sub);
  }
}

template <int NBW, int PRE, int KG>
__global__ __launch_bounds__(kThreads) void expand_pair_kernel(ExpandParams p0, ExpandParams p1, int* claim) {
  constexpr int NT = 4 * NBW * 32;
  constexpr int kD = static_cast<int>(sizeof(float)) * kTM * (NT + kOutPad);
  constexpr int kR = static_cast<int>(sizeof(float)) * 2 * kTM * (32 * kPairQB + kOutPad);
  __shared__ __align__(16) char buf[kD > kR ? kD : kR];   // the small item's delta tile, then the large items' partial deltas
  __shared__ int claimed;
  extern __shared__ __align__(16) char zs[];   // either class's shrink values
  auto& dtile = *reinterpret_cast<float(*)[kTM][NT + kOutPad]>(buf);
  auto& red = *reinterpret_cast<float(*)[2][kTM][32 * kPairQB + kOutPad]>(buf);
  int ticket = 0;
  bool early = false;                      // uniform: the small item ran and claimed
  {
    const int n_sub = (p0.out_total + NT - 1) / NT;
    int sub = 0, groups = 1, total = 0;
    const TileRef tr = locate_tile_by<kTM, kExpandBalanced>(p0.seg, p0.ranks, p0.b_off, p0.NA, p0.rw,
                                                            static_cast<int>(blockIdx.x), false,
                                                            [&](int tot) {
                                                              groups = expand_groups(tot, n_sub, p0.wt);
                                                              return groups;
                                                            }, sub, total);
    // the first claim goes out before the small item's last sub-tile, so
    // its round trip passes while that sub-tile is computed; its result is
    // written to LDS only afterwards (no wait for it before)
    if (tr.g != 0) {
      const int sub0 = (sub * n_sub) / groups;
      const int nsub = ((sub + 1) * n_sub) / groups - sub0;
      if (nsub > 0)
        expand_item<true, NBW, PRE, false>(p0, tr, sub0, nsub, p0.nparts, dtile, zs, [&]() {
          if (threadIdx.x == 0) ticket = claim_next(claim);
          early = true;
        });
    }
  }
  const int n_sub1 = p1.out_total / (32 * kPairQB);
  const int total1 = count_tiles<kTM>(p1.seg, p1.ranks, p1.NA, p1.rw);
  const int items1 = work_items(total1, n_sub1, true);
  const int nparts1 = sparse_nparts(p1);
  if (threadIdx.x == 0)
    claimed = early ? ticket : claim_next(claim);
  lds_barrier();                           // every wave is past the small item; `claimed` is written
  int it = claimed;
  while (it < items1) {
    int sub = 0;
    const TileRef tr = tile_at<kTM, kExpandBalanced>(p1.seg, p1.ranks, p1.b_off, p1.NA, p1.rw, it, true, total1, n_sub1, sub);
    if (tr.g != 0) expand_sparse_item<KG, kPairQB>(p1, tr, sub, nparts1, red, zs);
    lds_barrier();                         // zs, buf and `claimed` are free
    if (threadIdx.x == 0) claimed = claim_next(claim);
    lds_barrier();
    it = claimed;
  }
}

// ----------------------------------------------------------------------------
// Host-side planning (shared by the workspace query and the launches).
// ----------------------------------------------------------------------------
struct ShrinkPlan {
  int max_tiles, n_chunks, KS, KC, zw, NB;
  bool dma;               // shrink_dma_kernel (bf16, H % 64 == 0) instead of shrink_kernel
  bool flat;              // flat item layout (work_item)
  bool loop;              // the ring kernel's looping form (a capped grid)
  int ks_target;          // > 0: the k-split is chosen on the device, KS is its maximum
  int64_t grid;           // workgroups launched
  int64_t part_bytes;
};

#ifndef GS_SHRINK_DMA
#define GS_SHRINK_DMA 1
#endif
#ifndef GS_SHRINK_DMA_WGS_PER_4CU
#define GS_SHRINK_DMA_WGS_PER_4CU 8
#endif

// est_tokens: the tokens the launch's rank class is expected to hold (the
// k-split is sized for them); the items cover every tile the class can have
// (all T tokens over its NA adapters).  large: the class of ranks above
// GS_RANK_CLASS_SPLIT.
// The device k-split of a sparse class aims at half the shrink's usual
// workgroup target: its expand stages the split-K partials of every row for
// each 128-column item, so fewer, longer k-chunks measured faster overall
// (with one rank-512 adapter: decode QKV 46.0 us at the full target, 40.7 at
// half, 40.2 at a quarter; decoder step 8.87 / 8.85 / 8.90 ms).
#ifndef GS_SPARSE_KS_DIV
#define GS_SPARSE_KS_DIV 2
#endif
// sparse: a large-rank class expected to hold so few tokens that its tiles
// are laid out flat and its k-split is chosen on the device from the real
// count (ks_target, KS its maximum).  max_part_bytes caps the partial sums
// (the allocation-free entry point's static scratch).
static ShrinkPlan plan_shrink(int64_t T, int H, int S, int NA, int max_rank, bool bf16, int64_t est_tokens,
                              bool large = false, bool sparse = false, int64_t max_part_bytes = INT64_MAX) {
  ShrinkPlan pl{};
  pl.dma = GS_SHRINK_DMA && bf16 && H % kDmaBK == 0;
  pl.max_tiles = static_cast<int>((T + kTMS - 1) / kTMS + (NA < T ? NA : T));
  const int64_t est_tiles = (est_tokens + kTMS - 1) / kTMS + (NA < est_tokens ? NA : est_tokens);
  // the ring kernel holds two workgroups per CU: aim for one round of them
  const int64_t target = pl.dma ? int64_t(GS_SHRINK_DMA_WGS_PER_4CU) * device_cus() / 4 : kShrinkTargetWgs;
  pl.zw = S * max_rank;
  const int nblk = (pl.zw + 31) / 32;         // 32-column blocks of the widest adapter
  pl.NB = nblk >= 4 ? 4 : nblk;
  // A large-rank class expected to hold too few tiles to fill the GPU with
  // 128-column chunks takes 32-column chunks: its parallelism then comes from
  // its many columns instead of a deep k-split, and the expand adds fewer
  // partial sums.  Few tiles are laid out flat, so they spread over the XCDs.
  if (large && pl.dma && est_tiles * ((pl.zw + 127) / 128) < target) pl.NB = 1;
  pl.flat = sparse && pl.dma;
  pl.n_chunks = (pl.zw + 32 * pl.NB - 1) / (32 * pl.NB);
  const int unit = bf16 ? 256 : 128;          // k per batch of the shrink kernel
  const int units = (H + unit - 1) / unit;
  // split the hidden dimension for about 640 workgroups (the tile count is an
  // upper bound, T/64 + NA), at most 16 ways (the partial sums' consumers).
  // Where the grid stays at 512 workgroups or more, a workgroup takes at
  // least 3 batches, so its start (tile lookup, token rows, first batch) is
  // spread over enough streaming; measured on the prefill and decoder-step
  // shapes
  const int64_t wgs = est_tiles * pl.n_chunks;
  int ks = static_cast<int>((target + wgs / 2) / (wgs > 0 ? wgs : 1));
  if (ks < 1) ks = 1;
  if (ks > 16) ks = 16;
  if (ks > units) ks = units;
  if (pl.dma) {
    // the ring kernel splits the 64-k stages evenly over the KS chunks (at
    // least 4 stages each: ks <= units)
    pl.KS = ks;
    if (pl.flat) {
      // chosen on the device (dyn_ksplit): KS is the largest it may take,
      // within the partial sums' budget
      pl.ks_target = static_cast<int>(std::max<int64_t>(1, target / GS_SPARSE_KS_DIV));
      const int64_t row = T * pl.zw * 4;
      pl.KS = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(std::min(16, units), max_part_bytes / row)));
    }
    pl.KC = 0;
    pl.part_bytes = pl.KS > 1 ? static_cast<int64_t>(pl.KS) * T * pl.zw * 4 : 0;
    const int64_t nsub = static_cast<int64_t>(pl.n_chunks) * pl.KS;
    const auto items = [&](int64_t tiles) { return (pl.flat ? tiles : 8 * ((tiles + 7) / 8)) * nsub; };
    pl.grid = items(pl.max_tiles);
    // a large-rank class is expected to hold far fewer tiles than it could:
    // its grid is capped near the expected items and the workgroups loop
    // (workgroups with no item would each hold a ring of LDS through a lookup)
    if (large) {
      pl.loop = true;
      const int64_t cap = pl.flat ? target : std::max(target, std::min(items(est_tiles), 2 * target));
      pl.grid = std::min(pl.grid, (cap + 7) / 8 * 8);
    }
    return pl;
  }
  int per = (units + ks - 1) / ks;
  if (per < 3 && units >= 3 && wgs * ((units + 2) / 3) >= 512) per = 3;
  pl.KC = per * unit;
  pl.KS = (H + pl.KC - 1) / pl.KC;
  if (pl.KS < 1) pl.KS = 1;
  pl.part_bytes = pl.KS > 1 ? static_cast<int64_t>(pl.KS) * T * pl.zw * 4 : 0;
  pl.grid = 8 * ((static_cast<int64_t>(pl.max_tiles) + 7) / 8) * pl.n_chunks * pl.KS;
  return pl;
}

// ----------------------------------------------------------------------------
// Rank classes.  A module whose adapters' ranks differ widely (one rank-512
// adapter among rank-32 ones) runs its shrink and expand once per class, each
// planned for the class's own largest rank, so that the column tiles, k-split,
// LDS and registers a large adapter needs never apply to the small adapters'
// tokens: a large adapter costs large-rank work only for the tokens that use
// it.  The classes are ranks <= 64 (the expand's register-resident forms) and
// ranks above.  Without a host rank table a module is one class up to
// max_rank, as before.
// ----------------------------------------------------------------------------
constexpr int kRankClassSplit = GS_RANK_CLASS_SPLIT;

struct RankClass {
  RankWindow rw;
  int max_rank;         // the class's largest rank
  int adapters;         // its adapters (the grid's bound on part-filled tiles)
  int64_t est_tokens;   // the tokens it is expected to hold: ids spread evenly over the applicable adapters
};

// Fills cls[0..n) and sets n (0: no adapter is applicable, nothing to launch).
static int rank_classes(const char* who, const int32_t* ranks_host, int NA, int max_rank, int64_t T,
                        RankClass (&cls)[2], int& n) {
  n = 0;
  if (ranks_host == nullptr) {
    cls[n++] = RankClass{{1, max_rank}, max_rank, NA, T};
    return GS_OK;
  }
  RankClass c[2] = {RankClass{{1, kRankClassSplit}, 0, 0, 0}, RankClass{{kRankClassSplit + 1, GS_MAX_RANK}, 0, 0, 0}};
  int applicable = 0;
  for (int g = 1; g <= NA; ++g) {
    const int r = ranks_host[g];
    GS_CHECK_ARG(r >= 0 && r <= max_rank && r % 8 == 0, "%s: ranks_host[%d]=%d must be a multiple of 8 in [0, max_rank=%d]",
                 who, g, r, max_rank);
    if (r == 0) continue;
    RankClass& k = c[r <= kRankClassSplit ? 0 : 1];
    k.max_rank = r > k.max_rank ? r : k.max_rank;
    ++k.adapters;
    ++applicable;
  }
  for (RankClass& k : c) {
    if (k.adapters == 0) continue;
    k.est_tokens = (T * k.adapters + applicable - 1) / applicable;
    cls[n++] = k;
  }
  return GS_OK;
}

static bool large_class(const RankClass& k) { return k.rw.lo > kRankClassSplit; }

// A large-rank class expected to hold fewer than 8 tiles of 64 tokens: both
// kernels lay its tiles out flat (its few tiles spread over the XCDs), their
// workgroups loop over a grid of one round, and the shrink's k-split is
// chosen on the device from the real tile count.
static bool sparse_class(const RankClass& k) {
  const int64_t est_tiles = (k.est_tokens + kTMS - 1) / kTMS + std::min<int64_t>(k.adapters, k.est_tokens);
  return large_class(k) && est_tiles < 8;
}

// device_ks = false: the host's k-split even for a sparse class (gs_shrink,
// whose reduce into z must know it).
static ShrinkPlan plan_class(int64_t T, int H, int S, const RankClass& k, bool bf16,
                             int64_t max_part_bytes = INT64_MAX, bool device_ks = true) {
  return plan_shrink(T, H, S, k.adapters, k.max_rank, bf16, k.est_tokens, large_class(k),
                     device_ks && sparse_class(k), max_part_bytes);
}


}  // namespace gs

using namespace gs;

namespace {

// LDS of the expand: the row-major delta tile plus the tile's shrink values.
size_t expand_lds_bytes(bool bf16, int S, int max_rank) {
  return static_cast<size_t>(kTM) * (static_cast<size_t>(S) * max_rank + 8) * (bf16 ? 2 : 4);
}
constexpr size_t kMaxDynLds = 120 * 1024;

int check_common(const char* who, int32_t dtype, int64_t T, int32_t num_slices, int32_t num_adapters,
                 int32_t max_rank) {
  GS_CHECK_ARG(dtype == GS_DTYPE_BF16 || dtype == GS_DTYPE_FP32, "%s: dtype=%d", who, dtype);
  GS_CHECK_ARG(T >= 0 && T < (int64_t(1) << 31), "%s: num_tokens out of range", who);
  GS_CHECK_ARG(num_slices >= 1 && num_slices <= GS_MAX_SLICES, "%s: num_slices=%d", who, num_slices);
  GS_CHECK_ARG(num_adapters >= 1 && num_adapters <= GS_MAX_ADAPTERS, "%s: num_adapters=%d", who, num_adapters);
  GS_CHECK_ARG(max_rank >= 8 && max_rank <= GS_MAX_RANK && max_rank % 8 == 0,
               "%s: max_rank=%d must be a multiple of 8 in [8,%d]", who, max_rank, GS_MAX_RANK);
  return GS_OK;
}

int check_shrink(int32_t dtype, const void* x, int64_t ldx, int32_t hidden, const void* a_pack) {
  const int vec = dtype == GS_DTYPE_BF16 ? 8 : 4;
  GS_CHECK_ARG(hidden > 0 && hidden % 8 == 0, "gs_shrink: hidden=%d must be a positive multiple of 8", hidden);
  GS_CHECK_ARG(ldx >= hidden && ldx % vec == 0, "gs_shrink: ldx=%lld", (long long)ldx);
  GS_CHECK_ARG(aligned16(x) && aligned16(a_pack), "gs_shrink: x and a_pack must be 16-byte aligned");
  return GS_OK;
}

ShrinkParams make_shrink_params(const ShrinkPlan& pl, const void* x, int64_t ldx, int32_t hidden, const void* a_pack,
                                const int64_t* a_off, const int32_t* ranks, int32_t S, int32_t NA,
                                const int32_t* seg, const int32_t* perm, void* z, int64_t ldz, void* workspace,
                                int64_t T, RankWindow rw) {
  ShrinkParams p{};
  p.rw = rw;
  p.flat = pl.flat ? 1 : 0;
  p.ks_target = pl.ks_target;
  p.x = x;
  p.ldx = ldx;
  p.H = hidden;
  p.a_pack = a_pack;
  p.a_off = a_off;
  p.ranks = ranks;
  p.S = S;
  p.NA = NA;
  p.seg = seg;
  p.perm = perm;
  p.z = z;
  p.ldz = ldz;
  p.part = pl.KS > 1 ? static_cast<float*>(workspace) : nullptr;
  p.part_stride = T * pl.zw;
  p.zw = pl.zw;
  p.KS = pl.KS;
  p.KC = pl.KC;
  p.n_chunks = pl.n_chunks;
  return p;
}

int check_workspace(const ShrinkPlan& pl, const void* workspace, int64_t workspace_bytes) {
  if (pl.KS > 1 && (workspace == nullptr || workspace_bytes < pl.part_bytes || !aligned16(workspace))) {
    set_error("gs_shrink: workspace of %lld bytes needed (got %lld)", (long long)pl.part_bytes,
              (long long)workspace_bytes);
    return GS_ERR_WORKSPACE;
  }
  return GS_OK;
}

template <bool BF16>
void launch_shrink_t(const ShrinkPlan& pl, const ShrinkParams& p, hipStream_t st) {
  dim3 grid(static_cast<unsigned>(pl.grid));
  if (BF16 && pl.dma) {
    if (pl.loop) {
      if (pl.NB == 4) hipLaunchKernelGGL((shrink_dma_kernel<4, true>), grid, dim3(kThreads), 0, st, p);
      else if (pl.NB == 3) hipLaunchKernelGGL((shrink_dma_kernel<3, true>), grid, dim3(kThreads), 0, st, p);
      else if (pl.NB == 2) hipLaunchKernelGGL((shrink_dma_kernel<2, true>), grid, dim3(kThreads), 0, st, p);
      else hipLaunchKernelGGL((shrink_dma_kernel<1, true>), grid, dim3(kThreads), 0, st, p);
      return;
    }
    if (pl.NB == 4) hipLaunchKernelGGL((shrink_dma_kernel<4, false>), grid, dim3(kThreads), 0, st, p);
    else if (pl.NB == 3) hipLaunchKernelGGL((shrink_dma_kernel<3, false>), grid, dim3(kThreads), 0, st, p);
    else if (pl.NB == 2) hipLaunchKernelGGL((shrink_dma_kernel<2, false>), grid, dim3(kThreads), 0, st, p);
    else hipLaunchKernelGGL((shrink_dma_kernel<1, false>), grid, dim3(kThreads), 0, st, p);
    return;
  }
  if (pl.NB == 4) hipLaunchKernelGGL((shrink_kernel<BF16, 4>), grid, dim3(kThreads), 0, st, p);
  else if (pl.NB == 3) hipLaunchKernelGGL((shrink_kernel<BF16, 3>), grid, dim3(kThreads), 0, st, p);
  else if (pl.NB == 2) hipLaunchKernelGGL((shrink_kernel<BF16, 2>), grid, dim3(kThreads), 0, st, p);
  else hipLaunchKernelGGL((shrink_kernel<BF16, 1>), grid, dim3(kThreads), 0, st, p);
}

void launch_shrink(bool bf16, const ShrinkPlan& pl, const ShrinkParams& p, hipStream_t st) {
  if (bf16) launch_shrink_t<true>(pl, p, st);
  else launch_shrink_t<false>(pl, p, st);
}

int prepare_expand(ExpandParams& p, const char* who, int32_t dtype, void* y, int64_t ldy, int64_t T,
                   int32_t out_total, const int32_t* slice_bounds, int32_t num_slices, const void* b_pack,
                   const int64_t* b_off, const int32_t* ranks, int32_t NA, int32_t max_rank, const int32_t* seg,
                   const int32_t* perm) {
  const int vec = dtype == GS_DTYPE_BF16 ? 8 : 4;
  GS_CHECK_ARG(out_total > 0 && out_total % 32 == 0, "%s: out_total=%d must be a multiple of 32", who, out_total);
  GS_CHECK_ARG(slice_bounds != nullptr, "%s: slice_bounds is NULL", who);
  GS_CHECK_ARG(slice_bounds[0] == 0 && slice_bounds[num_slices] == out_total, "%s: slice_bounds must span [0,out_total]", who);
  for (int s = 0; s < num_slices; ++s)
    GS_CHECK_ARG(slice_bounds[s + 1] > slice_bounds[s] && (slice_bounds[s + 1] - slice_bounds[s]) % 32 == 0,
                 "%s: slice %d width must be a positive multiple of 32", who, s);
  GS_CHECK_ARG(ldy >= out_total && ldy % vec == 0, "%s: ldy=%lld", who, (long long)ldy);
  GS_CHECK_ARG(aligned16(y) && aligned16(b_pack), "%s: y and b_pack must be 16-byte aligned", who);
  GS_CHECK_ARG(max_tiles_for(T, NA) <= 65535, "%s: num_tokens too large for one launch", who);
  GS_CHECK_ARG(expand_lds_bytes(dtype == GS_DTYPE_BF16, num_slices, max_rank) <= kMaxDynLds,
               "%s: num_slices * max_rank = %d too large for the LDS-staged expand", who, num_slices * max_rank);
  p.y = y;
  p.ldy = ldy;
  p.out_total = out_total;
  p.si.S = num_slices;
  for (int s = 0; s <= num_slices; ++s) p.si.bounds[s] = slice_bounds[s];
  p.b_pack = b_pack;
  p.b_off = b_off;
  p.ranks = ranks;
  p.NA = NA;
  p.max_rank = max_rank;
  p.seg = seg;
  p.perm = perm;
  return GS_OK;
}

// Workgroups of a column-split expand launch: the items never exceed wt (or
// one per tile slot when the tiles alone exceed it) nor one per (tile slot,
// sub-tile); a flat launch is one round of workgroups that loop over its
// (tile, sub-tile) items.
int64_t expand_grid(int64_t wt, int max_tiles, int64_t n_sub, bool flat) {
  const int64_t t8 = 8 * ((static_cast<int64_t>(max_tiles) + 7) / 8);
  const int64_t items = flat ? std::min<int64_t>(wt, static_cast<int64_t>(max_tiles) * n_sub)
                             : std::min<int64_t>(std::max(wt, t8), t8 * n_sub);
  return (items + 7) / 8 * 8;
}

// Workgroups of a rank-split (sparse) expand launch: one round, at most one
// per (tile slot, sub-tile).
int64_t sparse_grid(int64_t wt, int max_tiles, int64_t n_sub) {
  return std::max<int64_t>(1, std::min<int64_t>(wt, static_cast<int64_t>(max_tiles) * n_sub));
}

template <bool BF16, int NBW, int PRE>
void launch_expand_t(int max_tiles, size_t lds, ExpandParams p, hipStream_t st) {
  auto kern = p.flat ? expand_kernel<BF16, NBW, PRE, true> : expand_kernel<BF16, NBW, PRE, false>;
  if (lds > 64 * 1024) (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  // workgroups resident per CU for this LDS size, queried once per size and
  // kernel form and kept as one word (lds << 16 | count) so concurrent
  // callers read a consistent pair
  static std::atomic<uint64_t> occ_of[2];
  std::atomic<uint64_t>& occ = occ_of[p.flat ? 1 : 0];
  uint64_t o = occ.load(std::memory_order_relaxed);
  if (o == 0 || (o >> 16) != lds) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(kern), kThreads, lds) != hipSuccess || n < 1) n = 1;
    o = (static_cast<uint64_t>(lds) << 16) | static_cast<uint64_t>(std::min(n, 0xffff));
    occ.store(o, std::memory_order_relaxed);
  }
  p.wt = static_cast<int>(o & 0xffff) * device_cus();
  constexpr int NT = 4 * NBW * 32;
  const int grid = static_cast<int>(expand_grid(p.wt, max_tiles, (p.out_total + NT - 1) / NT, p.flat != 0));
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), lds, st, p);
}

template <bool BF16, int NBW>
void launch_expand_pre(int max_tiles, size_t lds, const ExpandParams& p, hipStream_t st) {
  constexpr int KSTEP = BF16 ? 16 : 8;
  const int need = (p.max_rank + KSTEP - 1) / KSTEP;
  if (need <= 2) launch_expand_t<BF16, NBW, 2>(max_tiles, lds, p, st);
  else if (need <= 4) launch_expand_t<BF16, NBW, 4>(max_tiles, lds, p, st);
  else launch_expand_t<BF16, NBW, 8>(max_tiles, lds, p, st);
}

// The rank-split expand takes a sparse bf16 class whose sub-tiles of 128
// columns never straddle a slice.
bool sparse_expand_fits(bool bf16, const ExpandParams& p) {
  if (!bf16 || p.max_rank > 4 * 8 * 16) return false;
  for (int s = 0; s < p.si.S; ++s)
    if ((p.si.bounds[s + 1] - p.si.bounds[s]) % kSpNT != 0) return false;
  return true;
}

template <int KG>
void launch_sparse_t(int max_tiles, ExpandParams p, hipStream_t st) {
  auto kern = expand_sparse_kernel<KG>;
  const size_t lds = static_cast<size_t>(kTM) * (p.max_rank + 8) * 2;
  // workgroups resident per CU for this LDS size (one word: lds << 16 | count)
  static std::atomic<uint64_t> occ{0};
  uint64_t o = occ.load(std::memory_order_relaxed);
  if (o == 0 || (o >> 16) != lds) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(kern), kThreads, lds) != hipSuccess || n < 1) n = 1;
    o = (static_cast<uint64_t>(lds) << 16) | static_cast<uint64_t>(std::min(n, 0xffff));
    occ.store(o, std::memory_order_relaxed);
  }
  // one round of workgroups looping over the flat (tile, sub-tile) items
  const int64_t grid = sparse_grid(static_cast<int64_t>(o & 0xffff) * device_cus(), max_tiles, p.out_total / kSpNT);
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(kThreads), lds, st, p);
}

void launch_expand_sparse(int64_t T, int adapters, const ExpandParams& p, hipStream_t st) {
  const int max_tiles = max_tiles_for(T, adapters);
  if (p.max_rank <= 4 * 2 * 16) launch_sparse_t<2>(max_tiles, p, st);
  else if (p.max_rank <= 4 * 4 * 16) launch_sparse_t<4>(max_tiles, p, st);
  else launch_sparse_t<8>(max_tiles, p, st);
}

// Which expand form a launch takes (shared by the launch and the address
// model): the rank-split form for a sparse bf16 class, else the column-split
// form with NBW 32-column blocks per wave and PRE k-groups of lora_B in
// registers.
struct ExpandForm {
  bool sparse;
  int NBW, PRE, KG;
};
ExpandForm expand_form(bool bf16, int64_t T, const ExpandParams& p) {
  ExpandForm f{false, 1, 2, 0};
  if (p.flat && sparse_expand_fits(bf16, p)) {
    f.sparse = true;
    f.KG = p.max_rank <= 4 * 2 * 16 ? 2 : (p.max_rank <= 4 * 4 * 16 ? 4 : 8);
    return f;
  }
  // wider column tiles halve the z / partial reads per output byte, but
  // their lora_B registers grow with the rank: above rank 32 (bf16; 16 fp32
  // k per group) the wide kernel drops to 2 or 1 resident waves per SIMD and
  // the narrow one streams faster (multiswitch down, ranks to 64: expand
  // 21.5 -> 16.7 us)
  const int kstep = bf16 ? 16 : 8;
  const int need = (p.max_rank + kstep - 1) / kstep;
  f.NBW = ((T >= 2048 || p.nparts > 1) && need <= 2) ? 2 : 1;
  f.PRE = need <= 2 ? 2 : (need <= 4 ? 4 : 8);
  return f;
}


// adapters: the launch's rank class (bounds its part-filled tiles)
void launch_expand(bool bf16, int64_t T, int adapters, ExpandParams p, hipStream_t st) {
  const ExpandForm f = expand_form(bf16, T, p);
  if (f.sparse) {
    launch_expand_sparse(T, adapters, p, st);
    return;
  }
  const int max_tiles = max_tiles_for(T, adapters);
  const size_t lds = expand_lds_bytes(bf16, p.si.S, p.max_rank);
  if (bf16) {
    if (f.NBW == 2) launch_expand_pre<true, 2>(max_tiles, lds, p, st);
    else launch_expand_pre<true, 1>(max_tiles, lds, p, st);
  } else {
    if (f.NBW == 2) launch_expand_pre<false, 2>(max_tiles, lds, p, st);
    else launch_expand_pre<false, 1>(max_tiles, lds, p, st);
  }
}


// The pair launches (shrink_dma_pair_kernel, expand_pair_kernel) take a
// module's two classes when the small class's plans are the one-item ring
// shrink and column-split expand and the large class's are the sparse ones
// (bf16): the forms whose item functions the pair kernels run.
struct PairForm {
  bool ok = false;
  int NB0 = 1;            // the small class's shrink column blocks
  ExpandForm f0{};        // the small class's expand form
  int KG1 = 0;            // the large class's k-groups per wave
};
PairForm pair_form(bool bf16, int64_t T, const ShrinkPlan& pl0, const ShrinkPlan& pl1, const ExpandParams& e0,
                   const ExpandParams& e1) {
  PairForm f;
  if (!bf16 || !pl0.dma || pl0.loop || pl0.flat || !pl1.dma || !pl1.loop || !pl1.flat || pl1.NB != 1) return f;
  if (e1.max_rank > 4 * 8 * 16) return f;
  for (int s = 0; s < e1.si.S; ++s)
    if ((e1.si.bounds[s + 1] - e1.si.bounds[s]) % (32 * kPairQB) != 0) return f;
  f.f0 = expand_form(true, T, e0);
  if (f.f0.sparse || e0.flat || f.f0.PRE > 4) return f;
  f.NB0 = pl0.NB;
  f.KG1 = e1.max_rank <= 4 * 2 * 16 ? 2 : (e1.max_rank <= 4 * 4 * 16 ? 4 : 8);
  f.ok = true;
  return f;
}

// The launch-plan fields of a class's expand parameters (what the form
// choices read), as a call with these slices makes them.
ExpandParams class_expand_plan(const SliceInfo& si, int out_total, const RankClass& k, const ShrinkPlan& pl,
                               int64_t T, int64_t ldz) {
  ExpandParams e{};
  e.out_total = out_total;
  e.si = si;
  e.ldz = ldz;
  e.part_stride = T * pl.zw;
  e.zw = pl.zw;
  e.nparts = pl.KS > 1 ? pl.KS : 0;
  e.max_rank = k.max_rank;
  e.rw = k.rw;
  e.flat = pl.flat ? 1 : 0;
  e.ks_target = pl.ks_target;
  e.ks_chunks = pl.n_chunks;
  return e;
}

size_t pair_lds_bytes(int S, int max_rank0, int max_rank1) {
  return std::max(expand_lds_bytes(true, S, max_rank0), static_cast<size_t>(kTM) * (max_rank1 + 8) * 2);
}

template <int NBW, int PRE, int KG>
const void* expand_pair_fn() {
  return reinterpret_cast<const void*>(expand_pair_kernel<NBW, PRE, KG>);
}
template <int NBW, int PRE>
const void* expand_pair_fn_kg(int KG) {
  return KG == 2 ? expand_pair_fn<NBW, PRE, 2>() : (KG == 4 ? expand_pair_fn<NBW, PRE, 4>() : expand_pair_fn<NBW, PRE, 8>());
}
const void* expand_pair_fn_of(const PairForm& f) {
  if (f.f0.NBW == 2) return expand_pair_fn_kg<2, 2>(f.KG1);
  return f.f0.PRE <= 2 ? expand_pair_fn_kg<1, 2>(f.KG1) : expand_pair_fn_kg<1, 4>(f.KG1);
}

// Workgroups of the pair expand resident per CU at `lds` bytes of dynamic LDS
// (queried once per kernel and size, kept as one word: lds << 16 | count).
int pair_expand_occupancy(const void* kern, size_t lds) {
  static std::mutex mu;
  static std::vector<std::pair<const void*, uint64_t>> memo;
  std::lock_guard<std::mutex> lock(mu);
  for (const auto& m : memo)
    if (m.first == kern && (m.second >> 16) == lds) return static_cast<int>(m.second & 0xffff);
  if (lds > 64 * 1024) (void)hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, kThreads, lds) != hipSuccess || n < 1) n = 1;
  memo.emplace_back(kern, (static_cast<uint64_t>(lds) << 16) | static_cast<uint64_t>(std::min(n, 0xffff)));
  return n;
}

// The pair expand's grid: the small class's one-item grid at the pair
// kernel's occupancy (sets e0.wt, which its items' column groups follow).
int64_t pair_expand_grid(const PairForm& f, int64_t T, int adapters0, size_t lds, ExpandParams& e0) {
  e0.wt = pair_expand_occupancy(expand_pair_fn_of(f), lds) * device_cus();
  const int NT = 4 * f.f0.NBW * 32;
  return expand_grid(e0.wt, max_tiles_for(T, adapters0), (e0.out_total + NT - 1) / NT, false);
}

void launch_shrink_pair(const PairForm& f, int64_t grid, const ShrinkParams& p0, const ShrinkParams& p1, int* claim,
                        hipStream_t st) {
  const dim3 g(static_cast<unsigned>(grid));
  if (f.NB0 == 4) hipLaunchKernelGGL((shrink_dma_pair_kernel<4>), g, dim3(kThreads), 0, st, p0, p1, claim);
  else if (f.NB0 == 3) hipLaunchKernelGGL((shrink_dma_pair_kernel<3>), g, dim3(kThreads), 0, st, p0, p1, claim);
  else if (f.NB0 == 2) hipLaunchKernelGGL((shrink_dma_pair_kernel<2>), g, dim3(kThreads), 0, st, p0, p1, claim);
  else hipLaunchKernelGGL((shrink_dma_pair_kernel<1>), g, dim3(kThreads), 0, st, p0, p1, claim);
}

template <int NBW, int PRE>
void launch_expand_pair_kg(int KG, dim3 g, size_t lds, const ExpandParams& e0, const ExpandParams& e1, int* claim,
                           hipStream_t st) {
  if (KG == 2) hipLaunchKernelGGL((expand_pair_kernel<NBW, PRE, 2>), g, dim3(kThreads), lds, st, e0, e1, claim);
  else if (KG == 4) hipLaunchKernelGGL((expand_pair_kernel<NBW, PRE, 4>), g, dim3(kThreads), lds, st, e0, e1, claim);
  else hipLaunchKernelGGL((expand_pair_kernel<NBW, PRE, 8>), g, dim3(kThreads), lds, st, e0, e1, claim);
}
void launch_expand_pair(const PairForm& f, int64_t grid, size_t lds, const ExpandParams& e0, const ExpandParams& e1,
                        int* claim, hipStream_t st) {
  const dim3 g(static_cast<unsigned>(grid));
  if (f.f0.NBW == 2) launch_expand_pair_kg<2, 2>(f.KG1, g, lds, e0, e1, claim, st);
  else if (f.f0.PRE <= 2) launch_expand_pair_kg<1, 2>(f.KG1, g, lds, e0, e1, claim, st);
  else launch_expand_pair_kg<1, 4>(f.KG1, g, lds, e0, e1, claim, st);
}

// ----------------------------------------------------------------------------
// Address model (test support): replays the global and LDS accesses of the
// segment kernels on the host, with the launch plans and the addr:: formulas
// the kernels use, for every workgroup, wave, lane and loop step of every
// launch a call makes, and checks each access against its buffer.  It also
// checks that the launches cover every item of the batch (a one-item grid
// smaller than the items would skip work).  No HIP call is made.
// ----------------------------------------------------------------------------
struct AddrModel {
  // the call
  bool bf16;
  int64_t T;
  int H;
  int64_t ldx;
  int out_total;
  int64_t ldy;
  SliceInfo si;
  const int32_t* ranks;     // host copies of the module tables
  const int64_t* a_off;
  const int64_t* b_off;
  int64_t a_elems, b_elems;
  int NA;
  int max_rank;
  const int32_t* seg;
  const int32_t* perm;
  int64_t perm_len;
  // outcome
  int64_t checked = 0;
  int64_t bad = 0;
  char msg[512] = {0};

  int es() const { return bf16 ? 2 : 4; }
  void fail(const char* fmt, ...) {
    ++bad;
    if (bad > 1) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof msg, fmt, ap);
    va_end(ap);
  }
  // [lo, lo + len) inside [0, size)?
  bool in(const char* what, int64_t lo, int64_t len, int64_t size) {
    ++checked;
    if (lo < 0 || len < 0 || lo + len > size) {
      fail("%s: [%lld, %lld) outside [0, %lld)", what, (long long)lo, (long long)(lo + len), (long long)size);
      return false;
    }
    return true;
  }
  int token_at(int64_t slot_idx) {
    if (!in("perm", slot_idx, 1, perm_len)) return 0;
    const int tok = perm[slot_idx];
    in("token", tok, 1, T);
    return tok;
  }
  // a 16-byte (or len-byte) piece of row `tok` of a [T, ld] matrix whose rows hold `cols` valid elements
  void row_piece(const char* what, int64_t tok, int64_t elem, int64_t n_elems, int64_t cols) {
    in(what, elem, n_elems, cols);
    (void)tok;
  }
  // an adapter's block [off, off + rows * cols) inside a pack of `elems` elements
  void pack_piece(const char* what, int64_t off, int64_t rows, int64_t cols, int64_t elem, int64_t n, int64_t elems) {
    in(what, elem - off, n, rows * cols);
    in(what, elem, n, elems);
  }

  template <int TM, bool BAL>
  std::vector<TileRef> tiles(RankWindow rw, const int64_t* offs) const {
    std::vector<TileRef> v;
    for (int g = 1; g <= NA; ++g) {
      if (!in_window(rw, ranks[g])) continue;
      const int lo = seg[g - 1], hi = seg[g];
      const int nt = (hi - lo + TM - 1) / TM;
      for (int jj = 0; jj < nt; ++jj) {
        TileRef t{g, 0, 0, ranks[g], offs[g]};
        tile_span<TM, BAL>(lo, hi, jj, t.slot0, t.nrows);
        v.push_back(t);
      }
    }
    return v;
  }

  // Items processed by a grid: one per workgroup (loop = false) or
  // blockIdx.x, + grid, ... (loop = true); every real item must be taken
  // exactly once.
  template <typename F>
  void for_items(const char* who, int64_t grid, bool loop, int items, F&& fn) {
    int64_t seen = 0;
    for (int64_t b = 0; b < grid; ++b) {
      for (int64_t lin = b; lin < items; lin += grid) {
        fn(static_cast<int>(lin));
        ++seen;
        if (!loop) break;
      }
    }
    if (seen != items) fail("%s: the grid of %lld workgroups takes %lld of %d items", who, (long long)grid,
                            (long long)seen, items);
  }

  // ---- shrink_dma_kernel ----------------------------------------------------
  // grid / loop: the launch's (the plan's own unless the pair shrink carries
  // the items on the small class's grid)
  void shrink_dma(const ShrinkPlan& pl, RankWindow rw, int64_t ldz, int64_t z_elems, int64_t part_elems,
                  int64_t grid = -1, int loop = -1) {
    if (grid < 0) grid = pl.grid;
    if (loop < 0) loop = pl.loop ? 1 : 0;
    const std::vector<TileRef> tl = tiles<kTMS, false>(rw, a_off);
    const int total = static_cast<int>(tl.size());
    const int KS = pl.ks_target > 0 ? dyn_ksplit(total, pl.n_chunks, pl.ks_target, pl.KS) : pl.KS;
    const int nsub = pl.n_chunks * KS;
    const bool flat = pl.loop && pl.flat;
    const int COLS = 32 * pl.NB, ARW = COLS / 4, XT = kTMS / 4 / 8, AT = ARW / 8;
    const int NST = pl.NB == 1 ? GS_DMA_NST1 : (pl.NB == 2 ? GS_DMA_NST2 : (pl.NB == 3 ? GS_DMA_NST3 : GS_DMA_NST4));
    const int64_t stage = static_cast<int64_t>(kTMS + COLS) * kDmaRow, ring = NST * stage;
    const int64_t zw = pl.zw;
    for_items("shrink_dma_kernel", grid, loop != 0, work_items(total, nsub, flat), [&](int lin) {
      const XcdItem it = work_item(lin, total, nsub, flat);
      if (it.tile < 0) return;
      const TileRef& tr = tl[it.tile];
      const int chunk = it.sub % pl.n_chunks, ks = it.sub / pl.n_chunks;
      const int ncols = si.S * tr.rank, col0 = chunk * COLS;
      if (col0 >= ncols) return;
      int s_lo = 0, nst = 0;
      addr::dma_kchunk(H, ks, KS, s_lo, nst);
      in("shrink k-chunk", static_cast<int64_t>(s_lo) * kDmaBK, static_cast<int64_t>(nst) * kDmaBK, H);
      const int64_t k_lo = static_cast<int64_t>(s_lo) * kDmaBK;
      for (int wave = 0; wave < 4; ++wave)
        for (int l = 0; l < 64; ++l) {
          const int trow = addr::dma_trow(l);
          for (int t = 0; t < XT; ++t) {
            const int xrow = addr::dma_x_row(wave, t, trow);
            const int64_t gp = addr::dma_gpiece_bytes(l, xrow) / 2;
            const int tok = token_at(tr.slot0 + addr::tile_row(xrow, tr.nrows));
            for (int st = 0; st < nst; ++st) row_piece("shrink x", tok, k_lo + st * 64 + gp, 8, H);
            in("shrink x ring", (NST - 1) * stage + (16 * wave + 8 * t) * kDmaRow + 16 * l, 16, ring);
          }
          for (int t = 0; t < AT; ++t) {
            const int arow = addr::dma_a_row(col0, ARW, wave, t, trow, ncols);
            const int64_t gp = addr::dma_gpiece_bytes(l, kTMS + ARW * wave + 8 * t + trow) / 2;
            for (int st = 0; st < nst; ++st)
              pack_piece("shrink lora_A", tr.off, ncols, H, tr.off + static_cast<int64_t>(arow) * H + k_lo + st * 64 + gp,
                         8, a_elems);
            in("shrink A ring", (NST - 1) * stage + (kTMS + ARW * wave + 8 * t) * kDmaRow + 16 * l, 16, ring);
          }
        }
      const int PPR4 = COLS / 4, wcols = std::min(COLS, ncols - col0);
      in("shrink staged results", 0, static_cast<int64_t>(kTMS) * (COLS + 4) * 4, ring);
      for (int tid = 0; tid < kThreads; ++tid)
        for (int k = 0; k < kTMS * PPR4 / kThreads; ++k) {
          const int pc = tid + k * kThreads;
          const int row = addr::dma_res_row(pc, PPR4), c4 = addr::dma_res_col(pc, PPR4);
          if (row >= tr.nrows || c4 >= wcols) continue;
          const int64_t slot = tr.slot0 + row;
          if (KS == 1) {
            in("shrink z column", col0 + c4, 4, ldz);
            in("shrink z", slot * ldz + col0 + c4, 4, z_elems);
          } else {
            in("shrink partial column", col0 + c4, 4, zw);
            in("shrink partials", ks * T * zw + slot * zw + col0 + c4, 4, part_elems);
          }
        }
    });
  }

  // ---- shrink_kernel (register form) ----------------------------------------
  void shrink_reg(const ShrinkPlan& pl, RankWindow rw, int64_t ldz, int64_t z_elems, int64_t part_elems) {
    const std::vector<TileRef> tl = tiles<kTMS, false>(rw, a_off);
    const int total = static_cast<int>(tl.size());
    const int nsub = pl.n_chunks * pl.KS;
    const int P = bf16 ? 8 : 4, KSTEP = 4 * P, NPB = 8, BK = NPB * KSTEP, COLS = 32 * pl.NB;
    const int PPR = BK * es() / 16, RSTEP = kThreads / PPR, APT = COLS * PPR / kThreads;
    for_items("shrink_kernel", pl.grid, false, work_items(total, nsub, false), [&](int lin) {
      const XcdItem it = work_item(lin, total, nsub, false);
      if (it.tile < 0) return;
      const TileRef& tr = tl[it.tile];
      const int chunk = it.sub % pl.n_chunks, ks = it.sub / pl.n_chunks;
      const int ncols = si.S * tr.rank, col0 = chunk * COLS;
      if (col0 >= ncols) return;
      const int64_t k_lo = static_cast<int64_t>(ks) * pl.KC;
      const int64_t k_hi = std::min<int64_t>(H, k_lo + pl.KC);
      const int nbat = static_cast<int>((k_hi - k_lo + BK - 1) / BK);
      for (int tid = 0; tid < kThreads; ++tid) {
        const int wave = tid >> 6, l = tid & 63, i16 = l & 15, q4 = l >> 4;
        const int srow = 16 * wave + i16;
        const bool row_ok = srow < tr.nrows;
        const int tok = token_at(tr.slot0 + addr::tile_row(srow, tr.nrows));
        const int ar0 = tid / PPR, apc = tid % PPR, arows = ncols - col0 - ar0;
        const int64_t abase = tr.off + static_cast<int64_t>(col0 + ar0) * H;
        for (int b = 0; b <= nbat; ++b) {          // b = nbat: the prefetch past the chunk (masked)
          const int64_t kp_a = k_lo + static_cast<int64_t>(b) * BK + apc * P;
          for (int j = 0; j < APT; ++j) {
            const bool ok = j * RSTEP < arows && kp_a < k_hi;
            pack_piece("shrink lora_A", tr.off, ncols, H, abase + addr::reg_a_elem(ok, j, int64_t(RSTEP) * H, kp_a, k_lo),
                       P, a_elems);
          }
          for (int pp = 0; pp < NPB; ++pp) {
            const int64_t kp = k_lo + static_cast<int64_t>(b) * BK + pp * KSTEP + q4 * P;
            const bool ok = row_ok && kp < k_hi;
            row_piece("shrink x", tok, addr::reg_x_elem(ok, kp, k_lo), P, H);
          }
        }
        for (int c = 0; c < COLS / 16; ++c) {
          const int col = col0 + 16 * c + i16;
          if (col >= ncols) continue;
          for (int e = 0; e < 4; ++e) {
            const int row = 16 * wave + 4 * q4 + e;
            if (row >= tr.nrows) continue;
            const int64_t slot = tr.slot0 + row;
            if (pl.KS == 1) in("shrink z", slot * ldz + col, 1, z_elems);
            else in("shrink partials", ks * T * pl.zw + slot * pl.zw + col, 1, part_elems);
          }
        }
      }
    });
  }

  // ---- reduce_parts_kernel ---------------------------------------------------
  void reduce(const ShrinkPlan& pl, RankWindow rw, int64_t ldz, int64_t z_elems, int64_t part_elems) {
    const int64_t n8 = T * pl.zw / 8;
    const int64_t blocks = (n8 + kThreads - 1) / kThreads;
    for (int64_t e = 0; e < blocks * kThreads; ++e) {
      const int64_t e8 = e * 8, slot = e8 / pl.zw;
      const int col = static_cast<int>(e8 % pl.zw);
      if (!in("reduce seg", NA, 1, NA + 1) || slot >= seg[NA]) continue;
      int glo = 1, ghi = NA;
      while (glo < ghi) {
        const int mid = (glo + ghi) >> 1;
        if (seg[mid] > slot) ghi = mid;
        else glo = mid + 1;
      }
      if (!in_window(rw, ranks[glo])) continue;
      for (int ks = 0; ks < pl.KS; ++ks) in("reduce partials", ks * T * pl.zw + slot * pl.zw + col, 8, part_elems);
      in("reduce z", slot * ldz + col, 8, z_elems);
    }
  }

  // ---- expand_kernel and expand_sparse_kernel --------------------------------
  // z source: partials [nparts][T][zw] (nparts > 0), else z [z_rows, ldz]
  // by slot or by token (z_by_token), columns from z_off[g].
  // qb: 32-column blocks of a sparse item (the pair expand's are narrower);
  // claimed: the items are taken from a counter (each exactly once) instead
  // of by a grid.
  void expand(const ExpandParams& e, const ExpandForm& f, int adapters, int64_t wt, int64_t z_elems,
              int64_t part_elems, const int32_t* z_off, int qb = kSpNT / 32, bool claimed = false) {
    const bool flat = e.flat != 0;
    const int max_tiles = max_tiles_for(T, adapters);
    const std::vector<TileRef> tl = tiles<kTM, kExpandBalanced>(e.rw, b_off);
    const int total = static_cast<int>(tl.size());
    int nparts = e.nparts;
    if (flat && e.ks_target > 0) {
      const int ks = dyn_ksplit(static_cast<int>(tiles<kTMS, false>(e.rw, a_off).size()), e.ks_chunks, e.ks_target,
                                e.nparts);
      nparts = ks > 1 ? ks : 0;
    }
    const int ES = es(), EPL = 16 / ES;
    auto stage = [&](const TileRef& tr, int s_lo, int s_hi, int col_base_of_slice0, int64_t zs_ld, int64_t lds,
                     int nparts) {
      const int r = tr.rank, zo = z_off ? z_off[tr.g] : 0;
      const int per_row = ((s_hi - s_lo + 1) * r) >> 2;
      for (int it = 0; it < kTM * per_row; ++it) {
        const int row = addr::stage_row(it, per_row);
        const int c4 = addr::stage_col(it, row, per_row, col_base_of_slice0);
        in("expand staged shrink values", (row * zs_ld + c4) * ES, 4 * ES, lds);
        if (row >= tr.nrows) continue;
        const int64_t slot = tr.slot0 + row;
        const int zc = c4 + (s_lo * r - col_base_of_slice0);   // the value's column in the adapter's S*r
        if (nparts > 0) {
          in("expand partial column", zc, 4, e.zw);
          for (int ks = 0; ks < nparts; ++ks) in("expand partials", ks * e.part_stride + slot * e.zw + zc, 4, part_elems);
        } else {
          const int64_t zrow = e.z_by_token ? token_at(slot) : slot;
          in("expand z column", zo + zc, 4, e.ldz);
          in("expand z", zrow * e.ldz + zo + zc, 4, z_elems);
        }
      }
    };
    if (f.sparse) {
      const int NTC = 32 * qb;
      const int64_t n_sub = out_total / NTC;
      const int64_t zs_ld = e.max_rank + 8, lds = kTM * zs_ld * 2;
      const int LPR = NTC / 8, RPI = kThreads / LPR, PASSES = kTM / RPI;
      const int items = work_items(total, static_cast<int>(n_sub), true);
      for_items(claimed ? "expand_pair_kernel (claimed items)" : "expand_sparse_kernel",
                claimed ? items : sparse_grid(wt, max_tiles, n_sub), true, items, [&](int lin) {
        const XcdItem it = work_item(lin, total, static_cast<int>(n_sub), true);
        if (it.tile < 0) return;
        const TileRef& tr = tl[it.tile];
        const int r = tr.rank, n_tile0 = it.sub * NTC;
        int s = 0;
        while (s + 1 < si.S && n_tile0 >= si.bounds[s + 1]) ++s;
        in("sparse sub-tile inside its slice", n_tile0 - si.bounds[s], NTC, si.bounds[s + 1] - si.bounds[s]);
        for (int wave = 0; wave < 4; ++wave)
          for (int l = 0; l < 64; ++l) {
            const int i = l & 31, h = l >> 5;
            for (int q = 0; q < qb; ++q) {
              const int64_t n = n_tile0 + 32 * q + i;
              in("sparse lora_B column", n, 1, out_total);
              for (int kg = 0; kg < f.KG; ++kg) {
                const int k0 = (wave * f.KG + kg) * 16 + 8 * h;
                pack_piece("sparse lora_B", tr.off, out_total, r, tr.off + n * r + addr::k_or_zero(k0, r), 8, b_elems);
                in("sparse staged read", (static_cast<int64_t>(i) * zs_ld + addr::k_or_zero(k0, r)) * 2, 16, lds);
              }
            }
          }
        for (int tid = 0; tid < kThreads; ++tid)
          for (int ps = 0; ps < PASSES; ++ps) {
            const int row = ps * RPI + tid / LPR, cx = (tid % LPR) * 8;
            const int tok = token_at(tr.slot0 + addr::tile_row(row, tr.nrows));
            row_piece("sparse y", tok, n_tile0 + cx, 8, out_total);
          }
        if (nparts > 0) {
          stage(tr, s, s, 0, zs_ld, lds, nparts);
        } else {
          // every piece of the 2 KG per thread loaded (rows past the tile
          // and pieces past the rank read clamped addresses), then stored
          const int per_row = r >> 2, ZIT = 2 * f.KG, zo = z_off ? z_off[tr.g] : 0;
          for (int tid = 0; tid < kThreads; ++tid)
            for (int j = 0; j < ZIT; ++j) {
              const int it = tid + j * kThreads;
              const int row = addr::stage_row(it, per_row);
              const int64_t slot = tr.slot0 + addr::tile_row(row, tr.nrows);
              const int64_t zrow = e.z_by_token ? token_at(slot) : slot;
              const int c4 = it < kTM * per_row ? addr::stage_col(it, row, per_row, 0) : 0;
              in("sparse z column", zo + s * r + c4, 4, e.ldz);
              in("sparse z", zrow * e.ldz + zo + s * r + c4, 4, z_elems);
              if (it < kTM * per_row) in("sparse staged z", (row * zs_ld + c4) * 2, 8, lds);
            }
        }
      });
      return;
    }
    const int NT = 4 * f.NBW * 32, n_sub = (out_total + NT - 1) / NT;
    const int KSTEP = bf16 ? 16 : 8, KHALF = KSTEP / 2;
    const int LPR = NT / EPL, RPI = kThreads / LPR, PASSES = kTM / RPI;
    const int64_t zs_ld = static_cast<int64_t>(si.S) * e.max_rank + 8, lds = kTM * zs_ld * ES;
    const int groups = flat ? n_sub : expand_groups(total, n_sub, static_cast<int>(wt));
    for_items("expand_kernel", expand_grid(wt, max_tiles, n_sub, flat), flat, work_items(total, groups, flat),
              [&](int lin) {
      const XcdItem it = work_item(lin, total, groups, flat);
      if (it.tile < 0) return;
      const TileRef& tr = tl[it.tile];
      const int r = tr.rank;
      const int sub0 = (it.sub * n_sub) / groups, nsub = ((it.sub + 1) * n_sub) / groups - sub0;
      if (nsub <= 0) return;
      const int nchunk = (r + f.PRE * KSTEP - 1) / (f.PRE * KSTEP);
      for (int sb = sub0; sb < sub0 + nsub; ++sb) {
        for (int wave = 0; wave < 4; ++wave)
          for (int l = 0; l < 64; ++l) {
            const int i = l & 31, h = l >> 5;
            for (int q = 0; q < f.NBW; ++q) {
              const int n0 = sb * NT + 32 * (wave * f.NBW + q);
              const int n = addr::b_col(n0 + i, out_total);
              int s = 0;
              while (s + 1 < si.S && n0 >= si.bounds[s + 1]) ++s;
              for (int kc = 0; kc < nchunk; ++kc)
                for (int st = 0; st < f.PRE; ++st) {
                  const int k0 = (kc * f.PRE + st) * KSTEP + KHALF * h;
                  pack_piece("expand lora_B", tr.off, out_total, r,
                             tr.off + static_cast<int64_t>(n) * r + addr::k_or_zero(k0, r), EPL, b_elems);
                  in("expand staged read", (i * zs_ld + s * r + addr::k_or_zero(k0, r)) * ES, 16, lds);
                }
            }
          }
        for (int tid = 0; tid < kThreads; ++tid)
          for (int ps = 0; ps < PASSES; ++ps) {
            const int row = ps * RPI + tid / LPR, cx = (tid % LPR) * EPL;
            const int tok = token_at(tr.slot0 + addr::tile_row(row, tr.nrows));
            row_piece("expand y", tok, addr::y_col(sb, NT, cx, out_total, EPL), EPL, out_total);
          }
      }
      int s_lo = 0, s_hi = 0;
      const int c_first = sub0 * NT, c_last = std::min((sub0 + nsub) * NT, out_total) - 1;
      while (s_lo + 1 < si.S && c_first >= si.bounds[s_lo + 1]) ++s_lo;
      s_hi = s_lo;
      while (s_hi + 1 < si.S && c_last >= si.bounds[s_hi + 1]) ++s_hi;
      stage(tr, s_lo, s_hi, s_lo * r, zs_ld, lds, nparts);
    });
  }
};
}  // namespace

// ----------------------------------------------------------------------------
// The allocation-free variant's scratch: one static device array per GPU (each
// device holds its own copy at its own address), used for the split-K
// partials and z.  Host code never passes the array's name to a kernel -- on
// the host that name is only a stand-in -- but the device address that
// hipGetSymbolAddress returns for the current device, looked up once per
// device and kept.  Nothing in it needs to start at zero: every call writes
// the partials (or z) before its expand reads them.  Calls that overlap in
// time on one GPU share the array and race.
// ----------------------------------------------------------------------------
namespace {

constexpr int64_t kNoallocScratchBytes = GS_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kNoallocScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<char*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

int noalloc_scratch(const char* who, char** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("%s: no current HIP device (got %d)", who, dev);
    return GS_ERR_HIP;
  }
  char* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      void* addr = nullptr;
      const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || addr == nullptr) {
        set_error("%s: hipGetSymbolAddress of the static scratch failed on device %d: %s", who, dev,
                  hipGetErrorString(e));
        return GS_ERR_HIP;
      }
      p = static_cast<char*>(addr);
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return GS_OK;
}

// Shrink, then the expand reading its output, once per rank class (shared by
// gs_switched_lora and gs_switched_lora_noalloc, which differ only in where z
// and the partials live).  The classes run one after the other on the stream,
// so they share z and the workspace.
// Side stream and fork / join events of a device, on which the large rank
// class of a two-class module runs beside the small one (created on the
// first such call; default priority, non-blocking).  The mutex makes a call's
// record / wait / launch sequence atomic against other host threads.
struct ForkState {
  std::mutex mu;
  hipStream_t side = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  bool failed = false;
};
ForkState g_fork[kMaxDevices];

// nullptr (the classes then run in turn) when `stream` belongs to another
// device than the current one: the side stream is the current device's, and
// its kernels must run where the call's memory is.
ForkState* fork_state(hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess || sdev != dev) {
      (void)hipGetLastError();
      return nullptr;
    }
  }
  ForkState& f = g_fork[dev];
  std::lock_guard<std::mutex> lock(f.mu);
  if (f.side == nullptr && !f.failed) {
    if (hipStreamCreateWithFlags(&f.side, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&f.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&f.join, hipEventDisableTiming) != hipSuccess) {
      f.failed = true;
      (void)hipGetLastError();
    }
  }
  return f.failed ? nullptr : &f;
}

constexpr int64_t align256(int64_t b) { return (b + 255) & ~int64_t(255); }

// Workspace bytes of each rank class's partials and where they start when
// the classes run concurrently (side by side) or one after the other (both
// at 0).
struct ClassLayout {
  int64_t off[2] = {0, 0};
  int64_t bytes = 0;       // the span the call uses
  bool concurrent = false;
  int64_t claim = -1;      // byte offset of the pair launches' item counter (-1: no room for it)
};
// Two classes side by side: class 0's partials, class 1's from the next
// 256-byte boundary, then one 256-byte line holding the pair expand's item
// counter (what gs_shrink_workspace_bytes reports).  Without room for the
// counter but with room for both partials, the classes can still run
// concurrently on two streams.
ClassLayout class_layout(int64_t T, int H, int S, const RankClass* cls, int ncls, bool bf16, int64_t max_part_bytes,
                         bool want_concurrent, int64_t workspace_bytes) {
  ClassLayout L;
  int64_t part[2] = {0, 0};
  for (int c = 0; c < ncls; ++c) part[c] = plan_class(T, H, S, cls[c], bf16, max_part_bytes).part_bytes;
  L.bytes = ncls == 2 ? std::max(part[0], part[1]) : part[0];
  if (ncls == 2 && want_concurrent) {
    const int64_t both = part[0] == 0 ? part[1] : align256(part[0]) + part[1];
    const int64_t claim = align256(both);
    if (claim + 256 <= workspace_bytes) {
      L.concurrent = true;
      L.off[1] = part[0] == 0 ? 0 : align256(part[0]);
      L.claim = claim;
      L.bytes = claim + 256;
    } else if (both <= workspace_bytes || both == 0) {
      L.concurrent = true;
      L.off[1] = part[0] == 0 ? 0 : align256(part[0]);
      L.bytes = both;
    }
  }
  return L;
}

// concurrent: a two-class module runs its large class on the device's side
// stream, forked from and joined back into `stream`, when the workspace holds
// both classes' partials (gs_shrink_workspace_bytes); the classes touch
// disjoint y rows, z rows (both at the stride S * max_rank) and workspace
// ranges.  Otherwise (or with concurrent false) the classes run one after
// the other on `stream`, sharing z and the workspace.
int switched_lora_impl(const char* who, int32_t dtype, const void* x, int64_t ldx, void* y, int64_t ldy,
                       int64_t num_tokens, int32_t hidden, int32_t out_total, const int32_t* slice_bounds,
                       int32_t num_slices, const void* a_pack, const int64_t* a_off, const void* b_pack,
                       const int64_t* b_off, const int32_t* ranks, int32_t num_adapters, int32_t max_rank,
                       const int32_t* ranks_host, const int32_t* seg_offsets, const int32_t* perm, void* z,
                       void* workspace, int64_t workspace_bytes, void* stream,
                       int64_t max_part_bytes = INT64_MAX, bool concurrent = false) {
  int rc = check_common(who, dtype, num_tokens, num_slices, num_adapters, max_rank);
  if (rc != GS_OK) return rc;
  rc = check_shrink(dtype, x, ldx, hidden, a_pack);
  if (rc != GS_OK) return rc;
  ExpandParams ep{};
  rc = prepare_expand(ep, who, dtype, y, ldy, num_tokens, out_total, slice_bounds, num_slices, b_pack, b_off, ranks,
                      num_adapters, max_rank, seg_offsets, perm);
  if (rc != GS_OK) return rc;
  GS_CHECK_ARG(aligned16(z), "%s: z must be 16-byte aligned", who);
  RankClass cls[2];
  int ncls = 0;
  rc = rank_classes(who, ranks_host, num_adapters, max_rank, num_tokens, cls, ncls);
  if (rc != GS_OK) return rc;
  if (num_tokens == 0) return GS_OK;
  const bool bf16 = dtype == GS_DTYPE_BF16;
  for (int c = 0; c < ncls; ++c) {
    rc = check_workspace(plan_class(num_tokens, hidden, num_slices, cls[c], bf16, max_part_bytes), workspace,
                         workspace_bytes);
    if (rc != GS_OK) return rc;
  }
  const ClassLayout L = class_layout(num_tokens, hidden, num_slices, cls, ncls, bf16, max_part_bytes, concurrent,
                                     workspace_bytes);
  auto shrink_params = [&](const RankClass& k, const ShrinkPlan& pl, int64_t part_off, int64_t ldz) {
    void* ws = workspace ? static_cast<void*>(static_cast<char*>(workspace) + part_off) : nullptr;
    return make_shrink_params(pl, x, ldx, hidden, a_pack, a_off, ranks, num_slices, num_adapters, seg_offsets, perm, z,
                              ldz, ws, num_tokens, k.rw);
  };
  auto expand_params = [&](const RankClass& k, const ShrinkPlan& pl, const ShrinkParams& sp, int64_t ldz) {
    ExpandParams e = ep;
    e.max_rank = k.max_rank;
    e.rw = k.rw;
    e.flat = pl.flat ? 1 : 0;
    e.ks_target = pl.ks_target;
    e.ks_chunks = pl.n_chunks;
    e.z = z;
    e.ldz = ldz;
    e.z_by_token = 0;
    e.z_off = nullptr;
    e.part = sp.part;
    e.part_stride = sp.part_stride;
    e.zw = sp.zw;
    e.nparts = pl.KS > 1 ? pl.KS : 0;
    return e;
  };
  auto run_class = [&](const RankClass& k, hipStream_t st, int64_t part_off, int64_t ldz) -> int {
    const ShrinkPlan pl = plan_class(num_tokens, hidden, num_slices, k, bf16, max_part_bytes);
    const ShrinkParams sp = shrink_params(k, pl, part_off, ldz);
    launch_shrink(bf16, pl, sp, st);
    GS_CHECK_LAUNCH(who);
    launch_expand(bf16, num_tokens, k.adapters, expand_params(k, pl, sp, ldz), st);
    GS_CHECK_LAUNCH(who);
    return GS_OK;
  };
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (L.claim >= 0) {
    // both classes in the same two launches on `stream` when their forms allow
    const int64_t ldz = static_cast<int64_t>(num_slices) * max_rank;
    const ShrinkPlan pl0 = plan_class(num_tokens, hidden, num_slices, cls[0], bf16, max_part_bytes);
    const ShrinkPlan pl1 = plan_class(num_tokens, hidden, num_slices, cls[1], bf16, max_part_bytes);
    const ShrinkParams sp0 = shrink_params(cls[0], pl0, L.off[0], ldz);
    const ShrinkParams sp1 = shrink_params(cls[1], pl1, L.off[1], ldz);
    ExpandParams e0 = expand_params(cls[0], pl0, sp0, ldz);
    const ExpandParams e1 = expand_params(cls[1], pl1, sp1, ldz);
    const PairForm f = pair_form(bf16, num_tokens, pl0, pl1, e0, e1);
    if (f.ok) {
      int* claim = reinterpret_cast<int*>(static_cast<char*>(workspace) + L.claim);
      const size_t lds = pair_lds_bytes(num_slices, cls[0].max_rank, cls[1].max_rank);
      const int64_t egrid = pair_expand_grid(f, num_tokens, cls[0].adapters, lds, e0);
      launch_shrink_pair(f, pl0.grid, sp0, sp1, claim, st);
      GS_CHECK_LAUNCH(who);
      launch_expand_pair(f, egrid, lds, e0, e1, claim, st);
      GS_CHECK_LAUNCH(who);
      return GS_OK;
    }
  }
  ForkState* fs = L.concurrent ? fork_state(st) : nullptr;
  if (fs == nullptr) {
    for (int c = 0; c < ncls; ++c) {
      rc = run_class(cls[c], st, 0, static_cast<int64_t>(num_slices) * cls[c].max_rank);
      if (rc != GS_OK) return rc;
    }
    return GS_OK;
  }
  // the large class on the side stream once everything before this call on
  // `stream` is done, issued after the small class's kernels (decoder step
  // with one rank-512 adapter 9.23 ms; issued first, 9.29 ms); `stream` waits
  // for it before anything after this call
  const int64_t ldz = static_cast<int64_t>(num_slices) * max_rank;
  std::lock_guard<std::mutex> lock(fs->mu);
  if (hipEventRecord(fs->fork, st) != hipSuccess || hipStreamWaitEvent(fs->side, fs->fork, 0) != hipSuccess) {
    set_error("%s: forking the side stream failed: %s", who, hipGetErrorString(hipGetLastError()));
    return GS_ERR_HIP;
  }
  const int rc0 = run_class(cls[0], st, L.off[0], ldz);
  const int rc1 = run_class(cls[1], fs->side, L.off[1], ldz);
  const hipError_t ej = hipEventRecord(fs->join, fs->side);
  const hipError_t ew = ej == hipSuccess ? hipStreamWaitEvent(st, fs->join, 0) : ej;
  if (rc1 != GS_OK) return rc1;
  if (rc0 != GS_OK) return rc0;
  if (ew != hipSuccess) {
    set_error("%s: joining the side stream failed: %s", who, hipGetErrorString(ew));
    return GS_ERR_HIP;
  }
  return GS_OK;
}

}  // namespace

extern "C" {

int64_t gs_shrink_workspace_bytes(int64_t num_tokens, int32_t hidden, int32_t num_slices, int32_t num_adapters,
                                  int32_t max_rank, const int32_t* ranks_host) {
  if (num_tokens <= 0 || hidden <= 0) return 256;
  RankClass cls[2];
  int ncls = 0;
  if (rank_classes("gs_shrink_workspace_bytes", ranks_host, num_adapters, max_rank, num_tokens, cls, ncls) != GS_OK)
    return -1;
  // both dtypes; two classes side by side (gs_switched_lora runs them
  // concurrently in a workspace that holds both)
  int64_t b = 256;
  for (int bf16 = 0; bf16 < 2; ++bf16)
    b = std::max(b, class_layout(num_tokens, hidden, num_slices, cls, ncls, bf16 != 0, INT64_MAX, true, INT64_MAX).bytes);
  return b;
}

int32_t gs_shrink_ksplits(int32_t dtype, int64_t num_tokens, int32_t hidden, int32_t num_slices, int32_t num_adapters,
                          int32_t max_rank, const int32_t* ranks_host, int32_t* ksplit) {
  int rc = check_common("gs_shrink_ksplits", dtype, num_tokens, num_slices, num_adapters, max_rank);
  if (rc != GS_OK) return -rc;
  GS_CHECK_ARG(hidden > 0 && ksplit != nullptr, "gs_shrink_ksplits: hidden=%d / NULL ksplit", hidden);
  RankClass cls[2];
  int ncls = 0;
  rc = rank_classes("gs_shrink_ksplits", ranks_host, num_adapters, max_rank, num_tokens, cls, ncls);
  if (rc != GS_OK) return -rc;
  for (int c = 0; c < ncls; ++c)
    ksplit[c] = plan_class(num_tokens, hidden, num_slices, cls[c], dtype == GS_DTYPE_BF16, INT64_MAX, false).KS;
  return ncls;
}

int32_t gs_switched_lora_pair(int32_t dtype, int64_t num_tokens, int32_t hidden, int32_t out_total,
                              const int32_t* slice_bounds, int32_t num_slices, int32_t num_adapters, int32_t max_rank,
                              const int32_t* ranks_host) {
  const char* who = "gs_switched_lora_pair";
  int rc = check_common(who, dtype, num_tokens, num_slices, num_adapters, max_rank);
  if (rc != GS_OK) return -rc;
  GS_CHECK_ARG(hidden > 0 && out_total > 0 && slice_bounds != nullptr, "%s: hidden=%d out_total=%d", who, hidden,
               out_total);
  RankClass cls[2];
  int ncls = 0;
  rc = rank_classes(who, ranks_host, num_adapters, max_rank, num_tokens, cls, ncls);
  if (rc != GS_OK) return -rc;
  if (ncls != 2 || num_tokens == 0) return 0;
  SliceInfo si{};
  si.S = num_slices;
  for (int s = 0; s <= num_slices; ++s) si.bounds[s] = slice_bounds[s];
  const bool bf16 = dtype == GS_DTYPE_BF16;
  const int64_t ldz = static_cast<int64_t>(num_slices) * max_rank;
  const ShrinkPlan pl0 = plan_class(num_tokens, hidden, num_slices, cls[0], bf16);
  const ShrinkPlan pl1 = plan_class(num_tokens, hidden, num_slices, cls[1], bf16);
  return pair_form(bf16, num_tokens, pl0, pl1, class_expand_plan(si, out_total, cls[0], pl0, num_tokens, ldz),
                   class_expand_plan(si, out_total, cls[1], pl1, num_tokens, ldz))
                 .ok
             ? 1
             : 0;
}

int gs_shrink(int32_t dtype, const void* x, int64_t ldx, int64_t num_tokens, int32_t hidden, const void* a_pack,
              const int64_t* a_off, const int32_t* ranks, int32_t num_slices, int32_t num_adapters,
              int32_t max_rank, const int32_t* ranks_host, const int32_t* seg_offsets, const int32_t* perm, void* z,
              int64_t ldz, void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_common("gs_shrink", dtype, num_tokens, num_slices, num_adapters, max_rank);
  if (rc != GS_OK) return rc;
  rc = check_shrink(dtype, x, ldx, hidden, a_pack);
  if (rc != GS_OK) return rc;
  const bool bf16 = dtype == GS_DTYPE_BF16;
  GS_CHECK_ARG(z == nullptr || (ldz >= int64_t(num_slices) * max_rank && ldz % 8 == 0 && aligned16(z)),
               "gs_shrink: ldz=%lld / z alignment", (long long)ldz);
  RankClass cls[2];
  int ncls = 0;
  rc = rank_classes("gs_shrink", ranks_host, num_adapters, max_rank, num_tokens, cls, ncls);
  if (rc != GS_OK) return rc;
  if (num_tokens == 0) return GS_OK;
  for (int c = 0; c < ncls; ++c) {
    const ShrinkPlan pl = plan_class(num_tokens, hidden, num_slices, cls[c], bf16, INT64_MAX, false);
    GS_CHECK_ARG(z != nullptr || (pl.KS > 1 && ncls == 1),
                 "gs_shrink: z may be NULL only when the module is one rank class whose hidden dimension is split "
                 "(gs_shrink_ksplits)");
    rc = check_workspace(pl, workspace, workspace_bytes);
    if (rc != GS_OK) return rc;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int c = 0; c < ncls; ++c) {
    const RankClass& k = cls[c];
    const ShrinkPlan pl = plan_class(num_tokens, hidden, num_slices, k, bf16, INT64_MAX, false);
    const ShrinkParams p = make_shrink_params(pl, x, ldx, hidden, a_pack, a_off, ranks, num_slices, num_adapters,
                                              seg_offsets, perm, z, ldz, workspace, num_tokens, k.rw);
    launch_shrink(bf16, pl, p, st);
    GS_CHECK_LAUNCH("gs_shrink");
    if (pl.KS > 1 && z != nullptr) {
      const int64_t n8 = (num_tokens * pl.zw) / 8;
      const unsigned blocks = static_cast<unsigned>((n8 + kThreads - 1) / kThreads);
      if (bf16) hipLaunchKernelGGL(reduce_parts_kernel<true>, dim3(blocks), dim3(kThreads), 0, st, p.part,
                                   p.part_stride, pl.KS, pl.zw, seg_offsets, ranks, k.rw, num_adapters, z, ldz);
      else hipLaunchKernelGGL(reduce_parts_kernel<false>, dim3(blocks), dim3(kThreads), 0, st, p.part, p.part_stride,
                              pl.KS, pl.zw, seg_offsets, ranks, k.rw, num_adapters, z, ldz);
      GS_CHECK_LAUNCH("gs_shrink (reduce)");
    }
  }
  return GS_OK;
}

int gs_expand_add(int32_t dtype, void* y, int64_t ldy, int64_t num_tokens, int32_t out_total,
                  const int32_t* slice_bounds, int32_t num_slices, const void* z, int64_t ldz, int32_t z_by_token,
                  const int32_t* z_off, const void* b_pack, const int64_t* b_off, const int32_t* ranks,
                  int32_t num_adapters, int32_t max_rank, const int32_t* ranks_host, const int32_t* seg_offsets,
                  const int32_t* perm, void* stream) {
  int rc = check_common("gs_expand_add", dtype, num_tokens, num_slices, num_adapters, max_rank);
  if (rc != GS_OK) return rc;
  ExpandParams p{};
  rc = prepare_expand(p, "gs_expand_add", dtype, y, ldy, num_tokens, out_total, slice_bounds, num_slices, b_pack, b_off,
                      ranks, num_adapters, max_rank, seg_offsets, perm);
  if (rc != GS_OK) return rc;
  GS_CHECK_ARG(ldz % 8 == 0 && aligned16(z), "gs_expand_add: ldz=%lld / z alignment", (long long)ldz);
  RankClass cls[2];
  int ncls = 0;
  rc = rank_classes("gs_expand_add", ranks_host, num_adapters, max_rank, num_tokens, cls, ncls);
  if (rc != GS_OK) return rc;
  if (num_tokens == 0) return GS_OK;
  p.z = z;
  p.ldz = ldz;
  p.z_by_token = z_by_token;
  p.z_off = z_off;
  p.nparts = 0;
  for (int c = 0; c < ncls; ++c) {
    ExpandParams e = p;
    e.max_rank = cls[c].max_rank;
    e.rw = cls[c].rw;
    e.flat = sparse_class(cls[c]) ? 1 : 0;
    launch_expand(dtype == GS_DTYPE_BF16, num_tokens, cls[c].adapters, e, static_cast<hipStream_t>(stream));
    GS_CHECK_LAUNCH("gs_expand_add");
  }
  return GS_OK;
}

int gs_switched_lora(int32_t dtype, const void* x, int64_t ldx, void* y, int64_t ldy, int64_t num_tokens,
                     int32_t hidden, int32_t out_total, const int32_t* slice_bounds, int32_t num_slices,
                     const void* a_pack, const int64_t* a_off, const void* b_pack, const int64_t* b_off,
                     const int32_t* ranks, int32_t num_adapters, int32_t max_rank, const int32_t* ranks_host,
                     const int32_t* seg_offsets, const int32_t* perm, void* z, void* workspace,
                     int64_t workspace_bytes, void* stream) {
  return switched_lora_impl("gs_switched_lora", dtype, x, ldx, y, ldy, num_tokens, hidden, out_total, slice_bounds,
                            num_slices, a_pack, a_off, b_pack, b_off, ranks, num_adapters, max_rank, ranks_host,
                            seg_offsets, perm, z, workspace, workspace_bytes, stream, INT64_MAX, true);
}

int gs_switched_lora_noalloc(int32_t dtype, const void* x, int64_t ldx, void* y, int64_t ldy, int64_t num_tokens,
                             int32_t hidden, int32_t out_total, const int32_t* slice_bounds, int32_t num_slices,
                             const void* a_pack, const int64_t* a_off, const void* b_pack, const int64_t* b_off,
                             const int32_t* ranks, int32_t num_adapters, int32_t max_rank, const int32_t* ranks_host,
                             const int32_t* seg_offsets, const int32_t* perm, void* stream) {
  const char* who = "gs_switched_lora_noalloc";
  int rc = check_common(who, dtype, num_tokens, num_slices, num_adapters, max_rank);
  if (rc != GS_OK) return rc;
  GS_CHECK_ARG(hidden > 0, "%s: hidden=%d", who, hidden);
  RankClass cls[2];
  int ncls = 0;
  rc = rank_classes(who, ranks_host, num_adapters, max_rank, num_tokens, cls, ncls);
  if (rc != GS_OK) return rc;
  if (num_tokens == 0 || ncls == 0) return GS_OK;
  // scratch layout: [split-K partials][z], each 256-byte aligned; the rank
  // classes run one after the other and share both
  int64_t part_need = 0, zrank = 0;
  for (int c = 0; c < ncls; ++c) zrank = std::max<int64_t>(zrank, cls[c].max_rank);
  const int64_t zbytes = num_tokens * int64_t(num_slices) * zrank * (dtype == GS_DTYPE_BF16 ? 2 : 4);
  // a k-split chosen on the device is capped by what the array holds beside z
  const int64_t part_budget = std::max<int64_t>(0, (kNoallocScratchBytes - zbytes) & ~int64_t(255));
  for (int c = 0; c < ncls; ++c) {
    const ShrinkPlan pl = plan_class(num_tokens, hidden, num_slices, cls[c], dtype == GS_DTYPE_BF16, part_budget);
    part_need = std::max(part_need, pl.part_bytes);
  }
  const int64_t part = (part_need + 255) & ~int64_t(255);
  if (part + zbytes > kNoallocScratchBytes) {
    set_error("%s: this shape needs %lld bytes of scratch (split-K partials %lld + z %lld); the static scratch "
              "holds %lld (use gs_switched_lora with a caller workspace)", who, (long long)(part + zbytes),
              (long long)part_need, (long long)zbytes, (long long)kNoallocScratchBytes);
    return GS_ERR_WORKSPACE;
  }
  char* base = nullptr;
  rc = noalloc_scratch(who, &base);
  if (rc != GS_OK) return rc;
  return switched_lora_impl(who, dtype, x, ldx, y, ldy, num_tokens, hidden, out_total, slice_bounds, num_slices,
                            a_pack, a_off, b_pack, b_off, ranks, num_adapters, max_rank, ranks_host, seg_offsets, perm,
                            base + part, base, part, stream, part_budget);
}

int64_t gs_check_segment_addresses(int32_t dtype, int64_t num_tokens, int32_t hidden, int64_t ldx, int32_t out_total,
                                   int64_t ldy, const int32_t* slice_bounds, int32_t num_slices, const int64_t* a_off,
                                   int64_t a_pack_elems, const int64_t* b_off, int64_t b_pack_elems,
                                   const int32_t* ranks, int32_t num_adapters, int32_t max_rank,
                                   const int32_t* seg_offsets, const int32_t* perm, const int32_t* z_off,
                                   int64_t z_ld, char* msg, int64_t msg_len, int64_t* checked) {
  const char* who = "gs_check_segment_addresses";
  int rc = check_common(who, dtype, num_tokens, num_slices, num_adapters, max_rank);
  if (rc != GS_OK) return -rc;
  GS_CHECK_ARG(hidden > 0 && ldx >= hidden && out_total > 0 && ldy >= out_total, "%s: shape", who);
  GS_CHECK_ARG(slice_bounds && a_off && b_off && ranks && seg_offsets && (perm || num_tokens == 0), "%s: NULL table",
               who);
  const bool bf16 = dtype == GS_DTYPE_BF16;
  AddrModel m{};
  m.bf16 = bf16;
  m.T = num_tokens;
  m.H = hidden;
  m.ldx = ldx;
  m.out_total = out_total;
  m.ldy = ldy;
  m.si.S = num_slices;
  for (int s = 0; s <= num_slices; ++s) m.si.bounds[s] = slice_bounds[s];
  m.ranks = ranks;
  m.a_off = a_off;
  m.b_off = b_off;
  m.a_elems = a_pack_elems;
  m.b_elems = b_pack_elems;
  m.NA = num_adapters;
  m.max_rank = max_rank;
  m.seg = seg_offsets;
  m.perm = perm;
  m.perm_len = num_tokens > 0 ? num_tokens : 1;
  RankClass cls[2];
  int ncls = 0;
  rc = rank_classes(who, ranks, num_adapters, max_rank, num_tokens, cls, ncls);
  if (rc != GS_OK) return -rc;
  const int64_t T = num_tokens;
  const int cus = device_cus();
  const int64_t z_elems = std::max<int64_t>(T, 1) * num_slices * max_rank;   // z as switched.py allocates it
  const int64_t ws_elems = gs_shrink_workspace_bytes(T, hidden, num_slices, num_adapters, max_rank, ranks) / 4;
  if (T > 0) {
    // gs_switched_lora (caller workspace) and gs_switched_lora_noalloc (the
    // static array: the partial budget left beside z)
    for (int noalloc = 0; noalloc < 2; ++noalloc) {
      int64_t budget = INT64_MAX, zrank = 0;
      for (int c = 0; c < ncls; ++c) zrank = std::max<int64_t>(zrank, cls[c].max_rank);
      const int64_t zbytes = T * int64_t(num_slices) * zrank * (bf16 ? 2 : 4);
      if (noalloc) {
        budget = std::max<int64_t>(0, (kNoallocScratchBytes - zbytes) & ~int64_t(255));
        int64_t part = 0;
        for (int c = 0; c < ncls; ++c)
          part = std::max(part, plan_class(T, hidden, num_slices, cls[c], bf16, budget).part_bytes);
        if (((part + 255) & ~int64_t(255)) + zbytes > kNoallocScratchBytes) continue;   // rejected by the call
      }
      // gs_switched_lora runs two classes concurrently, their partials side
      // by side (each checked against its own range) and z at one stride
      const ClassLayout L = class_layout(T, hidden, num_slices, cls, ncls, bf16, budget, !noalloc, ws_elems * 4);
      if (L.claim >= 0) {
        // both classes in the pair launches when their forms allow
        const int64_t zl = static_cast<int64_t>(num_slices) * max_rank;
        const ShrinkPlan pl0 = plan_class(T, hidden, num_slices, cls[0], bf16, budget);
        const ShrinkPlan pl1 = plan_class(T, hidden, num_slices, cls[1], bf16, budget);
        const ExpandParams e0 = class_expand_plan(m.si, out_total, cls[0], pl0, T, zl);
        const ExpandParams e1 = class_expand_plan(m.si, out_total, cls[1], pl1, T, zl);
        const PairForm pf = pair_form(bf16, T, pl0, pl1, e0, e1);
        if (pf.ok) {
          m.in("pair item counter", L.claim / 4, 1, ws_elems);
          const int64_t part0 = L.off[1] > 0 ? L.off[1] / 4 : ws_elems, part1 = L.claim / 4 - L.off[1] / 4;
          m.shrink_dma(pl0, cls[0].rw, zl, z_elems, part0);
          m.shrink_dma(pl1, cls[1].rw, zl, z_elems, part1, pl0.grid, 1);
          for (int occ = 1; occ <= 4; ++occ)
            m.expand(e0, pf.f0, cls[0].adapters, int64_t(occ) * cus, z_elems, part0, nullptr);
          const ExpandForm f1{true, 1, 2, pf.KG1};
          m.expand(e1, f1, cls[1].adapters, cus, z_elems, part1, nullptr, kPairQB, true);
          continue;
        }
      }
      for (int c = 0; c < ncls; ++c) {
        const RankClass& k = cls[c];
        const ShrinkPlan pl = plan_class(T, hidden, num_slices, k, bf16, budget);
        const int64_t part_hi = noalloc ? budget / 4 : (L.concurrent && c == 0 && L.off[1] > 0 ? L.off[1] / 4 : ws_elems);
        const int64_t part_elems = part_hi - L.off[c] / 4;
        const int64_t zl = static_cast<int64_t>(num_slices) * (L.concurrent ? max_rank : k.max_rank);
        const int64_t zel = noalloc ? zbytes / (bf16 ? 2 : 4) : z_elems;
        if (pl.part_bytes / 4 > part_elems) m.fail("%s: partials of %lld bytes exceed the workspace", who,
                                                   (long long)pl.part_bytes);
        if (pl.dma) m.shrink_dma(pl, k.rw, zl, zel, part_elems);
        else m.shrink_reg(pl, k.rw, zl, zel, part_elems);
        ExpandParams e{};
        e.out_total = out_total;
        e.si = m.si;
        e.ldz = zl;
        e.part_stride = T * pl.zw;
        e.zw = pl.zw;
        e.nparts = pl.KS > 1 ? pl.KS : 0;
        e.max_rank = k.max_rank;
        e.rw = k.rw;
        e.flat = pl.flat ? 1 : 0;
        e.ks_target = pl.ks_target;
        e.ks_chunks = pl.n_chunks;
        const ExpandForm f = expand_form(bf16, T, e);
        for (int occ = 1; occ <= 4; ++occ) m.expand(e, f, k.adapters, int64_t(occ) * cus, zel, part_elems, nullptr);
      }
    }
    // gs_shrink writing z (reduced when split), then gs_expand_add from it;
    // and, when z_off is given, gs_expand_add reading its shrink values by
    // token from a [T, z_ld] matrix (the vLLM layer's x_ext columns)
    for (int c = 0; c < ncls; ++c) {
      const RankClass& k = cls[c];
      const ShrinkPlan pl = plan_class(T, hidden, num_slices, k, bf16, INT64_MAX, false);
      const int64_t zl = static_cast<int64_t>(num_slices) * max_rank;
      if (pl.dma) m.shrink_dma(pl, k.rw, zl, z_elems, ws_elems);
      else m.shrink_reg(pl, k.rw, zl, z_elems, ws_elems);
      if (pl.KS > 1) m.reduce(pl, k.rw, zl, z_elems, ws_elems);
      for (int by_token = 0; by_token < (z_off ? 2 : 1); ++by_token) {
        ExpandParams e{};
        e.out_total = out_total;
        e.si = m.si;
        e.ldz = by_token ? z_ld : zl;
        e.z_by_token = by_token;
        e.max_rank = k.max_rank;
        e.rw = k.rw;
        e.flat = sparse_class(k) ? 1 : 0;
        const ExpandForm f = expand_form(bf16, T, e);
        for (int occ = 1; occ <= 4; ++occ)
          m.expand(e, f, k.adapters, int64_t(occ) * cus, by_token ? T * z_ld : z_elems, 0, by_token ? z_off : nullptr);
      }
    }
  }
  if (checked) *checked = m.checked;
  if (msg && msg_len > 0) snprintf(msg, static_cast<size_t>(msg_len), "%s", m.msg);
  return m.bad;
}

}  // extern "C"
