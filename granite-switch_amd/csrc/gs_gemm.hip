// Dense bf16 GEMM C[M,N] = A[M,K] . B[N,K]^T for gfx950 -- the one GEMM of
// the reference's vLLM layer, x_ext = x . w_ext^T, where w_ext stacks the
// base weight and every adapter's lora_A rows, so one pass gives the base
// output and every shrink (src/granite_switch/vllm/core/lora.py:544;
// src/granite_switch/kernels/switch_lora_kernel.py:134-163).
//
// Both operands are K-contiguous rows, the layout MFMA reads directly.  A
// workgroup of 8 waves owns a 256 x 256 tile of C; wave (wm, wn) of the 2 x 4
// wave grid owns 128 x 64 of it as 4 x 2 blocks of v_mfma_f32_32x32x16_bf16,
// accumulated in fp32.  K is walked in tiles of 64 through two LDS stages
// (one barrier per k-tile).  The 256 x 256 tile gives 128 FLOP per byte moved
// from the L2 into the CU.  Tiles are numbered in groups of 8 tile rows
// (consecutive workgroups share B columns and A rows in the L2), and each XCD
// takes a contiguous range of that order, so the tiles running together on
// one XCD share its L2.  Partial tiles clamp their loads to the last row and
// mask their stores.
//
// Two kernels: for K % 64 == 0 the k-tiles go from global memory straight
// into LDS (gemm_bf16_tn_dma_kernel); otherwise they are loaded into
// registers, zero-filled past K, and written to padded LDS rows
// (gemm_bf16_tn_kernel).
#include <stdarg.h>

#include <algorithm>
#include <vector>

#include "gs_addr.h"
#include "gs_common.h"

namespace gs {

namespace {

constexpr int kGBM = 256;                       // C rows per workgroup
constexpr int kGBN = 256;                       // C columns per workgroup
constexpr int kGBK = 64;                        // k per tile
constexpr int kGRowBytes = kGBK * 2;            // bytes of one operand row per k-tile
constexpr int kGLd = kGRowBytes + 16;           // padded LDS row stride
constexpr int kGStage = (kGBM + kGBN) * kGLd;   // one k-tile of A and B in LDS
constexpr int kGLds = 2 * kGStage;              // double-buffered
constexpr int kGGroup = 8;                      // tile rows per group of the tile order
static_assert(kGBM == kGBN, "A and B tiles are staged with the same thread mapping");

struct GemmParams {
  const char* a;
  int64_t lda;            // elements
  const char* b;
  int64_t ldb;
  uint16_t* c;
  int64_t ldc;
  int M, N, K;
  int tiles_m, tiles_n;
};

// WM x WN waves; wave (wm, wn) owns rows wm*(256/WM) and columns wn*(256/WN)
// of the tile as MI x NJ blocks of 32 x 32.
template <bool KTAIL, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_bf16_tn_kernel(GemmParams p) {
  constexpr int kGThreads = 64 * WM * WN;
  constexpr int kGPieces = kGBM * (kGRowBytes / 16) / kGThreads;   // 16-byte pieces per thread and operand
  constexpr int kGRowStep = kGThreads / (kGRowBytes / 16);         // rows between a thread's pieces
  constexpr int MI = kGBM / WM / 32;
  constexpr int NJ = kGBN / WN / 32;
  extern __shared__ __align__(16) char smem[];

  // tile of this workgroup: XCD x = id % 8 takes tiles [x*per, (x+1)*per)
  int tm, tn;
  if (!addr::gemm_tile(static_cast<int>(blockIdx.x), p.tiles_m, p.tiles_n, kGGroup, tm, tn)) return;

  const int tid = threadIdx.x;
  // global -> LDS mapping: 8 consecutive threads move one row's 128 bytes
  const int lrow = tid >> 3;
  const int lpc = (tid & 7) * 16;
  const int kp = (tid & 7) * 8;                 // this thread's k within a tile
  const char* ga[kGPieces];
  const char* gb[kGPieces];
#pragma unroll
  for (int j = 0; j < kGPieces; ++j) {
    const int ra = addr::gemm_row(tm * kGBM + lrow + j * kGRowStep, p.M);
    const int rb = addr::gemm_row(tn * kGBN + lrow + j * kGRowStep, p.N);
    ga[j] = p.a + static_cast<int64_t>(ra) * p.lda * 2;
    gb[j] = p.b + static_cast<int64_t>(rb) * p.ldb * 2;
  }
  u32x4 va[kGPieces], vb[kGPieces];
  // loads from clamped in-bounds addresses, masked afterwards (K % 8 == 0, so
  // a 16-byte piece is entirely inside or entirely past K; a piece past K
  // re-reads the row's first 16 bytes)
  auto gload = [&](int kt) {
    const bool ok = !KTAIL || kt * kGBK + kp < p.K;
    const int64_t off = ok ? static_cast<int64_t>(kt) * kGRowBytes + lpc : 0;
#pragma unroll
    for (int j = 0; j < kGPieces; ++j) {
      va[j] = ld16(ga[j] + off);
      vb[j] = ld16(gb[j] + off);
    }
    if constexpr (KTAIL) {
#pragma unroll
      for (int j = 0; j < kGPieces; ++j) {
        va[j] = sel16(ok, va[j]);
        vb[j] = sel16(ok, vb[j]);
      }
    }
  };
  auto sstore = [&](int buf) {
    char* sa = smem + buf * kGStage;
    char* sb = sa + kGBM * kGLd;
#pragma unroll
    for (int j = 0; j < kGPieces; ++j) {
      st16(sa + (lrow + j * kGRowStep) * kGLd + lpc, va[j]);
      st16(sb + (lrow + j * kGRowStep) * kGLd + lpc, vb[j]);
    }
  };

  const int wave = tid >> 6;
  const int l = tid & 63;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int i32 = l & 31;
  const int h = l >> 5;
  f32x16 acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x16{};

  // MFMA operands: lane l reads row (l % 32) of a 32-row block, k 8*(l/32) .. +7
  // of each 16-k step
  auto compute = [&](int buf) {
    const char* sa = smem + buf * kGStage + (wm * MI * 32 + i32) * kGLd + h * 16;
    const char* sb = smem + buf * kGStage + kGBM * kGLd + (wn * NJ * 32 + i32) * kGLd + h * 16;
#pragma unroll
    for (int kk = 0; kk < kGBK / 16; ++kk) {
      u32x4 af[MI], bf[NJ];
#pragma unroll
      for (int i = 0; i < MI; ++i) af[i] = *reinterpret_cast<const u32x4*>(sa + i * 32 * kGLd + kk * 32);
#pragma unroll
      for (int j = 0; j < NJ; ++j) bf[j] = *reinterpret_cast<const u32x4*>(sb + j * 32 * kGLd + kk * 32);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = mfma32_bf16(af[i], bf[j], acc[i][j]);
    }
  };

  const int nk = (p.K + kGBK - 1) / kGBK;
  gload(0);
  sstore(0);
  lds_barrier();
  for (int kt = 0; kt < nk; ++kt) {
    // the next tile's loads go out before this tile's MFMAs (the scheduling
    // barrier keeps them there); the last iteration re-reads its own tile into
    // the idle buffer
    gload(min(kt + 1, nk - 1));
    __builtin_amdgcn_sched_barrier(0);
    compute(kt & 1);
    sstore((kt + 1) & 1);
    lds_barrier();
  }

  // lane (i32, h) holds column i32 and rows mfma32_row(v, l) of each 32 x 32 block
  const int row0 = tm * kGBM + wm * MI * 32;
  const int col0 = tn * kGBN + wn * NJ * 32 + i32;
#pragma unroll
  for (int i = 0; i < MI; ++i) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = col0 + j * 32;
      if (col >= p.N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = row0 + i * 32 + mfma32_row(v, l);
        if (row < p.M) p.c[static_cast<int64_t>(row) * p.ldc + col] = f32_to_bf16_bits(acc[i][j][v]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Direct-to-LDS variant (K % 64 == 0): the same 256 x 256 tile, wave grid and
// two-stage LDS ring, but the k-tiles travel from global memory straight into
// LDS with global_load_lds_dwordx4 -- no staging registers and no LDS writes
// by the waves.  A wave-wide transfer moves 1 KB: 8 rows x 128 bytes, so
// every request is one whole cache line (transfers of half lines doubled the
// L2 request count).  Each wave moves 32 rows of each operand per k-tile.  A
// transfer fills LDS contiguously, so bank spreading comes from an XOR
// swizzle instead of padding: the 16-byte piece p of row r sits at position
// p ^ addr::lds_swz(r), which puts the operand reads of 16 consecutive rows at
// one k (the lanes a 128-bit LDS read serves together) in distinct banks.
// The next k-tile's transfers are issued before the current tile's MFMAs;
// the waits are explicit (the transfers are written as assembly, so the
// compiler does not wait for them before every LDS read).
// ---------------------------------------------------------------------------
constexpr int kDBK = 64;                        // k per tile
constexpr int kDRow = kDBK * 2;                 // bytes of one operand row per tile (one cache line)
constexpr int kDOp = kGBM * kDRow;              // one operand of one stage

template <int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_bf16_tn_dma_kernel(GemmParams p) {
  constexpr int NW = WM * WN;
  constexpr int RPW = kGBM / NW;                // rows of each operand one wave moves per k-tile
  constexpr int TPO = RPW / 8;                  // its 1 KB transfers per operand
  static_assert(RPW % 8 == 0 && kGBM == kGBN, "waves move whole 8-row transfers");
  constexpr int MI = kGBM / WM / 32;
  constexpr int NJ = kGBN / WN / 32;
  __shared__ __align__(16) char sA0[kDOp], sB0[kDOp], sA1[kDOp], sB1[kDOp];

  int tm, tn;
  if (!addr::gemm_tile(static_cast<int>(blockIdx.x), p.tiles_m, p.tiles_n, kGGroup, tm, tn)) return;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  // transfer i of this wave: LDS row RPW*wave + 8*i + l/8, position l % 8,
  // which holds global piece (l % 8) ^ lds_swz(row) of that row
  const char* da[TPO];
  const char* db[TPO];
#pragma unroll
  for (int i = 0; i < TPO; ++i) {
    const int r = RPW * wave + 8 * i + (l >> 3);
    const int piece = addr::gemm_piece(l, r);
    da[i] = p.a + static_cast<int64_t>(addr::gemm_row(tm * kGBM + r, p.M)) * p.lda * 2 + piece * 16;
    db[i] = p.b + static_cast<int64_t>(addr::gemm_row(tn * kGBN + r, p.N)) * p.ldb * 2 + piece * 16;
  }
  auto issue = [&](int kt, char* sa, char* sb) {
    const int64_t off = static_cast<int64_t>(kt) * kDRow;
#pragma unroll
    for (int i = 0; i < TPO; ++i) {
      dma16(da[i] + off, sa + (RPW * wave + 8 * i) * kDRow);
      dma16(db[i] + off, sb + (RPW * wave + 8 * i) * kDRow);
    }
  };

  const int wm = wave / WN;
  const int wn = wave % WN;
  const int i32 = l & 31;
  const int h = l >> 5;
  const int sw = addr::lds_swz(i32);            // swizzle of this lane's rows (blocks start at multiples of 32)
  f32x16 acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x16{};
  auto compute = [&](const char* sa, const char* sb) {
    const char* pa = sa + (wm * MI * 32 + i32) * kDRow;
    const char* pb = sb + (wn * NJ * 32 + i32) * kDRow;
#pragma unroll
    for (int kk = 0; kk < kDBK / 16; ++kk) {
      const int pos = ((kk * 2 + h) ^ sw) * 16;
      u32x4 af[MI], bf[NJ];
#pragma unroll
      for (int i = 0; i < MI; ++i) af[i] = *reinterpret_cast<const u32x4*>(pa + i * 32 * kDRow + pos);
#pragma unroll
      for (int j = 0; j < NJ; ++j) bf[j] = *reinterpret_cast<const u32x4*>(pb + j * 32 * kDRow + pos);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = mfma32_bf16(af[i], bf[j], acc[i][j]);
    }
  };
  // wait until this wave's transfers landed, then the barrier makes every
  // wave's part visible (and every wave is done with the other stage)
  auto sync = [&]() {
    __builtin_amdgcn_s_waitcnt(wait_vm(0));
    mem_fence_compiler();
    __builtin_amdgcn_s_barrier();
    mem_fence_compiler();
  };
  const int nk = p.K / kDBK;
  // one k-tile: transfers of tile kt+1 into the stage every wave finished
  // with before the last barrier, the MFMAs of tile kt, then the wait
  auto step = [&](int kt, const char* ca, const char* cb, char* na, char* nb) {
    if (kt + 1 < nk) issue(kt + 1, na, nb);
    compute(ca, cb);
    sync();
  };
  issue(0, sA0, sB0);
  sync();
  for (int kt = 0; kt < nk; kt += 2) {
    step(kt, sA0, sB0, sA1, sB1);
    if (kt + 1 < nk) step(kt + 1, sA1, sB1, sA0, sB0);
  }

  const int row0 = tm * kGBM + wm * MI * 32;
  const int col0 = tn * kGBN + wn * NJ * 32 + i32;
#pragma unroll
  for (int i = 0; i < MI; ++i) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = col0 + j * 32;
      if (col >= p.N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = row0 + i * 32 + mfma32_row(v, l);
        if (row < p.M) p.c[static_cast<int64_t>(row) * p.ldc + col] = f32_to_bf16_bits(acc[i][j][v]);
      }
    }
  }
}

template <bool KTAIL>
void launch_gemm(unsigned grid, const GemmParams& p, hipStream_t st) {
  constexpr int WM = 2, WN = 4;
  auto kern = gemm_bf16_tn_kernel<KTAIL, WM, WN>;
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, kGLds);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * WM * WN), kGLds, st, p);
}

// ----------------------------------------------------------------------------
// Address model (test support): replays on the host every global and LDS
// access of both GEMM kernels for one shape -- every workgroup, thread and
// k-tile -- and checks each against its buffer, and that the grid takes
// every tile exactly once.  No HIP call is made.
// ----------------------------------------------------------------------------
struct GemmModel {
  int64_t M, N, K, lda, ldb, ldc;
  int tiles_m, tiles_n;
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
  int64_t a_elems() const { return (M - 1) * lda + K; }
  int64_t b_elems() const { return (N - 1) * ldb + K; }
  // the tiles of the grid, each once
  template <typename F>
  void tiles(F&& fn) {
    const int64_t total = int64_t(tiles_m) * tiles_n, grid = 8 * ((total + 7) / 8);
    std::vector<char> seen(total, 0);
    for (int64_t b = 0; b < grid; ++b) {
      int tm, tn;
      if (!addr::gemm_tile(static_cast<int>(b), tiles_m, tiles_n, kGGroup, tm, tn)) continue;
      if (!in("tile row", tm, 1, tiles_m) || !in("tile column", tn, 1, tiles_n)) continue;
      if (seen[int64_t(tm) * tiles_n + tn]++) fail("tile (%d, %d) taken twice", tm, tn);
      fn(tm, tn);
    }
    for (int64_t t = 0; t < total; ++t)
      if (!seen[t]) {
        fail("tile %lld of %lld is never taken", (long long)t, (long long)total);
        break;
      }
  }
  // The stage layout a writer mapping produces: slot (row, position) must be
  // written exactly once and hold the global piece position ^ lds_swz(row),
  // which is where the operand reads look for it.
  struct StageLayout {
    std::vector<int> piece = std::vector<int>(kGBM * 8, -1);
  };
  void put(StageLayout& st, int row, int pos, int gpiece) {
    ++checked;
    if (row < 0 || row >= kGBM || pos < 0 || pos >= 8) return fail("stage slot (%d, %d) outside the stage", row, pos);
    int& slot = st.piece[row * 8 + pos];
    if (slot >= 0) return fail("stage slot (%d, %d) written twice", row, pos);
    slot = gpiece;
  }
  void check_layout(const StageLayout& st, const char* who) {
    for (int r = 0; r < kGBM; ++r)
      for (int q = 0; q < 8; ++q) {
        ++checked;
        const int g = st.piece[r * 8 + q];
        if (g != (q ^ addr::lds_swz(r)))
          return fail("%s: stage slot (%d, %d) holds piece %d, the operand reads expect %d", who, r, q, g,
                      q ^ addr::lds_swz(r));
      }
  }
  void stores(int tm, int tn, int WM, int WN) {
    const int MI = kGBM / WM / 32, NJ = kGBN / WN / 32;
    for (int wave = 0; wave < WM * WN; ++wave)
      for (int l = 0; l < 64; ++l) {
        const int wm = wave / WN, wn = wave % WN;
        const int row0 = tm * kGBM + wm * MI * 32, col0 = tn * kGBN + wn * NJ * 32 + (l & 31);
        for (int i = 0; i < MI; ++i)
          for (int j = 0; j < NJ; ++j) {
            const int col = col0 + j * 32;
            if (col >= N) continue;
            for (int v = 0; v < 16; ++v) {
              const int row = row0 + i * 32 + ((v >> 2) << 3) + ((l >> 5) << 2) + (v & 3);
              if (row < M) in("C", int64_t(row) * ldc + col, 1, (M - 1) * ldc + N);
            }
          }
      }
  }
  // gemm_bf16_tn_dma_kernel<WM, WN> (K % 64 == 0)
  void dma(int WM, int WN) {
    const int NW = WM * WN, RPW = kGBM / NW, TPO = RPW / 8, MI = kGBM / WM / 32, NJ = kGBN / WN / 32;
    const int nk = static_cast<int>(K / kDBK);
    StageLayout st;
    for (int wave = 0; wave < NW; ++wave)
      for (int l = 0; l < 64; ++l)
        for (int i = 0; i < TPO; ++i) {
          // a transfer fills 8 rows x 128 bytes of LDS in lane order
          const int64_t lds = (RPW * wave + 8 * i) * kDRow + l * 16;
          put(st, static_cast<int>(lds / kDRow), static_cast<int>((lds % kDRow) / 16),
              addr::gemm_piece(l, RPW * wave + 8 * i + (l >> 3)));
        }
    check_layout(st, "dma");
    tiles([&](int tm, int tn) {
      for (int wave = 0; wave < NW; ++wave) {
        for (int l = 0; l < 64; ++l)
          for (int i = 0; i < TPO; ++i) {
            const int r = RPW * wave + 8 * i + (l >> 3);
            const int piece = addr::gemm_piece(l, r);
            const int64_t ra = addr::gemm_row(tm * kGBM + r, static_cast<int>(M));
            const int64_t rb = addr::gemm_row(tn * kGBN + r, static_cast<int>(N));
            in("stage row (LDS)", (RPW * wave + 8 * i) * kDRow + l * 16, 16, kDOp);
            for (int kt = 0; kt < nk; ++kt) {
              in("A", ra * lda + int64_t(kt) * kDBK + piece * 8, 8, a_elems());
              in("B", rb * ldb + int64_t(kt) * kDBK + piece * 8, 8, b_elems());
            }
          }
        const int wm = wave / WN, wn = wave % WN;
        for (int l = 0; l < 64; ++l)
          for (int kk = 0; kk < kDBK / 16; ++kk) {
            const int pos = ((kk * 2 + (l >> 5)) ^ addr::lds_swz(l & 31)) * 16;
            for (int i = 0; i < MI; ++i) in("A operand (LDS)", (wm * MI * 32 + (l & 31) + i * 32) * kDRow + pos, 16, kDOp);
            for (int j = 0; j < NJ; ++j) in("B operand (LDS)", (wn * NJ * 32 + (l & 31) + j * 32) * kDRow + pos, 16, kDOp);
          }
      }
      stores(tm, tn, WM, WN);
    });
  }
  // gemm_bf16_tn_kernel<KTAIL, WM, WN>
  void reg(bool KTAIL, int WM, int WN) {
    const int threads = 64 * WM * WN, pieces = kGBM * (kGRowBytes / 16) / threads, step = threads / (kGRowBytes / 16);
    const int MI = kGBM / WM / 32, NJ = kGBN / WN / 32;
    const int nk = static_cast<int>((K + kGBK - 1) / kGBK);
    tiles([&](int tm, int tn) {
      for (int tid = 0; tid < threads; ++tid) {
        const int lrow = tid >> 3, lpc = (tid & 7) * 16, kp = (tid & 7) * 8;
        for (int j = 0; j < pieces; ++j) {
          const int64_t ra = addr::gemm_row(tm * kGBM + lrow + j * step, static_cast<int>(M));
          const int64_t rb = addr::gemm_row(tn * kGBN + lrow + j * step, static_cast<int>(N));
          for (int kt = 0; kt < nk; ++kt) {
            const bool ok = !KTAIL || kt * kGBK + kp < K;
            const int64_t off = ok ? int64_t(kt) * kGBK + lpc / 2 : 0;
            in("A", ra * lda + off, 8, a_elems());
            in("B", rb * ldb + off, 8, b_elems());
          }
          for (int buf = 0; buf < 2; ++buf) {
            in("A stage (LDS)", buf * kGStage + (lrow + j * step) * kGLd + lpc, 16, kGLds);
            in("B stage (LDS)", buf * kGStage + kGBM * kGLd + (lrow + j * step) * kGLd + lpc, 16, kGLds);
          }
        }
      }
      for (int wave = 0; wave < WM * WN; ++wave) {
        const int wm = wave / WN, wn = wave % WN;
        for (int l = 0; l < 64; ++l)
          for (int buf = 0; buf < 2; ++buf)
            for (int kk = 0; kk < kGBK / 16; ++kk) {
              const int64_t sa = buf * kGStage + (wm * MI * 32 + (l & 31)) * kGLd + (l >> 5) * 16 + kk * 32;
              const int64_t sb = buf * kGStage + kGBM * kGLd + (wn * NJ * 32 + (l & 31)) * kGLd + (l >> 5) * 16 + kk * 32;
              for (int i = 0; i < MI; ++i) in("A operand (LDS)", sa + i * 32 * kGLd, 16, kGLds);
              for (int j = 0; j < NJ; ++j) in("B operand (LDS)", sb + j * 32 * kGLd, 16, kGLds);
            }
      }
      stores(tm, tn, WM, WN);
    });
  }
};
}  // namespace

}  // namespace gs

using namespace gs;

extern "C" {

int gs_gemm_bf16_tn(const void* a, int64_t lda, const void* b, int64_t ldb, void* c, int64_t ldc, int64_t M,
                    int64_t N, int64_t K, void* stream) {
  const char* who = "gs_gemm_bf16_tn";
  GS_CHECK_ARG(M >= 0 && N >= 0 && M < (int64_t(1) << 31) && N < (int64_t(1) << 31), "%s: M=%lld N=%lld", who,
               (long long)M, (long long)N);
  GS_CHECK_ARG(K > 0 && K % 8 == 0 && K < (int64_t(1) << 31), "%s: K=%lld must be a positive multiple of 8", who,
               (long long)K);
  GS_CHECK_ARG(lda >= K && ldb >= K && lda % 8 == 0 && ldb % 8 == 0, "%s: lda=%lld ldb=%lld", who, (long long)lda,
               (long long)ldb);
  GS_CHECK_ARG(ldc >= N, "%s: ldc=%lld < N", who, (long long)ldc);
  GS_CHECK_ARG(aligned16(a) && aligned16(b) && (reinterpret_cast<uintptr_t>(c) & 1u) == 0,
               "%s: a and b must be 16-byte aligned, c 2-byte aligned", who);
  if (M == 0 || N == 0) return GS_OK;
  GemmParams p{};
  p.a = static_cast<const char*>(a);
  p.lda = lda;
  p.b = static_cast<const char*>(b);
  p.ldb = ldb;
  p.c = static_cast<uint16_t*>(c);
  p.ldc = ldc;
  p.M = static_cast<int>(M);
  p.N = static_cast<int>(N);
  p.K = static_cast<int>(K);
  p.tiles_m = static_cast<int>((M + kGBM - 1) / kGBM);
  p.tiles_n = static_cast<int>((N + kGBN - 1) / kGBN);
  const int64_t total = static_cast<int64_t>(p.tiles_m) * p.tiles_n;
  GS_CHECK_ARG(total <= (int64_t(1) << 30), "%s: too many tiles", who);
  const unsigned grid = static_cast<unsigned>(8 * ((total + 7) / 8));
  hipStream_t st = static_cast<hipStream_t>(stream);
#ifndef GS_GEMM_NO_DMA
  if (K % kDBK == 0) {
    hipLaunchKernelGGL((gemm_bf16_tn_dma_kernel<2, 4>), dim3(grid), dim3(512), 0, st, p);
  } else
#endif
  if (K % kGBK == 0) launch_gemm<false>(grid, p, st);
  else launch_gemm<true>(grid, p, st);
  GS_CHECK_LAUNCH(who);
  return GS_OK;
}

int64_t gs_check_gemm_addresses(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, char* msg,
                                int64_t msg_len, int64_t* checked) {
  const char* who = "gs_check_gemm_addresses";
  GS_CHECK_ARG(M > 0 && N > 0 && K > 0 && K % 8 == 0 && lda >= K && ldb >= K && ldc >= N, "%s: shape", who);
  GemmModel m{};
  m.M = M;
  m.N = N;
  m.K = K;
  m.lda = lda;
  m.ldb = ldb;
  m.ldc = ldc;
  m.tiles_m = static_cast<int>((M + kGBM - 1) / kGBM);
  m.tiles_n = static_cast<int>((N + kGBN - 1) / kGBN);
  if (K % kDBK == 0) {
    m.dma(2, 4);
    m.reg(false, 2, 4);      // the register-staged form of the same shape
  } else {
    m.reg(true, 2, 4);
  }
  if (checked) *checked = m.checked;
  if (msg && msg_len > 0) snprintf(msg, static_cast<size_t>(msg_len), "%s", m.msg);
  return m.bad;
}

}  // extern "C"
