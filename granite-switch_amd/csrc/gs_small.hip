// Small-batch (decode-sized) switched-LoRA for gfx950: the whole op in two
// launches, with no separate segment build.
//
// Both grids are adapter-major and static: a workgroup owns ONE adapter g and
// a slice of its work (shrink: a k-chunk x 32 shrink columns; expand: a
// column tile of y).  A shrink workgroup first lists the batch's tokens of
// adapter g itself: every thread gates a few tokens exactly like
// gs_build_segments does (ids outside [0, NA] are base; aLoRA: a token before
// its sequence's activation offset is base), and one ballot per token chunk
// plus a 16-entry prefix in LDS gives the list in ascending token order -- the
// order of the reference HF loop.  That costs one round trip to memory (the
// ids, cache-resident after the first workgroup), after which all of its
// lora_A and x loads are issued at once.  One shrink workgroup per adapter
// also stores the list and its length, so an expand workgroup reads them in
// one cache-hot trip and then issues its lora_B, partial-sum and y loads
// together.  Each kernel is therefore launch + two memory trips + its stores,
// and an adapter with no tokens in the batch reads no weights.
//
// The shrink splits the hidden dimension into KS chunks and writes fp32
// partial sums at part[ks][g-1][j][col], j = the token's rank among adapter
// g's tokens.  The expand sums them in ks order (deterministic) and rounds to
// the element type exactly as a materialised z would be, then MFMAs with
// lora_B and read-modify-writes only its adapter's token rows of y.
//
// Workspace: part [KS][NA][cap][zw] fp32, then lists [NA][cap] int32.
#include "gs_common.h"

namespace gs {

namespace {

constexpr int kSmT = 256;                    // threads per workgroup (4 waves)
constexpr int kSmMaxTokens = 1024;           // largest batch of this path
constexpr int kSmMaxAdapters = 64;           // adapters whose tables ride in the kernel arguments
constexpr int kSmMaxRank = 64;               // largest (padded) rank of this path
constexpr int kSmU = kSmMaxTokens / kSmT;    // tokens per thread in the routing pass
constexpr int kPartGrp = 8;                  // split-K partials loaded together by the expand
constexpr int kTokBits = 11;                 // token-list entry: (count << kTokBits) | token
constexpr int kTokMask = (1 << kTokBits) - 1;
static_assert(kSmMaxTokens < kTokMask, "token ids must fit below the list marker");

// Per-adapter weight offsets and ranks, passed by value (load-time constants of
// the module) so no workgroup waits on a table load before its weight loads.
struct SmallTab {
  int64_t off[kSmMaxAdapters + 1];
  int32_t rank[kSmMaxAdapters + 1];
};

// Routing input: either pre-gated ids (eff, int32, e.g. the eff_ids output of
// gs_build_segments) or the raw request (req + positions + cu + act_off).
struct SmallRoute {
  const int64_t* req;
  const int64_t* pos;
  const int32_t* cu;
  const int64_t* act_off;
  const int32_t* eff;
  int T;
  int num_seqs;
  int NA;
};

struct RouteLds {
  int tok[kSmMaxTokens];
  int32_t cu[kSmMaxTokens];
  int64_t off[kSmMaxTokens];
  int wreq[4];
  int wcnt[kSmU * 4];
};

// Routing in two halves so the caller can issue its weight loads in between.
// route_load: token t = u*256 + tid of every thread; loads the ids (and the
// raw routing), stages sequence boundaries and activation offsets in LDS, and
// returns whether any token REQUESTS adapter g (before gating; exact for
// pre-gated ids) -- workgroup-uniform, read after one barrier.
struct RouteRegs {
  int id[kSmU];
};

__device__ bool route_load(const SmallRoute& r, int g, RouteLds& s, RouteRegs& rr) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int64_t rq[kSmU], q[kSmU];
  if (r.eff != nullptr) {
#pragma unroll
    for (int u = 0; u < kSmU; ++u) {
      const int t = u * kSmT + tid;
      rq[u] = t < r.T ? r.eff[t] : 0;
    }
  } else {
#pragma unroll
    for (int u = 0; u < kSmU; ++u) {
      const int t = u * kSmT + tid;
      rq[u] = t < r.T ? r.req[t] : 0;
      q[u] = (t < r.T && r.pos != nullptr) ? r.pos[t] : 0;
    }
  }
  const bool gate = r.eff == nullptr && r.act_off != nullptr;
  const int ns = (gate && r.cu != nullptr) ? r.num_seqs : 1;
  if (gate) {
    if (r.cu != nullptr) {
#pragma unroll
      for (int u = 0; u < kSmU; ++u) {
        const int k = u * kSmT + tid;
        if (k < ns) {
          s.cu[k] = r.cu[k];
          s.off[k] = r.act_off[k];
        }
      }
    } else if (tid == 0) {
      s.cu[0] = 0;
      s.off[0] = r.act_off[0];
    }
  }
  bool req_g = false;
#pragma unroll
  for (int u = 0; u < kSmU; ++u) req_g |= (u * kSmT + tid < r.T) && rq[u] == g;
  const uint64_t any = __ballot(req_g);
  if (lane == 0) s.wreq[wave] = any != 0;
  lds_barrier();
  const bool used = (s.wreq[0] | s.wreq[1] | s.wreq[2] | s.wreq[3]) != 0;
  // gating (sequence of token t: the largest sq with cu[sq] <= t, by a
  // fixed-step search whose per-token chains interleave)
  int sq[kSmU];
#pragma unroll
  for (int u = 0; u < kSmU; ++u) sq[u] = 0;
  if (gate) {
    // First guess: token t is sequence t (a decode batch, one token per
    // sequence); it is right iff cu[t] <= t < cu[t+1].  Lanes whose guess
    // fails run a fixed-step search (one LDS read per token slot and step,
    // all issued before any is compared; clamped indices stay in bounds).
    bool ok[kSmU];
    bool all_ok = true;
#pragma unroll
    for (int u = 0; u < kSmU; ++u) {
      const int t = u * kSmT + tid;
      const int gs = min(t, ns - 1);
      const int c0 = s.cu[gs];
      const int c1 = gs + 1 < ns ? s.cu[gs + 1] : 0x7fffffff;
      ok[u] = t >= r.T || (c0 <= t && t < c1);
      sq[u] = ok[u] ? gs : 0;
      all_ok = all_ok && ok[u];
    }
    if (!all_ok) {
#pragma unroll
      for (int step = kSmMaxTokens / 2; step > 0; step >>= 1) {
        if (step < ns) {
          int c[kSmU];
#pragma unroll
          for (int u = 0; u < kSmU; ++u) c[u] = s.cu[min(sq[u] + step, ns - 1)];
#pragma unroll
          for (int u = 0; u < kSmU; ++u)
            sq[u] = (!ok[u] && sq[u] + step < ns && c[u] <= u * kSmT + tid) ? sq[u] + step : sq[u];
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kSmU; ++u) {
    const int t = u * kSmT + tid;
    int64_t v = rq[u];
    if (gate && t < r.T) {
      const int64_t qq = r.pos != nullptr ? q[u] : static_cast<int64_t>(t - s.cu[sq[u]]);
      if (qq < s.off[sq[u]]) v = 0;
    }
    if (t >= r.T || v < 0 || v > r.NA) v = 0;
    rr.id[u] = static_cast<int>(v);
  }
  return used;
}

// route_list: lists adapter g's tokens (ascending) in s.tok and returns their
// count; position = earlier (u, wave) chunks' counts + matches in lower lanes.
// Called by all threads of the workgroup; ends with a barrier.
__device__ int route_list(int g, RouteLds& s, const RouteRegs& rr) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  uint64_t bal[kSmU];
#pragma unroll
  for (int u = 0; u < kSmU; ++u) {
    bal[u] = __ballot(rr.id[u] == g);
    if (lane == 0) s.wcnt[u * 4 + wave] = __popcll(bal[u]);
  }
  lds_barrier();
  int before[kSmU];
  int total = 0;
#pragma unroll
  for (int u = 0; u < kSmU; ++u) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if (w == wave) before[u] = total;
      total += s.wcnt[u * 4 + w];
    }
  }
#pragma unroll
  for (int u = 0; u < kSmU; ++u) {
    if (rr.id[u] == g) s.tok[before[u] + __popcll(bal[u] & lanemask_lt())] = u * kSmT + tid;
  }
  lds_barrier();
  return total;
}

// ----------------------------------------------------------------------------
// Shrink.  Grid (32-column block, k-chunk, adapter).  The 4 waves
// split the k-chunk; each holds its share of the adapter's 32 lora_A rows in
// registers (NPW 16-byte pieces per lane) for every 32-token row tile.
// ----------------------------------------------------------------------------
struct SmallShrinkParams {
  SmallRoute rt;
  const void* x;
  int64_t ldx;
  int H;
  const void* a_pack;
  int S;
  int KS;
  int NCB;
  float* part;    // [KS][NA][cap][zw]
  int32_t* lists; // [NA][cap] the adapter's tokens, ascending (see the shrink)
  int cap;
  int zw;
  SmallTab tab;
};

template <bool BF16, int NPW>
__global__ __launch_bounds__(kSmT) void shrink_small_kernel(SmallShrinkParams p) {
  __shared__ RouteLds rl;
  __shared__ float red[3][16][64];
  __shared__ float tile_s[32][32 + 4];
  constexpr int P = Elt<BF16>::kPerPiece;
  constexpr int ES = Elt<BF16>::kSize;
  constexpr int KW = NPW * 2 * P;   // k per wave

  const int cb = blockIdx.x;
  const int kc = blockIdx.y;
  const int g = blockIdx.z + 1;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int i = l & 31;
  const int h = l >> 5;
  // Trip 1: the routing loads (and the adapter's table entry, a kernel
  // argument).
  RouteRegs rr;
  const bool requested = route_load(p.rt, g, rl, rr);
  const int r = p.tab.rank[g];
  const int ncols = p.S * r;
  const bool active = r > 0 && cb * 32 < ncols;
  // Trip 2 starts here: lora_A of this workgroup's 32 shrink columns and its
  // waves' k ranges, issued while the tokens are gated and listed -- only if
  // some token requested the adapter, so an adapter absent from the batch
  // reads no weights.
  const int64_t k_lo = (static_cast<int64_t>(kc) * 4 + wave) * KW;
  const int64_t k_hi = min(static_cast<int64_t>(p.H), k_lo + KW);
  const int n = cb * 32 + i;
  const bool n_ok = active && requested && n < ncols;
  const char* arow =
      static_cast<const char*>(p.a_pack) + (p.tab.off[g] + static_cast<int64_t>(n_ok ? n : 0) * p.H) * ES;
  u32x4 av[NPW];
#pragma unroll
  for (int pp = 0; pp < NPW; ++pp) {
    const int64_t kp = k_lo + (2 * pp + h) * P;
    av[pp] = u32x4{0u, 0u, 0u, 0u};
    if (n_ok && kp < k_hi) av[pp] = ld16(arow + kp * ES);
  }
  const int n_g = route_list(g, rl, rr);
  if (!active) return;
  if (kc == 0 && cb == 0) {
    // The expand reads the token list instead of routing again.  Each entry
    // is (count << kTokBits) | token; the first 32 entries are always written
    // (token kTokMask past the count), so an expand workgroup learns the count
    // from its own first-tile entries.
    const int nw = n_g > 32 ? n_g : 32;
    for (int j = tid; j < nw; j += kSmT)
      p.lists[static_cast<int64_t>(g - 1) * p.cap + j] = (n_g << kTokBits) | (j < n_g ? rl.tok[j] : kTokMask);
  }
  if (n_g == 0) return;

  for (int rt0 = 0; rt0 < n_g; rt0 += 32) {
    const int row = rt0 + i;
    const bool row_ok = row < n_g;
    const int token = rl.tok[row_ok ? row : rt0];
    const char* xrow = static_cast<const char*>(p.x) + static_cast<int64_t>(token) * p.ldx * ES;
    u32x4 xv[NPW];
#pragma unroll
    for (int pp = 0; pp < NPW; ++pp) {
      const int64_t kp = k_lo + (2 * pp + h) * P;
      xv[pp] = u32x4{0u, 0u, 0u, 0u};
      if (row_ok && kp < k_hi) xv[pp] = ld16(xrow + kp * ES);
    }
    f32x16 acc = f32x16{};
#pragma unroll
    for (int pp = 0; pp < NPW; ++pp) acc = mfma_piece<BF16>(xv[pp], av[pp], acc);

    // fixed-order cross-wave sum: ((w0 + w1) + w2) + w3
    if (wave > 0) {
#pragma unroll
      for (int v = 0; v < 16; ++v) red[wave - 1][v][l] = acc[v];
    }
    lds_barrier();
    if (wave == 0) {
#pragma unroll
      for (int v = 0; v < 16; ++v) tile_s[mfma32_row(v, l)][i] = ((acc[v] + red[0][v][l]) + red[1][v][l]) + red[2][v][l];
    }
    lds_barrier();
    const int srow = tid >> 3;
    const int c4 = (tid & 7) * 4;
    if (rt0 + srow < n_g && cb * 32 + c4 < ncols) {
      float* dst = p.part +
                   ((static_cast<int64_t>(kc) * p.rt.NA + (g - 1)) * p.cap + rt0 + srow) * p.zw + cb * 32 + c4;
      *reinterpret_cast<f32x4*>(dst) =
          f32x4{tile_s[srow][c4], tile_s[srow][c4 + 1], tile_s[srow][c4 + 2], tile_s[srow][c4 + 3]};
    }
    lds_barrier();   // red / tile_s are reused by the next row tile
  }
}

// ----------------------------------------------------------------------------
// Expand.  Grid (column tile of NT = 128*NBW columns inside one slice,
// adapter).  Each wave owns NBW 32-column blocks and holds their lora_B rows
// for the whole rank in registers.  Per 32-token row tile: the partial sums
// become the tile's shrink rows in LDS, y rows are loaded, the MFMA deltas go
// through LDS to a row-major tile, and each thread adds and stores 16-byte
// pieces of its token rows.
// ----------------------------------------------------------------------------
struct SmallExpandParams {
  const int32_t* lists;   // [NA][cap] written by the shrink
  int NA;
  void* y;
  int64_t ldy;
  int out_total;
  SliceInfo si;
  const void* b_pack;
  const float* part;
  int KS;
  int cap;
  int zw;
  int NNT;          // column tiles per adapter
  SmallTab tab;
};

template <bool BF16, int NBW>
__global__ __launch_bounds__(kSmT) void expand_small_kernel(SmallExpandParams p) {
  constexpr int NT = 4 * NBW * 32;
  constexpr int ES = Elt<BF16>::kSize;
  constexpr int EPL = 16 / ES;          // elements per 16-byte piece
  constexpr int LPR = NT / EPL;         // lanes per y row
  constexpr int RPI = kSmT / LPR;       // rows per workgroup-wide access
  constexpr int PASSES = 32 / RPI;
  constexpr int KSTEP = BF16 ? 16 : 8;  // rank per MFMA group (both lane halves)
  constexpr int KHALF = KSTEP / 2;
  constexpr int KG = kSmMaxRank / KSTEP;
  constexpr int ZLD = kSmMaxRank + 8;   // elements per LDS shrink row
  __shared__ __align__(16) char zs[32 * ZLD * ES];
  __shared__ float dtile[32][NT + 4];

  const int nt = blockIdx.x;
  const int g = blockIdx.y + 1;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int i = l & 31;
  const int h = l >> 5;
  const int32_t* list = p.lists + static_cast<int64_t>(g - 1) * p.cap;
  // Trip 1: this thread's entries of the first row tile.  Every entry also
  // carries the adapter's token count, so the exit test below depends on
  // these loads and they are issued before it.
  int ent[PASSES];
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) ent[ps] = list[ps * RPI + tid / LPR];
  const int r = p.tab.rank[g];
  const int n_g = __builtin_amdgcn_readfirstlane(ent[0] >> kTokBits);
  if (r == 0 || n_g == 0) return;

  const int n_tile0 = nt * NT;
  int s = 0;                             // slice of this column tile
#pragma unroll
  for (int k = 1; k < GS_MAX_SLICES; ++k)
    if (k < p.si.S && n_tile0 >= p.si.bounds[k]) s = k;
  const int zc0 = s * r;                 // this slice's columns in the adapter's shrink row
  const int64_t goff = static_cast<int64_t>(g - 1) * p.cap;
  const int64_t kstride = static_cast<int64_t>(p.NA) * p.cap * p.zw;
  const int cx = (tid % LPR) * EPL;
  const int per_row = r >> 2;            // 4-element items per shrink row
  const int nitems = 32 * per_row;       // <= 2 items per thread (rank <= 64)

  // Trip 2 (first tile): lora_B rows of this wave's column blocks (all
  // k-groups of the rank), the first kPartGrp split-K partials of the tile's
  // shrink rows, and the tile's y rows -- all in flight before any is used.
  u32x4 bv[NBW][KG];
#pragma unroll
  for (int q = 0; q < NBW; ++q) {
    const int n = n_tile0 + 32 * (wave * NBW + q) + i;
    const char* br = static_cast<const char*>(p.b_pack) + (p.tab.off[g] + static_cast<int64_t>(n) * r) * ES;
#pragma unroll
    for (int kg = 0; kg < KG; ++kg) {
      const int k0 = kg * KSTEP + KHALF * h;
      bv[q][kg] = u32x4{0u, 0u, 0u, 0u};
      if (k0 < r) bv[q][kg] = ld16(br + k0 * ES);
    }
  }

  auto tile = [&](const int rt0) {
    const float* src[2];
    bool iok[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int it = tid + j * kSmT;
      const int row = it / per_row;
      const int c4 = (it - row * per_row) * 4;
      iok[j] = it < nitems && rt0 + row < n_g;
      src[j] = p.part + (goff + rt0 + (iok[j] ? row : 0)) * p.zw + zc0 + (iok[j] ? c4 : 0);
    }
    f32x4 a[2][kPartGrp];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int u = 0; u < kPartGrp; ++u) {
        a[j][u] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (iok[j] && u < p.KS) a[j][u] = *reinterpret_cast<const f32x4*>(src[j] + u * kstride);
      }
    u32x4 yv[PASSES];
    int64_t yoff[PASSES];
    bool rok[PASSES];
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      const int row = ps * RPI + tid / LPR;
      rok[ps] = rt0 + row < n_g;
      yoff[ps] = static_cast<int64_t>(rok[ps] ? (ent[ps] & kTokMask) : 0) * p.ldy + n_tile0 + cx;
      yv[ps] = u32x4{0u, 0u, 0u, 0u};
      if (rok[ps]) yv[ps] = ld16(static_cast<const char*>(p.y) + yoff[ps] * ES);
    }
    // shrink rows: partials summed in ks order, rounded like a stored z
    f32x4 sum[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int u = 0; u < kPartGrp; ++u)
        if (u < p.KS) sum[j] += a[j][u];
    for (int ks0 = kPartGrp; ks0 < p.KS; ks0 += kPartGrp) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int u = 0; u < kPartGrp; ++u) {
          a[j][u] = f32x4{0.f, 0.f, 0.f, 0.f};
          if (iok[j] && ks0 + u < p.KS) a[j][u] = *reinterpret_cast<const f32x4*>(src[j] + (ks0 + u) * kstride);
        }
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int u = 0; u < kPartGrp; ++u)
          if (ks0 + u < p.KS) sum[j] += a[j][u];
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int it = tid + j * kSmT;
      if (it < nitems) {
        const int row = it / per_row;
        const int c4 = (it - row * per_row) * 4;
        char* dst = zs + (row * ZLD + c4) * ES;
        if constexpr (BF16) {
          *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(sum[j].x, sum[j].y), pack_bf16x2(sum[j].z, sum[j].w));
        } else {
          *reinterpret_cast<f32x4*>(dst) = sum[j];
        }
      }
    }
    lds_barrier();

    f32x16 acc[NBW];
#pragma unroll
    for (int q = 0; q < NBW; ++q) {
      acc[q] = f32x16{};
#pragma unroll
      for (int kg = 0; kg < KG; ++kg) {
        if (kg * KSTEP < r) {
          const int k0 = kg * KSTEP + KHALF * h;
          u32x4 za = u32x4{0u, 0u, 0u, 0u};
          if (k0 < r) za = *reinterpret_cast<const u32x4*>(zs + (i * ZLD + k0) * ES);
          acc[q] = mfma_piece<BF16>(za, bv[q][kg], acc[q]);
        }
      }
    }
#pragma unroll
    for (int q = 0; q < NBW; ++q)
#pragma unroll
      for (int v = 0; v < 16; ++v) dtile[mfma32_row(v, l)][32 * (wave * NBW + q) + i] = acc[q][v];
    lds_barrier();
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      if (rok[ps]) {
        const int row = ps * RPI + tid / LPR;
        float d[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) d[e] = dtile[row][cx + e];
        add_store_y<BF16>(p.y, yoff[ps], yv[ps], d);
      }
    }
  };

  tile(0);
  for (int rt0 = 32; rt0 < n_g; rt0 += 32) {
    lds_barrier();   // zs / dtile are reused by this tile
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      const int row = rt0 + ps * RPI + tid / LPR;
      ent[ps] = row < n_g ? list[row] : 0;
    }
    tile(rt0);
  }
}

// ----------------------------------------------------------------------------
// Host-side plan.
// ----------------------------------------------------------------------------
struct SmallPlan {
  int NPW, KS, NCB, cap, zw, NBW, NNT;
  int64_t part_bytes, ws_bytes;
};

constexpr int kSmTargetShrinkWgs = 192;

SmallPlan plan_small(int64_t T, int H, int S, int NA, int max_rank, bool bf16, int out_total,
                     const int32_t* slice_bounds) {
  SmallPlan pl{};
  pl.zw = S * max_rank;
  pl.NCB = (pl.zw + 31) / 32;
  const int kpair = bf16 ? 16 : 8;       // k covered by one piece of each lane half
  // smallest k-split (fewest partials for the expand to add) that still gives
  // about kSmTargetShrinkWgs workgroups, with at most 2 partial groups
  int npw = 16;
  int ks = 1;
  for (;;) {
    ks = (H + 4 * npw * kpair - 1) / (4 * npw * kpair);
    if (static_cast<int64_t>(NA) * pl.NCB * ks >= kSmTargetShrinkWgs || npw == 2) break;
    const int ks_next = (H + 2 * npw * kpair - 1) / (2 * npw * kpair);
    if (ks_next > 2 * kPartGrp) break;
    npw >>= 1;
  }
  pl.NPW = npw;
  pl.KS = ks;
  pl.cap = static_cast<int>(((T + 31) / 32) * 32);
  bool all256 = true;
  for (int s = 0; s < S; ++s)
    if ((slice_bounds[s + 1] - slice_bounds[s]) % 256 != 0) all256 = false;
  pl.NBW = all256 ? 2 : 1;
  pl.NNT = out_total / (128 * pl.NBW);
  pl.part_bytes = static_cast<int64_t>(pl.KS) * NA * pl.cap * pl.zw * 4;
  pl.ws_bytes = pl.part_bytes + static_cast<int64_t>(NA) * pl.cap * 4;
  return pl;
}

template <bool BF16>
void launch_small(const SmallPlan& pl, const SmallShrinkParams& sp, const SmallExpandParams& ep, int NA,
                  hipStream_t st) {
  const dim3 g1(static_cast<unsigned>(pl.NCB), static_cast<unsigned>(pl.KS), static_cast<unsigned>(NA));
  switch (pl.NPW) {
    case 16: hipLaunchKernelGGL((shrink_small_kernel<BF16, 16>), g1, dim3(kSmT), 0, st, sp); break;
    case 8: hipLaunchKernelGGL((shrink_small_kernel<BF16, 8>), g1, dim3(kSmT), 0, st, sp); break;
    case 4: hipLaunchKernelGGL((shrink_small_kernel<BF16, 4>), g1, dim3(kSmT), 0, st, sp); break;
    default: hipLaunchKernelGGL((shrink_small_kernel<BF16, 2>), g1, dim3(kSmT), 0, st, sp); break;
  }
  const dim3 g2(static_cast<unsigned>(pl.NNT), static_cast<unsigned>(NA));
  if (pl.NBW == 2) hipLaunchKernelGGL((expand_small_kernel<BF16, 2>), g2, dim3(kSmT), 0, st, ep);
  else hipLaunchKernelGGL((expand_small_kernel<BF16, 1>), g2, dim3(kSmT), 0, st, ep);
}

}  // namespace

}  // namespace gs

using namespace gs;

extern "C" {

int gs_small_eligible(int64_t num_tokens, int32_t num_seqs, int32_t num_slices, const int32_t* slice_bounds,
                      int32_t num_adapters, int32_t max_rank) {
  if (num_tokens < 0 || num_tokens > kSmMaxTokens) return 0;
  if (num_seqs > kSmMaxTokens) return 0;
  if (num_adapters < 1 || num_adapters > kSmMaxAdapters) return 0;
  if (max_rank < 8 || max_rank > kSmMaxRank || max_rank % 8 != 0) return 0;
  if (num_slices < 1 || num_slices > GS_MAX_SLICES || slice_bounds == nullptr || slice_bounds[0] != 0) return 0;
  for (int s = 0; s < num_slices; ++s) {
    const int w = slice_bounds[s + 1] - slice_bounds[s];
    if (w <= 0 || w % 128 != 0) return 0;
  }
  return 1;
}

int64_t gs_small_workspace_bytes(int32_t dtype, int64_t num_tokens, int32_t hidden, int32_t num_slices,
                                 int32_t num_adapters, int32_t max_rank, int32_t out_total,
                                 const int32_t* slice_bounds) {
  if (num_tokens <= 0 || hidden <= 0 || slice_bounds == nullptr) return 256;
  const SmallPlan pl = plan_small(num_tokens, hidden, num_slices, num_adapters, max_rank, dtype == GS_DTYPE_BF16,
                                  out_total, slice_bounds);
  return pl.ws_bytes < 256 ? 256 : pl.ws_bytes;
}

int gs_switched_lora_small(int32_t dtype, const int64_t* req_ids, const int64_t* positions,
                           const int32_t* cu_seqlens, const int64_t* act_offsets, int32_t num_seqs,
                           const int32_t* eff_ids, const void* x, int64_t ldx, void* y, int64_t ldy,
                           int64_t num_tokens, int32_t hidden, int32_t out_total, const int32_t* slice_bounds,
                           int32_t num_slices, const void* a_pack, const int64_t* a_off, const void* b_pack,
                           const int64_t* b_off, const int32_t* ranks, int32_t num_adapters, int32_t max_rank,
                           void* workspace, int64_t workspace_bytes, void* stream) {
  const char* who = "gs_switched_lora_small";
  GS_CHECK_ARG(dtype == GS_DTYPE_BF16 || dtype == GS_DTYPE_FP32, "%s: dtype=%d", who, dtype);
  const int nseq = (cu_seqlens != nullptr) ? num_seqs : 1;
  GS_CHECK_ARG(gs_small_eligible(num_tokens, nseq, num_slices, slice_bounds, num_adapters, max_rank),
               "%s: shape outside the small-batch path (T <= %d, <= %d adapters, max_rank <= %d, slice widths "
               "multiples of 128)", who, kSmMaxTokens, kSmMaxAdapters, kSmMaxRank);
  GS_CHECK_ARG(nseq >= 1, "%s: num_seqs=%d", who, num_seqs);
  GS_CHECK_ARG(eff_ids != nullptr || req_ids != nullptr || num_tokens == 0, "%s: no routing input", who);
  GS_CHECK_ARG(slice_bounds[num_slices] == out_total, "%s: slice_bounds must end at out_total", who);
  GS_CHECK_ARG(hidden > 0 && hidden % 8 == 0, "%s: hidden=%d must be a positive multiple of 8", who, hidden);
  const int vec = dtype == GS_DTYPE_BF16 ? 8 : 4;
  GS_CHECK_ARG(ldx >= hidden && ldx % vec == 0 && ldy >= out_total && ldy % vec == 0, "%s: ldx/ldy", who);
  GS_CHECK_ARG(aligned16(x) && aligned16(y) && aligned16(a_pack) && aligned16(b_pack) && aligned16(workspace),
               "%s: x, y, a_pack, b_pack and workspace must be 16-byte aligned", who);
  GS_CHECK_ARG(a_off != nullptr && b_off != nullptr && ranks != nullptr, "%s: NULL adapter tables", who);
  GS_CHECK_ARG(ranks[0] == 0, "%s: ranks[0] must be 0 (base)", who);
  for (int g = 1; g <= num_adapters; ++g) {
    GS_CHECK_ARG(ranks[g] >= 0 && ranks[g] <= max_rank && ranks[g] % 8 == 0, "%s: ranks[%d]=%d", who, g, ranks[g]);
    GS_CHECK_ARG(a_off[g] >= 0 && a_off[g] % 8 == 0 && b_off[g] >= 0 && b_off[g] % 8 == 0,
                 "%s: adapter %d offsets must be non-negative multiples of 8", who, g);
  }
  if (num_tokens == 0) return GS_OK;
  const bool bf16 = dtype == GS_DTYPE_BF16;
  const SmallPlan pl = plan_small(num_tokens, hidden, num_slices, num_adapters, max_rank, bf16, out_total,
                                  slice_bounds);
  if (workspace_bytes < pl.ws_bytes) {
    set_error("%s: workspace of %lld bytes needed (got %lld)", who, (long long)pl.ws_bytes,
              (long long)workspace_bytes);
    return GS_ERR_WORKSPACE;
  }
  SmallRoute rt{eff_ids != nullptr ? nullptr : req_ids, positions, cu_seqlens, act_offsets, eff_ids,
                static_cast<int>(num_tokens), nseq, num_adapters};
  SmallTab at{}, bt{};
  for (int g = 0; g <= num_adapters; ++g) {
    at.off[g] = a_off[g];
    at.rank[g] = ranks[g];
    bt.off[g] = b_off[g];
    bt.rank[g] = ranks[g];
  }
  SmallShrinkParams sp{};
  sp.rt = rt;
  sp.x = x;
  sp.ldx = ldx;
  sp.H = hidden;
  sp.a_pack = a_pack;
  sp.S = num_slices;
  sp.KS = pl.KS;
  sp.NCB = pl.NCB;
  sp.part = static_cast<float*>(workspace);
  int32_t* lists = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + pl.part_bytes);
  sp.lists = lists;
  sp.cap = pl.cap;
  sp.zw = pl.zw;
  sp.tab = at;
  SmallExpandParams ep{};
  ep.lists = lists;
  ep.NA = num_adapters;
  ep.y = y;
  ep.ldy = ldy;
  ep.out_total = out_total;
  ep.si.S = num_slices;
  for (int s = 0; s <= num_slices; ++s) ep.si.bounds[s] = slice_bounds[s];
  ep.b_pack = b_pack;
  ep.part = static_cast<const float*>(workspace);
  ep.KS = pl.KS;
  ep.cap = pl.cap;
  ep.zw = pl.zw;
  ep.NNT = pl.NNT;
  ep.tab = bt;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (bf16) launch_small<true>(pl, sp, ep, num_adapters, st);
  else launch_small<false>(pl, sp, ep, num_adapters, st);
  GS_CHECK_LAUNCH(who);
  return GS_OK;
}

}  // extern "C"
