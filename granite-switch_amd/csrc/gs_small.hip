// Small-batch (decode-sized) switched-LoRA for gfx950: the whole op in ONE
// launch, with no separate segment build.
//
// The grid is 1-D: NP producer workgroups, then NC consumer workgroups.
//   producer (cb, kc, g, rs): the shrink of adapter g's 32-column block cb over
//     the k-chunk kc, written as fp32 partial sums;
//   consumer (nt, g, rs): the expand of adapter g into the NT-column tile nt of
//     y (inside one slice), which adds the partials of its slice in ks order.
// An adapter's token list is cut into 32-token row chunks; row split rs of RS
// takes chunks rs, rs + RS, rs + 2 RS, ..., so an adapter with many tokens is
// spread over RS times the workgroups.
// Every workgroup gates and lists the tokens of its own adapter from the
// routing input (ids outside [0, NA] are base; aLoRA: a token before its
// sequence's activation offset is base), with one ballot per token chunk and a
// 16-entry prefix in LDS, giving the list in ascending token order -- the
// iteration order of the reference HF loop.
//
// Hand-off inside the launch: tagged partials.  Each adapter g has a 64-bit
// launch counter C_g in the sync buffer whose epoch is E_g = C_g >> 20.
// Every workgroup of adapter g reads C_g when it starts; a producer stores each
// partial as one 64-bit pair (tag = E_g + 1, fp32 bits) with agent-coherent
// stores (sc1: written through past the XCD's L2), and a consumer issues its
// lora_B and y loads first, then polls its partials with agent-coherent 64-bit
// loads until every tag equals E_g + 1 (a pair is read in one access, so a
// value is never taken without its tag).  Once it has its partials, a consumer
// adds its weight to C_g without waiting for the result; the weights of g's
// NNT * RS consumers in one launch sum to exactly 2^20, so E_g moves to E_g + 1
// only when the last of them has added (a consumer whose row split holds no
// chunk adds its weight without waiting).  Every workgroup of g in the launch reads
// E_g: consumers read it before adding, and every producer that writes
// partials is waited for by some consumer of its slice, which has not added
// yet.  No counters on the critical path, no cache writeback or invalidate,
// no device-scope fence.  Adapter g's partials live in a fixed region of the
// workspace whatever the module's shape, so a stale pair there carries a tag
// of an earlier epoch of the same g and never the current one (until the
// 32-bit tag wraps, after 2^32 launches with tokens for g).
//
// Forward progress: producers have the lowest workgroup ids and never wait, and
// workgroups are dispatched in id order, so a waiting consumer never holds a
// slot a producer still needs.  The wait is nevertheless bounded: after
// max_polls looks at a group of partials a consumer sets bit 0 of the error
// word and goes on, so every wave of the grid always ends.  The bound counts
// looks, not time, so a queue preempted mid-wait does not use it up.
//
// MFMA shapes: 16x16x32 bf16 (16x16x4 fp32) throughout, so each global load
// instruction reads 64 contiguous bytes of 16 rows (4 lanes per row) instead
// of 32 bytes of 32 rows.
//
// Workspace: kSmMaxAdapters equal regions, adapter g's holding its tagged
// partials [KS][cap][zw] uint64; used by nothing else.
// Sync buffer (int32 words): [2] error word; [32*g .. 32*g + 1] the 64-bit
// launch counter of adapter g (one 128-byte line per adapter).  Both buffers
// are zeroed once before the first call.
#include <stdarg.h>

#include <algorithm>
#include <vector>

#include "gs_addr.h"
#include "gs_common.h"

namespace gs {

namespace {

// y rows (consumers) are read and written once per launch and lora_A
// (producers) once per row split: both go through the streaming (nt) cache
// policy, so the x rows, lora_B and the partials that several workgroups
// read stay in L2 (decode QKV 11.38 -> 11.12 us, the fp32 aLoRA batch with
// row split 4 15.38 -> 14.81 us).
__device__ __forceinline__ u32x4 ld_y(const void* p) { return ld16_nt(p); }
__device__ __forceinline__ u32x4 ld_a(const void* p) { return ld16_nt(p); }
__device__ __forceinline__ void st_y(void* p, const u32x4& v) { st16_nt(p, v); }

constexpr int kSmT = 256;                    // threads per workgroup (4 waves)
constexpr int kSmMaxTokens = 1024;           // largest batch of this path
constexpr int kSmMaxAdapters = 64;           // adapters whose tables ride in the kernel arguments
constexpr int kSmMaxRank = 64;               // largest (padded) rank of this path
constexpr int kSmMaxU = kSmMaxTokens / kSmT; // tokens per thread in the routing pass (at most)
#ifndef GS_SMALL_KS_GROUP
#define GS_SMALL_KS_GROUP 4
#endif
constexpr int kKsGrp = GS_SMALL_KS_GROUP;     // split-K partials a consumer polls together
constexpr int kErrTimeout = 1;               // error word bits
constexpr int kSyncErrWord = 2;              // int32 index of the error word
constexpr int kSyncLine = 32;                // int32 words per adapter (its 64-bit launch counter)
constexpr int kEpochShift = 20;              // a launch adds 2^20 to the counter of each adapter with tokens
constexpr int kSmMaxRowSplit = 32;           // row splits: at most one 32-token chunk each at 1024 tokens

// Per-adapter weight offsets and ranks, passed by value (load-time constants of
// the module) so no workgroup waits on a table load before its weight loads.
struct SmallTab {
  int64_t a_off[kSmMaxAdapters + 1];
  int64_t b_off[kSmMaxAdapters + 1];
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

// U = tokens per thread in the routing pass: batches (and sequence counts) of
// up to U*256 tokens.
template <int U>
struct RouteLds {
  int tok[U * kSmT];
  int32_t cu[U * kSmT];
  int64_t off[U * kSmT];
  int wreq[4];
  int wcnt[U * 4];
};

// Routing in three steps so the caller can issue its weight loads between the
// routing loads and their first use (loads return in order, so a wait for the
// routing loads does not wait for weight loads issued after them).
template <int U>
struct RouteRegs {
  int64_t rq[U];        // requested ids (req path) or pre-gated ids (eff path)
  int64_t q[U];
  int32_t cu[U];
  int64_t off[U];
  int id[U];
};

__device__ __forceinline__ bool route_gated(const SmallRoute& r) { return r.eff == nullptr && r.act_off != nullptr; }
__device__ __forceinline__ int route_nseq(const SmallRoute& r) {
  return (route_gated(r) && r.cu != nullptr) ? r.num_seqs : 1;
}

// Step 1: issue the routing loads for tokens t = u*256 + tid.  The pointer
// checks are uniform and sit outside the loops; inside, every load is issued
// unconditionally from a clamped in-bounds index (T >= 1, ns >= 1), so the
// loads stay in flight together.  Entries past T / ns are masked by the users.
template <int U>
__device__ __forceinline__ void route_issue(const SmallRoute& r, RouteRegs<U>& rr) {
  const int tid = threadIdx.x;
  if (r.eff != nullptr) {
    // zero-extended: a negative id becomes a large one, base either way, and
    // no instruction depends on the load before the routing wait
#pragma unroll
    for (int u = 0; u < U; ++u) rr.rq[u] = static_cast<uint32_t>(r.eff[addr::small_route_index(u, tid, r.T)]);
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) rr.rq[u] = r.req[addr::small_route_index(u, tid, r.T)];
  }
  if (r.eff == nullptr && r.pos != nullptr) {
#pragma unroll
    for (int u = 0; u < U; ++u) rr.q[u] = r.pos[addr::small_route_index(u, tid, r.T)];
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) rr.q[u] = 0;
  }
  if (route_gated(r)) {
    const int ns = route_nseq(r);
#pragma unroll
    for (int u = 0; u < U; ++u) rr.off[u] = r.act_off[addr::small_route_index(u, tid, ns)];
    if (r.cu != nullptr) {
#pragma unroll
      for (int u = 0; u < U; ++u) rr.cu[u] = r.cu[addr::small_route_index(u, tid, ns)];
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) rr.cu[u] = 0;
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      rr.off[u] = 0;
      rr.cu[u] = 0;
    }
  }
}

// Step 2: stage sequence boundaries and offsets in LDS, gate every token, and
// return whether any token REQUESTS adapter g (before gating; exact for
// pre-gated ids) -- workgroup-uniform.  Ends with a barrier.
template <int U>
__device__ __forceinline__ bool route_gate(const SmallRoute& r, int g, RouteLds<U>& s, RouteRegs<U>& rr) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const bool gate = route_gated(r);
  const int ns = route_nseq(r);
  if (gate) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = u * kSmT + tid;
      if (k < ns) {
        s.cu[k] = rr.cu[u];
        s.off[k] = rr.off[u];
      }
    }
  }
  bool req_g = false;
#pragma unroll
  for (int u = 0; u < U; ++u) req_g |= (u * kSmT + tid < r.T) && rr.rq[u] == g;
  const uint64_t any = __ballot(req_g);
  if (lane == 0) s.wreq[wave] = any != 0;
  lds_barrier();
  const bool used = (s.wreq[0] | s.wreq[1] | s.wreq[2] | s.wreq[3]) != 0;
  // sequence of token t: the largest sq with cu[sq] <= t.  First guess: token t
  // is sequence t (a decode batch, one token per sequence), right iff
  // cu[t] <= t < cu[t+1].  Lanes whose guess fails run a fixed-step search
  // (one LDS read per token slot and step; clamped indices stay in bounds).
  int sq[U];
#pragma unroll
  for (int u = 0; u < U; ++u) sq[u] = 0;
  if (gate) {
    bool ok[U];
    bool all_ok = true;
#pragma unroll
    for (int u = 0; u < U; ++u) {
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
      for (int step = U * kSmT / 2; step > 0; step >>= 1) {
        if (step < ns) {
          int c[U];
#pragma unroll
          for (int u = 0; u < U; ++u) c[u] = s.cu[min(sq[u] + step, ns - 1)];
#pragma unroll
          for (int u = 0; u < U; ++u)
            sq[u] = (!ok[u] && sq[u] + step < ns && c[u] <= u * kSmT + tid) ? sq[u] + step : sq[u];
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int t = u * kSmT + tid;
    int64_t v = rr.rq[u];
    if (gate && t < r.T) {
      const int64_t qq = r.pos != nullptr ? rr.q[u] : static_cast<int64_t>(t - s.cu[sq[u]]);
      if (qq < s.off[sq[u]]) v = 0;
    }
    if (t >= r.T || v < 0 || v > r.NA) v = 0;
    rr.id[u] = static_cast<int>(v);
  }
  return used;
}

// Step 3: list adapter g's tokens (ascending) in s.tok and return their count;
// position = earlier (u, wave) chunks' counts + matches in lower lanes.
// Ends with a barrier.
template <int U>
__device__ __forceinline__ int route_list(int g, RouteLds<U>& s, const RouteRegs<U>& rr) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  uint64_t bal[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    bal[u] = __ballot(rr.id[u] == g);
    if (lane == 0) s.wcnt[u * 4 + wave] = __popcll(bal[u]);
  }
  lds_barrier();
  int before[U];
  int total = 0;
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if (w == wave) before[u] = total;
      total += s.wcnt[u * 4 + w];
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (rr.id[u] == g) s.tok[before[u] + __popcll(bal[u] & lanemask_lt())] = u * kSmT + tid;
  }
  lds_barrier();
  return total;
}

// 16x16 MFMA, K = 32 bf16 (one 16-byte piece per lane) or 4 x K = 4 fp32.
// Lane l supplies row (l % 16) of the A operand and column (l % 16) of the B
// operand, elements [8*(l/16), +8) of K (bf16).  Both operands pair their
// elements by (lane group, element), so any fixed assignment of k to pieces is
// a correct contraction.  Result: lane l holds D[4*(l/16) + e][l % 16], e < 4.
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

struct FusedParams {
  SmallRoute rt;
  // shrink side
  const void* x;
  int64_t ldx;
  int H;
  const void* a_pack;
  int S;
  int KS;
  int NCB;
  int RS;                 // row splits: split rs takes row chunks rs, rs + RS, ...
  int NP;                 // producer workgroups (the first NP ids)
  uint64_t* part;         // tagged partials: region (g-1) at part + (g-1)*region, [KS][cap][zw]
  int64_t region;
  int cap;
  int zw;
  // expand side
  void* y;
  int64_t ldy;
  int out_total;
  SliceInfo si;
  const void* b_pack;
  int NNT;                // column tiles per adapter
  int TG;                 // tiles per consumer (consecutive, inside one slice)
  int NG;                 // consumer tile groups per adapter (NNT / TG)
  // hand-off
  int32_t* sync;
  int64_t max_polls;      // looks at a partial group before giving up (sets the error word)
  SmallTab tab;
};

// Slice of column tile nt (tiles never straddle a slice).
template <int NT>
__device__ __forceinline__ int tile_slice(const SliceInfo& si, int nt) {
  const int n0 = nt * NT;
  int s = 0;
#pragma unroll
  for (int k = 1; k < GS_MAX_SLICES; ++k)
    if (k < si.S && n0 >= si.bounds[k]) s = k;
  return s;
}

constexpr int kZld = kSmMaxRank + 8;         // elements per LDS shrink row
constexpr int kHalf = 128;                   // y columns per delta staging pass

template <bool BF16, int U>
struct FusedLds {
  RouteLds<U> rt;
  uint32_t epoch;
  union {
    f32x4 red[4][4][64];                     // producer: per-wave sums [wave][rt*2 + c2][lane]
    struct {                                 // consumer
      __attribute__((aligned(16))) char zs[32 * kZld * Elt<BF16>::kSize];
      float dtile[32][kHalf + 4];
    } co;
  } u;
};

__device__ __forceinline__ uint64_t* launch_counter(const FusedParams& p, int g) {
  return reinterpret_cast<uint64_t*>(p.sync + kSyncLine * g);
}

// Adapter g's epoch at the start of this launch (thread 0 only).
// Adapter g's launch counter; its epoch is the value >> kEpochShift.  Issued
// with the workgroup's first loads and consumed after the routing wait, so
// the read adds no memory round trip of its own.
__device__ __forceinline__ uint64_t read_counter(const FusedParams& p, int g) {
  return __hip_atomic_load(launch_counter(p, g), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ----------------------------------------------------------------------------
// Producer: the 4 waves split the k-chunk; each holds its share of the
// adapter's 32 lora_A rows (two 16-row blocks) in registers, NPW 16-byte
// pieces per lane and block, and streams x rows in 32-token chunks (two
// 16-row tiles).  The waves' sums are added in a fixed order in LDS and wave 0
// stores the tagged partials straight from its registers.
// ----------------------------------------------------------------------------
template <bool BF16, int NPW, int NT, bool SPEC, int U>
__device__ __forceinline__ void produce(const FusedParams& p, FusedLds<BF16, U>& L, int bid) {
  constexpr int P = Elt<BF16>::kPerPiece;
  constexpr int ES = Elt<BF16>::kSize;
  constexpr int KSTEP = 4 * P;      // k per piece over the 4 lane groups
  constexpr int KW = NPW * KSTEP;   // k per wave
  // Workgroups are dealt to the 8 XCDs round-robin by id, so the NCB * RS
  // column-block and row-split siblings of one (k-chunk, adapter) -- which
  // read the same x rows or the same lora_A rows -- get ids 8 apart and share
  // an XCD's L2.  Ids past the last (k-chunk, adapter) pair have no work.
  int q, cb, rs;
  addr::small_producer(bid, p.NCB, p.RS, q, cb, rs);
  if (q >= p.KS * p.rt.NA) return;
  const int kc = q % p.KS;
  const int g = q / p.KS + 1;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int i16 = l & 15;
  const int q4 = l >> 4;
  const int r = p.tab.rank[g];
  const int ncols = p.S * r;
  const bool active = r > 0 && cb * 32 < ncols;
  const int64_t k_lo = (static_cast<int64_t>(kc) * 4 + wave) * KW;
  const int64_t k_hi = min(static_cast<int64_t>(p.H), k_lo + KW);
  int n[2];
  bool nok[2];
  const char* arow[2];
#pragma unroll
  for (int c2 = 0; c2 < 2; ++c2) {
    n[c2] = cb * 32 + 16 * c2 + i16;
    nok[c2] = active && n[c2] < ncols;
    // rows past the adapter's columns (and adapters with rank 0, whose offset
    // is 0) read row 0 of the block and are masked
    arow[c2] = static_cast<const char*>(p.a_pack) +
               (p.tab.a_off[g] + static_cast<int64_t>(nok[c2] ? n[c2] : 0) * p.H) * ES;
  }

  // lora_A: a piece outside the adapter's columns or past the k-chunk reads
  // row 0 at k 0 (finite weights) and is not masked -- past the chunk its x
  // piece is zero, and outside the columns the result is never stored -- so
  // no instruction waits on these loads before the MFMAs
  u32x4 av[2][NPW];

  const uint64_t counter = read_counter(p, g);   // one 8-byte request per wave
  RouteRegs<U> rr;
  route_issue<U>(p.rt, rr);
  // Order of the memory trips: the routing loads go out first, then the first
  // 16-row block of lora_A, so HBM streams weights while the routing is
  // waited for (loads complete in order: the routing wait does not wait for
  // them).  Once the token list is known, the x rows of the first row chunk,
  // then the second lora_A block.  Issuing all of lora_A before the wait
  // measured the same but delays the routing under load; issuing none of it
  // leaves HBM idle during the routing (3.5 % slower).
#pragma unroll
  for (int pp = 0; pp < NPW; ++pp) {
    const int64_t kp = k_lo + pp * KSTEP + q4 * P;
    const bool ok = nok[0] && kp < k_hi;
    av[0][pp] = ld_a(arow[0] + addr::reg_x_elem(ok, kp, 0) * ES);
  }
  route_gate<U>(p.rt, g, L.rt, rr);
  if (tid == 0) L.epoch = static_cast<uint32_t>(counter >> kEpochShift);   // visible after route_list's barriers
  const int n_g = route_list<U>(g, L.rt, rr);
  const int first = 32 * rs;             // this row split's first chunk
  if (!active || n_g <= first) return;
  const uint64_t tag = static_cast<uint64_t>(L.epoch + 1u) << 32;

  // x rows of one 32-token chunk.  Rows past the adapter's tokens re-read its
  // first token (their sums are never stored) and pieces past the k-chunk
  // read the row's first piece and are zeroed where they are multiplied, so
  // the loads are unconditional and go out back to back with lora_A's second
  // block: no wait for x sits between them.
  u32x4 xv[2][NPW];
  bool xk[NPW];
  auto load_x = [&](int rt0) {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int slot = rt0 + 16 * rt + i16;
      const char* xrow =
          static_cast<const char*>(p.x) + static_cast<int64_t>(L.rt.tok[addr::small_slot(slot, n_g, rt0)]) * p.ldx * ES;
#pragma unroll
      for (int pp = 0; pp < NPW; ++pp) {
        const int64_t kp = k_lo + pp * KSTEP + q4 * P;
        xk[pp] = kp < k_hi;
        xv[rt][pp] = ld16(xrow + addr::reg_x_elem(xk[pp], kp, 0) * ES);
      }
    }
  };
  load_x(first);
#pragma unroll
  for (int pp = 0; pp < NPW; ++pp) {
    const int64_t kp = k_lo + pp * KSTEP + q4 * P;
    const bool ok = nok[1] && kp < k_hi;
    av[1][pp] = ld_a(arow[1] + addr::reg_x_elem(ok, kp, 0) * ES);
  }
  __builtin_amdgcn_sched_barrier(0);   // every load above is issued before the MFMAs wait

  for (int rt0 = first; rt0 < n_g; rt0 += 32 * p.RS) {
    if (rt0 > first) load_x(rt0);
    // acc[rt][c2]: token slots rt0 + 16*rt + 4*q4 + e, column n[c2]
    f32x4 acc[2][2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        acc[rt][c2] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int pp = 0; pp < NPW; ++pp) acc[rt][c2] = mfma16<BF16>(sel16(xk[pp], xv[rt][pp]), av[c2][pp], acc[rt][c2]);
      }

    // fixed-order cross-wave sum ((w0 + w1) + w2) + w3; wave w finishes and
    // stores the 16x16 tile rc = w (row tile rc >> 1, column block rc & 1)
#pragma unroll
    for (int rc = 0; rc < 4; ++rc) L.u.red[wave][rc][l] = acc[rc >> 1][rc & 1];
    lds_barrier();
    {
      const int rt = wave >> 1;
      const int nw = cb * 32 + 16 * (wave & 1) + i16;
      const f32x4 v = ((L.u.red[0][wave][l] + L.u.red[1][wave][l]) + L.u.red[2][wave][l]) + L.u.red[3][wave][l];
      uint64_t* dst = p.part + addr::small_part(p.region, g, kc, p.cap, rt0 + 16 * rt + 4 * q4, p.zw, nw);
      const int slots = n_g - (rt0 + 16 * rt + 4 * q4);    // rows of this lane's 4 still in the batch
      if (active && nw < ncols) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (e < slots)
            __hip_atomic_store(dst + static_cast<int64_t>(e) * p.zw, tag | __float_as_uint(v[e]), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    lds_barrier();   // red is reused by the next row chunk
  }
}

// ----------------------------------------------------------------------------
// Consumer: each wave owns NQ 16-column blocks of the tile (block q*4 + wave)
// and holds their lora_B rows for the whole rank in registers.  Per 32-token
// row chunk: y rows are loaded, the tagged partials are polled and summed in
// ks order into the chunk's shrink rows in LDS (rounded like a stored z), the
// MFMA deltas go through LDS in 128-column halves, and each thread adds and
// stores 16-byte pieces of its token rows.
// ----------------------------------------------------------------------------
// RMAX: the module's largest rank rounded up to 32 or 64 (lora_B pieces held
// per column block); tile groups (TG > 1) are compiled for bf16 at RMAX = 32
// only, where the next tile's lora_B and y fit beside the current tile's.
template <bool BF16, int NQ, bool SPEC, int U, int RMAX>
__device__ __forceinline__ void consume(const FusedParams& p, FusedLds<BF16, U>& L, int cid) {
  constexpr int NT = 64 * NQ;
  constexpr int NH = NQ / 2;            // 128-column halves
  constexpr int P = Elt<BF16>::kPerPiece;
  constexpr int ES = Elt<BF16>::kSize;
  constexpr int KSTEP = 4 * P;          // rank per MFMA (over the 4 lane groups)
  constexpr int KG = RMAX / KSTEP;
  constexpr int EPL = 16 / ES;          // y elements per 16-byte piece
  constexpr int LPR = kHalf / EPL;      // lanes per y row in a half
  constexpr int RPP = kSmT / LPR;       // y rows per workgroup-wide access
  constexpr int PASSES = 32 / RPP;
  constexpr int EPT = 4;                // shrink elements per thread and batch
  constexpr int NEB = 32 * kSmMaxRank / (kSmT * EPT);   // batches (rank <= 64)
  constexpr bool kTileGroups = BF16 && RMAX == 32;       // the next tile's lora_B and y fit beside the current's

  // (tile group, adapter) items are dealt to the XCDs by the low 3 id bits;
  // the RS row-split siblings of an item, which read the same lora_B rows, get
  // ids 8 apart and share an XCD's L2.  Ids past the last item have no work.
  int item, rs;
  addr::small_consumer(cid, p.RS, item, rs);
  if (item >= p.NG * p.rt.NA) return;
  const int grp = item % p.NG;
  const int g = item / p.NG + 1;
  const int nt0 = grp * p.TG;            // the group's first tile (all of its tiles lie in one slice)
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int i16 = l & 15;
  const int q4 = l >> 4;
  const int r = p.tab.rank[g];
  const int s = tile_slice<NT>(p.si, nt0);
  const int zc0 = s * r;                 // this slice's columns in the adapter's shrink row

  const uint64_t counter = read_counter(p, g);   // one 8-byte request per wave
  RouteRegs<U> rr;
  route_issue<U>(p.rt, rr);
  // lora_B rows of this wave's column blocks of tile nt (n < out_total always;
  // rank 0 reads element 0 of the pack and is masked).  Pieces past the rank
  // read the row's first piece and are not masked: the MFMAs multiply them by
  // shrink values that are zeroed there, so no instruction waits on these
  // loads before later loads go out.
  auto load_b = [&](int nt, u32x4 (&bv)[NQ][KG]) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int n = nt * NT + 16 * (q * 4 + wave) + i16;
      const char* brow = static_cast<const char*>(p.b_pack) + (p.tab.b_off[g] + static_cast<int64_t>(n) * r) * ES;
#pragma unroll
      for (int kg = 0; kg < KG; ++kg) {
        const int k0 = kg * KSTEP + q4 * P;
        bv[q][kg] = ld16(brow + addr::k_or_zero(k0, r) * ES);
      }
    }
  };
  u32x4 bv[NQ][KG];
  // SPEC: tile nt0's lora_B in the first memory trip, while the producers
  // wait for their token lists
  if constexpr (SPEC) load_b(nt0, bv);
  const bool requested = route_gate<U>(p.rt, g, L.rt, rr);
  if (tid == 0) L.epoch = static_cast<uint32_t>(counter >> kEpochShift);   // visible after route_list's barriers
  if constexpr (!SPEC) {
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
      for (int kg = 0; kg < KG; ++kg) bv[q][kg] = u32x4{0u, 0u, 0u, 0u};
    if (requested) load_b(nt0, bv);
  }
  const int n_g = route_list<U>(g, L.rt, rr);
  if (r == 0 || n_g == 0) return;       // no producer wrote partials for it
  const uint32_t want = L.epoch + 1u;
  const int64_t kstride = static_cast<int64_t>(p.cap) * p.zw;
  // this consumer's share of the 2^20 that g's NG * RS consumers add per launch
  const int ncons = p.NG * p.RS;
  const int cidx = rs * p.NG + grp;
  const uint64_t weight = (uint64_t{1} << kEpochShift) / ncons + (cidx < (1 << kEpochShift) % ncons ? 1 : 0);
  const int cx = (tid % LPR) * EPL;

  for (int rt0 = 32 * rs; rt0 < n_g; rt0 += 32 * p.RS) {
    // tile nt0's lora_B again for a later row chunk when other tiles of the
    // group have used the registers since
    if (p.TG > 1 && rt0 != 32 * rs) load_b(nt0, bv);
    // y pieces of tile nt0 for this row chunk (issued before the wait)
    u32x4 yv[NH][PASSES];
    int64_t yoff[PASSES];
    bool rok[PASSES];
    // (rows past the adapter's tokens re-read the chunk's first row and are
    // never stored: unconditional loads keep the wait counts exact)
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      const int row = rt0 + ps * RPP + tid / LPR;
      rok[ps] = row < n_g;
      yoff[ps] = static_cast<int64_t>(L.rt.tok[addr::small_slot(row, n_g, rt0)]) * p.ldy + nt0 * NT + cx;
#pragma unroll
      for (int hf = 0; hf < NH; ++hf) yv[hf][ps] = ld_y(static_cast<const char*>(p.y) + (yoff[ps] + hf * kHalf) * ES);
    }

    // shrink rows of the chunk: element m of batch eb of this thread is
    // (row, c) = divmod(tid + 256*(EPT*eb + m), r); partials polled kKsGrp at
    // a time and summed in ks order, then rounded like a stored z
    for (int eb = 0; eb < NEB; ++eb) {
      if (kSmT * EPT * eb >= 32 * r) break;
      float sum[EPT];
      const uint64_t* src[EPT];
      bool eok[EPT];
#pragma unroll
      for (int m = 0; m < EPT; ++m) {
        const int e = tid + kSmT * (EPT * eb + m);
        const int row = e / r;
        const int c = e - row * r;
        eok[m] = e < 32 * r && rt0 + row < n_g;
        src[m] = p.part + addr::small_part(p.region, g, 0, p.cap, rt0 + (eok[m] ? row : 0), p.zw, zc0 + (eok[m] ? c : 0));
        sum[m] = 0.f;
      }
      for (int ks0 = 0; ks0 < p.KS; ks0 += kKsGrp) {
        uint64_t pv[EPT][kKsGrp];
#pragma unroll
        for (int m = 0; m < EPT; ++m)
#pragma unroll
          for (int u = 0; u < kKsGrp; ++u) pv[m][u] = static_cast<uint64_t>(want) << 32;
        // At most max_polls looks: counting looks instead of time keeps the
        // bound from expiring while the queue is preempted
        for (int64_t polls = 0;; ++polls) {
          if (polls >= p.max_polls) {
            __hip_atomic_fetch_or(p.sync + kSyncErrWord, kErrTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
          bool ready = true;
#pragma unroll
          for (int m = 0; m < EPT; ++m)
#pragma unroll
            for (int u = 0; u < kKsGrp; ++u) {
              pv[m][u] = static_cast<uint64_t>(want) << 32;
              if (eok[m] && ks0 + u < p.KS)
                pv[m][u] = __hip_atomic_load(src[m] + (ks0 + u) * kstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
          for (int m = 0; m < EPT; ++m)
#pragma unroll
            for (int u = 0; u < kKsGrp; ++u) ready = ready && static_cast<uint32_t>(pv[m][u] >> 32) == want;
          if (ready) break;
          __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int m = 0; m < EPT; ++m)
#pragma unroll
          for (int u = 0; u < kKsGrp; ++u)
            if (ks0 + u < p.KS) sum[m] += __uint_as_float(static_cast<uint32_t>(pv[m][u]));
      }
#pragma unroll
      for (int m = 0; m < EPT; ++m) {
        const int e = tid + kSmT * (EPT * eb + m);
        if (e < 32 * r) {
          const int row = e / r;
          const int c = e - row * r;
          char* dst = L.u.co.zs + (row * kZld + c) * ES;
          if constexpr (BF16) *reinterpret_cast<uint16_t*>(dst) = f32_to_bf16_bits(sum[m]);
          else *reinterpret_cast<float*>(dst) = sum[m];
        }
      }
    }
    lds_barrier();

    // One tile of the group: D[t][n] = sum_k z[t][k] B[n][k] (acc[rt][q]: token
    // 16*rt + 4*q4 + e of the chunk, column 16*(q*4 + wave) + i16 of the tile),
    // through LDS in 128-column halves, added to the tile's y pieces and stored.
    // Every y piece is combined with its delta before the tile's first store:
    // on gfx9 stores count in the same in-order counter as loads.
    auto tile_out = [&](const u32x4 (&b)[NQ][KG], const u32x4 (&yin)[NH][PASSES], int col) {
      f32x4 acc[2][NQ];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int q = 0; q < NQ; ++q) acc[rt][q] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kg = 0; kg < KG; ++kg) {
        if (kg * KSTEP < r) {
          const int k0 = kg * KSTEP + q4 * P;
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            const bool kin = k0 < r;
            const u32x4 za =
                sel16(kin, *reinterpret_cast<const u32x4*>(L.u.co.zs + ((16 * rt + i16) * kZld + (kin ? k0 : 0)) * ES));
#pragma unroll
            for (int q = 0; q < NQ; ++q) acc[rt][q] = mfma16<BF16>(za, b[q][kg], acc[rt][q]);
          }
        }
      }
      u32x4 yo[NH][PASSES];
#pragma unroll
      for (int hf = 0; hf < NH; ++hf) {
#pragma unroll
        for (int qq = 0; qq < 2; ++qq) {
          const int q = 2 * hf + qq;
          const int cc = 16 * (qq * 4 + wave) + i16;      // within the half
#pragma unroll
          for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int e = 0; e < 4; ++e) L.u.co.dtile[16 * rt + 4 * q4 + e][cc] = acc[rt][q][e];
        }
        lds_barrier();
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps) {
          const int row = ps * RPP + tid / LPR;
          float d[EPL];
#pragma unroll
          for (int e = 0; e < EPL; ++e) d[e] = L.u.co.dtile[row][cx + e];
          yo[hf][ps] = add_y16<BF16>(yin[hf][ps], d);
        }
        lds_barrier();   // dtile is reused
      }
#pragma unroll
      for (int hf = 0; hf < NH; ++hf)
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps)
          if (rok[ps]) st_y(static_cast<char*>(p.y) + (yoff[ps] + col + hf * kHalf) * ES, yo[hf][ps]);
    };

    if (!kTileGroups || p.TG == 1) {
      tile_out(bv, yv, 0);
    } else if constexpr (kTileGroups) {
      // tiles 1.. of the group: the next tile's lora_B and y go out before the
      // current tile is computed
      u32x4 bn[NQ][KG], yn[NH][PASSES];
      auto load_y = [&](int t, u32x4 (&yt)[NH][PASSES]) {
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps)
#pragma unroll
          for (int hf = 0; hf < NH; ++hf)
            yt[hf][ps] = ld_y(static_cast<const char*>(p.y) + (yoff[ps] + t * NT + hf * kHalf) * ES);
      };
      load_b(nt0 + 1, bn);
      load_y(1, yn);
      tile_out(bv, yv, 0);
      for (int t = 1; t < p.TG; ++t) {
#pragma unroll
        for (int q = 0; q < NQ; ++q)
#pragma unroll
          for (int kg = 0; kg < KG; ++kg) bv[q][kg] = bn[q][kg];
#pragma unroll
        for (int hf = 0; hf < NH; ++hf)
#pragma unroll
          for (int ps = 0; ps < PASSES; ++ps) yv[hf][ps] = yn[hf][ps];
        const int tn = t + 1 < p.TG ? t + 1 : t;      // the last tile re-reads itself (no extra line)
        load_b(nt0 + tn, bn);
        load_y(tn, yn);
        tile_out(bv, yv, t * NT);
      }
    }
  }
  // every thread has had all its partials (barriers since): add this
  // consumer's weight; issued last and never waited for, since on gfx9 a
  // wait for any later load would also wait for it
  if (tid == 0)
    __hip_atomic_fetch_add(launch_counter(p, g), weight, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool BF16, int NPW, int NQ, bool SPEC, int U, int RMAX>
__global__ __launch_bounds__(kSmT) void small_fused_kernel(FusedParams p) {
  __shared__ FusedLds<BF16, U> lds;
  const int bid = static_cast<int>(blockIdx.x);
  if (bid < p.NP) produce<BF16, NPW, 64 * NQ, SPEC, U>(p, lds, bid);
  else consume<BF16, NQ, SPEC, U, RMAX>(p, lds, bid - p.NP);
}

// ----------------------------------------------------------------------------
// Host-side plan.
// ----------------------------------------------------------------------------
struct SmallPlan {
  int NPW, KS, NCB, cap, zw, NQ, NNT, TG;
  int64_t region_bytes;       // one adapter's tagged partials
};

// about this many producer workgroups: fewer means fewer split-K partials for
// each consumer to wait for and add, more means more loads in flight
#ifndef GS_SMALL_TARGET_PRODUCERS
#define GS_SMALL_TARGET_PRODUCERS 128
#endif
constexpr int kSmTargetShrinkWgs = GS_SMALL_TARGET_PRODUCERS;
#ifndef GS_SMALL_TILE_GROUP
#define GS_SMALL_TILE_GROUP 8
#endif
constexpr int kSmTileGroup = GS_SMALL_TILE_GROUP;      // most column tiles one consumer walks
// Looks a consumer takes at one group of partials before it gives up.  One
// look is a coherent load round trip (>= ~0.3 us) plus a short sleep, so the
// default bounds the wait at tens to hundreds of milliseconds; a completed
// hand-off takes a few microseconds.
constexpr int64_t kDefaultWaitPolls = 200000;
std::atomic<int64_t> g_wait_polls{kDefaultWaitPolls};
constexpr int64_t kSyncBytes = 4 * kSyncLine * (kSmMaxAdapters + 1);

// The row split RS multiplies the producers like the k-split does, so it
// counts towards the target: a larger RS never gives a larger KS (and so
// never a larger workspace than RS = 1).
SmallPlan plan_small(int64_t T, int H, int S, int NA, int max_rank, bool bf16, int out_total,
                     const int32_t* slice_bounds, int RS = 1) {
  SmallPlan pl{};
  pl.zw = S * max_rank;
  pl.NCB = (pl.zw + 31) / 32;
  const int kstep = bf16 ? 32 : 16;      // k of one piece over the 4 lane groups
  // largest pieces per wave (fewest partials for the consumers to add) that
  // still gives about kSmTargetShrinkWgs producers
  int npw = 8;
  int ks = 1;
  for (;;) {
    ks = (H + 4 * npw * kstep - 1) / (4 * npw * kstep);
    if (static_cast<int64_t>(NA) * pl.NCB * ks * RS >= kSmTargetShrinkWgs || npw == 4) break;
    npw >>= 1;
  }
  pl.NPW = npw;
  pl.KS = ks;
  pl.cap = static_cast<int>(((T + 31) / 32) * 32);
  bool all256 = true;
  for (int s = 0; s < S; ++s)
    if ((slice_bounds[s + 1] - slice_bounds[s]) % 256 != 0) all256 = false;
  pl.NQ = all256 ? 4 : 2;
  pl.NNT = out_total / (64 * pl.NQ);
  // Tiles per consumer: the smallest group (a divisor of every slice's tile
  // count, so it never straddles a slice) that brings the consumers within 2
  // per CU, else the largest allowed.  Each consumer polls its partials once
  // and walks its tiles, so long groups serialise: measured on decode batches
  // (gate_up 4096 -> 25600, 24 adapters, T = 128: no groups 30.6 us, groups
  // of 5 18.1, of 10 20.3; groups of 16 on a 4096-wide down projection were
  // 1.5x slower than none).
  const int64_t limit = 2 * static_cast<int64_t>(device_cus());
  pl.TG = 1;
  for (int d = 1; d <= (bf16 && max_rank <= 32 ? kSmTileGroup : 1); ++d) {
    bool ok = true;
    for (int s = 0; s < S; ++s)
      if (((slice_bounds[s + 1] - slice_bounds[s]) / (64 * pl.NQ)) % d != 0) ok = false;
    if (!ok) continue;
    pl.TG = d;
    if (8 * static_cast<int64_t>(RS) * ((static_cast<int64_t>(pl.NNT / d) * NA + 7) / 8) <= limit) break;
  }
  pl.region_bytes = static_cast<int64_t>(pl.KS) * pl.cap * pl.zw * 8;
  return pl;
}

// Producers: NCB * RS siblings for each group of 8 (k-chunk, adapter) pairs.
// Consumers: RS siblings for each group of 8 (tile, adapter) items.
int64_t producer_wgs(const SmallPlan& pl, int NA, int RS) {
  return 8 * static_cast<int64_t>(pl.NCB) * RS * ((static_cast<int64_t>(pl.KS) * NA + 7) / 8);
}
int64_t consumer_wgs(const SmallPlan& pl, int NA, int RS) {
  return 8 * static_cast<int64_t>(RS) * ((static_cast<int64_t>(pl.NNT / pl.TG) * NA + 7) / 8);
}

template <bool BF16, int NQ, bool SPEC, int U, int RMAX>
void launch_fused_r(const SmallPlan& pl, const FusedParams& fp, unsigned grid, hipStream_t st) {
  switch (pl.NPW) {
    case 8: hipLaunchKernelGGL((small_fused_kernel<BF16, 8, NQ, SPEC, U, RMAX>), dim3(grid), dim3(kSmT), 0, st, fp); break;
    default: hipLaunchKernelGGL((small_fused_kernel<BF16, 4, NQ, SPEC, U, RMAX>), dim3(grid), dim3(kSmT), 0, st, fp); break;
  }
}

template <bool BF16, int NQ, bool SPEC, int U>
void launch_fused_nq(const SmallPlan& pl, const FusedParams& fp, unsigned grid, hipStream_t st) {
  if (pl.zw <= 32 * fp.S) launch_fused_r<BF16, NQ, SPEC, U, 32>(pl, fp, grid, st);
  else launch_fused_r<BF16, NQ, SPEC, U, 64>(pl, fp, grid, st);
}

template <bool BF16, bool SPEC, int U>
void launch_fused_spec(const SmallPlan& pl, const FusedParams& fp, unsigned grid, hipStream_t st) {
  if (pl.NQ == 4) launch_fused_nq<BF16, 4, SPEC, U>(pl, fp, grid, st);
  else launch_fused_nq<BF16, 2, SPEC, U>(pl, fp, grid, st);
}

// U = 1 routes batches of up to 256 tokens and sequences, U = 4 up to 1024.
template <bool BF16, int U>
void launch_fused_u(const SmallPlan& pl, const FusedParams& fp, unsigned grid, bool spec, hipStream_t st) {
  if (spec) launch_fused_spec<BF16, true, U>(pl, fp, grid, st);
  else launch_fused_spec<BF16, false, U>(pl, fp, grid, st);
}

template <bool BF16>
void launch_fused(const SmallPlan& pl, const FusedParams& fp, unsigned grid, bool spec, hipStream_t st) {
  if (fp.rt.T <= kSmT && fp.rt.num_seqs <= kSmT) launch_fused_u<BF16, 1>(pl, fp, grid, spec, st);
  else launch_fused_u<BF16, kSmMaxU>(pl, fp, grid, spec, st);
}

// ----------------------------------------------------------------------------
// Address model (test support): replays on the host every global and LDS
// access of small_fused_kernel for one call -- routing, every producer and
// consumer workgroup, wave, lane and loop step, with the call's own plan and
// the addr:: formulas the kernel uses -- and checks each access against its
// buffer.  The adapters' token lists (which the kernel's routing computes)
// come from the host copy of the gated ids.  No HIP call is made.
// ----------------------------------------------------------------------------
struct SmallModel {
  bool bf16;
  int64_t T;
  int H;
  int64_t ldx;
  int out_total;
  int64_t ldy;
  int S;
  const int64_t* a_off;
  const int64_t* b_off;
  const int32_t* rank;
  int64_t a_elems, b_elems;
  int NA;
  int nseq;
  bool has_eff, has_pos, has_cu, has_act;
  int64_t ws_elems;                 // 8-byte elements of the workspace
  int64_t sync_words;
  std::vector<std::vector<int>> toks;   // toks[g]: adapter g's tokens, ascending
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
  int es() const { return bf16 ? 2 : 4; }
  int P() const { return bf16 ? 8 : 4; }
  // the routing of one workgroup (route_issue / route_gate / route_list)
  void routing(int U) {
    for (int tid = 0; tid < kSmT; ++tid)
      for (int u = 0; u < U; ++u) {
        const int k = u * kSmT + tid;
        if (has_eff) in("eff_ids", addr::small_route_index(u, tid, static_cast<int>(T)), 1, T);
        else in("req_ids", addr::small_route_index(u, tid, static_cast<int>(T)), 1, T);
        if (!has_eff && has_pos) in("positions", addr::small_route_index(u, tid, static_cast<int>(T)), 1, T);
        if (!has_eff && has_act) {
          in("act_offsets", addr::small_route_index(u, tid, nseq), 1, nseq);
          if (has_cu) in("cu_seqlens", addr::small_route_index(u, tid, nseq), 1, nseq + 1);
          if (k < nseq) in("sequence table (LDS)", k, 1, U * kSmT);
        }
        in("token list (LDS)", k, 1, U * kSmT);
      }
  }
  void counter(int g) { in("launch counter", static_cast<int64_t>(kSyncLine) * g, 2, sync_words); }

  void produce(const SmallPlan& pl, int RS, int bid, int U) {
    int q, cb, rs;
    addr::small_producer(bid, pl.NCB, RS, q, cb, rs);
    if (q >= pl.KS * NA) return;
    const int kc = q % pl.KS, g = q / pl.KS + 1;
    const int r = rank[g], ncols = S * r;
    const bool active = r > 0 && cb * 32 < ncols;
    const int KSTEP = 4 * P(), KW = pl.NPW * KSTEP;
    const std::vector<int>& tk = toks[g];
    const int n_g = static_cast<int>(tk.size());
    const int first = 32 * rs;
    counter(g);
    routing(U);
    for (int c2 = 0; c2 < 2; ++c2) {
      if (c2 == 1 && (!active || n_g <= first)) break;   // the second block goes out with the first x rows
      for (int wave = 0; wave < 4; ++wave) {
        const int64_t k_lo = (static_cast<int64_t>(kc) * 4 + wave) * KW;
        const int64_t k_hi = std::min<int64_t>(H, k_lo + KW);
        for (int l = 0; l < 64; ++l) {
          const int i16 = l & 15, q4 = l >> 4;
          const int n = cb * 32 + 16 * c2 + i16;
          const bool nok = active && n < ncols;
          for (int pp = 0; pp < pl.NPW; ++pp) {
            const int64_t kp = k_lo + pp * KSTEP + q4 * P();
            const bool ok = nok && kp < k_hi;
            const int64_t e = a_off[g] + static_cast<int64_t>(nok ? n : 0) * H + addr::reg_x_elem(ok, kp, 0);
            if (in("lora_A row", nok ? n : 0, 1, std::max(ncols, 1))) in("lora_A", e, P(), a_elems);
          }
        }
      }
    }
    if (!active || n_g <= first) return;
    for (int rt0 = first; rt0 < n_g; rt0 += 32 * RS) {
      for (int wave = 0; wave < 4; ++wave) {
        const int64_t k_lo = (static_cast<int64_t>(kc) * 4 + wave) * KW;
        const int64_t k_hi = std::min<int64_t>(H, k_lo + KW);
        for (int l = 0; l < 64; ++l) {
          const int i16 = l & 15, q4 = l >> 4;
          for (int rt = 0; rt < 2; ++rt) {
            const int sl = addr::small_slot(rt0 + 16 * rt + i16, n_g, rt0);
            in("token list read (LDS)", sl, 1, U * kSmT);
            if (!in("token slot (the adapter's listed tokens)", sl, 1, n_g)) continue;
            const int tok = tk[sl];
            for (int pp = 0; pp < pl.NPW; ++pp) {
              const int64_t kp = k_lo + pp * KSTEP + q4 * P();
              if (in("x row", tok, 1, T)) in("x", static_cast<int64_t>(tok) * ldx + addr::reg_x_elem(kp < k_hi, kp, 0), P(), (T - 1) * ldx + H);
            }
          }
          // the stores of the tile wave w finishes
          const int rt = wave >> 1, nw = cb * 32 + 16 * (wave & 1) + i16;
          const int slot0 = rt0 + 16 * rt + 4 * q4;
          if (active && nw < ncols)
            for (int e = 0; e < 4; ++e)
              if (e < n_g - slot0) {
                in("partial slot", slot0 + e, 1, pl.cap);
                in("partial column", nw, 1, pl.zw);
                in("tagged partials", addr::small_part(pl.region_bytes / 8, g, kc, pl.cap, slot0 + e, pl.zw, nw), 1,
                   ws_elems);
              }
        }
      }
    }
  }

  void consume(const SmallPlan& pl, int RS, int cid, int U, int64_t region) {
    int item, rs;
    addr::small_consumer(cid, RS, item, rs);
    const int NG = pl.NNT / pl.TG;
    if (item >= NG * NA) return;
    const int grp = item % NG, g = item / NG + 1, nt0 = grp * pl.TG;
    const int NQ = pl.NQ, NT = 64 * NQ, NH = NQ / 2;
    const int r = rank[g];
    int s = 0;
    for (int k = 1; k < S; ++k)
      if (nt0 * NT >= sb[k]) s = k;
    const int zc0 = s * r;
    const int KSTEP = 4 * P(), RMAX = pl.zw <= 32 * S ? 32 : 64, KG = RMAX / KSTEP;
    const int EPL = 16 / es(), LPR = kHalf / EPL, RPP = kSmT / LPR, PASSES = 32 / RPP;
    const std::vector<int>& tk = toks[g];
    const int n_g = static_cast<int>(tk.size());
    counter(g);
    routing(U);
    auto load_b = [&](int nt) {
      in("column tile", nt, 1, pl.NNT);
      for (int wave = 0; wave < 4; ++wave)
        for (int l = 0; l < 64; ++l) {
          const int i16 = l & 15, q4 = l >> 4;
          for (int q = 0; q < NQ; ++q) {
            const int64_t n = static_cast<int64_t>(nt) * NT + 16 * (q * 4 + wave) + i16;
            in("lora_B column", n, 1, out_total);
            for (int kg = 0; kg < KG; ++kg)
              in("lora_B", b_off[g] + n * r + addr::k_or_zero(kg * KSTEP + q4 * P(), r), P(), b_elems);
          }
        }
    };
    load_b(nt0);
    if (r == 0 || n_g == 0) return;
    for (int rt0 = 32 * rs; rt0 < n_g; rt0 += 32 * RS) {
      if (pl.TG > 1 && rt0 != 32 * rs) load_b(nt0);
      for (int tid = 0; tid < kSmT; ++tid) {
        const int cx = (tid % LPR) * EPL;
        for (int ps = 0; ps < PASSES; ++ps) {
          const int row = rt0 + ps * RPP + tid / LPR;
          const int sl = addr::small_slot(row, n_g, rt0);
          in("token list read (LDS)", sl, 1, U * kSmT);
          if (!in("token slot (the adapter's listed tokens)", sl, 1, n_g)) continue;
          const int64_t yoff = static_cast<int64_t>(tk[sl]) * ldy + static_cast<int64_t>(nt0) * NT + cx;
          for (int t = 0; t < pl.TG; ++t)
            for (int hf = 0; hf < NH; ++hf) {
              in("y column", static_cast<int64_t>(nt0) * NT + cx + t * NT + hf * kHalf, EPL, out_total);
              in("y", yoff + t * NT + hf * kHalf, EPL, (T - 1) * ldy + out_total);
            }
          in("delta tile read (LDS)", (ps * RPP + tid / LPR) * (kHalf + 4) + cx, EPL, 32 * (kHalf + 4));
        }
        // the chunk's shrink rows: partials polled and staged
        for (int eb = 0; eb < 2; ++eb) {
          if (kSmT * 4 * eb >= 32 * r) break;
          for (int m = 0; m < 4; ++m) {
            const int e = tid + kSmT * (4 * eb + m);
            const int row = e / r, c = e - row * r;
            const bool eok = e < 32 * r && rt0 + row < n_g;
            if (eok)
              for (int ks = 0; ks < pl.KS; ++ks) {
                in("partial column (consumer)", zc0 + c, 1, pl.zw);
                in("tagged partials (consumer)",
                   addr::small_part(region, g, ks, pl.cap, rt0 + row, pl.zw, zc0 + c), 1, ws_elems);
              }
            if (e < 32 * r) in("shrink rows (LDS)", (static_cast<int64_t>(row) * kZld + c) * es(), es(), 32 * kZld * es());
          }
        }
      }
      // the MFMAs' shrink-row reads
      for (int l = 0; l < 64; ++l) {
        const int i16 = l & 15, q4 = l >> 4;
        for (int kg = 0; kg < KG; ++kg) {
          if (kg * KSTEP >= r) continue;
          const int k0 = kg * KSTEP + q4 * P();
          for (int rt = 0; rt < 2; ++rt)
            in("shrink rows read (LDS)", ((16 * rt + i16) * kZld + (k0 < r ? k0 : 0)) * es(), 16, 32 * kZld * es());
        }
      }
      for (int t = 1; t < pl.TG; ++t) load_b(nt0 + t);
    }
    in("error word", kSyncErrWord, 1, sync_words);
  }
  int sb[GS_MAX_SLICES + 1];
};
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
  return kSmMaxAdapters * pl.region_bytes;
}

int64_t gs_small_sync_bytes(void) { return kSyncBytes; }

int64_t gs_small_set_wait_limit(int64_t polls) {
  const int64_t v = polls < 0 ? kDefaultWaitPolls : polls;
  return g_wait_polls.exchange(v, std::memory_order_relaxed);
}

int64_t gs_small_workgroups(int32_t dtype, int64_t num_tokens, int32_t hidden, int32_t num_slices,
                            int32_t num_adapters, int32_t max_rank, int32_t out_total,
                            const int32_t* slice_bounds, int32_t row_split) {
  if (num_tokens <= 0 || hidden <= 0 || slice_bounds == nullptr || num_adapters < 1) return 0;
  if (row_split < 1 || row_split > kSmMaxRowSplit) return 0;
  const SmallPlan pl = plan_small(num_tokens, hidden, num_slices, num_adapters, max_rank, dtype == GS_DTYPE_BF16,
                                  out_total, slice_bounds, row_split);
  return producer_wgs(pl, num_adapters, row_split) + consumer_wgs(pl, num_adapters, row_split);
}

int gs_switched_lora_small(int32_t dtype, const int64_t* req_ids, const int64_t* positions,
                           const int32_t* cu_seqlens, const int64_t* act_offsets, int32_t num_seqs,
                           const int32_t* eff_ids, const void* x, int64_t ldx, void* y, int64_t ldy,
                           int64_t num_tokens, int32_t hidden, int32_t out_total, const int32_t* slice_bounds,
                           int32_t num_slices, const void* a_pack, const int64_t* a_off, const void* b_pack,
                           const int64_t* b_off, const int32_t* ranks, int32_t num_adapters, int32_t max_rank,
                           void* workspace, int64_t workspace_bytes, int32_t* sync, int64_t sync_bytes,
                           int32_t row_split, int32_t speculate, void* stream) {
  const char* who = "gs_switched_lora_small";
  GS_CHECK_ARG(dtype == GS_DTYPE_BF16 || dtype == GS_DTYPE_FP32, "%s: dtype=%d", who, dtype);
  const int nseq = (cu_seqlens != nullptr) ? num_seqs : 1;
  GS_CHECK_ARG(gs_small_eligible(num_tokens, nseq, num_slices, slice_bounds, num_adapters, max_rank),
               "%s: shape outside the small-batch path (T <= %d, <= %d adapters, max_rank <= %d, slice widths "
               "multiples of 128)", who, kSmMaxTokens, kSmMaxAdapters, kSmMaxRank);
  GS_CHECK_ARG(nseq >= 1, "%s: num_seqs=%d", who, num_seqs);
  GS_CHECK_ARG(row_split >= 1 && row_split <= kSmMaxRowSplit, "%s: row_split=%d outside [1, %d]", who, row_split,
               kSmMaxRowSplit);
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
  GS_CHECK_ARG(sync != nullptr && (reinterpret_cast<uintptr_t>(sync) & 7u) == 0, "%s: sync must be 8-byte aligned",
               who);
  GS_CHECK_ARG(sync_bytes >= kSyncBytes, "%s: sync buffer of %lld bytes needed (got %lld)", who,
               (long long)kSyncBytes, (long long)sync_bytes);
  if (num_tokens == 0) return GS_OK;
  const bool bf16 = dtype == GS_DTYPE_BF16;
  const SmallPlan pl = plan_small(num_tokens, hidden, num_slices, num_adapters, max_rank, bf16, out_total,
                                  slice_bounds, row_split);
  // adapter regions are a fixed fraction of the workspace, whatever the shape
  const int64_t region_bytes = (workspace_bytes / kSmMaxAdapters) & ~int64_t(15);
  if (region_bytes < pl.region_bytes) {
    set_error("%s: workspace of %lld bytes needed (got %lld)", who, (long long)(kSmMaxAdapters * pl.region_bytes),
              (long long)workspace_bytes);
    return GS_ERR_WORKSPACE;
  }
  FusedParams fp{};
  fp.rt = SmallRoute{eff_ids != nullptr ? nullptr : req_ids, positions, cu_seqlens, act_offsets, eff_ids,
                     static_cast<int>(num_tokens), nseq, num_adapters};
  for (int g = 0; g <= num_adapters; ++g) {
    fp.tab.a_off[g] = a_off[g];
    fp.tab.b_off[g] = b_off[g];
    fp.tab.rank[g] = ranks[g];
  }
  fp.x = x;
  fp.ldx = ldx;
  fp.H = hidden;
  fp.a_pack = a_pack;
  fp.S = num_slices;
  fp.KS = pl.KS;
  fp.NCB = pl.NCB;
  fp.RS = row_split;
  fp.NP = static_cast<int>(producer_wgs(pl, num_adapters, row_split));
  fp.part = static_cast<uint64_t*>(workspace);
  fp.region = region_bytes / 8;
  fp.cap = pl.cap;
  fp.zw = pl.zw;
  fp.y = y;
  fp.ldy = ldy;
  fp.out_total = out_total;
  fp.si.S = num_slices;
  for (int s = 0; s <= num_slices; ++s) fp.si.bounds[s] = slice_bounds[s];
  fp.b_pack = b_pack;
  fp.NNT = pl.NNT;
  fp.TG = pl.TG;
  fp.NG = pl.NNT / pl.TG;
  // tile groups exist only in the bf16, rank <= 32 instantiation (kTileGroups)
  GS_CHECK_ARG(pl.TG == 1 || (bf16 && max_rank <= 32 && pl.NNT % pl.TG == 0), "%s: tile group %d for this module",
               who, pl.TG);
  fp.sync = sync;
  fp.max_polls = g_wait_polls.load(std::memory_order_relaxed);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>(fp.NP + consumer_wgs(pl, num_adapters, row_split));
  if (bf16) launch_fused<true>(pl, fp, grid, speculate != 0, st);
  else launch_fused<false>(pl, fp, grid, speculate != 0, st);
  GS_CHECK_LAUNCH(who);
  return GS_OK;
}

int64_t gs_check_small_addresses(int32_t dtype, int64_t num_tokens, int32_t hidden, int64_t ldx, int32_t out_total,
                                 int64_t ldy, const int32_t* slice_bounds, int32_t num_slices, const int64_t* a_off,
                                 int64_t a_pack_elems, const int64_t* b_off, int64_t b_pack_elems,
                                 const int32_t* ranks, int32_t num_adapters, int32_t max_rank, const int32_t* eff_ids,
                                 int32_t num_seqs, int32_t route_flags, int32_t row_split, char* msg, int64_t msg_len,
                                 int64_t* checked) {
  const char* who = "gs_check_small_addresses";
  GS_CHECK_ARG(dtype == GS_DTYPE_BF16 || dtype == GS_DTYPE_FP32, "%s: dtype=%d", who, dtype);
  const bool has_cu = (route_flags & 4) != 0;
  const int nseq = has_cu ? num_seqs : 1;
  GS_CHECK_ARG(gs_small_eligible(num_tokens, nseq, num_slices, slice_bounds, num_adapters, max_rank),
               "%s: shape outside the small-batch path", who);
  GS_CHECK_ARG(row_split >= 1 && row_split <= kSmMaxRowSplit && nseq >= 1, "%s: row_split / num_seqs", who);
  GS_CHECK_ARG(a_off && b_off && ranks && (eff_ids || num_tokens == 0), "%s: NULL table", who);
  SmallModel m{};
  m.bf16 = dtype == GS_DTYPE_BF16;
  m.T = num_tokens;
  m.H = hidden;
  m.ldx = ldx;
  m.out_total = out_total;
  m.ldy = ldy;
  m.S = num_slices;
  for (int s = 0; s <= num_slices; ++s) m.sb[s] = slice_bounds[s];
  m.a_off = a_off;
  m.b_off = b_off;
  m.rank = ranks;
  m.a_elems = a_pack_elems;
  m.b_elems = b_pack_elems;
  m.NA = num_adapters;
  m.nseq = nseq;
  m.has_eff = (route_flags & 1) != 0;
  m.has_pos = (route_flags & 2) != 0;
  m.has_cu = has_cu;
  m.has_act = (route_flags & 8) != 0;
  m.sync_words = kSyncBytes / 4;
  m.toks.assign(num_adapters + 1, {});
  for (int64_t t = 0; t < num_tokens; ++t) {
    const int v = eff_ids[t];
    if (v >= 1 && v <= num_adapters) m.toks[v].push_back(static_cast<int>(t));
  }
  if (num_tokens > 0) {
    const int64_t ws_bytes = gs_small_workspace_bytes(dtype, num_tokens, hidden, num_slices, num_adapters, max_rank,
                                                      out_total, slice_bounds);
    m.ws_elems = ws_bytes / 8;
    const SmallPlan pl = plan_small(num_tokens, hidden, num_slices, num_adapters, max_rank, m.bf16, out_total,
                                    slice_bounds, row_split);
    const int64_t region = ((ws_bytes / kSmMaxAdapters) & ~int64_t(15)) / 8;   // as the launch derives it
    if (region < pl.region_bytes / 8) m.fail("%s: adapter region of %lld elements is too small", who, (long long)region);
    const int U = (num_tokens <= kSmT && nseq <= kSmT) ? 1 : kSmMaxU;
    const int64_t NP = producer_wgs(pl, num_adapters, row_split);
    const int64_t NC = consumer_wgs(pl, num_adapters, row_split);
    SmallPlan plr = pl;
    plr.region_bytes = region * 8;           // the producers' stride is the launch's region
    for (int64_t b = 0; b < NP; ++b) m.produce(plr, row_split, static_cast<int>(b), U);
    for (int64_t c = 0; c < NC; ++c) m.consume(pl, row_split, static_cast<int>(c), U, region);
  }
  if (checked) *checked = m.checked;
  if (msg && msg_len > 0) snprintf(msg, static_cast<size_t>(msg_len), "%s", m.msg);
  return m.bad;
}

}  // extern "C"
