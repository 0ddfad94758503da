// Metadata kernels: segment builder, latest-wins routing, reference bitmasks.
#include <stdarg.h>

#include <algorithm>
#include <vector>

#include "gs_common.h"

namespace gs {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

// ---------------------------------------------------------------------------
// Segment builder: one workgroup of 1024 threads (16 waves) per chunk of 1024
// tokens, with no communication between workgroups.
//
// Every workgroup gates ALL tokens (aLoRA activation offsets; sequence
// boundaries staged in LDS) and counts them per adapter: the whole batch's
// histogram gives seg_offsets (written by workgroup 0), the histogram of the
// tokens before its own chunk gives the chunk's starting cursor per adapter.
// Counting is per wave: lanes with equal ids are matched with one ballot per
// id bit, and the lowest lane of each group adds the group's size to LDS.  Then
// the workgroup scatters its own chunk: a token's rank among equal ids of lower
// lanes is a popcount, per-wave counts in LDS give the rank across waves.  The
// result is a stable sort (ascending token order within each adapter), the
// iteration order of the reference HF loop.
// ---------------------------------------------------------------------------
constexpr int kBuildThreads = 1024;
constexpr int kBuildWaves = kBuildThreads / 64;
constexpr int kCuCap = 2048;            // sequences whose boundaries and offsets are staged in LDS
constexpr int kPre = 8;                 // token chunks whose ids and positions are loaded together

// largest s with cu[s] <= t (cu non-decreasing, cu[0] = 0), over n = num_seqs entries
__device__ __forceinline__ int find_seq(const int32_t* cu, int n, int t) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

struct BuildArgs {
  const int64_t* req;
  const int64_t* pos;
  const int32_t* cu;
  const int64_t* act_off;
  int T;
  int num_seqs;
  int NA;
  int32_t* eff;
  int32_t* seg;
  int32_t* perm;
};

// Effective id of token t from its requested id and position (already
// loaded): base unless the token's position reaches its sequence's activation
// offset; ids outside [0, NA] are base.  Sequence boundaries and offsets come
// from LDS when they fit there.
__device__ __forceinline__ int gate_id(const BuildArgs& a, const int32_t* cu_lds, const int64_t* off_lds, int t,
                                       int64_t id, int64_t pos) {
  if (a.act_off != nullptr) {
    int s = 0;
    if (a.cu != nullptr) s = cu_lds != nullptr ? find_seq(cu_lds, a.num_seqs, t) : find_seq(a.cu, a.num_seqs, t);
    const int64_t q = (a.pos != nullptr) ? pos
                                         : static_cast<int64_t>(t - (a.cu != nullptr ? (cu_lds ? cu_lds[s] : a.cu[s]) : 0));
    if (q < (off_lds != nullptr ? off_lds[s] : a.act_off[s])) id = 0;
  }
  if (id < 0 || id > a.NA) id = 0;
  return static_cast<int>(id);
}

// Lanes of the wave whose id equals this lane's (one ballot per id bit).
__device__ __forceinline__ uint64_t match_id(int id, bool active, int nbits) {
  uint64_t match = __ballot(active);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (id >> b) & 1;
    const uint64_t bal = __ballot(bit);
    match &= bit ? bal : ~bal;
  }
  return match;
}

// Segment starts from the per-adapter totals (an exclusive scan by wave 0;
// workgroup 0 writes seg), the chunk's cursor per adapter (segment start +
// tokens of the adapter before the chunk, already in cursor), then the
// chunk's stable scatter: a token's rank among equal ids of lower lanes is a
// popcount, per-wave counts in LDS give the rank across waves.
__device__ __forceinline__ void finish_chunk(const BuildArgs& a, const int* total, int* cursor,
                                             int (*wcnt)[GS_MAX_ADAPTERS + 1], int mine, int c0, int nbits) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int NA = a.NA;
  if (wave == 0) {
    const int lane = tid & 63;
    int carry = 0;
    if (lane == 0 && blockIdx.x == 0) a.seg[0] = 0;
    for (int g0 = 1; g0 <= NA; g0 += 64) {
      const int g = g0 + lane;
      const int v = (g <= NA) ? total[g] : 0;
      int incl = v;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        int u = __shfl_up(incl, d, 64);
        if (lane >= d) incl += u;
      }
      if (g <= NA) {
        cursor[g] += carry + incl - v;
        if (blockIdx.x == 0) a.seg[g] = carry + incl;
      }
      carry += __shfl(incl, 63, 64);
    }
  }
  lds_barrier();

  const int t = c0 + tid;
  const bool active = t < a.T && mine > 0;
  const uint64_t match = match_id(mine, active, nbits);
  const uint64_t below = match & lanemask_lt();
  if (active && below == 0) wcnt[wave][mine] = __popcll(match);
  lds_barrier();
  if (active) {
    int pp = cursor[mine] + __popcll(below);
    for (int w = 0; w < wave; ++w) pp += wcnt[w][mine];   // zero where wave w has none of this id
    a.perm[pp] = t;
  }
}

__global__ __launch_bounds__(kBuildThreads) void build_segments_kernel(BuildArgs a) {
  __shared__ int total[GS_MAX_ADAPTERS + 1];
  __shared__ int cursor[GS_MAX_ADAPTERS + 1];     // counts before this chunk, then the chunk's cursors
  __shared__ int wcnt[kBuildWaves][GS_MAX_ADAPTERS + 1];
  __shared__ int32_t cu_s[kCuCap];
  __shared__ int64_t off_s[kCuCap];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int NA = a.NA;
  const int T = a.T;
  const int c0 = static_cast<int>(blockIdx.x) * kBuildThreads;   // this workgroup's chunk

  for (int i = tid; i <= NA; i += kBuildThreads) {
    total[i] = 0;
    cursor[i] = 0;
  }
  for (int i = tid; i < kBuildWaves * (GS_MAX_ADAPTERS + 1); i += kBuildThreads) (&wcnt[0][0])[i] = 0;
  const int nseq = a.cu != nullptr ? a.num_seqs : 1;
  const bool seq_in_lds = a.act_off != nullptr && nseq <= kCuCap;
  if (seq_in_lds) {
    for (int i = tid; i < nseq; i += kBuildThreads) {
      cu_s[i] = a.cu != nullptr ? a.cu[i] : 0;
      off_s[i] = a.act_off[i];
    }
  }
  lds_barrier();
  const int32_t* cu_lds = seq_in_lds && a.cu != nullptr ? cu_s : nullptr;
  const int64_t* off_lds = seq_in_lds ? off_s : nullptr;
  int nbits = 0;
  while ((1 << nbits) <= NA) ++nbits;

  // Pass 1: gate every token of the batch and count per adapter.  The ids and
  // positions of kPre chunks are loaded together (clamped, in bounds) before
  // any is used.  Every workgroup reads the whole batch, at the rate one CU
  // fetches from beyond its L2, so positions are read only when gating uses
  // them.
  int mine = 0;                                   // this thread's token of the own chunk
  const int nchunks = (T + kBuildThreads - 1) / kBuildThreads;
  const bool need_pos = a.pos != nullptr && a.act_off != nullptr;
  for (int k0 = 0; k0 < nchunks; k0 += kPre) {
    int64_t rq[kPre], ps[kPre];
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      const int tc = min((k0 + u) * kBuildThreads + tid, T - 1);
      rq[u] = a.req[tc];
      ps[u] = need_pos ? a.pos[tc] : 0;
    }
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      const int b0 = (k0 + u) * kBuildThreads;
      if (b0 < T) {
        const int t = b0 + tid;
        const int id = t < T ? gate_id(a, cu_lds, off_lds, t, rq[u], ps[u]) : 0;
        if (b0 == c0) {
          mine = id;
          if (t < T) a.eff[t] = id;
        }
        const bool active = id > 0;
        const uint64_t match = match_id(id, active, nbits);
        if (active && (match & lanemask_lt()) == 0) {
          const int n = __popcll(match);
          atomicAdd(&total[id], n);
          if (b0 < c0) atomicAdd(&cursor[id], n);
        }
      }
    }
  }
  lds_barrier();

  finish_chunk(a, total, cursor, wcnt, mine, c0, nbits);
}

// ---------------------------------------------------------------------------
// Two-launch form for long batches, where every workgroup re-reading the
// whole batch would cost more than a second launch: build_count_kernel gates
// one chunk per workgroup and writes the chunk's per-adapter histogram to a
// workspace ([chunks][NA+1] int32); build_scatter_kernel sums the histograms
// (all chunks: totals; chunks before its own: cursors) and scatters its chunk
// exactly as the one-launch kernel does.  The workspace is written in full by
// the first launch before the second reads it, so it needs no clearing.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBuildThreads) void build_count_kernel(BuildArgs a, int32_t* __restrict__ hist) {
  __shared__ int cnt[GS_MAX_ADAPTERS + 1];
  __shared__ int32_t cu_s[kCuCap];
  __shared__ int64_t off_s[kCuCap];
  const int tid = threadIdx.x;
  const int NA = a.NA;
  const int t = static_cast<int>(blockIdx.x) * kBuildThreads + tid;
  const int tc = min(t, a.T - 1);
  const int64_t rq = a.req[tc];
  const int64_t ps = (a.pos != nullptr && a.act_off != nullptr) ? a.pos[tc] : 0;
  for (int i = tid; i <= NA; i += kBuildThreads) cnt[i] = 0;
  const int nseq = a.cu != nullptr ? a.num_seqs : 1;
  const bool seq_in_lds = a.act_off != nullptr && nseq <= kCuCap;
  if (seq_in_lds) {
    for (int i = tid; i < nseq; i += kBuildThreads) {
      cu_s[i] = a.cu != nullptr ? a.cu[i] : 0;
      off_s[i] = a.act_off[i];
    }
  }
  lds_barrier();
  int nbits = 0;
  while ((1 << nbits) <= NA) ++nbits;
  const int id = t < a.T ? gate_id(a, seq_in_lds && a.cu != nullptr ? cu_s : nullptr, seq_in_lds ? off_s : nullptr, t,
                                   rq, ps)
                         : 0;
  if (t < a.T) a.eff[t] = id;
  const bool active = id > 0;
  const uint64_t match = match_id(id, active, nbits);
  if (active && (match & lanemask_lt()) == 0) atomicAdd(&cnt[id], __popcll(match));
  lds_barrier();
  for (int i = tid; i <= NA; i += kBuildThreads) hist[static_cast<int64_t>(blockIdx.x) * (NA + 1) + i] = cnt[i];
}

constexpr int kHistPre = 8;

// Chunks from which the two-launch form is the faster one (its workspace
// query returns 0 below), and its workspace size.
#ifndef GS_BUILD_SPLIT_CHUNKS
#define GS_BUILD_SPLIT_CHUNKS 2
#endif
constexpr int64_t kBuildSplitChunks = GS_BUILD_SPLIT_CHUNKS;
inline int64_t build_hist_bytes(int64_t chunks, int num_adapters) { return chunks * (num_adapters + 1) * 4; }   // histogram entries loaded per thread before any is added

__global__ __launch_bounds__(kBuildThreads) void build_scatter_kernel(BuildArgs a, const int32_t* __restrict__ hist,
                                                                      int nchunks) {
  __shared__ int total[GS_MAX_ADAPTERS + 1];
  __shared__ int cursor[GS_MAX_ADAPTERS + 1];
  __shared__ int wcnt[kBuildWaves][GS_MAX_ADAPTERS + 1];
  const int tid = threadIdx.x;
  const int NA = a.NA;
  const int c = static_cast<int>(blockIdx.x);
  const int c0 = c * kBuildThreads;
  const int mine = c0 + tid < a.T ? a.eff[c0 + tid] : 0;
  for (int i = tid; i <= NA; i += kBuildThreads) {
    total[i] = 0;
    cursor[i] = 0;
  }
  for (int i = tid; i < kBuildWaves * (GS_MAX_ADAPTERS + 1); i += kBuildThreads) (&wcnt[0][0])[i] = 0;
  lds_barrier();
  const int width = NA + 1;
  const int n = nchunks * width;
  for (int i0 = 0; i0 < n; i0 += kHistPre * kBuildThreads) {
    int v[kHistPre];
#pragma unroll
    for (int u = 0; u < kHistPre; ++u) {
      const int i = i0 + u * kBuildThreads + tid;
      v[u] = i < n ? hist[i] : 0;
    }
#pragma unroll
    for (int u = 0; u < kHistPre; ++u) {
      const int i = i0 + u * kBuildThreads + tid;
      if (v[u] != 0) {
        const int cc = i / width;
        const int g = i - cc * width;
        atomicAdd(&total[g], v[u]);
        if (cc < c) atomicAdd(&cursor[g], v[u]);
      }
    }
  }
  lds_barrier();
  int nbits = 0;
  while ((1 << nbits) <= NA) ++nbits;
  finish_chunk(a, total, cursor, wcnt, mine, c0, nbits);
}

// ---------------------------------------------------------------------------
// Latest-wins routing: one workgroup per sequence; an inclusive max-scan of
// "index of the last control token" over the sequence, chunk by chunk.
// ---------------------------------------------------------------------------
constexpr int kRouteThreads = 256;

__global__ __launch_bounds__(kRouteThreads) void route_latest_wins_kernel(
    const int64_t* __restrict__ input_ids, const int32_t* __restrict__ cu, int T, const int64_t* __restrict__ ctl,
    int num_control, int id_offset, const int64_t* __restrict__ start_ids, int64_t* __restrict__ out) {
  __shared__ int64_t ctl_s[GS_MAX_ADAPTERS + 1];
  __shared__ int wave_max[kRouteThreads / 64];
  __shared__ int wave_id[kRouteThreads / 64];
  const int s = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  for (int i = tid; i < num_control; i += kRouteThreads) ctl_s[i] = ctl[i];
  lds_barrier();
  const int lo = (cu != nullptr) ? cu[s] : 0;
  const int hi = (cu != nullptr) ? cu[s + 1] : T;
  // carry: (index of last control token so far, its fired id); index -1 = none
  int carry_idx = -1;
  int carry_id = (start_ids != nullptr) ? static_cast<int>(start_ids[s]) : 0;
  for (int base = lo; base < hi; base += kRouteThreads) {
    const int t = base + tid;
    int my_idx = -1, my_id = 0;
    if (t < hi) {
      const int64_t tok = input_ids[t];
      for (int k = 0; k < num_control; ++k) {
        if (ctl_s[k] == tok) {  // the first matching slot, like list.index
          my_idx = t;
          my_id = k + id_offset;
          break;
        }
      }
    }
    // inclusive max-scan of (idx, id) by idx inside the wave
    int sidx = my_idx, sid = my_id;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      int oi = __shfl_up(sidx, d, 64);
      int od = __shfl_up(sid, d, 64);
      if (lane >= d && oi > sidx) {
        sidx = oi;
        sid = od;
      }
    }
    if (lane == 63) {
      wave_max[wave] = sidx;
      wave_id[wave] = sid;
    }
    lds_barrier();
    // combine with earlier waves of this chunk, then with the carry
    for (int w = 0; w < wave; ++w) {
      if (wave_max[w] > sidx) {
        sidx = wave_max[w];
        sid = wave_id[w];
      }
    }
    if (carry_idx > sidx) {
      sidx = carry_idx;
      sid = carry_id;
    }
    if (t < hi) out[t] = (sidx >= 0) ? sid : carry_id;
    // new carry: the max over the whole chunk
    int cidx = carry_idx, cid = carry_id;
    for (int w = 0; w < kRouteThreads / 64; ++w) {
      if (wave_max[w] > cidx) {
        cidx = wave_max[w];
        cid = wave_id[w];
      }
    }
    lds_barrier();
    carry_idx = cidx;
    carry_id = cid;
  }
}

// ---------------------------------------------------------------------------
// Reference bitmasks and remap gather.  Grid: (ceil(M / 256), num_modules).
// Each thread gathers one token; tiles of a power-of-two block_m <= 64 are
// OR-reduced with lane shuffles, other block_m by the tile's first thread.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t load_idx(const void* p, int bytes, int64_t i) {
  return bytes == 8 ? static_cast<const int64_t*>(p)[i] : static_cast<int64_t>(static_cast<const int32_t*>(p)[i]);
}

__device__ __forceinline__ uint64_t loc_bit(int64_t loc) {
  return (loc > 0 && loc <= 64) ? (1ull << (loc - 1)) : 0ull;
}

__global__ __launch_bounds__(256) void bitmask_kernel(const void* __restrict__ ids, int idx_bytes, int M,
                                                      const int64_t* __restrict__ remap_t, int na_plus_1,
                                                      int num_modules, int block_m, int64_t* __restrict__ bitmasks,
                                                      int64_t* __restrict__ remapped) {
  const int mod = blockIdx.y;
  const int t = blockIdx.x * 256 + threadIdx.x;
  const int num_tiles = (M + block_m - 1) / block_m;
  int64_t loc = 0;
  if (t < M) {
    int64_t id = load_idx(ids, idx_bytes, t);
    id = id < 0 ? 0 : (id > na_plus_1 - 1 ? na_plus_1 - 1 : id);
    loc = remap_t[id * num_modules + mod];
    if (remapped != nullptr) remapped[static_cast<int64_t>(mod) * M + t] = loc;
  }
  const bool pow2 = block_m <= 64 && (block_m & (block_m - 1)) == 0;
  if (pow2) {
    uint64_t bits = loc_bit(loc);
    for (int d = 1; d < block_m; d <<= 1) bits |= __shfl_xor(bits, d, 64);
    if ((t % block_m) == 0 && t < M) bitmasks[static_cast<int64_t>(mod) * num_tiles + t / block_m] = static_cast<int64_t>(bits);
  } else if (t < M && (t % block_m) == 0) {
    uint64_t bits = 0;
    const int end = min(M, t + block_m);
    for (int u = t; u < end; ++u) {
      int64_t id = load_idx(ids, idx_bytes, u);
      id = id < 0 ? 0 : (id > na_plus_1 - 1 ? na_plus_1 - 1 : id);
      bits |= loc_bit(remap_t[id * num_modules + mod]);
    }
    bitmasks[static_cast<int64_t>(mod) * num_tiles + t / block_m] = static_cast<int64_t>(bits);
  }
}

// Probe-slot split: one thread per token.  The kind table (<= 257 bytes) is
// staged in LDS.  An index outside the table (negative or past its last
// slot) is neither a probe nor an adapter: both streams get 0, so the token
// takes the base model, as the segment builder treats such ids.
__global__ __launch_bounds__(256) void split_indices_kernel(const uint8_t* __restrict__ kind_lut, int lut_len,
                                                            const void* __restrict__ ids, int idx_bytes, int64_t n,
                                                            void* lora_out, void* probe_out) {
  __shared__ uint8_t lut[GS_MAX_ADAPTERS + 1];
  for (int k = threadIdx.x; k < lut_len; k += blockDim.x) lut[k] = kind_lut[k];
  __syncthreads();
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n) return;
  const int64_t v = load_idx(ids, idx_bytes, t);
  const bool in_table = v >= 0 && v < lut_len;
  const bool probe = in_table && lut[v] != 0;
  const int64_t lora = in_table && !probe ? v : 0;
  if (idx_bytes == 8) {
    if (lora_out) static_cast<int64_t*>(lora_out)[t] = lora;
    if (probe_out) static_cast<int64_t*>(probe_out)[t] = probe ? v : 0;
  } else {
    if (lora_out) static_cast<int32_t*>(lora_out)[t] = static_cast<int32_t>(lora);
    if (probe_out) static_cast<int32_t*>(probe_out)[t] = probe ? static_cast<int32_t>(v) : 0;
  }
}

// ---------------------------------------------------------------------------
// Address model (test support): replays on the host every global and LDS
// access of the metadata kernels for one call, following the values that
// steer them (the ids, positions, sequence table and offsets), and checks
// each against its buffer.  No HIP call is made.
// ---------------------------------------------------------------------------
struct MetaModel {
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

  // ---- the segment builder (both forms) ----------------------------------
  int T = 0, nseq = 1, NA = 1;
  const int64_t* req = nullptr;
  const int64_t* pos = nullptr;
  const int32_t* cu = nullptr;
  const int64_t* act = nullptr;
  // find_seq over the staged or the global table (n entries), as the kernel
  int seq_of(int t, bool lds) {
    int lo = 0, hi = nseq - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      in(lds ? "sequence table (LDS)" : "cu_seqlens", mid, 1, lds ? kCuCap : nseq + 1);
      if (cu[mid] <= t) lo = mid; else hi = mid - 1;
    }
    return lo;
  }
  int gate(int t, bool lds) {
    int64_t id = req[t];
    if (act != nullptr) {
      int sq = 0;
      if (cu != nullptr) sq = seq_of(t, lds && cu != nullptr);
      if (cu != nullptr) in(lds ? "sequence table (LDS)" : "cu_seqlens", sq, 1, lds ? kCuCap : nseq + 1);
      in(lds ? "offsets (LDS)" : "act_offsets", sq, 1, lds ? kCuCap : nseq);
      const int64_t q = pos != nullptr ? pos[t] : static_cast<int64_t>(t - (cu != nullptr ? cu[sq] : 0));
      if (q < act[sq]) id = 0;
    }
    if (id < 0 || id > NA) id = 0;
    return static_cast<int>(id);
  }
  void build(bool two_launch) {
    const int chunks = T > 0 ? (T + kBuildThreads - 1) / kBuildThreads : 1;
    const bool lds = act != nullptr && nseq <= kCuCap;
    const bool need_pos = pos != nullptr && act != nullptr;
    // the stable order's slot of every token (what the scatter writes)
    std::vector<int> eff(T), start(NA + 2, 0), seen(NA + 1, 0);
    for (int t = 0; t < T; ++t) eff[t] = gate(t, lds);
    for (int t = 0; t < T; ++t) ++start[eff[t] + 1];
    for (int g = 1; g <= NA + 1; ++g) start[g] += start[g - 1];
    const int64_t lds_adapters = GS_MAX_ADAPTERS + 1;
    for (int b = 0; b < chunks; ++b) {
      const int c0 = b * kBuildThreads;
      if (lds)
        for (int i = 0; i < nseq; ++i) {
          in("sequence table (LDS)", i, 1, kCuCap);
          if (cu) in("cu_seqlens", i, 1, nseq + 1);
          in("act_offsets", i, 1, nseq);
        }
      for (int i = 0; i <= NA; ++i) in("per-adapter counts (LDS)", i, 1, lds_adapters);
      if (!two_launch) {
        // pass 1: every chunk of the batch, loads clamped
        const int nch = (T + kBuildThreads - 1) / kBuildThreads;
        for (int k = 0; k < nch; ++k)
          for (int tid = 0; tid < kBuildThreads; ++tid) {
            const int tc = std::min(k * kBuildThreads + tid, T - 1);
            in("req_ids", tc, 1, T);
            if (need_pos) in("positions", tc, 1, T);
          }
      } else {
        for (int tid = 0; tid < kBuildThreads; ++tid) {
          const int tc = std::min(c0 + tid, T - 1);
          if (T > 0) {
            in("req_ids", tc, 1, T);
            if (need_pos) in("positions", tc, 1, T);
          }
        }
        for (int i = 0; i <= NA; ++i) in("histograms", static_cast<int64_t>(b) * (NA + 1) + i, 1, int64_t(chunks) * (NA + 1));
        for (int i = 0; i < chunks * (NA + 1); ++i) in("histograms (scatter)", i, 1, int64_t(chunks) * (NA + 1));
      }
      // the own chunk: eff written, seg by workgroup 0, perm by the scatter
      if (b == 0)
        for (int g = 0; g <= NA; ++g) in("seg_offsets", g, 1, NA + 1);
      for (int tid = 0; tid < kBuildThreads; ++tid) {
        const int t = c0 + tid;
        if (t >= T) continue;
        in("eff_ids", t, 1, T);
        const int g = eff[t];
        in("wave counts (LDS)", (tid >> 6) * lds_adapters + g, 1, kBuildWaves * lds_adapters);
        if (g > 0) in("perm", start[g] + seen[g]++, 1, T);
      }
    }
  }

  // ---- route_latest_wins_kernel: one workgroup per sequence ----------------
  void route(int num_control) {
    for (int sq = 0; sq < nseq; ++sq) {
      for (int i = 0; i < num_control; ++i) {
        in("control tokens", i, 1, num_control);
        in("control tokens (LDS)", i, 1, GS_MAX_ADAPTERS + 1);
      }
      int lo = 0, hi = T;
      if (cu != nullptr) {
        in("cu_seqlens", sq, 2, nseq + 1);
        lo = cu[sq];
        hi = cu[sq + 1];
      }
      in("start ids (when given)", sq, 1, nseq);
      for (int base = lo; base < hi; base += kRouteThreads)
        for (int tid = 0; tid < kRouteThreads; ++tid) {
          const int t = base + tid;
          if (t < hi) {
            in("input_ids", t, 1, T);
            in("routed ids", t, 1, T);
          }
        }
    }
  }
  // ---- bitmask_kernel: grid (ceil(M / 256), num_modules) ---------------------
  void bitmask(const int64_t* ids, int na_plus_1, int num_modules, int block_m) {
    const int M = T;
    const int64_t tiles = (M + block_m - 1) / block_m;
    const bool pow2 = block_m <= 64 && (block_m & (block_m - 1)) == 0;
    auto remap_at = [&](int u, int mod) {
      int64_t id = ids[u];
      id = id < 0 ? 0 : (id > na_plus_1 - 1 ? na_plus_1 - 1 : id);
      in("remap table", id * num_modules + mod, 1, int64_t(na_plus_1) * num_modules);
    };
    for (int mod = 0; mod < num_modules; ++mod)
      for (int t = 0; t < M; ++t) {
        in("adapter ids", t, 1, M);
        remap_at(t, mod);
        in("remapped ids", int64_t(mod) * M + t, 1, int64_t(num_modules) * M);
        if (t % block_m == 0) {
          in("bitmasks", int64_t(mod) * tiles + t / block_m, 1, int64_t(num_modules) * tiles);
          if (!pow2)
            for (int u = t; u < std::min(M, t + block_m); ++u) {
              in("adapter ids", u, 1, M);
              remap_at(u, mod);
            }
        }
      }
  }
  // ---- split_indices_kernel ----------------------------------------------------
  void split(const int64_t* ids, int lut_len) {
    for (int k = 0; k < lut_len; ++k) {
      in("kind table", k, 1, lut_len);
      in("kind table (LDS)", k, 1, GS_MAX_ADAPTERS + 1);
    }
    for (int t = 0; t < T; ++t) {
      in("adapter ids", t, 1, T);
      const int64_t v = ids[t];
      if (v >= 0 && v < lut_len) in("kind table (LDS)", v, 1, GS_MAX_ADAPTERS + 1);
      in("split outputs", t, 1, T);
    }
  }
};
}  // namespace gs

using namespace gs;

extern "C" {

int gs_version(void) { return 100; }

int gs_split_adapter_indices(const uint8_t* kind_lut, int32_t lut_len, const void* adapter_indices,
                             int32_t idx_bytes, int64_t num_tokens, void* lora_indices, void* probe_indices,
                             void* stream) {
  const char* who = "gs_split_adapter_indices";
  GS_CHECK_ARG(idx_bytes == 4 || idx_bytes == 8, "%s: idx_bytes=%d", who, idx_bytes);
  GS_CHECK_ARG(lut_len >= 1 && lut_len <= GS_MAX_ADAPTERS + 1 && kind_lut != nullptr,
               "%s: kind table of %d entries (1..%d)", who, lut_len, GS_MAX_ADAPTERS + 1);
  GS_CHECK_ARG(num_tokens >= 0 && num_tokens < (int64_t(1) << 31), "%s: num_tokens out of range", who);
  GS_CHECK_ARG(num_tokens == 0 || adapter_indices != nullptr, "%s: NULL adapter_indices", who);
  if (num_tokens == 0 || (lora_indices == nullptr && probe_indices == nullptr)) return GS_OK;
  hipLaunchKernelGGL(split_indices_kernel, dim3(static_cast<unsigned>((num_tokens + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), kind_lut, lut_len, adapter_indices, idx_bytes, num_tokens,
                     lora_indices, probe_indices);
  GS_CHECK_LAUNCH(who);
  return GS_OK;
}

const char* gs_last_error(void) { return g_err; }

int64_t gs_build_segments_workspace_bytes(int64_t num_tokens, int32_t num_adapters) {
  if (num_tokens <= 0 || num_tokens >= (int64_t(1) << 31) || num_adapters < 1 || num_adapters > GS_MAX_ADAPTERS) return 0;
  const int64_t chunks = (num_tokens + kBuildThreads - 1) / kBuildThreads;
  return chunks >= kBuildSplitChunks ? build_hist_bytes(chunks, num_adapters) : 0;
}

int gs_build_segments(const int64_t* req_ids, const int64_t* positions, const int32_t* cu_seqlens,
                      const int64_t* act_offsets, int64_t num_tokens, int32_t num_seqs, int32_t num_adapters,
                      int32_t* eff_ids, int32_t* seg_offsets, int32_t* perm, void* workspace, int64_t workspace_bytes,
                      void* stream) {
  GS_CHECK_ARG(num_adapters >= 1 && num_adapters <= GS_MAX_ADAPTERS, "gs_build_segments: num_adapters=%d not in [1,%d]",
               num_adapters, GS_MAX_ADAPTERS);
  GS_CHECK_ARG(num_tokens >= 0 && num_tokens < (int64_t(1) << 31), "gs_build_segments: num_tokens=%lld out of range",
               (long long)num_tokens);
  GS_CHECK_ARG(seg_offsets != nullptr, "gs_build_segments: seg_offsets is NULL");
  GS_CHECK_ARG(num_tokens == 0 || (req_ids && eff_ids && perm), "gs_build_segments: NULL token array");
  GS_CHECK_ARG(act_offsets == nullptr || cu_seqlens == nullptr || num_seqs >= 1,
               "gs_build_segments: num_seqs=%d with cu_seqlens", num_seqs);
  GS_CHECK_ARG(workspace == nullptr || (reinterpret_cast<uintptr_t>(workspace) & 3) == 0,
               "gs_build_segments: workspace must be 4-byte aligned");
  BuildArgs a{req_ids, positions, cu_seqlens, act_offsets, static_cast<int>(num_tokens), cu_seqlens ? num_seqs : 1,
              num_adapters, eff_ids, seg_offsets, perm};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t chunks = num_tokens > 0 ? (num_tokens + kBuildThreads - 1) / kBuildThreads : 1;
  if (workspace != nullptr && num_tokens > 0) {
    const int64_t need = build_hist_bytes(chunks, num_adapters);
    if (workspace_bytes < need) {
      set_error("gs_build_segments: workspace of %lld bytes, the two-launch form needs %lld "
                "(see gs_build_segments_workspace_bytes; NULL selects the one-launch form)",
                (long long)workspace_bytes, (long long)need);
      return GS_ERR_WORKSPACE;
    }
    int32_t* hist = static_cast<int32_t*>(workspace);
    hipLaunchKernelGGL(build_count_kernel, dim3(static_cast<unsigned>(chunks)), dim3(kBuildThreads), 0, st, a, hist);
    GS_CHECK_LAUNCH("gs_build_segments (count)");
    hipLaunchKernelGGL(build_scatter_kernel, dim3(static_cast<unsigned>(chunks)), dim3(kBuildThreads), 0, st, a,
                       static_cast<const int32_t*>(hist), static_cast<int>(chunks));
    GS_CHECK_LAUNCH("gs_build_segments (scatter)");
    return GS_OK;
  }
  hipLaunchKernelGGL(build_segments_kernel, dim3(static_cast<unsigned>(chunks)), dim3(kBuildThreads), 0, st, a);
  GS_CHECK_LAUNCH("gs_build_segments");
  return GS_OK;
}

int gs_route_latest_wins(const int64_t* input_ids, const int32_t* cu_seqlens, int64_t num_tokens,
                         int32_t num_seqs, const int64_t* control_tokens, int32_t num_control, int32_t id_offset,
                         const int64_t* start_ids, int64_t* out_ids, void* stream) {
  GS_CHECK_ARG(num_control >= 0 && num_control <= GS_MAX_ADAPTERS + 1, "gs_route_latest_wins: num_control=%d",
               num_control);
  GS_CHECK_ARG(num_tokens >= 0 && num_tokens < (int64_t(1) << 31), "gs_route_latest_wins: num_tokens out of range");
  const int nseq = cu_seqlens ? num_seqs : 1;
  GS_CHECK_ARG(nseq >= 1, "gs_route_latest_wins: num_seqs=%d", num_seqs);
  if (num_tokens == 0) return GS_OK;
  hipLaunchKernelGGL(route_latest_wins_kernel, dim3(nseq), dim3(kRouteThreads), 0, static_cast<hipStream_t>(stream),
                     input_ids, cu_seqlens, static_cast<int>(num_tokens), control_tokens, num_control, id_offset,
                     start_ids, out_ids);
  GS_CHECK_LAUNCH("gs_route_latest_wins");
  return GS_OK;
}

int gs_compute_bitmasks(const void* adapter_indices, int32_t idx_bytes, int64_t M, const int64_t* remap_tables_t,
                        int32_t na_plus_1, int32_t num_modules, int32_t block_m, int64_t* bitmasks,
                        int64_t* remapped, void* stream) {
  GS_CHECK_ARG(idx_bytes == 4 || idx_bytes == 8, "gs_compute_bitmasks: idx_bytes=%d", idx_bytes);
  GS_CHECK_ARG(block_m >= 1 && block_m <= 1024, "gs_compute_bitmasks: block_m=%d", block_m);
  GS_CHECK_ARG(na_plus_1 >= 1 && num_modules >= 1, "gs_compute_bitmasks: bad remap table shape");
  GS_CHECK_ARG(M >= 0 && M < (int64_t(1) << 31), "gs_compute_bitmasks: M out of range");
  if (M == 0) return GS_OK;
  dim3 grid(static_cast<unsigned>((M + 255) / 256), static_cast<unsigned>(num_modules));
  hipLaunchKernelGGL(bitmask_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), adapter_indices, idx_bytes,
                     static_cast<int>(M), remap_tables_t, na_plus_1, num_modules, block_m, bitmasks, remapped);
  GS_CHECK_LAUNCH("gs_compute_bitmasks");
  return GS_OK;
}

int64_t gs_check_build_addresses(int64_t num_tokens, int32_t num_seqs, int32_t num_adapters, const int64_t* req_ids,
                                 const int64_t* positions, const int32_t* cu_seqlens, const int64_t* act_offsets,
                                 int32_t two_launch, char* msg, int64_t msg_len, int64_t* checked) {
  GS_CHECK_ARG(num_adapters >= 1 && num_adapters <= GS_MAX_ADAPTERS && num_tokens >= 0 && num_tokens < (1ll << 31),
               "gs_check_build_addresses: shape");
  GS_CHECK_ARG(num_tokens == 0 || req_ids, "gs_check_build_addresses: NULL req_ids");
  MetaModel m{};
  m.T = static_cast<int>(num_tokens);
  m.nseq = cu_seqlens ? num_seqs : 1;
  m.NA = num_adapters;
  m.req = req_ids;
  m.pos = positions;
  m.cu = cu_seqlens;
  m.act = act_offsets;
  m.build(two_launch != 0 && num_tokens > 0);
  if (checked) *checked = m.checked;
  if (msg && msg_len > 0) snprintf(msg, static_cast<size_t>(msg_len), "%s", m.msg);
  return m.bad;
}

int64_t gs_check_token_addresses(int64_t num_tokens, int32_t num_seqs, const int32_t* cu_seqlens,
                                 int32_t num_control, const int64_t* ids, int32_t na_plus_1, int32_t num_modules,
                                 int32_t block_m, int32_t lut_len, char* msg, int64_t msg_len, int64_t* checked) {
  const char* who = "gs_check_token_addresses";
  GS_CHECK_ARG(num_tokens >= 0 && num_tokens < (1ll << 31) && (ids || num_tokens == 0), "%s: tokens", who);
  GS_CHECK_ARG(num_control >= 0 && num_control <= GS_MAX_ADAPTERS + 1 && (cu_seqlens == nullptr || num_seqs >= 1),
               "%s: num_control / num_seqs", who);
  GS_CHECK_ARG(na_plus_1 >= 1 && num_modules >= 1 && block_m >= 1 && block_m <= 1024, "%s: remap shape", who);
  GS_CHECK_ARG(lut_len >= 1 && lut_len <= GS_MAX_ADAPTERS + 1, "%s: lut_len", who);
  MetaModel m{};
  m.T = static_cast<int>(num_tokens);
  m.nseq = cu_seqlens ? num_seqs : 1;
  m.cu = cu_seqlens;
  if (num_tokens > 0) {
    m.route(num_control);
    m.bitmask(ids, na_plus_1, num_modules, block_m);
    m.split(ids, lut_len);
  }
  if (checked) *checked = m.checked;
  if (msg && msg_len > 0) snprintf(msg, static_cast<size_t>(msg_len), "%s", m.msg);
  return m.bad;
}

}  // extern "C"
