// Metadata kernels: segment builder, latest-wins routing, reference bitmasks.
#include <stdarg.h>

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
// Segment builder: one workgroup of 1024 threads (16 waves).
//
// Pass 1 computes every token's effective id (aLoRA gating) and a histogram in
// LDS.  A wave-0 scan turns the histogram into seg_offsets.  Pass 2 walks the
// tokens in chunks of 1024, in order; inside a wave, tokens with equal ids are
// found with one ballot per id bit, so a token's rank among equal ids of lower
// lanes is a popcount; per-wave counts in LDS give the rank across waves, and a
// running cursor per adapter carries the order across chunks.  The result is a
// stable sort (ascending token order within each adapter).
// ---------------------------------------------------------------------------
constexpr int kBuildThreads = 1024;
constexpr int kBuildWaves = kBuildThreads / 64;
constexpr int kBuildRegChunks = 8;      // chunks of 1024 tokens whose ids stay in registers
constexpr int kCuCap = 2048;            // sequences whose boundaries are staged in LDS

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

__device__ __forceinline__ int effective_id(const BuildArgs& a, const int32_t* cu_lds, int t) {
  int64_t id = a.req[t];
  if (a.act_off != nullptr) {
    int s = 0;
    if (a.cu != nullptr) s = cu_lds != nullptr ? find_seq(cu_lds, a.num_seqs, t) : find_seq(a.cu, a.num_seqs, t);
    const int64_t q = (a.pos != nullptr) ? a.pos[t]
                                         : static_cast<int64_t>(t - (a.cu != nullptr ? (cu_lds ? cu_lds[s] : a.cu[s]) : 0));
    if (q < a.act_off[s]) id = 0;
  }
  if (id < 0 || id > a.NA) id = 0;
  return static_cast<int>(id);
}

__global__ __launch_bounds__(kBuildThreads) void build_segments_kernel(BuildArgs a) {
  __shared__ int hist[GS_MAX_ADAPTERS + 1];
  __shared__ int cursor[GS_MAX_ADAPTERS + 1];
  __shared__ int wcnt[kBuildWaves][GS_MAX_ADAPTERS + 1];
  __shared__ int32_t cu_s[kCuCap];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int NA = a.NA;
  const int T = a.T;

  for (int i = tid; i <= NA; i += kBuildThreads) {
    hist[i] = 0;
    for (int w = 0; w < kBuildWaves; ++w) wcnt[w][i] = 0;
  }
  const bool cu_in_lds = a.cu != nullptr && a.act_off != nullptr && a.num_seqs <= kCuCap;
  if (cu_in_lds)
    for (int i = tid; i < a.num_seqs; i += kBuildThreads) cu_s[i] = a.cu[i];
  lds_barrier();
  const int32_t* cu_lds = cu_in_lds ? cu_s : nullptr;

  // Pass 1: effective ids + histogram; the first chunks keep their ids in registers.
  int ereg[kBuildRegChunks];
#pragma unroll
  for (int c = 0; c < kBuildRegChunks; ++c) {
    const int t = c * kBuildThreads + tid;
    ereg[c] = 0;
    if (t < T) {
      const int id = effective_id(a, cu_lds, t);
      ereg[c] = id;
      a.eff[t] = id;
      if (id > 0) atomicAdd(&hist[id], 1);
    }
  }
  for (int t = kBuildRegChunks * kBuildThreads + tid; t < T; t += kBuildThreads) {
    const int id = effective_id(a, cu_lds, t);
    a.eff[t] = id;
    if (id > 0) atomicAdd(&hist[id], 1);
  }
  lds_barrier();

  // Exclusive scan of hist[1..NA] by wave 0 -> cursor, seg.
  if (wave == 0) {
    const int lane = tid & 63;
    int carry = 0;
    if (lane == 0) a.seg[0] = 0;
    for (int g0 = 1; g0 <= NA; g0 += 64) {
      const int g = g0 + lane;
      const int v = (g <= NA) ? hist[g] : 0;
      int incl = v;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        int u = __shfl_up(incl, d, 64);
        if (lane >= d) incl += u;
      }
      if (g <= NA) {
        cursor[g] = carry + incl - v;
        a.seg[g] = carry + incl;
      }
      carry += __shfl(incl, 63, 64);
    }
  }
  lds_barrier();

  int nbits = 0;
  while ((1 << nbits) <= NA) ++nbits;

  // Pass 2: stable scatter, chunk by chunk in token order.
  const int nchunks = (T + kBuildThreads - 1) / kBuildThreads;
  for (int c = 0; c < nchunks; ++c) {
    const int t = c * kBuildThreads + tid;
    int id = 0;
    if (c < kBuildRegChunks) {
#pragma unroll
      for (int u = 0; u < kBuildRegChunks; ++u)
        if (u == c) id = ereg[u];
    } else if (t < T) {
      id = a.eff[t];    // written by this same thread in pass 1
    }
    const bool active = id > 0;
    uint64_t match = __ballot(active);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (id >> b) & 1;
      const uint64_t bal = __ballot(bit);
      match &= bit ? bal : ~bal;
    }
    const uint64_t below = match & lanemask_lt();
    if (active && below == 0) wcnt[wave][id] = __popcll(match);
    lds_barrier();
    if (active) {
      int pp = cursor[id] + __popcll(below);
      for (int w = 0; w < wave; ++w) pp += wcnt[w][id];
      a.perm[pp] = t;
    }
    lds_barrier();
    for (int g = tid + 1; g <= NA; g += kBuildThreads) {
      int add = 0;
      for (int w = 0; w < kBuildWaves; ++w) {
        add += wcnt[w][g];
        wcnt[w][g] = 0;
      }
      cursor[g] += add;
    }
    lds_barrier();
  }
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

}  // namespace gs

using namespace gs;

extern "C" {

int gs_version(void) { return 100; }

const char* gs_last_error(void) { return g_err; }

int gs_build_segments(const int64_t* req_ids, const int64_t* positions, const int32_t* cu_seqlens,
                      const int64_t* act_offsets, int64_t num_tokens, int32_t num_seqs, int32_t num_adapters,
                      int32_t* eff_ids, int32_t* seg_offsets, int32_t* perm, void* stream) {
  GS_CHECK_ARG(num_adapters >= 1 && num_adapters <= GS_MAX_ADAPTERS, "gs_build_segments: num_adapters=%d not in [1,%d]",
               num_adapters, GS_MAX_ADAPTERS);
  GS_CHECK_ARG(num_tokens >= 0 && num_tokens < (int64_t(1) << 31), "gs_build_segments: num_tokens=%lld out of range",
               (long long)num_tokens);
  GS_CHECK_ARG(seg_offsets != nullptr, "gs_build_segments: seg_offsets is NULL");
  GS_CHECK_ARG(num_tokens == 0 || (req_ids && eff_ids && perm), "gs_build_segments: NULL token array");
  GS_CHECK_ARG(act_offsets == nullptr || cu_seqlens == nullptr || num_seqs >= 1,
               "gs_build_segments: num_seqs=%d with cu_seqlens", num_seqs);
  BuildArgs a{req_ids, positions, cu_seqlens, act_offsets, static_cast<int>(num_tokens), cu_seqlens ? num_seqs : 1,
              num_adapters, eff_ids, seg_offsets, perm};
  hipLaunchKernelGGL(build_segments_kernel, dim3(1), dim3(kBuildThreads), 0, static_cast<hipStream_t>(stream), a);
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

}  // extern "C"
