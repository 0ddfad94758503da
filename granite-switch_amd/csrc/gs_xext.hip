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
  const uint16_t* xrow = static_cast<const uint16_t*>(a.x_ext) + (m0 + i) * a.stride_m;
  while (todo) {
    const int b = __builtin_amdgcn_readfirstlane(__ffsll(static_cast<long long>(todo)) - 1);   // uniform
    todo &= todo - 1;
    const int kid = b + 1;   // kernel-local id
    // tier lookup: ids are numbered 1.. across tiers in ascending-rank order
    int t = 0, first = 1;
    int64_t lb_off = 0;
    while (t < 6 && kid >= first + a.na[t]) {
      first += a.na[t];
      lb_off += static_cast<int64_t>(a.na[t]) * a.N * (16 << t);   // tier t holds rank 16 << t
      ++t;
    }
    if (t >= 6) break;   // cannot happen: the loop runs only over bits <= total count
    const int r = 16 << t;
    const int idx = kid - first;
    const int64_t c0 = static_cast<int64_t>(scr[s * 6 + t]) + static_cast<int64_t>(idx) * a.S * r;
    const uint16_t* brow = a.lb + lb_off + static_cast<int64_t>(idx) * a.N * r + static_cast<int64_t>(n0 + i) * r;
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

// Only bits for kernel-local ids that exist (1..sum(na)) may be followed.
__device__ __forceinline__ uint64_t valid_bits(const int na[6]) {
  int tot = 0;
  for (int t = 0; t < 6; ++t) tot += na[t];
  return tot >= 64 ? ~0ull : ((1ull << tot) - 1ull);
}

__global__ __launch_bounds__(256) void xext_expand_kernel(XextArgs a, uint16_t* x_out, const int32_t* __restrict__ tile_slice,
                                                          int block_n) {
  __shared__ float dtile[32][128 + 4];
  __shared__ int scr[GS_MAX_SLICES * 6];
  const int64_t pm = blockIdx.y;
  const uint64_t bm = static_cast<uint64_t>(a.bitmask[pm * a.stride_bm]) & valid_bits(a.na);
  if (a.bitmask[pm * a.stride_bm] == 0) return;
  // the slice column table, staged once (the adapter loop reads it per adapter)
  if (threadIdx.x < a.S * 6) scr[threadIdx.x] = a.slice_col_r[threadIdx.x];
  const int n_tile0 = blockIdx.x * 128;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int i = l & 31;
  const int64_t m0 = pm * 32;
  const bool row_ok = (m0 + i) < a.M;
  const int id = row_ok ? load_id(a.ids, a.idx_bytes, m0 + i) : 0;

  const int n0 = n_tile0 + 32 * wave;
  const int s = tile_slice[(n0 < a.N ? n0 : n_tile0) / block_n];
  lds_barrier();
  f32x16 acc = f32x16{};
  if (n0 < a.N) acc = xext_block_delta(a, scr, m0, n0, s, id, row_ok, bm);
#pragma unroll
  for (int v = 0; v < 16; ++v) dtile[mfma32_row(v, l)][32 * wave + i] = acc[v];
  lds_barrier();

  const int row = tid >> 3;
  const int cx = (tid & 7) * 16;
  const int64_t m = m0 + row;
  if (m >= a.M || n_tile0 + cx >= a.N) return;
  if (load_id(a.ids, a.idx_bytes, m) == 0) return;   // base rows are never written
  uint16_t* p = x_out + m * a.stride_m + n_tile0 + cx;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const u32x4 in = *reinterpret_cast<const u32x4*>(p + half * 8);
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = bf16_bits_to_f32(static_cast<uint16_t>(in[e] & 0xffffu)) + dtile[row][cx + half * 8 + 2 * e];
      const float hi = bf16_bits_to_f32(static_cast<uint16_t>(in[e] >> 16)) + dtile[row][cx + half * 8 + 2 * e + 1];
      o[e] = static_cast<uint32_t>(f32_to_bf16_bits(lo)) | (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
    }
    *reinterpret_cast<u32x4*>(p + half * 8) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// W-less expand (the reference's switch_lora_shrink_expand): x_ext holds only
// shrink columns, and out[M, N] receives the delta itself.  The reference
// zeroes out and then stores the delta of every tile with a nonzero bitmask;
// here every workgroup stores its whole 32 x 128 tile -- the delta, exactly
// zero for base rows (they select no adapter), and zeros for a tile whose
// bitmask is 0 -- so out is written once and no zeroing pass is needed.
template <bool F32OUT>
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
    if (n0 < a.N) acc = xext_block_delta(a, scr, m0, n0, s, id, row_ok, bm);
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

__global__ __launch_bounds__(256) void xext_swiglu_kernel(XextArgs a, uint16_t* out, int64_t stride_om, int H) {
  __shared__ float dg[32][128 + 4];
  __shared__ float du[32][128 + 4];
  __shared__ int scr[GS_MAX_SLICES * 6];
  const int64_t pm = blockIdx.y;
  const int64_t bm_raw = a.bitmask[pm * a.stride_bm];
  const uint64_t bm = static_cast<uint64_t>(bm_raw) & valid_bits(a.na);
  const int h_tile0 = blockIdx.x * 128;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int i = l & 31;
  const int64_t m0 = pm * 32;
  const bool row_ok = (m0 + i) < a.M;
  // this thread's gate and up pieces (row tid / 8, 16 columns) do not depend
  // on the delta: they go out first, from a clamped in-bounds address
  const int row = tid >> 3;
  const int cx = (tid & 7) * 16;
  const int64_t m = m0 + row;
  const bool out_ok = m < a.M && h_tile0 + cx < H;
  const uint16_t* xr = static_cast<const uint16_t*>(a.x_ext) + (out_ok ? m : m0) * a.stride_m +
                       (out_ok ? h_tile0 + cx : h_tile0);
  u32x4 gi[2], ui[2];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    gi[half] = *reinterpret_cast<const u32x4*>(xr + half * 8);
    ui[half] = *reinterpret_cast<const u32x4*>(xr + H + half * 8);
  }

  if (bm_raw != 0) {
    if (tid < a.S * 6) scr[tid] = a.slice_col_r[tid];
    const int id = row_ok ? load_id(a.ids, a.idx_bytes, m0 + i) : 0;
    lds_barrier();
    const int h0 = h_tile0 + 32 * wave;
    f32x16 ag = f32x16{}, au = f32x16{};
    if (h0 < H) {
      ag = xext_block_delta(a, scr, m0, h0, 0, id, row_ok, bm);
      au = xext_block_delta(a, scr, m0, H + h0, 1, id, row_ok, bm);
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      dg[mfma32_row(v, l)][32 * wave + i] = ag[v];
      du[mfma32_row(v, l)][32 * wave + i] = au[v];
    }
  }
  lds_barrier();

  if (!out_ok) return;
  uint16_t* orow = out + m * stride_om + h_tile0 + cx;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float r2[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = half * 8 + 2 * e + j;
        float g = bf16_bits_to_f32(static_cast<uint16_t>((gi[half][e] >> (16 * j)) & 0xffffu));
        float u = bf16_bits_to_f32(static_cast<uint16_t>((ui[half][e] >> (16 * j)) & 0xffffu));
        if (bm_raw != 0) {
          g += dg[row][cx + c];
          u += du[row][cx + c];
        }
        r2[j] = g / (1.0f + expf(-g)) * u;
      }
      o[e] = static_cast<uint32_t>(f32_to_bf16_bits(r2[0])) | (static_cast<uint32_t>(f32_to_bf16_bits(r2[1])) << 16);
    }
    *reinterpret_cast<u32x4*>(orow + half * 8) = u32x4{o[0], o[1], o[2], o[3]};
  }
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
  hipLaunchKernelGGL(xext_expand_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a,
                     static_cast<uint16_t*>(x_ext), tile_slice, block_n);
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
  if (out_dtype == GS_DTYPE_FP32)
    hipLaunchKernelGGL(xext_shrink_expand_kernel<true>, grid, dim3(256), 0, st, a, out, stride_om, tile_slice, block_n);
  else
    hipLaunchKernelGGL(xext_shrink_expand_kernel<false>, grid, dim3(256), 0, st, a, out, stride_om, tile_slice, block_n);
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
  hipLaunchKernelGGL(xext_swiglu_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a,
                     static_cast<uint16_t*>(out), stride_om, H);
  GS_CHECK_LAUNCH("gs_switch_lora_expand_swiglu");
  return GS_OK;
}

}  // extern "C"
