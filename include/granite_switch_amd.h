/*
 * granite_switch_amd.h -- C ABI of the MI355X (gfx950) switched-LoRA library.
 *
 * One shared library, libgranite_switch_amd.so, built with hipcc for gfx950.
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * (passed as void*), launches on that stream, never synchronises, never
 * allocates, and returns a GS_* status.  On failure gs_last_error() returns a
 * message for the calling thread.  Tensors are row-major; "ld" arguments are
 * row strides in ELEMENTS.  Token / adapter id convention is the reference's:
 * 0 = base (no LoRA), 1..num_adapters = adapters.
 *
 * Element types (dtype argument): GS_DTYPE_BF16 or GS_DTYPE_FP32.  Compute is
 * fp32-accumulated; bf16 paths use bf16 MFMA on gfx950, fp32 paths fp32 MFMA.
 *
 * Reference interfaces replaced (paths relative to the Granite Switch repo):
 *   gs_build_segments      the per-adapter token grouping of the HF loop
 *                          (src/granite_switch/hf/core/lora.py:127-135, 317-325)
 *                          fed by latest-wins / aLoRA routing
 *                          (src/granite_switch/vllm/switch/multi.py:516-518)
 *   gs_route_latest_wins   control-token routing semantics of MultiSwitch
 *                          (src/granite_switch/vllm/switch/multi.py:348-525)
 *   gs_shrink, gs_expand_add, gs_switched_lora
 *                          the shrink/expand/add of
 *                          src/granite_switch/hf/core/lora.py:127-161, 308-348
 *   gs_switched_lora_small the same shrink/expand/add for decode-sized batches,
 *                          with the per-adapter token grouping of
 *                          src/granite_switch/hf/core/lora.py:127-135 done
 *                          inside the one kernel
 *   gs_compute_bitmasks    torch.ops.granite_switch.compute_per_module_bitmasks
 *                          (src/granite_switch/vllm/core/lora_kernel_meta.py:61-91,
 *                          169-182) plus the remap gather at :294
 *   gs_switch_lora_expand  torch.ops.granite_switch.switch_lora_expand
 *                          (src/granite_switch/vllm/core/lora_ops.py:30-60,192-202;
 *                          src/granite_switch/kernels/switch_lora_kernel.py:414-458)
 *   gs_switch_lora_expand_swiglu
 *                          torch.ops.granite_switch.switch_lora_expand_swiglu
 *                          (lora_ops.py:82-113,204-214; switch_lora_kernel.py:809-857)
 *   gs_switch_lora_shrink_expand
 *                          torch.ops.granite_switch.switch_lora_shrink_expand, the
 *                          Shadow-Residual W_cross shunt's W-less expand
 *                          (lora_ops.py:137-226; switch_lora_kernel.py:883-1146)
 *   gs_split_adapter_indices
 *                          granite_switch.probe_routing.split_adapter_indices
 *                          (src/granite_switch/probe_routing.py:36-58)
 *   gs_gemm_bf16_tn        the layer's one GEMM x_ext = x . w_ext^T over the base
 *                          weight stacked with every adapter's lora_A rows
 *                          (src/granite_switch/vllm/core/lora.py:544;
 *                          w_ext from src/granite_switch/kernels/switch_lora_kernel.py:134-163)
 */
#ifndef GRANITE_SWITCH_AMD_H_
#define GRANITE_SWITCH_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GS_OK 0
#define GS_ERR_INVALID 1     /* bad argument (shape, alignment, limit)            */
#define GS_ERR_HIP 2         /* a HIP runtime call or kernel launch failed         */
#define GS_ERR_WORKSPACE 3   /* workspace too small: see gs_shrink_workspace_bytes */

#define GS_DTYPE_BF16 0
#define GS_DTYPE_FP32 1

#define GS_MAX_ADAPTERS 256  /* global adapter ids handled by the segment builder */
#define GS_MAX_SLICES 8      /* output slices per projection (QKV = 3, gate_up = 2) */
#define GS_MAX_RANK 512      /* largest LoRA rank (the reference's top tier)       */

/* Library version (major*10000 + minor*100 + patch) and last error text. */
int gs_version(void);
const char* gs_last_error(void);

/* ------------------------------------------------------------------------
 * Segment builder.
 *
 * eff_ids[t] = req_ids[t] if the token is activated, else 0, where a token t of
 * sequence s (cu_seqlens[s] <= t < cu_seqlens[s+1]) at absolute position
 * q = positions[t] (or t - cu_seqlens[s] when positions is NULL) is activated
 * iff act_offsets == NULL or q >= act_offsets[s] (aLoRA: tokens before the
 * invocation point are base only).  Ids outside [0, num_adapters] become 0.
 *
 * Then a stable counting sort of the active tokens by adapter:
 *   seg_offsets[0] = 0, seg_offsets[g] = number of active tokens with id <= g;
 *   perm[seg_offsets[g-1] .. seg_offsets[g]) = the tokens of adapter g in
 *   ascending token order.  perm entries past seg_offsets[num_adapters] are
 *   left untouched.
 *
 * req_ids [T] int64; positions [T] int64 or NULL; cu_seqlens [num_seqs+1]
 * int32 or NULL (one sequence); act_offsets [num_seqs] int64 or NULL.
 * Outputs: eff_ids [T] int32, seg_offsets [num_adapters+1] int32, perm [T] int32.
 * Limits: 1 <= num_adapters <= GS_MAX_ADAPTERS; 0 <= T < 2^31.
 *
 * workspace NULL: one launch, in which every 1024-token chunk's workgroup
 * counts the whole batch (its cost grows with T per workgroup).  Non-NULL
 * (4-byte aligned, at least ceil(T/1024) * (num_adapters+1) * 4 bytes, else
 * GS_ERR_WORKSPACE): two launches, each workgroup counting only its chunk,
 * through per-chunk histograms in the workspace.  Both give identical
 * outputs.  gs_build_segments_workspace_bytes returns the size to pass for
 * batches where the two-launch form is the faster one, and 0 where the
 * one-launch form is (pass NULL then).
 * ---------------------------------------------------------------------- */
int64_t gs_build_segments_workspace_bytes(int64_t num_tokens, int32_t num_adapters);
int gs_build_segments(const int64_t* req_ids, const int64_t* positions, const int32_t* cu_seqlens,
                      const int64_t* act_offsets, int64_t num_tokens, int32_t num_seqs, int32_t num_adapters,
                      int32_t* eff_ids, int32_t* seg_offsets, int32_t* perm, void* workspace, int64_t workspace_bytes,
                      void* stream);

/* Test support (no counterpart in the reference; makes no HIP call).  Replays
 * on the host every global and LDS access of gs_build_segments for these
 * inputs (host copies; the same NULL conventions) -- the one-launch form, or
 * the two-launch form when two_launch is nonzero -- gating every token as the
 * kernels do and following each token to the perm slot its scatter writes.
 * Returns the number of accesses outside their buffers (0: clean), the first
 * described in msg, *checked the number checked; a negated GS_* status on bad
 * arguments. */
int64_t gs_check_build_addresses(int64_t num_tokens, int32_t num_seqs, int32_t num_adapters, const int64_t* req_ids,
                                 const int64_t* positions, const int32_t* cu_seqlens, const int64_t* act_offsets,
                                 int32_t two_launch, char* msg, int64_t msg_len, int64_t* checked);

/* Test support (no counterpart in the reference; makes no HIP call).  The
 * replay of the per-token kernels over one token stream of num_tokens:
 * gs_route_latest_wins (num_control control tokens, cu_seqlens host copy or
 * NULL), gs_compute_bitmasks of the ids (host copy; a [na_plus_1,
 * num_modules] remap table, tiles of block_m) with the remapped output, and
 * gs_split_adapter_indices of the same ids with a kind table of lut_len.
 * Returns the number of accesses outside their buffers (0: clean), the first
 * described in msg, *checked the number checked; a negated GS_* status on bad
 * arguments. */
int64_t gs_check_token_addresses(int64_t num_tokens, int32_t num_seqs, const int32_t* cu_seqlens,
                                 int32_t num_control, const int64_t* ids, int32_t na_plus_1, int32_t num_modules,
                                 int32_t block_m, int32_t lut_len, char* msg, int64_t msg_len, int64_t* checked);

/* ------------------------------------------------------------------------
 * Probe-slot split of the per-token index stream (reference ids, 0 = base).
 *
 * kind_lut [lut_len] bytes (torch.bool): entry i != 0 marks adapter index i as
 * an activation-probe slot (build_adapter_kind_lut; entry 0, base, is 0).
 * lora_indices[t] = 0 where adapter_indices[t] is a probe, else the index;
 * probe_indices[t] = the index where it is a probe, else 0.  Either output may
 * be NULL.  Indices outside [0, lut_len) are neither probes nor adapters:
 * both outputs hold 0 there, so the token takes the base model (the
 * reference's table lookup would wrap a negative index and reject one past
 * the end).  adapter_indices and both outputs have
 * element size idx_bytes (4 or 8).  Limits: 1 <= lut_len <= GS_MAX_ADAPTERS+1.
 * ---------------------------------------------------------------------- */
int gs_split_adapter_indices(const uint8_t* kind_lut, int32_t lut_len, const void* adapter_indices,
                             int32_t idx_bytes, int64_t num_tokens, void* lora_indices, void* probe_indices,
                             void* stream);

/* ------------------------------------------------------------------------
 * Latest-wins routing from control tokens (per sequence, across chunks).
 *
 * out_ids[t] = the adapter fired by the most recent control token at or before
 * token t within its sequence, else start_ids[s] (the id in force at the end of
 * the sequence's cached prefix; NULL = 0).  A token equal to
 * control_tokens[k] fires id k + id_offset (id_offset = 1 for the layout with no
 * base slot, 0 for the base-reset layout whose slot 0 re-selects base).
 * input_ids [T] int64; cu_seqlens [num_seqs+1] int32 or NULL;
 * control_tokens [num_control] int64; start_ids [num_seqs] int64 or NULL;
 * out_ids [T] int64.  Limits: num_control <= GS_MAX_ADAPTERS + 1.
 * ---------------------------------------------------------------------- */
int gs_route_latest_wins(const int64_t* input_ids, const int32_t* cu_seqlens, int64_t num_tokens,
                         int32_t num_seqs, const int64_t* control_tokens, int32_t num_control, int32_t id_offset,
                         const int64_t* start_ids, int64_t* out_ids, void* stream);

/* ------------------------------------------------------------------------
 * Per-module packed adapter weights (built once at load time by the host):
 *   ranks [num_adapters+1] int32: rank of adapter g in this module, 0 if g is
 *       not applicable here (ranks[0] = 0).  bf16 ranks must be multiples of 8.
 *   a_pack + a_off[g]: S*r_g rows of `hidden` elements, row s*r_g + j is
 *       lora_A of slice s, rank row j (the reference's w_ext tail order).
 *   b_pack + b_off[g]: [out_total, r_g] row-major (slices concatenated along
 *       out, rank contiguous -- the reference's lora_B_merged / lb_packed
 *       layout), already scaled by alpha/r.
 *   slice_bounds [S+1] int32 (host array): output column where each slice
 *       starts; every slice width must be a multiple of 32.
 *   ranks_host [num_adapters+1] int32 (host array) or NULL: the same values
 *       as ranks, on the host.  With it the module's adapters are split into
 *       rank classes (ranks <= 64 and ranks above) and each class is planned
 *       and launched for its own largest rank, so a large adapter's tile
 *       widths, k-split, LDS and registers apply only to its own tokens (the
 *       reference's per-adapter rank tiers, docs/SWITCH_KERNELS.md "per-adapter
 *       rank tiers").  An entry of 0 skips that adapter.  NULL: one class of
 *       every rank up to max_rank.
 * ---------------------------------------------------------------------- */
#define GS_RANK_CLASS_SPLIT 64

/* Workspace for gs_shrink / gs_switched_lora: fp32 split-K partial sums.
 * The hidden dimension is split over several workgroups when there are too
 * few tiles to fill the GPU; each writes its own partial and the consumer adds
 * them in a fixed order (deterministic).  No initialisation is needed.  Calls
 * that share a workspace must not overlap in time (stream order is enough).
 * For a module of two rank classes the size holds both classes' partials
 * side by side and then one 256-byte line for the item counter of
 * gs_switched_lora's pair launches (which the call itself zeroes); a
 * workspace without that line but with both partials runs the classes on two
 * streams, and one that holds only the larger class's partials runs them in
 * turn.  All three give the same bits. */
int64_t gs_shrink_workspace_bytes(int64_t num_tokens, int32_t hidden, int32_t num_slices, int32_t num_adapters,
                                  int32_t max_rank, const int32_t* ranks_host);

/* The hidden-dimension split (k-chunks) of each rank class of a module for
 * this batch size and dtype: writes ksplit[0..n) (n <= 2) and returns n (0
 * when no adapter is applicable, a negated GS_* status on bad arguments).  No
 * counterpart in the reference (its shrink is the fused GEMM); it tells a
 * caller whether gs_shrink may write partials only (one class split >1). */
int32_t gs_shrink_ksplits(int32_t dtype, int64_t num_tokens, int32_t hidden, int32_t num_slices,
                          int32_t num_adapters, int32_t max_rank, const int32_t* ranks_host, int32_t* ksplit);

/* Whether gs_switched_lora, with a workspace of gs_shrink_workspace_bytes,
 * runs this module's two rank classes in its pair launches for this batch
 * size and dtype: 1 yes, 0 no (one class, fp32, a large class that is not
 * sparse, or forms the pair kernels do not take), a negated GS_* status on
 * bad arguments.  No counterpart in the reference; it lets a caller choose
 * between the segment kernels and the one-launch decode kernel for a module
 * with a rank above GS_RANK_CLASS_SPLIT (switched.path_plan). */
int32_t gs_switched_lora_pair(int32_t dtype, int64_t num_tokens, int32_t hidden, int32_t out_total,
                              const int32_t* slice_bounds, int32_t num_slices, int32_t num_adapters, int32_t max_rank,
                              const int32_t* ranks_host);

/* z[slot, s*r_g + j] = sum_k x[perm[slot], k] * lora_A_{g,s}[j, k] for every
 * active slot (slot < seg_offsets[num_adapters]) whose adapter is applicable.
 * x [T, hidden] (ld ldx); z [T, ldz] with ldz >= S*max_rank; same dtype.
 * When the module is one rank class whose hidden dimension is split
 * (gs_shrink_ksplits), z may be NULL: only the fp32 partials
 * [KS][T][S*max_rank] are written to the workspace, the shrink half of
 * gs_switched_lora. */
int gs_shrink(int32_t dtype, const void* x, int64_t ldx, int64_t num_tokens, int32_t hidden, const void* a_pack,
              const int64_t* a_off, const int32_t* ranks, int32_t num_slices, int32_t num_adapters,
              int32_t max_rank, const int32_t* ranks_host, const int32_t* seg_offsets, const int32_t* perm, void* z,
              int64_t ldz, void* workspace, int64_t workspace_bytes, void* stream);

/* y[perm[slot], n] = round(y + sum_k z[row, zcol + k] * B_g[n, k]) for every
 * active slot and output column n, k < r_g, where n lies in slice s,
 * zcol = z_off[g] + s*r_g, and row = perm[slot] if z_by_token else slot.
 * Rows of base tokens and of non-applicable adapters are not touched.
 * z_off [num_adapters+1] int32 or NULL (all zero). */
int gs_expand_add(int32_t dtype, void* y, int64_t ldy, int64_t num_tokens, int32_t out_total,
                  const int32_t* slice_bounds, int32_t num_slices, const void* z, int64_t ldz, int32_t z_by_token,
                  const int32_t* z_off, const void* b_pack, const int64_t* b_off, const int32_t* ranks,
                  int32_t num_adapters, int32_t max_rank, const int32_t* ranks_host, const int32_t* seg_offsets,
                  const int32_t* perm, void* stream);

/* The whole switched-LoRA delta added into y in two launches: the shrink,
 * then the expand reading the shrink's output directly (split-K partials are
 * summed while they are staged, so z is only written when the shrink is not
 * split), once per rank class.  z [T, S*max_rank] scratch of the same dtype.
 * A module of two rank classes with a workspace of gs_shrink_workspace_bytes:
 *   - bf16 with a sparse large class (e.g. one rank-512 adapter among rank-32
 *     ones): both classes in the same two launches, the small class's
 *     workgroups taking the large class's items once their own are done;
 *   - otherwise, when `stream` belongs to the current device: the large class
 *     on the library's side stream of the current device (default priority,
 *     created on the first such call: make it eagerly, outside graph capture),
 *     forked from `stream` after the work queued before the call and joined
 *     back into it before the work queued after (events; captured into a graph
 *     like any other work on `stream`).
 * The classes write disjoint rows of y and z and disjoint ranges of the
 * workspace. */
int gs_switched_lora(int32_t dtype, const void* x, int64_t ldx, void* y, int64_t ldy, int64_t num_tokens,
                     int32_t hidden, int32_t out_total, const int32_t* slice_bounds, int32_t num_slices,
                     const void* a_pack, const int64_t* a_off, const void* b_pack, const int64_t* b_off,
                     const int32_t* ranks, int32_t num_adapters, int32_t max_rank, const int32_t* ranks_host,
                     const int32_t* seg_offsets, const int32_t* perm, void* z, void* workspace,
                     int64_t workspace_bytes, void* stream);

/* Test support (no counterpart in the reference; makes no HIP call).  Replays
 * on the host every global and LDS access the segment kernels would make for
 * this call -- the launches of gs_switched_lora with a caller workspace and
 * with gs_switched_lora_noalloc's static scratch, and gs_shrink (z written,
 * split partials reduced) followed by gs_expand_add; with z_off given, also
 * gs_expand_add reading its shrink values by token from a [T, z_ld] matrix
 * (the vLLM layer's x_ext columns) -- for every workgroup, wave, lane and loop
 * step, with the launches' own plans and the kernels' address arithmetic
 * (gs_addr.h), and for each possible number of resident expand workgroups
 * per CU (1..4).  Host copies of the tables: a_off / b_off / ranks
 * [num_adapters+1], seg_offsets [num_adapters+1], perm [num_tokens] (as
 * gs_build_segments writes them).  Returns the number of accesses outside
 * their buffers plus items a grid leaves uncovered (0: clean), the first one
 * described in msg; *checked receives the number of accesses checked; a
 * negated GS_* status on bad arguments. */
int64_t gs_check_segment_addresses(int32_t dtype, int64_t num_tokens, int32_t hidden, int64_t ldx, int32_t out_total,
                                   int64_t ldy, const int32_t* slice_bounds, int32_t num_slices, const int64_t* a_off,
                                   int64_t a_pack_elems, const int64_t* b_off, int64_t b_pack_elems,
                                   const int32_t* ranks, int32_t num_adapters, int32_t max_rank,
                                   const int32_t* seg_offsets, const int32_t* perm, const int32_t* z_off,
                                   int64_t z_ld, char* msg, int64_t msg_len, int64_t* checked);

/* Test support (no counterpart in the reference; makes no HIP call).  The
 * same replay for the reference-semantics ops over x_ext: op 0
 * gs_switch_lora_expand (the launch form this device would take and every
 * other column-block shape, plus the per-tile forms), op 1
 * gs_switch_lora_shrink_expand into out [M, >= N] (stride_om, out_dtype),
 * op 2 gs_switch_lora_expand_swiglu into out [M, H] (stride_om).  x_ext has M
 * rows of x_cols valid elements, stride_m apart.  Host copies of the values
 * that steer the kernels: ids [M] (kernel-local, as idx_bytes-wide ids would
 * hold them), bitmask (bitmask_elems, tile pm at pm * stride_bm),
 * tile_slice [tile_slice_len] (unused by op 2), slice_col_r [S * 6], na[6];
 * lb_elems: the packed lora_B's size.  Returns the number of accesses outside
 * their buffers (0: clean), the first described in msg, *checked the number
 * checked; a negated GS_* status on bad arguments. */
int64_t gs_check_xext_addresses(int32_t op, int64_t M, int64_t stride_m, int64_t x_cols, const int64_t* ids,
                                int32_t idx_bytes, const int64_t* bitmask, int64_t stride_bm, int64_t bitmask_elems,
                                int64_t lb_elems, const int32_t* tile_slice, int64_t tile_slice_len,
                                const int32_t* slice_col_r, const int32_t* na, int32_t S, int32_t block_n, int32_t N,
                                int32_t H, int64_t stride_om, int32_t out_dtype, char* msg, int64_t msg_len,
                                int64_t* checked);

/* Test support (no counterpart in the reference; makes no HIP call).  The
 * same replay for the one-launch small-batch kernel (gs_switched_lora_small):
 * the routing loads, every producer and consumer workgroup, wave, lane and
 * loop step, with the call's own plan (row_split) and the workspace size
 * gs_small_workspace_bytes gives.  eff_ids [num_tokens]: the gated ids the
 * kernel's routing produces (host copy; they give each adapter's token
 * list).  route_flags: which routing inputs the call passes -- 1 eff_ids,
 * 2 positions, 4 cu_seqlens (num_seqs sequences), 8 act_offsets.  Returns
 * the number of accesses outside their buffers (0: clean), the first
 * described in msg, *checked the number checked; a negated GS_* status on
 * bad arguments. */
int64_t gs_check_small_addresses(int32_t dtype, int64_t num_tokens, int32_t hidden, int64_t ldx, int32_t out_total,
                                 int64_t ldy, const int32_t* slice_bounds, int32_t num_slices, const int64_t* a_off,
                                 int64_t a_pack_elems, const int64_t* b_off, int64_t b_pack_elems,
                                 const int32_t* ranks, int32_t num_adapters, int32_t max_rank, const int32_t* eff_ids,
                                 int32_t num_seqs, int32_t route_flags, int32_t row_split, char* msg, int64_t msg_len,
                                 int64_t* checked);

/* The same op with its scratch (split-K partials and z) in a static device
 * array of GS_NOALLOC_SCRATCH_BYTES per GPU, so it allocates nothing: no
 * workspace, no z, no hipMalloc.  No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation).  The array is looked up once per
 * device (hipGetSymbolAddress, on the first call with that device current):
 * make that first call outside graph capture (one eager call); launch on a
 * stream of the current device.  Shapes whose partials plus z
 * exceed the array are rejected with GS_ERR_WORKSPACE (use gs_switched_lora
 * with a workspace then).  Every call on a GPU shares that GPU's array, which
 * keeps the last call's contents (nothing needs to start at zero): calls that
 * overlap in time on one GPU race; stream order keeps them apart. */
#define GS_NOALLOC_SCRATCH_BYTES (64ll << 20)
int gs_switched_lora_noalloc(int32_t dtype, const void* x, int64_t ldx, void* y, int64_t ldy, int64_t num_tokens,
                             int32_t hidden, int32_t out_total, const int32_t* slice_bounds, int32_t num_slices,
                             const void* a_pack, const int64_t* a_off, const void* b_pack, const int64_t* b_off,
                             const int32_t* ranks, int32_t num_adapters, int32_t max_rank, const int32_t* ranks_host,
                             const int32_t* seg_offsets, const int32_t* perm, void* stream);

/* ------------------------------------------------------------------------
 * Small-batch switched-LoRA in ONE launch, no segment build (decode-sized
 * batches).  Same result as gs_build_segments + gs_switched_lora: every
 * workgroup gates and lists the tokens of its own adapter from the routing
 * input, so no metadata kernel runs first, and the expand workgroups of the
 * launch wait (bounded) for the shrink partials they read, which carry the
 * launch's epoch tag.
 *
 * Routing input, one of:
 *   eff_ids [T] int32 -- ids already gated (e.g. gs_build_segments' eff_ids);
 *   req_ids [T] int64 (+ positions, cu_seqlens, act_offsets, num_seqs with the
 *   meaning of gs_build_segments) when eff_ids is NULL.
 * a_off, b_off [num_adapters+1] int64 and ranks [num_adapters+1] int32 are
 * HOST arrays here (load-time constants of the module; they travel in the
 * kernel arguments), with the layout described above.
 * Limits (gs_small_eligible): T <= 1024, num_seqs <= 1024,
 * num_adapters <= 64, max_rank <= 64, every slice width a multiple of 128.
 * workspace: gs_small_workspace_bytes(...) bytes, 16-byte aligned, ZEROED
 * before the first call and used by nothing but this entry point (it holds
 * epoch-tagged partial sums; any size change may reuse the same buffer).
 * sync: gs_small_sync_bytes() bytes, 8-byte aligned, ZEROED before the first
 * call: int32 word 2 is an error word whose bit 0 means an expand workgroup
 * gave up waiting for its shrink partials (gs_small_set_wait_limit) and that
 * call's output is wrong -- callers read it at a point that already
 * synchronises and treat a nonzero word as a failed call; int32 words
 * [32*g, 32*g + 1] hold adapter g's 64-bit launch counter (each launch with
 * tokens for g adds 2^20; bits 20 and up are g's epoch, the tag of its
 * partials).  Zeroing sync again requires zeroing the workspace too.  Calls
 * sharing a workspace or sync buffer must not overlap in time (stream order
 * is enough).
 * row_split (1..32) cuts each adapter's token list into 32-token chunks and
 * gives chunks rs, rs + row_split, ... to a workgroup set of their own, so an
 * adapter with many tokens runs on row_split times the workgroups; the result
 * does not depend on it.  1 suits decode (a few tokens per adapter); about
 * (largest adapter group) / 64 suits larger batches.
 * speculate != 0 issues every adapter's weight loads before the routing is
 * known (saves a memory round trip when most adapters have tokens); 0 reads
 * only the weights of adapters some token requests.
 * ---------------------------------------------------------------------- */
int gs_small_eligible(int64_t num_tokens, int32_t num_seqs, int32_t num_slices, const int32_t* slice_bounds,
                      int32_t num_adapters, int32_t max_rank);
int64_t gs_small_workspace_bytes(int32_t dtype, int64_t num_tokens, int32_t hidden, int32_t num_slices,
                                 int32_t num_adapters, int32_t max_rank, int32_t out_total,
                                 const int32_t* slice_bounds);
int64_t gs_small_sync_bytes(void);
/* Process-wide bound on the expand workgroups' wait: each gives up after
 * `polls` looks at a group of its shrink partials (a look is one coherent
 * load round trip plus a short sleep), sets bit 0 of the error word and
 * finishes, so every launch ends.  The bound counts looks, not time, so a
 * preempted queue does not use it up.  polls < 0 restores the default
 * (200000, tens to hundreds of milliseconds); 0 never looks and always
 * reports the error (a test hook: the launch still completes normally).
 * Returns the previous value.  Applies to launches made after the call.
 * No counterpart in the reference (its kernels never wait on each other). */
int64_t gs_small_set_wait_limit(int64_t polls);
/* Workgroups of one gs_switched_lora_small launch for this shape and row split
 * (producers + consumers; 0 for arguments outside the limits).  No
 * counterpart in the reference: this library's path choice uses it -- the
 * one-launch kernel wins while its grid fits the GPU about once, the segment
 * kernels beyond. */
int64_t gs_small_workgroups(int32_t dtype, int64_t num_tokens, int32_t hidden, int32_t num_slices,
                            int32_t num_adapters, int32_t max_rank, int32_t out_total,
                            const int32_t* slice_bounds, int32_t row_split);
int gs_switched_lora_small(int32_t dtype, const int64_t* req_ids, const int64_t* positions,
                           const int32_t* cu_seqlens, const int64_t* act_offsets, int32_t num_seqs,
                           const int32_t* eff_ids, const void* x, int64_t ldx, void* y, int64_t ldy,
                           int64_t num_tokens, int32_t hidden, int32_t out_total, const int32_t* slice_bounds,
                           int32_t num_slices, const void* a_pack, const int64_t* a_off, const void* b_pack,
                           const int64_t* b_off, const int32_t* ranks, int32_t num_adapters, int32_t max_rank,
                           void* workspace, int64_t workspace_bytes, int32_t* sync, int64_t sync_bytes,
                           int32_t row_split, int32_t speculate, void* stream);

/* ------------------------------------------------------------------------
 * Reference op: per-module tile bitmasks and kernel-local ids.
 * bitmasks[m, tile] (int64, [num_modules, ceil(M/block_m)]) has bit (loc-1) set
 * iff some token of the tile has kernel-local id loc = remap_t[clamp(id,0,NA), m]
 * > 0 (loc 64 sets the sign bit); the tail tile is padded with id 0.
 * remapped (int64 [num_modules, M], NULL to skip) = remap_t[clamp(id), m].
 * adapter_indices [M] with element size idx_bytes (4 or 8);
 * remap_tables_t [NA+1, num_modules] int64.  1 <= block_m <= 1024.
 * ---------------------------------------------------------------------- */
int gs_compute_bitmasks(const void* adapter_indices, int32_t idx_bytes, int64_t M, const int64_t* remap_tables_t,
                        int32_t na_plus_1, int32_t num_modules, int32_t block_m, int64_t* bitmasks,
                        int64_t* remapped, void* stream);

/* ------------------------------------------------------------------------
 * Reference op: in-place expand over x_ext (bf16), reference semantics.
 * x_ext [M, >= N + shrink cols] with strides (stride_m, stride_n) in elements;
 * adapter_indices [M] kernel-local ids (element size idx_bytes 4 or 8);
 * bitmask [ceil(M/32)] int64 with stride stride_bm; lb_packed bf16 (tiers
 * concatenated, each [NA_r, N, r]); tile_slice [ceil(N/block_n)] int32;
 * slice_col_r [S, 6] int32; na[6] = NA_16..NA_512 (host array).
 * Requires block_n % 32 == 0 and N % 32 == 0.
 * ---------------------------------------------------------------------- */
int gs_switch_lora_expand(void* x_ext, int64_t stride_m, int64_t stride_n, int64_t M, const void* adapter_indices,
                          int32_t idx_bytes, const int64_t* bitmask, int64_t stride_bm, const void* lb_packed,
                          const int32_t* tile_slice, const int32_t* slice_col_r, const int32_t* na, int32_t S,
                          int32_t block_n, int32_t N, void* stream);

/* Reference op: out[M, H] = silu(gate + dgate) * (up + dup), always written.
 * gate = x_ext[:, 0:H], up = x_ext[:, H:2H]; out dtype bf16 with strides
 * (stride_om, stride_on).  S must be 2 and N = 2H.  H % 32 == 0. */
int gs_switch_lora_expand_swiglu(void* out, int64_t stride_om, int64_t stride_on, const void* x_ext,
                                 int64_t stride_m, int64_t stride_n, int64_t M, const void* adapter_indices,
                                 int32_t idx_bytes, const int64_t* bitmask, int64_t stride_bm,
                                 const void* lb_packed, const int32_t* slice_col_r, const int32_t* na, int32_t S,
                                 int32_t block_n, int32_t H, int32_t N, void* stream);

/* Reference op: the W-less expand of the Shadow-Residual cross-stream shunt.
 * out[m, n] = sum over the tier adapters present in m's 32-row tile of
 * shrink[m, :r] . lb[n, :r] for a row whose kernel-local id selects that
 * adapter, 0 for base rows and for every row of a tile whose bitmask is 0;
 * out[:M, :N] is written in full (the reference zeroes out first and stores
 * the delta of the tiles it does not skip).  x_ext [M, >= shrink cols] holds
 * only shrink columns (slice_col_r bases start at 0); other arguments as for
 * gs_switch_lora_expand.  out_dtype GS_DTYPE_BF16 or GS_DTYPE_FP32, row
 * stride stride_om >= N (elements), stride_on == 1, rows 16-byte aligned. */
int gs_switch_lora_shrink_expand(void* out, int32_t out_dtype, int64_t stride_om, int64_t stride_on,
                                 const void* x_ext, int64_t stride_m, int64_t stride_n, int64_t M,
                                 const void* adapter_indices, int32_t idx_bytes, const int64_t* bitmask,
                                 int64_t stride_bm, const void* lb_packed, const int32_t* tile_slice,
                                 const int32_t* slice_col_r, const int32_t* na, int32_t S, int32_t block_n, int32_t N,
                                 void* stream);

/* ------------------------------------------------------------------------
 * Dense bf16 GEMM C[M,N] = A[M,K] . B[N,K]^T with fp32 accumulation and one
 * bf16 rounding per element (round-to-nearest-even).  A, B, C row-major with
 * row strides lda, ldb, ldc in elements; A and B rows K-contiguous (the
 * layer's x and w_ext).  K a positive multiple of 8, lda and ldb multiples
 * of 8, A and B 16-byte aligned.  No size limit on M and N.
 * ---------------------------------------------------------------------- */
int gs_gemm_bf16_tn(const void* a, int64_t lda, const void* b, int64_t ldb, void* c, int64_t ldc, int64_t M,
                    int64_t N, int64_t K, void* stream);

/* Test support (no counterpart in the reference; makes no HIP call).  Replays
 * on the host every global and LDS access of gs_gemm_bf16_tn's kernels for
 * this shape (the direct-to-LDS form when K % 64 == 0, plus the
 * register-staged form) -- every workgroup, thread and k-tile -- and checks
 * that the grid takes every tile exactly once.  Returns the number of
 * violations (0: clean), the first described in msg, *checked the number of
 * accesses checked; a negated GS_* status on bad arguments. */
int64_t gs_check_gemm_addresses(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, char* msg,
                                int64_t msg_len, int64_t* checked);

#ifdef __cplusplus
}
#endif

#endif /* GRANITE_SWITCH_AMD_H_ */
