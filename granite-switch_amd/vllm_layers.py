"""vLLM-form ``SwitchedLoRALinear`` on MI355X.

Same constructor, parameter names, ``weight_loader``s, ``finalize_weights``
and ``forward`` contract as src/granite_switch/vllm/core/lora.py:40-686, with
the vLLM-specific pieces (parallel linear classes, distributed groups) taken
as arguments so the class works without vLLM:

  forward(x) -> (out, output_bias):
    x_ext = x . w_ext^T           one GEMM: base output + every adapter's shrink
                                  (torch.mm, i.e. hipBLASLt; this library's own
                                  MFMA GEMM gs_gemm_bf16_tn with
                                  ``native_gemm = True``, bf16 only)
    expand, in place into x_ext[:, :N_total]
    [row-parallel all-reduce] [bias]

The expand runs on the shared context's adapter-sorted segments
(``gs_expand_add`` reading the shrink columns straight out of x_ext), or, when
the context carries only the reference metadata, through
``torch.ops.granite_switch.switch_lora_expand`` -- both give the reference's
result.  The gate/up projection with ``fuse_swiglu`` uses the fused
expand+SwiGLU op.
"""

from __future__ import annotations

import logging

import numpy as np
import torch
from torch import nn

from . import _lib, ops
from .kernels import BLOCK_M, BLOCK_N, SUPPORTED_RANKS, build_w_ext, promote_rank
from . import switched
from .switched import _dtype_code, _i32_array

logger = logging.getLogger(__name__)


class _FusionPlan:
    """Host-side tables of the fused layer, derived from the checkpoint.

    Definitions (src/granite_switch/vllm/core/lora.py:353-492 and :637-657
    compute the same tables):

    * adapter ``a`` (0-based) is *applicable* iff some value in the first
      ``rank[a]`` rows of its lora_A is nonzero in some slice;
    * its *tier* is ``promote_rank(rank[a])``;
    * kernel-local numbering: tiers in ascending order, and inside a tier the
      applicable adapters in ascending index -- ``order`` lists (a, tier) in
      that numbering, ``remap[a + 1]`` is a's kernel-local id (0 = none);
    * ``na[t]`` counts the adapters of tier ``SUPPORTED_RANKS[t]``;
    * shrink columns of x_ext follow the N base columns tier by tier, each
      adapter taking S * tier columns (slice-major), so slice s of tier t
      starts at ``slice_col_r[s][t] = N + sum_{t' < t} na[t'] S r_t' + s r_t``;
    * ``tile_slice[j]`` is the slice holding output column ``j * block_n``.
    """

    def __init__(self, A_slices, ranks, output_slices, block_n):
        NA, _, stored, _ = A_slices[0].shape
        dev = A_slices[0].device
        rk = torch.as_tensor([int(r) for r in ranks], device=dev)
        live = torch.zeros(NA, stored, dtype=torch.bool, device=dev)
        for A in A_slices:
            live |= A[:, 0].ne(0).any(dim=-1)
        within = torch.arange(stored, device=dev).unsqueeze(0) < rk.unsqueeze(1)
        applicable = (live & within).any(dim=1).tolist()          # the one host sync
        self.tier = [promote_rank(int(r)) for r in ranks]
        self.order = [(a, r) for r in SUPPORTED_RANKS for a in range(NA) if applicable[a] and self.tier[a] == r]
        self.remap = [0] * (NA + 1)
        for local, (a, _) in enumerate(self.order, start=1):
            self.remap[a + 1] = local
        self.na = tuple(sum(1 for _, r in self.order if r == t) for t in SUPPORTED_RANKS)
        self.S = len(output_slices)
        self.bounds = [0] + list(np.cumsum(output_slices, dtype=np.int64).tolist())
        self.n_total = int(self.bounds[-1])
        self.tier_base = (self.n_total + np.concatenate(
            [[0], np.cumsum([n * self.S * r for n, r in zip(self.na, SUPPORTED_RANKS)])[:-1]])).astype(np.int64)
        self.slice_col_r = (self.tier_base[None, :]
                            + np.arange(self.S)[:, None] * np.asarray(SUPPORTED_RANKS)[None, :]).tolist()
        starts = np.arange(-(-self.n_total // block_n)) * block_n
        self.tile_slice = (np.searchsorted(np.asarray(self.bounds), starts, side="right") - 1).tolist()

    @staticmethod
    def _rows(mat, r):
        """The first r rows of ``mat``, zero rows appended past its end."""
        if mat.shape[0] >= r:
            return mat[:r]
        return torch.cat([mat, mat.new_zeros(r - mat.shape[0], *mat.shape[1:])])

    def lora_A_by_tier(self, A_slices) -> dict:
        """{tier: [n_t, S, tier, K]} in kernel-local order (build_w_ext's input)."""
        out = {}
        for r in SUPPORTED_RANKS:
            members = [a for a, t in self.order if t == r]
            if members:
                out[r] = torch.stack([torch.stack([self._rows(A[a, 0], r) for A in A_slices]) for a in members])
        return out

    def lb_packed(self, B_slices) -> torch.Tensor:
        """Every kernel-local adapter's [N, tier] lora_B (slices stacked along N,
        rank contiguous), concatenated in kernel-local order."""
        parts = [torch.cat([self._rows(B[a, 0].t(), r).t() for B in B_slices]).reshape(-1) for a, r in self.order]
        if not parts:
            return B_slices[0].new_zeros(8)
        return torch.cat(parts).contiguous()

    def segment_tables(self, NA):
        """Per global adapter id g: its tier rank, the element offset of its
        lora_B block in lb_packed, and its first shrink column in x_ext (all 0
        when g is not applicable)."""
        rank, boff, zoff = [0] * (NA + 1), [0] * (NA + 1), [0] * (NA + 1)
        b = 0
        seen = [0] * len(SUPPORTED_RANKS)
        for a, r in self.order:
            t = SUPPORTED_RANKS.index(r)
            rank[a + 1] = r
            boff[a + 1] = b
            zoff[a + 1] = int(self.tier_base[t]) + seen[t] * self.S * r
            seen[t] += 1
            b += self.n_total * r
        return rank, boff, zoff


class SwitchedLoRALinear(nn.Module):
    """Fused switched-LoRA linear layer (reference: vllm/core/lora.py:40-130 for the layout)."""

    _lora_ctx = None
    # x . w_ext^T through this library's MFMA GEMM gs_gemm_bf16_tn (True) or
    # torch.mm, i.e. hipBLASLt (False, the default: measured faster at every
    # workload shape)
    native_gemm = False

    def __init__(self, base_layer: nn.Module, num_adapters: int, max_lora_rank: int, num_slices: int = 1,
                 output_slices: tuple | None = None, fuse_swiglu: bool = False, *, tp_size: int = 1,
                 tp_rank: int = 0, parallel: str | None = None, reduce_results: bool = True,
                 all_reduce=None):
        super().__init__()
        self.base_layer = base_layer
        self.num_adapters = num_adapters
        self.max_lora_rank = max_lora_rank
        self.num_slices = num_slices
        self.fuse_swiglu = fuse_swiglu
        if hasattr(base_layer, "weight"):
            out_features, in_features = base_layer.weight.shape
            device, dtype = base_layer.weight.device, base_layer.weight.dtype
        elif hasattr(base_layer, "qweight"):
            # a quantized base layer: sizes from the layer, fp16 adapters, as
            # src/granite_switch/vllm/core/lora.py:157-161; finalize_weights
            # needs the dense weight and says so
            in_features, out_features = base_layer.input_size, base_layer.output_size
            device, dtype = base_layer.qweight.device, torch.float16
        else:
            raise ValueError(f"Unsupported base layer type: {type(base_layer)}")
        self.in_features = in_features
        self.out_features = out_features
        self._device = device
        self._dtype = dtype

        # Tensor parallelism (vllm/core/lora.py:170-195): column-parallel layers
        # shard lora_B along out, row-parallel ones shard lora_A along in and
        # all-reduce the partial output (LoRA delta included) before the bias.
        self.tp_size = tp_size
        self.tp_rank = tp_rank
        self._is_column_parallel = parallel == "column"
        self._is_row_parallel = parallel == "row"
        self._row_parallel_reduce = self._is_row_parallel and tp_size > 1 and reduce_results
        self._all_reduce = all_reduce

        if num_slices > 1:
            if output_slices is None:
                raise ValueError("output_slices required for packed modules")
            if self._is_column_parallel and tp_size > 1:
                self.output_slices = tuple(s // tp_size for s in output_slices)
            else:
                self.output_slices = tuple(output_slices)
        else:
            self.output_slices = (out_features,)

        if num_slices == 1:
            self.lora_A = nn.Parameter(torch.zeros(num_adapters, 1, max_lora_rank, in_features, dtype=dtype, device=device))
            self.lora_B = nn.Parameter(torch.zeros(num_adapters, 1, out_features, max_lora_rank, dtype=dtype, device=device))
            self.lora_A.weight_loader = self._make_weight_loader("a")
            self.lora_B.weight_loader = self._make_weight_loader("b")
        else:
            self.lora_A_slices = nn.ParameterList([
                nn.Parameter(torch.zeros(num_adapters, 1, max_lora_rank, in_features, dtype=dtype, device=device))
                for _ in range(num_slices)])
            self.lora_B_slices = nn.ParameterList([
                nn.Parameter(torch.zeros(num_adapters, 1, o, max_lora_rank, dtype=dtype, device=device))
                for o in self.output_slices])
            for i, p in enumerate(self.lora_A_slices):
                p.weight_loader = self._make_weight_loader("a", i)
            for i, p in enumerate(self.lora_B_slices):
                p.weight_loader = self._make_weight_loader("b", i)
        self._finalized = False
        self._module_idx = 0

    @property
    def weight(self):
        return self.base_layer.weight

    # -- TP slicing of the full checkpoint tensors (vllm/core/lora.py:270-297)
    def slice_lora_a_weight(self, full_weight: torch.Tensor, slice_idx: int = 0) -> torch.Tensor:
        if self.tp_size <= 1 or not self._is_row_parallel:
            return full_weight
        shard = full_weight.shape[-1] // self.tp_size
        return full_weight[..., self.tp_rank * shard:(self.tp_rank + 1) * shard]

    def slice_lora_b_weight(self, full_weight: torch.Tensor, slice_idx: int = 0) -> torch.Tensor:
        if self.tp_size <= 1 or not self._is_column_parallel:
            return full_weight
        shard = full_weight.shape[-2] // self.tp_size
        return full_weight[..., self.tp_rank * shard:(self.tp_rank + 1) * shard, :]

    def _make_weight_loader(self, ab: str, slice_idx: int = 0):
        slicer = self.slice_lora_a_weight if ab == "a" else self.slice_lora_b_weight

        def weight_loader(param: torch.Tensor, loaded_weight: torch.Tensor):
            param.data.copy_(slicer(loaded_weight, slice_idx))

        return weight_loader

    # -- load time -----------------------------------------------------------
    def _checkpoint_slices(self):
        if self.num_slices == 1:
            return [self.lora_A.data], [self.lora_B.data]
        return [p.data for p in self.lora_A_slices], [p.data for p in self.lora_B_slices]

    def finalize_weights(self, adapter_ranks: list, block_n: int | None = None):
        """Checkpoint layout -> the fused layout the expand ops read.

        Produces the tables of src/granite_switch/vllm/core/lora.py:299-538
        (see ``_FusionPlan`` for their definitions): ``remap_table``,
        ``w_ext`` (base rows, then every kernel-local adapter's lora_A rows),
        ``_lb_packed``, ``tile_to_slice``, ``slice_col_r``, ``_na``; plus the
        per-global-adapter tables of the segment expand (rank, lora_B offset,
        first shrink column in x_ext).  One host sync (the applicability scan).
        The checkpoint parameters are emptied afterwards.
        """
        if self._finalized:
            return
        if not hasattr(self.base_layer, "weight"):
            raise NotImplementedError(
                f"{type(self.base_layer).__name__} is quantized (qweight): the fused layout stacks lora_A under a "
                "dense base weight (w_ext = [W; A...]), so dequantize the base layer to bf16 first")
        bn = BLOCK_N if block_n is None else int(block_n)
        if any(w % bn for w in self.output_slices):
            raise AssertionError(f"block_n={bn} must divide the width of every output slice, got {self.output_slices}")
        A_ck, B_ck = self._checkpoint_slices()
        plan = _FusionPlan(A_ck, adapter_ranks, self.output_slices, bn)
        dev = self._device

        self.register_buffer("remap_table", torch.tensor(plan.remap, dtype=torch.long, device=dev), persistent=False)
        W = self.base_layer.weight.data
        self.register_buffer("w_ext", build_w_ext(W, plan.lora_A_by_tier(A_ck)), persistent=False)
        self._N_total = plan.n_total
        self.base_layer.weight.data = self.w_ext[:plan.n_total]          # the base rows are a view of w_ext
        self.register_buffer("_lb_packed", plan.lb_packed(B_ck), persistent=False)
        self.register_buffer("tile_to_slice", torch.tensor(plan.tile_slice, dtype=torch.int32, device=dev),
                             persistent=False)
        self.register_buffer("slice_col_r", torch.tensor(plan.slice_col_r, dtype=torch.int32, device=dev),
                             persistent=False)
        self._na = plan.na
        self._S = self.num_slices
        self._block_n = bn
        self._num_applicable = len(plan.order)
        self._block_cfg_key = (self.in_features, plan.n_total, self._num_applicable)

        seg_rank, seg_boff, seg_zoff = plan.segment_tables(self.num_adapters)
        self.register_buffer("_seg_ranks", torch.tensor(seg_rank, dtype=torch.int32, device=dev), persistent=False)
        self._seg_boff = torch.tensor(seg_boff, dtype=torch.int64, device=dev)
        self._seg_zoff = torch.tensor(seg_zoff, dtype=torch.int32, device=dev)
        self._seg_max_rank = max([16] + seg_rank)
        self._seg_ranks_host = _i32_array(seg_rank)
        self._slice_bounds = _i32_array(plan.bounds)

        if self.fuse_swiglu:
            gate, up = (self.output_slices + (None, None))[:2]
            if self.num_slices != 2 or gate != up:
                raise AssertionError(f"fuse_swiglu needs two equal (gate, up) slices, got {self.output_slices}")
            if getattr(self.base_layer, "bias", None) is not None:
                raise AssertionError("fuse_swiglu: the gate/up projection must have no bias")
            self._H = plan.n_total // 2

        bias = getattr(self.base_layer, "bias", None)
        self._fused_bias = None
        self._output_bias = None
        if bias is not None:
            if getattr(self.base_layer, "skip_bias_add", False):
                self._output_bias = bias          # the caller adds it (vLLM's skip_bias_add contract)
            else:
                self._fused_bias = bias.data

        for p in self._checkpoint_params():
            p.requires_grad_(False)
            p.data = p.data.new_empty(0)
        self._finalized = True

    def _checkpoint_params(self):
        if self.num_slices == 1:
            return [self.lora_A, self.lora_B]
        return [*self.lora_A_slices, *self.lora_B_slices]

    # -- forward -------------------------------------------------------------
    def forward(self, x: torch.Tensor):
        assert self._finalized, "finalize_weights() must be called before forward()"
        x_ext = self._gemm(x)
        if self.fuse_swiglu:
            return self._forward_swiglu(x, x_ext)
        base_out = x_ext[:, :self._N_total]
        ctx = self._lora_ctx
        if ctx is not None and ctx.adapter_indices is not None and self._num_applicable > 0:
            segs = getattr(ctx, "segments", None)
            if (segs is not None and segs.num_tokens == x.shape[0]
                    and segs.num_adapters == self.num_adapters):
                self._run_segment_expand(x_ext, segs)
            else:
                M = x.shape[0]
                self._run_expand(x_ext, ctx.remapped_indices[self._module_idx, :M], ctx)
        if self._row_parallel_reduce:
            base_out = base_out.contiguous()
            if self._all_reduce is not None:
                base_out = self._all_reduce(base_out)
            else:
                torch.distributed.all_reduce(base_out)
        if self._fused_bias is not None:
            base_out = base_out + self._fused_bias
        return base_out, self._output_bias

    def _gemm(self, x: torch.Tensor) -> torch.Tensor:
        """x_ext = x . w_ext^T (src/granite_switch/vllm/core/lora.py:544)."""
        if (self.native_gemm and x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(-1) == 1
                and x.shape[1] % 8 == 0 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0):
            return switched.linear_bf16(x, self.w_ext)
        return torch.mm(x, self.w_ext.T)

    def _forward_swiglu(self, x: torch.Tensor, x_ext: torch.Tensor):
        M = x.shape[0]
        H = self._H
        out = torch.empty(M, H, device=x_ext.device, dtype=x_ext.dtype)
        ctx = self._lora_ctx
        if ctx is not None and ctx.adapter_indices is not None and self._num_applicable > 0:
            adapter_indices = ctx.remapped_indices[self._module_idx, :M]
            bitmask = ctx.per_module_bitmasks[self._module_idx]
        else:
            num_tiles_m = (M + BLOCK_M - 1) // BLOCK_M
            adapter_indices = torch.zeros(M, dtype=torch.long, device=x_ext.device)
            bitmask = torch.zeros(num_tiles_m, dtype=torch.int64, device=x_ext.device)
        ops.op("switch_lora_expand_swiglu")(out, x_ext, adapter_indices, bitmask, self._lb_packed, self.slice_col_r,
                                             *self._na, self._S, self._block_n, H, self._N_total)
        return out, self._output_bias

    def _run_expand(self, x_ext, adapter_indices, ctx):
        """Reference path: the in-place expand op with the tile bitmask (vllm/core/lora.py:659-686)."""
        bitmask = ctx.per_module_bitmasks[self._module_idx]
        ops.op("switch_lora_expand")(x_ext, adapter_indices, bitmask, self._lb_packed, self.tile_to_slice,
                                      self.slice_col_r, *self._na, self._S, self._block_n, self._N_total)

    def _run_segment_expand(self, x_ext, segs):
        """MI355X path: segment expand reading the shrink columns of x_ext by token."""
        M = x_ext.shape[0]
        _lib.call("gs_expand_add", _dtype_code(x_ext), x_ext.data_ptr(), x_ext.stride(0), M, self._N_total,
                  self._slice_bounds, self._S, x_ext.data_ptr(), x_ext.stride(0), 1, self._seg_zoff.data_ptr(),
                  self._lb_packed.data_ptr(), self._seg_boff.data_ptr(), self._seg_ranks.data_ptr(),
                  self.num_adapters, self._seg_max_rank, self._seg_ranks_host, segs.seg_offsets.data_ptr(),
                  segs.perm.data_ptr(),
                  _lib.stream_ptr(x_ext.device))

