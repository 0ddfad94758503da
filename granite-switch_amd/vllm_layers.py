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
from collections import OrderedDict

import torch
from torch import nn

from . import _lib, ops
from .kernels import BLOCK_M, BLOCK_N, SUPPORTED_RANKS, build_w_ext, promote_rank
from . import switched
from .switched import _dtype_code, _i32_array

logger = logging.getLogger(__name__)


class SwitchedLoRALinear(nn.Module):
    """Fused switched-LoRA linear layer (reference: vllm/core/lora.py:40-130 for the layout)."""

    _lora_ctx = None
    # x . w_ext^T through gs_gemm_bf16_tn (True) or torch.mm (False); the
    # library GEMM is faster at every measured workload shape
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
        if not hasattr(base_layer, "weight"):
            raise ValueError(f"Unsupported base layer type: {type(base_layer)}")
        out_features, in_features = base_layer.weight.shape
        device, dtype = base_layer.weight.device, base_layer.weight.dtype
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
    def finalize_weights(self, adapter_ranks: list, block_n: int | None = None):
        """Checkpoint layout -> fused layout (vllm/core/lora.py:299-538).

        Applicability scan (one host sync), rank promotion with zero padding,
        stable ascending-rank order -> ``remap_table``, ``w_ext``, packed lora_B,
        ``tile_to_slice``, ``slice_col_r``; plus the per-global-adapter tables
        the segment expand reads (rank, lora_B offset, shrink column in x_ext).
        """
        if self._finalized:
            return
        if block_n is None:
            block_n = BLOCK_N
        device, dtype = self._device, self._dtype
        NA, S = self.num_adapters, self.num_slices
        if S == 1:
            lora_A_all = [self.lora_A.data]
            lora_B_all = [self.lora_B.data]
        else:
            lora_A_all = [p.data for p in self.lora_A_slices]
            lora_B_all = [p.data for p in self.lora_B_slices]
        max_rank = lora_A_all[0].shape[2]
        ranks_t = torch.tensor(adapter_ranks, device=device)
        rank_mask = torch.arange(max_rank, device=device)[None, :] < ranks_t[:, None]
        applicable_t = torch.zeros(NA, dtype=torch.bool, device=device)
        for s in range(S):
            nz = lora_A_all[s][:, 0, :, :].ne(0).any(dim=-1)
            applicable_t |= (nz & rank_mask).any(dim=1)
        applicable = applicable_t.tolist()
        applicable_adapters = [i for i in range(NA) if applicable[i]]

        eff_ranks = [promote_rank(int(r)) for r in adapter_ranks]
        pad_to = max((eff_ranks[i] for i in applicable_adapters), default=0)
        if pad_to > max_rank:
            pad = pad_to - max_rank
            lora_A_all = [torch.nn.functional.pad(a, (0, 0, 0, pad)) for a in lora_A_all]
            lora_B_all = [torch.nn.functional.pad(b, (0, pad)) for b in lora_B_all]
        adapter_ranks = eff_ranks

        rank_order = sorted(applicable_adapters, key=lambda i: adapter_ranks[i])
        remap = torch.zeros(NA + 1, dtype=torch.long, device=device)
        for k, orig in enumerate(rank_order):
            remap[orig + 1] = k + 1
        self.register_buffer("remap_table", remap, persistent=False)

        tiers = OrderedDict()
        for orig in rank_order:
            tiers.setdefault(adapter_ranks[orig], []).append(orig)

        lora_A_by_rank = {}
        for rank, idxs in tiers.items():
            lora_A_by_rank[rank] = torch.stack(
                [torch.stack([lora_A_all[s][oi, 0, :rank, :] for s in range(S)], dim=0) for oi in idxs], dim=0)
        W_base = self.base_layer.weight.data
        w_ext = build_w_ext(W_base, lora_A_by_rank)
        self.register_buffer("w_ext", w_ext, persistent=False)
        N_total = W_base.shape[0]
        self._N_total = N_total
        self.base_layer.weight.data = self.w_ext[:N_total]
        del W_base

        tier_info, lora_B_merged = {}, {}
        for rank, idxs in tiers.items():
            lora_B_merged[rank] = torch.stack(
                [torch.cat([lora_B_all[s][oi, 0, :, :rank] for s in range(S)], dim=0) for oi in idxs], dim=0)
            tier_info[rank] = len(idxs)
        self._num_applicable = sum(tier_info.values())
        self._block_cfg_key = (self.in_features, N_total, self._num_applicable)

        self._block_n = block_n
        assert all(n_s % block_n == 0 for n_s in self.output_slices), (
            f"block_n={block_n} must divide every output slice: {self.output_slices}")
        num_tiles_n = (N_total + block_n - 1) // block_n
        cum = [0]
        for n_s in self.output_slices:
            cum.append(cum[-1] + n_s)
        tile_slice = torch.zeros(num_tiles_n, dtype=torch.int32)
        for t in range(num_tiles_n):
            c = t * block_n
            for s in range(S):
                if cum[s] <= c < cum[s + 1]:
                    tile_slice[t] = s
                    break
        self.register_buffer("tile_to_slice", tile_slice.to(device), persistent=False)

        tier_col_bases, off = [], N_total
        for r in SUPPORTED_RANKS:
            tier_col_bases.append(off)
            off += tier_info.get(r, 0) * S * r
        self.register_buffer("slice_col_r", torch.tensor(
            [[tier_col_bases[t] + s * SUPPORTED_RANKS[t] for t in range(6)] for s in range(S)],
            dtype=torch.int32, device=device), persistent=False)

        self._na = tuple(tier_info.get(r, 0) for r in SUPPORTED_RANKS)
        self._S = S
        parts = [lora_B_merged[r].reshape(-1) for r in SUPPORTED_RANKS if r in lora_B_merged]
        lb = torch.cat(parts) if parts else torch.zeros(8, device=device, dtype=dtype)
        self.register_buffer("_lb_packed", lb.contiguous(), persistent=False)

        # per-GLOBAL-adapter tables for the segment expand (0 = not applicable)
        g_rank = [0] * (NA + 1)
        g_boff = [0] * (NA + 1)
        g_zoff = [0] * (NA + 1)
        lb_off = 0
        for t, r in enumerate(SUPPORTED_RANKS):
            for idx, orig in enumerate(tiers.get(r, [])):
                g = orig + 1
                g_rank[g] = r
                g_boff[g] = lb_off + idx * N_total * r
                g_zoff[g] = tier_col_bases[t] + idx * S * r
            lb_off += tier_info.get(r, 0) * N_total * r
        self.register_buffer("_seg_ranks", torch.tensor(g_rank, dtype=torch.int32, device=device), persistent=False)
        self._seg_boff = torch.tensor(g_boff, dtype=torch.int64, device=device)
        self._seg_zoff = torch.tensor(g_zoff, dtype=torch.int32, device=device)
        self._seg_max_rank = max([16] + g_rank)
        self._slice_bounds = _i32_array(cum)

        if self.fuse_swiglu:
            assert S == 2 and self.output_slices[0] == self.output_slices[1], (
                "fuse_swiglu requires the merged 2-slice (gate, up) layout with "
                f"equal widths; got S={S}, output_slices={self.output_slices}")
            assert getattr(self.base_layer, "bias", None) is None, (
                "fuse_swiglu does not support a biased gate/up projection")
            self._H = N_total // 2

        self._fused_bias = None
        self._output_bias = None
        if getattr(self.base_layer, "bias", None) is not None:
            if not getattr(self.base_layer, "skip_bias_add", False):
                self._fused_bias = self.base_layer.bias.data
            else:
                self._output_bias = self.base_layer.bias

        ckpt = [self.lora_A, self.lora_B] if S == 1 else [*self.lora_A_slices, *self.lora_B_slices]
        for p in ckpt:
            p.requires_grad_(False)
            p.data = p.data.new_empty(0)
        self._finalized = True

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
                  self.num_adapters, self._seg_max_rank, segs.seg_offsets.data_ptr(), segs.perm.data_ptr(),
                  _lib.stream_ptr(x_ext.device))

