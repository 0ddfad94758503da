"""``torch.ops.granite_switch.*`` registrations backed by the HIP library.

The reference registers its Triton launchers as custom ops in a dedicated
``granite_switch`` namespace so torch.compile / graph capture treat them as
opaque (src/granite_switch/vllm/core/lora_ops.py:25-27,192-226;
src/granite_switch/vllm/core/lora_kernel_meta.py:166-182).  This module
registers the same op names with the same argument lists, ``mutates_args`` and
fake implementations, so callers such as ``SwitchedLoRALinear._run_expand``
(src/granite_switch/vllm/core/lora.py:659-686) and ``WCrossShunt.forward``
(src/granite_switch/vllm/decoder/shadow_residual/wcross_shunt.py:198-242) run
unchanged on MI355X, plus three new ops for the y-given switched-LoRA path.

Only one provider of the ``granite_switch`` ops can be loaded in a process.
"""

from __future__ import annotations

import torch

from . import kernels, switched

_NS = "granite_switch"


def _registered(name: str) -> bool:
    try:
        getattr(getattr(torch.ops, _NS), name)
        return True
    except (AttributeError, RuntimeError):
        return False


# ---------------------------------------------------------------------------
# Reference ops (same schemas)
# ---------------------------------------------------------------------------
if not _registered("switch_lora_expand"):

    @torch.library.custom_op(f"{_NS}::switch_lora_expand", mutates_args=("x_ext",))
    def switch_lora_expand(x_ext: torch.Tensor, adapter_indices: torch.Tensor, bitmask: torch.Tensor,
                           lb_packed: torch.Tensor, tile_slice: torch.Tensor, slice_col_r: torch.Tensor, NA_16: int,
                           NA_32: int, NA_64: int, NA_128: int, NA_256: int, NA_512: int, S: int, block_n: int,
                           N: int) -> None:
        kernels.switch_lora_expand(x_ext, adapter_indices, bitmask, lb_packed, tile_slice, slice_col_r,
                                   (NA_16, NA_32, NA_64, NA_128, NA_256, NA_512), S, block_n, N)

    @switch_lora_expand.register_fake
    def _(x_ext, adapter_indices, bitmask, lb_packed, tile_slice, slice_col_r, NA_16, NA_32, NA_64, NA_128, NA_256,
          NA_512, S, block_n, N):
        return None


if not _registered("switch_lora_expand_swiglu"):

    @torch.library.custom_op(f"{_NS}::switch_lora_expand_swiglu", mutates_args=("out",))
    def switch_lora_expand_swiglu(out: torch.Tensor, x_ext: torch.Tensor, adapter_indices: torch.Tensor,
                                  bitmask: torch.Tensor, lb_packed: torch.Tensor, slice_col_r: torch.Tensor,
                                  NA_16: int, NA_32: int, NA_64: int, NA_128: int, NA_256: int, NA_512: int, S: int,
                                  block_n: int, H: int, N: int) -> None:
        kernels.switch_lora_expand_swiglu(out, x_ext, adapter_indices, bitmask, lb_packed, slice_col_r,
                                          (NA_16, NA_32, NA_64, NA_128, NA_256, NA_512), S, block_n, H, N)

    @switch_lora_expand_swiglu.register_fake
    def _(out, x_ext, adapter_indices, bitmask, lb_packed, slice_col_r, NA_16, NA_32, NA_64, NA_128, NA_256, NA_512,
          S, block_n, H, N):
        return None


if not _registered("switch_lora_shrink_expand"):

    @torch.library.custom_op(f"{_NS}::switch_lora_shrink_expand", mutates_args=("out",))
    def switch_lora_shrink_expand(out: torch.Tensor, x_ext: torch.Tensor, adapter_indices: torch.Tensor,
                                  bitmask: torch.Tensor, lb_packed: torch.Tensor, tile_slice: torch.Tensor,
                                  slice_col_r: torch.Tensor, NA_16: int, NA_32: int, NA_64: int, NA_128: int,
                                  NA_256: int, NA_512: int, S: int, block_n: int, N: int) -> None:
        kernels.switch_lora_shrink_expand(out, x_ext, adapter_indices, bitmask, lb_packed, tile_slice, slice_col_r,
                                          (NA_16, NA_32, NA_64, NA_128, NA_256, NA_512), S, block_n, N)

    @switch_lora_shrink_expand.register_fake
    def _(out, x_ext, adapter_indices, bitmask, lb_packed, tile_slice, slice_col_r, NA_16, NA_32, NA_64, NA_128,
          NA_256, NA_512, S, block_n, N):
        return None


if not _registered("compute_per_module_bitmasks"):

    @torch.library.custom_op(f"{_NS}::compute_per_module_bitmasks", mutates_args=())
    def compute_per_module_bitmasks(adapter_indices: torch.Tensor, remap_tables_t: torch.Tensor) -> torch.Tensor:
        return kernels.compute_per_module_bitmasks(adapter_indices, remap_tables_t)

    @compute_per_module_bitmasks.register_fake
    def _(adapter_indices, remap_tables_t):
        M = adapter_indices.shape[0]
        num_modules = remap_tables_t.shape[1]
        bm = kernels.BLOCK_M
        return torch.empty(num_modules, (M + bm - 1) // bm, dtype=torch.int64, device=adapter_indices.device)


# ---------------------------------------------------------------------------
# y-given switched-LoRA ops
# ---------------------------------------------------------------------------
if not _registered("build_segments"):

    @torch.library.custom_op(f"{_NS}::build_segments", mutates_args=())
    def build_segments(adapter_ids: torch.Tensor, num_adapters: int, positions: torch.Tensor | None,
                       cu_seqlens: torch.Tensor | None,
                       act_offsets: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        s = switched.build_segments(adapter_ids, num_adapters, positions, cu_seqlens, act_offsets)
        return s.eff_ids, s.seg_offsets, s.perm

    @build_segments.register_fake
    def _(adapter_ids, num_adapters, positions, cu_seqlens, act_offsets):
        T = adapter_ids.numel()
        dev = adapter_ids.device
        return (torch.empty(T, dtype=torch.int32, device=dev), torch.empty(num_adapters + 1, dtype=torch.int32, device=dev),
                torch.empty(max(T, 1), dtype=torch.int32, device=dev))


def _packed_view(a_pack, b_pack, a_off, b_off, ranks, slice_bounds, hidden, max_rank):
    out_slices = tuple(int(slice_bounds[i + 1] - slice_bounds[i]) for i in range(len(slice_bounds) - 1))
    return switched.PackedAdapters(a_pack=a_pack, b_pack=b_pack, a_off=a_off, b_off=b_off, ranks=ranks,
                                   ranks_host=[], output_slices=out_slices, hidden=int(hidden),
                                   num_adapters=int(ranks.numel() - 1), max_rank=int(max_rank))


def _segs(seg_offsets, perm, T):
    return switched.Segments(eff_ids=perm, seg_offsets=seg_offsets, perm=perm, num_tokens=int(T),
                             num_adapters=int(seg_offsets.numel() - 1))


if not _registered("switched_lora_shrink"):

    @torch.library.custom_op(f"{_NS}::switched_lora_shrink", mutates_args=())
    def switched_lora_shrink(x: torch.Tensor, seg_offsets: torch.Tensor, perm: torch.Tensor, a_pack: torch.Tensor,
                             a_off: torch.Tensor, ranks: torch.Tensor, num_slices: int, max_rank: int) -> torch.Tensor:
        bounds = list(range(num_slices + 1))   # only the slice count matters for the shrink
        pk = _packed_view(a_pack, a_pack, a_off, a_off, ranks, bounds, x.shape[-1], max_rank)
        return switched.shrink(x, _segs(seg_offsets, perm, x.shape[0]), pk)

    @switched_lora_shrink.register_fake
    def _(x, seg_offsets, perm, a_pack, a_off, ranks, num_slices, max_rank):
        return torch.empty(max(x.shape[0], 1), num_slices * max_rank, dtype=x.dtype, device=x.device)


if not _registered("switched_lora_expand_add"):

    @torch.library.custom_op(f"{_NS}::switched_lora_expand_add", mutates_args=("y",))
    def switched_lora_expand_add(y: torch.Tensor, z: torch.Tensor, seg_offsets: torch.Tensor, perm: torch.Tensor,
                                 b_pack: torch.Tensor, b_off: torch.Tensor, ranks: torch.Tensor,
                                 slice_bounds: list[int], max_rank: int) -> None:
        pk = _packed_view(b_pack, b_pack, b_off, b_off, ranks, slice_bounds, 0, max_rank)
        switched.expand_add_(y, z, _segs(seg_offsets, perm, y.shape[0]), pk)

    @switched_lora_expand_add.register_fake
    def _(y, z, seg_offsets, perm, b_pack, b_off, ranks, slice_bounds, max_rank):
        return None


def op(name: str):
    """``torch.ops.granite_switch.<name>``."""
    return getattr(getattr(torch.ops, _NS), name)
