"""Per-forward LoRA metadata: the reference's ``LoRAContext`` / ``FusedLoRAKernelMeta``.

Mirrors src/granite_switch/vllm/core/lora_kernel_meta.py:185-298.  Once per
forward, ``prepare_and_store`` fills the shared context every
``SwitchedLoRALinear`` reads:

  per_module_bitmasks [num_modules, ceil(M/32)] int64  (reference contract)
  remapped_indices    [num_modules, M] int64           (reference contract)
  segments            adapter-sorted segments of the global ids (MI355X path)

The bitmasks and the remapped ids come out of ONE launch
(``gs_compute_bitmasks``), the segments out of one more
(``gs_build_segments``); nothing syncs with the host.
"""

from __future__ import annotations

import torch
from torch import nn

from . import kernels, switched
from . import ops  # noqa: F401  -- registers torch.ops.granite_switch.*

BLOCK_M = kernels.BLOCK_M


class LoRAContext:
    """Shared per-forward LoRA metadata (lora_kernel_meta.py:185-210) plus segments."""

    __slots__ = ("adapter_indices", "num_tokens", "per_module_bitmasks", "remapped_indices", "segments")

    def __init__(self):
        self.adapter_indices: torch.Tensor | None = None
        self.remapped_indices: torch.Tensor | None = None
        self.per_module_bitmasks: torch.Tensor | None = None
        self.segments: switched.Segments | None = None
        self.num_tokens: int = 0

    def reset(self):
        self.adapter_indices = None
        self.remapped_indices = None
        self.per_module_bitmasks = None
        self.segments = None
        self.num_tokens = 0


class FusedLoRAKernelMeta(nn.Module):
    """Computes every module's metadata in a batched launch (lora_kernel_meta.py:213-298)."""

    def __init__(self, device: torch.device):
        super().__init__()
        self.device = device
        self.register_buffer("_remap_tables_t", None, persistent=False)
        self._module_cfg_keys = None

    def register_remap_tables(self, all_remap_tables: torch.Tensor, module_cfg_keys: list) -> None:
        """Register the stacked per-module remap tables [num_modules, NA+1].

        Same contract as lora_kernel_meta.py:235-262, including the assertion
        that no module numbers more than 64 kernel-local adapters (the int64
        tile mask holds 64 bits).
        """
        assert all_remap_tables.max() <= 64, (
            f"int64 bitmask supports at most 64 kernel-local adapters per module, "
            f"got {all_remap_tables.max().item()}")
        self._remap_tables_t = all_remap_tables.T.contiguous()
        self._module_cfg_keys = module_cfg_keys

    def prepare_and_store(self, adapter_indices: torch.Tensor, ctx: LoRAContext, positions=None, cu_seqlens=None,
                          act_offsets=None) -> None:
        """Fill ``ctx`` for one forward (lora_kernel_meta.py:264-298).

        ``adapter_indices`` are the switch's global ids [M] (0 = base).  The
        optional aLoRA arguments gate them first (see
        ``switched.build_segments``); the bitmasks and remapped ids are then
        computed from the gated ids so every path sees the same routing.
        """
        assert self._remap_tables_t is not None, (
            "register_remap_tables() must be called before prepare_and_store(). "
            "Ensure _finalize_fused_lora() has run.")
        M = adapter_indices.shape[0]
        na1, num_modules = self._remap_tables_t.shape
        segs = switched.build_segments(adapter_indices, na1 - 1, positions, cu_seqlens, act_offsets)
        ids = adapter_indices if act_offsets is None else segs.eff_ids
        remapped = torch.empty(num_modules, M, dtype=torch.int64, device=adapter_indices.device)
        bitmasks = kernels.compute_per_module_bitmasks(ids, self._remap_tables_t, BLOCK_M, remapped_out=remapped)
        ctx.per_module_bitmasks = bitmasks
        ctx.remapped_indices = remapped
        ctx.segments = segs
        ctx.adapter_indices = adapter_indices
        ctx.num_tokens = M
