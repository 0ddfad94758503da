"""Drop-in for ``granite_switch.probe_routing`` (src/granite_switch/probe_routing.py).

An adapter slot is either a generation adapter or an activation-probe head,
both selected by the same control token.  The switch's one per-token index
stream is split so that probe positions leave the LoRA path (their LoRA id is
0) and feed the probe stream instead.  The split runs on the GPU
(``gs_split_adapter_indices``), on torch's current stream, without a host
sync, so it can sit inside a captured forward before the LoRA metadata is
built (src/granite_switch/vllm/granite_switch_model.py:396).
"""

from __future__ import annotations

import torch

from . import _lib


def build_adapter_kind_lut(config) -> torch.Tensor | None:
    """Bool table over adapter indices marking the probe slots.

    Same contract as src/granite_switch/probe_routing.py:17-33:
    ``[num_adapters + 1]``, entry ``i`` True when adapter index ``i`` (slot
    ``i - 1``) is a probe, entry 0 (base) False; None when no slot is a probe.
    ``config`` is an object with ``adapter_kinds`` (a list of "lora" / "probe"
    per slot), or that list itself.
    """
    kinds = config if isinstance(config, (list, tuple)) or config is None else getattr(config, "adapter_kinds", None)
    if kinds is None or "probe" not in kinds:
        return None
    flags = [False] + [kind == "probe" for kind in kinds]
    return torch.tensor(flags, dtype=torch.bool)


def split_adapter_indices(kind_lut: torch.Tensor | None,
                          adapter_indices: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(LoRA stream, probe stream) of a per-token index stream.

    Same contract as src/granite_switch/probe_routing.py:36-58: shapes are
    preserved; the LoRA stream has probe positions zeroed, the probe stream
    holds the index at probe positions and 0 elsewhere; with ``kind_lut``
    None the LoRA stream IS ``adapter_indices`` and the probe stream is zeros.
    Indices must be int32 or int64 on the GPU; ``kind_lut`` is moved to their
    device if it is not there (keep it there, e.g. as a module buffer, to stay
    capture-safe).  An index outside the table (negative, or past the last
    slot) is neither a probe nor an adapter: both streams hold 0 there, so the
    token takes the base model.  (The reference indexes the table directly: a
    negative index wraps and one past the end raises.)
    """
    if kind_lut is None:
        return adapter_indices, torch.zeros_like(adapter_indices)
    if not adapter_indices.is_cuda:
        raise ValueError("split_adapter_indices: adapter_indices must live on the GPU")
    if adapter_indices.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"split_adapter_indices: int32 or int64 indices expected, got {adapter_indices.dtype}")
    if kind_lut.dtype != torch.bool or kind_lut.dim() != 1 or not 1 <= kind_lut.numel() <= _lib.GS_MAX_ADAPTERS + 1:
        raise ValueError("split_adapter_indices: kind_lut must be a 1-D bool table of 1..257 entries")
    lut = kind_lut.to(adapter_indices.device).contiguous()
    ids = adapter_indices.contiguous()
    lora = torch.empty_like(ids)
    probe = torch.empty_like(ids)
    _lib.call("gs_split_adapter_indices", lut.data_ptr(), lut.numel(), ids.data_ptr(), ids.element_size(),
              ids.numel(), lora.data_ptr(), probe.data_ptr(), _lib.stream_ptr(ids.device))
    return lora, probe


__all__ = ["build_adapter_kind_lut", "split_adapter_indices"]
