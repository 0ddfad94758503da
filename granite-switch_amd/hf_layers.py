"""HF-form ``SwitchedLoRALinear`` / ``MergedSwitchedLoRALinear`` on MI355X.

Same constructor, parameters (``lora_A``/``lora_B`` or ``lora_A_slices``/
``lora_B_slices``, stacked ``[NA, 1, max_r, in]`` / ``[NA, 1, out, max_r]``,
lora_B pre-scaled), ``weight``/``bias`` properties, context-passing
``_adapter_indices`` and ``forward(x, adapter_indices=None)`` as
src/granite_switch/hf/core/lora.py:23-348.  The per-adapter Python loop with
its host syncs (``torch.any``, ``unique``) is replaced by the three device
steps of ``switched`` (segments, shrink, expand-add), so forward never syncs
once the adapters are packed: ``freeze()`` packs them once; without it the
pack is cached and rebuilt only when a LoRA parameter changes.  The kernels
compute no gradients, so a forward that autograd would track raises.

The layers run the segment kernels (``path = "segments"``), in which no
workgroup waits for another, so a forward either completes correctly or
raises.  Setting a layer's ``path`` to ``"auto"`` lets decode-sized batches
take the one-launch kernel, whose consumers wait for their producers with a
bounded wait; a wait that runs out leaves a wrong output and sets an error
word, which ``check()`` (or ``switched.check()``) turns into an exception.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import switched


class _SwitchedBase(nn.Module):
    def _slices(self):
        raise NotImplementedError

    def freeze(self, adapter_ranks=None) -> None:
        """Pack the current adapter weights once and stop tracking them.

        ``adapter_ranks`` (true rank per adapter) limits the bytes read to the
        true-rank rows; the default reads all max_lora_rank rows (zero rows of
        a smaller adapter contribute nothing, so the result is the same).  The
        LoRA parameters stop requiring grad.  ``unfreeze()`` goes back to
        packing on demand.
        """
        A_sl, B_sl = self._slices()
        for p in (*A_sl, *B_sl):
            p.requires_grad_(False)
        with torch.no_grad():
            self._packed = switched.PackedAdapters.from_slices([a.detach() for a in A_sl], [b.detach() for b in B_sl],
                                                               adapter_ranks)

    def unfreeze(self) -> None:
        self._packed = None
        self._auto_pack = None
        self._auto_key = None

    def _weights_key(self):
        A_sl, B_sl = self._slices()
        return tuple((p.data_ptr(), p._version) for p in (*A_sl, *B_sl))

    def _current_pack(self) -> "switched.PackedAdapters":
        """The frozen pack, else a pack cached until the weights change.

        A change is seen through each parameter's storage address and version
        counter: in-place updates under ``no_grad`` or through ``detach()``,
        optimizer steps and reassignment all move them.  Writes through
        ``.data`` bypass the version counter; call ``unfreeze()`` after those.
        """
        if self._packed is not None:
            return self._packed
        key = self._weights_key()
        if getattr(self, "_auto_pack", None) is None or self._auto_key != key:
            A_sl, B_sl = self._slices()
            with torch.no_grad():
                self._auto_pack = switched.PackedAdapters.from_slices([a.detach() for a in A_sl],
                                                                      [b.detach() for b in B_sl])
            self._auto_key = key
        return self._auto_pack

    def _apply_lora(self, output: torch.Tensor, x: torch.Tensor, adapter_indices: torch.Tensor) -> torch.Tensor:
        if torch.is_grad_enabled():
            A_sl, B_sl = self._slices()
            if x.requires_grad or any(p.requires_grad for p in (*A_sl, *B_sl)):
                raise RuntimeError(
                    "the MI355X switched-LoRA kernels compute no gradients: run the forward under torch.no_grad() / "
                    "torch.inference_mode(), or freeze() the layer and pass inputs that do not require grad")
        packed = self._current_pack()
        x_flat = x.reshape(-1, self.in_features)
        out_flat = output.view(-1, output.shape[-1])
        ids = adapter_indices.reshape(-1)
        if ids.numel() != x_flat.shape[0]:
            raise ValueError("adapter_indices must have one entry per token")
        segs = switched.build_segments(ids, self.num_adapters)
        switched.switched_lora_(out_flat, x_flat.to(packed.dtype), segs, packed, path=self.path)
        return output

    # "segments": no workgroup waits for another (a forward is correct or
    # raises); "auto": decode-sized batches take the one-launch kernel -- call
    # check() at a point that synchronises anyway
    path = "segments"

    def check(self) -> None:
        """Raise ``switched.SmallPathError`` if a one-launch call on this layer's
        device has reported a failed hand-off (its output was wrong) since the
        last ``switched.small_reset``; synchronises.  Only ``path = "auto"``
        can take that kernel."""
        switched.check(self.base_layer.weight.device)

    @property
    def weight(self):
        return self.base_layer.weight

    @property
    def bias(self):
        return self.base_layer.bias


class SwitchedLoRALinear(_SwitchedBase):
    """Single-slice switched-LoRA linear (hf/core/lora.py:23-169)."""

    def __init__(self, in_features: int, out_features: int, num_adapters: int, max_lora_rank: int, bias: bool = True):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.num_adapters = num_adapters
        self.max_lora_rank = max_lora_rank
        self.base_layer = nn.Linear(in_features, out_features, bias=bias)
        self.lora_A = nn.Parameter(torch.zeros(num_adapters, 1, max_lora_rank, in_features))
        self.lora_B = nn.Parameter(torch.zeros(num_adapters, 1, out_features, max_lora_rank))
        nn.init.kaiming_uniform_(self.lora_A, a=5 ** 0.5)
        nn.init.zeros_(self.lora_B)
        self._adapter_indices: torch.Tensor | None = None
        self._packed = None
        self._auto_pack = None
        self._auto_key = None

    def _slices(self):
        return [self.lora_A], [self.lora_B]

    def forward(self, x: torch.Tensor, adapter_indices: torch.Tensor | None = None) -> torch.Tensor:
        if adapter_indices is None:
            adapter_indices = self._adapter_indices
        output = self.base_layer(x)
        if adapter_indices is None:
            return output
        return self._apply_lora(output, x, adapter_indices)


class MergedSwitchedLoRALinear(_SwitchedBase):
    """Fused multi-slice projection (QKV, gate/up) with per-slice adapters (hf/core/lora.py:172-348)."""

    def __init__(self, in_features: int, output_slices: tuple, num_adapters: int, max_lora_rank: int,
                 bias: bool = False):
        super().__init__()
        self.in_features = in_features
        self.output_slices = tuple(output_slices)
        self.num_slices = len(output_slices)
        self.num_adapters = num_adapters
        self.max_lora_rank = max_lora_rank
        self.base_layer = nn.Linear(in_features, sum(output_slices), bias=bias)
        self.lora_A_slices = nn.ParameterList(
            [nn.Parameter(torch.zeros(num_adapters, 1, max_lora_rank, in_features)) for _ in range(self.num_slices)])
        self.lora_B_slices = nn.ParameterList(
            [nn.Parameter(torch.zeros(num_adapters, 1, o, max_lora_rank)) for o in output_slices])
        for A in self.lora_A_slices:
            nn.init.kaiming_uniform_(A, a=5 ** 0.5)
        for B in self.lora_B_slices:
            nn.init.zeros_(B)
        self._adapter_indices: torch.Tensor | None = None
        self._packed = None
        self._auto_pack = None
        self._auto_key = None

    def _slices(self):
        return list(self.lora_A_slices), list(self.lora_B_slices)

    def forward(self, x: torch.Tensor, adapter_indices: torch.Tensor | None = None) -> torch.Tensor:
        if adapter_indices is None:
            adapter_indices = self._adapter_indices
        output = self.base_layer(x)
        if adapter_indices is None:
            return output
        return self._apply_lora(output, x, adapter_indices)
