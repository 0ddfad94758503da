"""granite_switch_amd -- Granite Switch's per-token switched-LoRA path on MI355X.

Hand-written gfx950 HIP kernels behind a C ABI (include/granite_switch_amd.h),
driven from Python on PyTorch-ROCm:

  switched     y-given switched LoRA: segments, shrink, expand-add
  kernels      drop-in for ``granite_switch.kernels`` (reference launchers)
  ops          ``torch.ops.granite_switch.*`` registrations (reference schemas)
  meta         ``LoRAContext`` / ``FusedLoRAKernelMeta``
  vllm_layers  vLLM-form ``SwitchedLoRALinear`` (fused w_ext GEMM + expand)
  hf_layers    HF-form ``SwitchedLoRALinear`` / ``MergedSwitchedLoRALinear``
  probe_routing  drop-in for ``granite_switch.probe_routing`` (probe-slot split)
  workloads    seeded synthetic benchmark shapes

The directory name carries a dash, so the package is imported under the name
``granite_switch_amd`` with ``__graft_entry__.load_package()`` (or any loader
that maps that name to this directory).
"""

from . import _lib
from ._lib import GraniteSwitchError

__all__ = ["GraniteSwitchError", "library_path", "load_library"]


def library_path() -> str:
    return _lib.LIB_PATH


def load_library():
    """Load the HIP library (raises ImportError when it has not been built)."""
    return _lib.load()
