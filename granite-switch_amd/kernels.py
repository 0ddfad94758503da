"""Drop-in for ``granite_switch.kernels`` (src/granite_switch/kernels/__init__.py:4-30).

Same names, constants and launcher signatures as the reference's
backend-agnostic kernel module; the launchers call the gfx950 HIP library
instead of Triton.  Launches go on torch's current stream; no host sync.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

# src/granite_switch/kernels/switch_lora_kernel.py:79
SUPPORTED_RANKS = (16, 32, 64, 128, 256, 512)

# Tiling constants of the reference (switch_lora_kernel.py:107-110).  BLOCK_M is
# the token tile of the per-module bitmask and of the expand op's row tiles;
# BLOCK_N the default output tile that ``block_n`` must divide every slice by.
# NUM_WARPS / NUM_STAGES are Triton launch knobs with no meaning for the HIP
# kernels (which always use 256-thread workgroups = 4 wave64s); they are kept
# so callers that read them keep working.
BLOCK_M: int = 32
BLOCK_N: int = 32
NUM_WARPS: int = 4
NUM_STAGES: int = 1


def promote_rank(rank: int) -> int:
    """Round a LoRA rank up to the next supported tier.

    Same contract as src/granite_switch/kernels/switch_lora_kernel.py:82-101:
    rank <= 0 is returned unchanged; ranks above 512 raise ValueError.
    """
    if rank <= 0:
        return rank
    for supported in SUPPORTED_RANKS:
        if supported >= rank:
            return supported
    raise ValueError(f"LoRA rank {rank} exceeds the largest supported rank {SUPPORTED_RANKS[-1]}.")


def get_switch_lora_expand_config() -> dict:
    """Tiling parameters (switch_lora_kernel.py:113-126 contract: a dict)."""
    return {"block_m": BLOCK_M, "block_n": BLOCK_N, "num_warps": NUM_WARPS, "num_stages": NUM_STAGES}


def build_w_ext(W: torch.Tensor, lora_A_by_rank: dict) -> torch.Tensor:
    """``cat([W] + [A_r.reshape(n_r*S*r, K) for r in tiers])`` (switch_lora_kernel.py:134-163).

    Rows are appended in tier -> adapter -> slice -> rank order; only ranks in
    SUPPORTED_RANKS are read.  A load-time concatenation, done with torch.
    """
    parts = [W]
    for r in SUPPORTED_RANKS:
        lA = lora_A_by_rank.get(r)
        if lA is not None and lA.shape[0] > 0:
            n_r, S = lA.shape[0], lA.shape[1]
            parts.append(lA.reshape(n_r * S * r, lA.shape[3]))
    return torch.cat(parts, dim=0)


def _idx_bytes(t: torch.Tensor) -> int:
    if t.dtype == torch.int64:
        return 8
    if t.dtype == torch.int32:
        return 4
    raise TypeError(f"adapter_indices must be int32 or int64, got {t.dtype}")


def _na_array(na) -> ctypes.Array:
    if len(na) != 6:
        raise ValueError("na must be the 6-tuple (NA_16, NA_32, NA_64, NA_128, NA_256, NA_512)")
    return (ctypes.c_int32 * 6)(*[int(v) for v in na])


def _check_tables(who, x_ext, lb_packed, slice_col_r, na, S, N) -> None:
    """Shape checks the kernels rely on (host metadata only, no device sync).

    x_ext must hold the base columns plus every tier's shrink columns, and
    lb_packed every tier's [NA_r, N, r] block, in the layout finalize_weights
    produces (src/granite_switch/vllm/core/lora.py:435-492).
    """
    if len(na) != 6:
        raise ValueError(f"{who}: na must have 6 tier counts")
    shrink_cols = sum(int(n) * int(S) * r for n, r in zip(na, SUPPORTED_RANKS))
    if x_ext.dim() != 2 or x_ext.shape[1] < int(N) + shrink_cols:
        raise ValueError(f"{who}: x_ext has {x_ext.shape[-1]} columns, needs N + shrink columns = "
                         f"{int(N) + shrink_cols}")
    lb_need = sum(int(n) * int(N) * r for n, r in zip(na, SUPPORTED_RANKS))
    if lb_packed.numel() < lb_need:
        raise ValueError(f"{who}: lb_packed holds {lb_packed.numel()} elements, needs {lb_need}")
    if slice_col_r.numel() < int(S) * 6:
        raise ValueError(f"{who}: slice_col_r must be [S, 6]")


def switch_lora_expand(x_ext: torch.Tensor, adapter_indices: torch.Tensor, bitmask: torch.Tensor,
                       lb_packed: torch.Tensor, tile_slice: torch.Tensor, slice_col_r: torch.Tensor, na: tuple,
                       S: int, block_n: int, N: int) -> None:
    """Accumulate the LoRA expand delta in place into ``x_ext[:, :N]``.

    Signature and semantics of src/granite_switch/kernels/switch_lora_kernel.py:
    414-458 (kernel :171-411): 32-row tiles with a zero bitmask are skipped;
    rows with kernel-local id 0 are never written; each present adapter's
    delta ``shrink[:, :r] . lb^T`` is accumulated in fp32 and added with one
    bf16 rounding.  ``adapter_indices`` may be int32 or int64.
    """
    if x_ext.dtype != torch.bfloat16 or lb_packed.dtype != torch.bfloat16:
        raise TypeError("switch_lora_expand: x_ext and lb_packed must be bfloat16")
    if tile_slice.dtype != torch.int32 or slice_col_r.dtype != torch.int32 or bitmask.dtype != torch.int64:
        raise TypeError("switch_lora_expand: tile_slice/slice_col_r int32, bitmask int64 expected")
    M = x_ext.shape[0]
    if adapter_indices.numel() < M or bitmask.numel() < (M + BLOCK_M - 1) // BLOCK_M:
        raise ValueError("switch_lora_expand: adapter_indices / bitmask shorter than x_ext's rows")
    _check_tables("switch_lora_expand", x_ext, lb_packed, slice_col_r, na, S, N)
    if tile_slice.numel() < (int(N) + int(block_n) - 1) // int(block_n):
        raise ValueError("switch_lora_expand: tile_slice has fewer than ceil(N / block_n) entries")
    ids = adapter_indices if adapter_indices.stride(-1) == 1 else adapter_indices.contiguous()
    _lib.call("gs_switch_lora_expand", x_ext.data_ptr(), x_ext.stride(0), x_ext.stride(1), M, ids.data_ptr(),
              _idx_bytes(ids), bitmask.data_ptr(), bitmask.stride(0), lb_packed.data_ptr(),
              tile_slice.data_ptr(), slice_col_r.data_ptr(), _na_array(na), int(S), int(block_n), int(N),
              _lib.stream_ptr(x_ext.device))


def switch_lora_expand_swiglu(out: torch.Tensor, x_ext: torch.Tensor, adapter_indices: torch.Tensor,
                              bitmask: torch.Tensor, lb_packed: torch.Tensor, slice_col_r: torch.Tensor, na: tuple,
                              S: int, block_n: int, H: int, N: int) -> None:
    """``out[M, H] = silu(gate + dgate) * (up + dup)`` (switch_lora_kernel.py:809-857).

    gate/up are x_ext columns [0,H) / [H,2H) plus their LoRA delta (computed
    only for tiles with a nonzero bitmask); ``out`` is always written.
    """
    if x_ext.dtype != torch.bfloat16 or out.dtype != torch.bfloat16:
        raise TypeError("switch_lora_expand_swiglu: bfloat16 x_ext and out expected")
    M = x_ext.shape[0]
    if out.shape[0] < M or out.shape[1] < H:
        raise ValueError("switch_lora_expand_swiglu: out is smaller than [M, H]")
    if adapter_indices.numel() < M or bitmask.numel() < (M + BLOCK_M - 1) // BLOCK_M:
        raise ValueError("switch_lora_expand_swiglu: adapter_indices / bitmask shorter than x_ext's rows")
    _check_tables("switch_lora_expand_swiglu", x_ext, lb_packed, slice_col_r, na, S, N)
    ids = adapter_indices if adapter_indices.stride(-1) == 1 else adapter_indices.contiguous()
    _lib.call("gs_switch_lora_expand_swiglu", out.data_ptr(), out.stride(0), out.stride(1), x_ext.data_ptr(),
              x_ext.stride(0), x_ext.stride(1), M, ids.data_ptr(), _idx_bytes(ids), bitmask.data_ptr(),
              bitmask.stride(0), lb_packed.data_ptr(), slice_col_r.data_ptr(), _na_array(na), int(S),
              int(block_n), int(H), int(N), _lib.stream_ptr(x_ext.device))


def compute_per_module_bitmasks(adapter_indices: torch.Tensor, remap_tables_t: torch.Tensor,
                                block_m: int | None = None, remapped_out: torch.Tensor | None = None) -> torch.Tensor:
    """Per-module tile bitmasks [num_modules, ceil(M/block_m)] int64.

    Semantics of src/granite_switch/vllm/core/lora_kernel_meta.py:30-91 and the
    spec :104-151.  ``remapped_out`` ([num_modules, M] int64), when given, also
    receives ``remap_t[clamp(ids)].T`` (lora_kernel_meta.py:294) in the same
    launch.
    """
    bm = BLOCK_M if block_m is None else int(block_m)
    if remap_tables_t.dtype != torch.int64:
        raise TypeError("remap_tables_t must be int64")
    M = adapter_indices.shape[0]
    na1, num_modules = remap_tables_t.shape
    ids = adapter_indices if adapter_indices.stride(-1) == 1 else adapter_indices.contiguous()
    rt = remap_tables_t.contiguous()
    out = torch.empty(num_modules, (M + bm - 1) // bm, dtype=torch.int64, device=adapter_indices.device)
    if remapped_out is not None and (remapped_out.shape != (num_modules, M) or not remapped_out.is_contiguous()):
        raise ValueError("remapped_out must be a contiguous [num_modules, M] int64 tensor")
    _lib.call("gs_compute_bitmasks", ids.data_ptr(), _idx_bytes(ids), M, rt.data_ptr(), na1, num_modules, bm,
              out.data_ptr(), _lib.ptr(remapped_out), _lib.stream_ptr(adapter_indices.device))
    return out


def switch_lora_shrink_expand(out: torch.Tensor, x_ext: torch.Tensor, adapter_indices: torch.Tensor,
                              bitmask: torch.Tensor, lb_packed: torch.Tensor, tile_slice: torch.Tensor,
                              slice_col_r: torch.Tensor, na: tuple, S: int, block_n: int, N: int) -> None:
    """W-less expand of the Shadow-Residual cross-stream shunt into ``out[M, N]``.

    Signature and semantics of src/granite_switch/kernels/switch_lora_kernel.py:
    1094-1146 (kernel :883-1091): ``x_ext`` holds only shrink columns (the
    cross weight has no base rows, so ``slice_col_r`` bases start at 0); a row
    of an adapter gets ``shrink[:, :r] . lb^T`` in ``out``'s dtype, a base row
    and every row of a skipped tile read back exactly zero.  The kernel writes
    all of ``out[:M, :N]``; a larger ``out`` is zeroed first, as the
    reference's launcher zeroes all of it.
    """
    if x_ext.dtype != torch.bfloat16 or lb_packed.dtype != torch.bfloat16:
        raise TypeError("switch_lora_shrink_expand: x_ext and lb_packed must be bfloat16")
    if out.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"switch_lora_shrink_expand: out must be bfloat16 or float32, got {out.dtype}")
    if tile_slice.dtype != torch.int32 or slice_col_r.dtype != torch.int32 or bitmask.dtype != torch.int64:
        raise TypeError("switch_lora_shrink_expand: tile_slice/slice_col_r int32, bitmask int64 expected")
    M = x_ext.shape[0]
    if out.dim() != 2 or out.shape[0] < M or out.shape[1] < int(N):
        raise ValueError(f"switch_lora_shrink_expand: out {tuple(out.shape)} is smaller than [M, N] = [{M}, {N}]")
    if adapter_indices.numel() < M or bitmask.numel() < (M + BLOCK_M - 1) // BLOCK_M:
        raise ValueError("switch_lora_shrink_expand: adapter_indices / bitmask shorter than x_ext's rows")
    if len(na) != 6:
        raise ValueError("switch_lora_shrink_expand: na must have 6 tier counts")
    shrink_cols = sum(int(n) * int(S) * r for n, r in zip(na, SUPPORTED_RANKS))
    if x_ext.dim() != 2 or x_ext.shape[1] < shrink_cols:
        raise ValueError(f"switch_lora_shrink_expand: x_ext has {x_ext.shape[-1]} columns, the tiers need "
                         f"{shrink_cols}")
    lb_need = sum(int(n) * int(N) * r for n, r in zip(na, SUPPORTED_RANKS))
    if lb_packed.numel() < lb_need:
        raise ValueError(f"switch_lora_shrink_expand: lb_packed holds {lb_packed.numel()} elements, needs {lb_need}")
    if slice_col_r.numel() < int(S) * 6:
        raise ValueError("switch_lora_shrink_expand: slice_col_r must be [S, 6]")
    if tile_slice.numel() < (int(N) + int(block_n) - 1) // int(block_n):
        raise ValueError("switch_lora_shrink_expand: tile_slice has fewer than ceil(N / block_n) entries")
    if tuple(out.shape) != (M, int(N)):
        out.zero_()
    ids = adapter_indices if adapter_indices.stride(-1) == 1 else adapter_indices.contiguous()
    code = _lib.GS_DTYPE_BF16 if out.dtype == torch.bfloat16 else _lib.GS_DTYPE_FP32
    _lib.call("gs_switch_lora_shrink_expand", out.data_ptr(), code, out.stride(0), out.stride(1), x_ext.data_ptr(),
              x_ext.stride(0), x_ext.stride(1), M, ids.data_ptr(), _idx_bytes(ids), bitmask.data_ptr(),
              bitmask.stride(0), lb_packed.data_ptr(), tile_slice.data_ptr(), slice_col_r.data_ptr(),
              _na_array(na), int(S), int(block_n), int(N), _lib.stream_ptr(x_ext.device))


__all__ = [
    "BLOCK_M",
    "BLOCK_N",
    "NUM_STAGES",
    "NUM_WARPS",
    "SUPPORTED_RANKS",
    "build_w_ext",
    "get_switch_lora_expand_config",
    "promote_rank",
    "switch_lora_expand",
    "switch_lora_expand_swiglu",
    "switch_lora_shrink_expand",
    "compute_per_module_bitmasks",
]
