"""Floating-point side of the switched-LoRA path (numpy, float64 arithmetic).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

bf16 data is carried as float32 arrays holding exactly-representable bf16
values; ``bf16_round`` rounds float arrays to the nearest bf16 (ties to even),
which is what torch's ``.to(torch.bfloat16)`` and a ``v_cvt`` to bf16 do.
"""

from __future__ import annotations

import numpy as np

from .mapping import SUPPORTED_RANKS


def bf16_round(a) -> np.ndarray:
    """Round to the nearest bf16 value (ties to even); returns float32."""
    f = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = rounded.astype(np.uint32).view(np.float32).copy()
    out[nan] = np.nan
    return out


def round_to(a, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_round(a)
    if dtype == "fp32":
        return np.asarray(a, dtype=np.float32)
    if dtype == "f64":
        return np.asarray(a, dtype=np.float64)
    raise ValueError(dtype)


def switched_lora_apply(y, x, ids, lora_A_slices, lora_B_slices, output_slices,
                        ranks=None, dtype: str = "bf16", mode: str = "exact"):
    """``y[t] += sum_s (x[t] . A_{a,s}^T) . B_{a,s}^T`` for tokens with id a > 0.

    Restates src/granite_switch/hf/core/lora.py:127-161 (single slice) and
    :280-298 / :308-348 (per-slice loop of ``MergedSwitchedLoRALinear``): base
    rows (id 0) are never written; for each active adapter ``a`` (ascending, as
    ``unique`` returns them) its rows are gathered, shrunk with
    ``lora_A[a-1, 0]`` and expanded with the pre-scaled ``lora_B[a-1, 0]``
    (src/granite_switch/composer/weight_transfer.py:564-568 folds alpha/r into
    B), then added in place.

    lora_A_slices[s]: [NA, 1, max_r, H]; lora_B_slices[s]: [NA, 1, O_s, max_r]
    ranks: optional per-adapter true rank; rows/cols past it are zero in the
           stored layout, so truncating to it is exact (vllm/core/lora.py:368-379)
    mode:
      "exact" -- float64 math, one rounding of ``y + delta`` to ``dtype``
      "hf"    -- the HF loop's rounding sequence: shrink rounded to ``dtype``,
                 expand rounded to ``dtype``, then ``y + d`` rounded
    Returns a float64 array [T, O] (values representable in ``dtype``).
    """
    y = np.asarray(y, dtype=np.float64)
    x = np.asarray(x, dtype=np.float64)
    ids = np.asarray(ids, dtype=np.int64)
    out = y.copy()
    NA = np.asarray(lora_A_slices[0]).shape[0]
    offs = np.cumsum([0] + list(output_slices))
    active = np.unique(ids[(ids > 0) & (ids <= NA)])
    for a in active:
        idx = np.nonzero(ids == a)[0]
        xa = x[idx]
        for s in range(len(output_slices)):
            A = np.asarray(lora_A_slices[s][a - 1, 0], dtype=np.float64)
            B = np.asarray(lora_B_slices[s][a - 1, 0], dtype=np.float64)
            if ranks is not None:
                r = int(ranks[a - 1])
                A = A[:r]
                B = B[:, :r]
            z = xa @ A.T
            if mode == "hf":
                z = round_to(z, dtype).astype(np.float64)
                d = round_to(z @ B.T, dtype).astype(np.float64)
                out[idx, offs[s]:offs[s + 1]] = round_to(out[idx, offs[s]:offs[s + 1]] + d, dtype)
            else:
                out[idx, offs[s]:offs[s + 1]] += z @ B.T
    if mode != "hf":
        touched = (ids > 0) & (ids <= NA)
        out[touched] = round_to(out[touched], dtype)
    return out


def per_token_reference(y, x, ids, lora_A_slices, lora_B_slices, output_slices, ranks):
    """Explicit per-token loop, float64 (independent formulation).

    Restates ``_reference_forward`` of tests/unit/test_switched_lora_linear.py:
    199-241: for every token m with id > 0 and every slice s,
    ``out[m, slice] += (x[m] @ A[a,s,:r].T) @ B[a,s,:,:r].T``.
    """
    out = np.asarray(y, dtype=np.float64).copy()
    x = np.asarray(x, dtype=np.float64)
    offs = np.cumsum([0] + list(output_slices))
    for m, ai in enumerate(np.asarray(ids, dtype=np.int64)):
        if ai == 0:
            continue
        a = ai - 1
        r = int(ranks[a])
        for s in range(len(output_slices)):
            A = np.asarray(lora_A_slices[s], dtype=np.float64)[a, 0, :r]
            B = np.asarray(lora_B_slices[s], dtype=np.float64)[a, 0, :, :r]
            out[m, offs[s]:offs[s + 1]] += (x[m] @ A.T) @ B.T
    return out


def shrink_rows(x, perm, seg_offsets, lora_A_slices, ranks, zw: int):
    """Shrink values in segment order: ``z[slot, s*r_a + j] = x[perm[slot]] . A_{a,s}[j]``.

    The slot layout is this build's (adapter-sorted, see
    ``mapping.build_segments``); the values are the reference's
    ``x[idx] @ lora_A[a-1,0].T`` (src/granite_switch/hf/core/lora.py:156).
    Returns float64 [T_act, zw] (unused columns zero).
    """
    x = np.asarray(x, dtype=np.float64)
    seg = np.asarray(seg_offsets, dtype=np.int64)
    perm = np.asarray(perm, dtype=np.int64)
    S = len(lora_A_slices)
    z = np.zeros((int(seg[-1]), zw), dtype=np.float64)
    for g in range(1, seg.shape[0]):
        lo, hi = int(seg[g - 1]), int(seg[g])
        if hi == lo:
            continue
        r = int(ranks[g - 1])
        if r == 0:
            continue
        for s in range(S):
            A = np.asarray(lora_A_slices[s], dtype=np.float64)[g - 1, 0, :r]
            z[lo:hi, s * r:(s + 1) * r] = x[perm[lo:hi]] @ A.T
    return z


def _xext_tile_delta(x_ext, ids_tile, rows, bitmask, lb_packed, slice_cols, na, S, N, n_cols):
    """fp64 LoRA delta for one row-tile and a set of output columns.

    Shared body of the two reference expand kernels
    (src/granite_switch/kernels/switch_lora_kernel.py:264-403 and :478-665):
    tier by tier, each adapter whose bit is set contributes
    ``shrink[rows of that adapter, :r] @ lb[n, :r]^T``; shrink columns start at
    ``slice_cols[tier] + a*S*r``; lora_B of tier adapter ``a`` is
    ``lb_packed[lb_off_t + a*N*r + n*r + k]``.
    """
    delta = np.zeros((rows.shape[0], n_cols.shape[0]), dtype=np.float64)
    lb_off = 0
    id_off = 0
    lb = np.asarray(lb_packed, dtype=np.float64)
    bm = int(np.int64(bitmask)) & ((1 << 64) - 1)
    for t, r in enumerate(SUPPORTED_RANKS):
        for a in range(na[t]):
            kid = id_off + a + 1
            if (bm >> (kid - 1)) & 1:
                sel = ids_tile == kid
                if np.any(sel):
                    c0 = int(slice_cols[t]) + a * S * r
                    sh = np.asarray(x_ext[rows[sel], c0:c0 + r], dtype=np.float64)
                    B = lb[lb_off + a * N * r: lb_off + (a + 1) * N * r].reshape(N, r)[n_cols]
                    delta[sel] += sh @ B.T
        lb_off += na[t] * N * r
        id_off += na[t]
    return delta


def switch_lora_expand_xext(x_ext, adapter_indices, bitmask, lb_packed, tile_slice, slice_col_r,
                            na, S, block_n, N, block_m=32, dtype="bf16"):
    """In-place expand over ``x_ext[:, :N]`` (returns the updated copy).

    Restates src/granite_switch/kernels/switch_lora_kernel.py:171-411: per
    (32-row tile, ``block_n`` columns): skip if the tile bitmask is 0; look up
    the tile's slice (``tile_slice``) and that slice's shrink-column bases
    (``slice_col_r[s]``); accumulate each present adapter's delta in fp32
    (here fp64); write ``round(existing + delta)`` only on rows with id != 0.
    """
    xe = np.array(x_ext, dtype=np.float64, copy=True)
    ids = np.asarray(adapter_indices, dtype=np.int64)
    M = xe.shape[0]
    bms = np.asarray(bitmask, dtype=np.int64).reshape(-1)
    for pm in range((M + block_m - 1) // block_m):
        if bms[pm] == 0:
            continue
        rows = np.arange(pm * block_m, min(M, (pm + 1) * block_m))
        ids_tile = ids[rows]
        act = ids_tile != 0
        if not np.any(act):
            continue
        for pn in range((N + block_n - 1) // block_n):
            cols = np.arange(pn * block_n, min(N, (pn + 1) * block_n))
            s = int(tile_slice[pn])
            d = _xext_tile_delta(xe, ids_tile, rows, bms[pm], lb_packed, slice_col_r[s], na, S, N, cols)
            blk = xe[np.ix_(rows[act], cols)] + d[act]
            xe[np.ix_(rows[act], cols)] = round_to(blk, dtype)
    return xe


def shrink_expand_xext(x_ext, adapter_indices, bitmask, lb_packed, tile_slice, slice_col_r, na, S, block_n, N,
                       block_m=32, dtype="bf16"):
    """W-less expand: a fresh ``out[M, N]`` holding only the LoRA delta.

    Restates src/granite_switch/kernels/switch_lora_kernel.py:883-1146: the
    launcher zeroes ``out`` (:1117); tiles whose bitmask is 0 are skipped and
    stay zero; every other tile gets the same per-adapter delta as the in-place
    expand (shrink columns at ``slice_col_r[s][tier] + a*S*r``, which start at
    0 because the cross weight has no base rows) and STORES it, rounded to the
    output dtype, on every row of the tile -- a base row (id 0) selects no
    adapter, so it stores an exact zero.
    """
    xe = np.asarray(x_ext, dtype=np.float64)
    ids = np.asarray(adapter_indices, dtype=np.int64)
    M = xe.shape[0]
    bms = np.asarray(bitmask, dtype=np.int64).reshape(-1)
    out = np.zeros((M, N), dtype=np.float64)
    for pm in range((M + block_m - 1) // block_m):
        if bms[pm] == 0:
            continue
        rows = np.arange(pm * block_m, min(M, (pm + 1) * block_m))
        for pn in range((N + block_n - 1) // block_n):
            cols = np.arange(pn * block_n, min(N, (pn + 1) * block_n))
            s = int(tile_slice[pn])
            d = _xext_tile_delta(xe, ids[rows], rows, bms[pm], lb_packed, slice_col_r[s], na, S, N, cols)
            out[np.ix_(rows, cols)] = round_to(d, dtype)
    return out


def expand_swiglu_xext(x_ext, adapter_indices, bitmask, lb_packed, slice_col_r, na, S, H, N,
                       block_m=32, dtype="bf16"):
    """``out[M, H] = silu(gate + dgate) * (up + dup)``, always written.

    Restates src/granite_switch/kernels/switch_lora_kernel.py:668-806: gate is
    x_ext[:, 0:H], up is x_ext[:, H:2H]; the LoRA delta (slice 0 columns for
    gate, slice 1 for up) is added in fp32 only for tiles with a nonzero
    bitmask; ``silu(g) = g * sigmoid(g)``; one rounding at the store.
    """
    xe = np.asarray(x_ext, dtype=np.float64)
    ids = np.asarray(adapter_indices, dtype=np.int64)
    M = xe.shape[0]
    bms = np.asarray(bitmask, dtype=np.int64).reshape(-1)
    gate = xe[:, :H].copy()
    up = xe[:, H:2 * H].copy()
    hcols = np.arange(H)
    for pm in range((M + block_m - 1) // block_m):
        if bms[pm] == 0:
            continue
        rows = np.arange(pm * block_m, min(M, (pm + 1) * block_m))
        ids_tile = ids[rows]
        gate[rows] += _xext_tile_delta(xe, ids_tile, rows, bms[pm], lb_packed, slice_col_r[0], na, S, N, hcols)
        up[rows] += _xext_tile_delta(xe, ids_tile, rows, bms[pm], lb_packed, slice_col_r[1], na, S, N, H + hcols)
    out = gate / (1.0 + np.exp(-gate)) * up
    return round_to(out, dtype).astype(np.float64)
