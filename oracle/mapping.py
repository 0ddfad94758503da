"""Integer side of the switched-LoRA path: routing, remap tables, bitmasks, segments.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Pure numpy / Python.
Every function cites the reference code it restates.
"""

from __future__ import annotations

import numpy as np

# src/granite_switch/kernels/switch_lora_kernel.py:79
SUPPORTED_RANKS = (16, 32, 64, 128, 256, 512)
# src/granite_switch/kernels/switch_lora_kernel.py:107
BLOCK_M = 32


def promote_rank(rank: int) -> int:
    """Smallest supported tier >= rank; rank <= 0 unchanged; > 512 raises.

    Restates src/granite_switch/kernels/switch_lora_kernel.py:82-101.
    """
    if rank <= 0:
        return rank
    for tier in SUPPORTED_RANKS:
        if tier >= rank:
            return tier
    raise ValueError(f"rank {rank} exceeds the largest supported rank {SUPPORTED_RANKS[-1]}")


def latest_wins_ids(tokens, adapter_token_ids, base_reset: bool, start_id: int = 0) -> list[int]:
    """Latest-wins routing (tests/vllm/test_multi_switch_serving.py:141-153).

    ``base_reset``: slot 0 of ``adapter_token_ids`` re-selects base (id = slot
    index); otherwise slot k fires adapter k+1.  ``start_id`` is the id in force
    before the first token (the routing state carried from a cached prefix in
    chunked prefill / decode, tests/vllm/test_multi_switch_serving.py:168-243).
    """
    offset = 0 if base_reset else 1
    out, cur = [], int(start_id)
    for t in tokens:
        if t in adapter_token_ids:
            cur = adapter_token_ids.index(t) + offset
        out.append(cur)
    return out


def alora_effective_ids(req_ids, positions, cu_seqlens, act_offsets) -> np.ndarray:
    """aLoRA gating on a ragged packed batch.

    Token ``t`` of sequence ``s`` (absolute position ``q = positions[t]``) keeps
    its requested adapter iff ``q >= act_offsets[s]``; otherwise it is base (0).
    This is latest-wins routing (tests/vllm/test_multi_switch_serving.py:141-153)
    with one control token at the activation offset: the control token's own
    position is already adapted (tests/shared/multi_switch_cases.py:139-144).

    req_ids   : [T] int, 0 = base, 1..NA adapters (reference convention)
    positions : [T] int absolute positions, or None (then position = index in
                the sequence)
    cu_seqlens: [B+1] int token boundaries, or None (one sequence)
    act_offsets: [B] int, or None (no gating)
    """
    req = np.asarray(req_ids, dtype=np.int64)
    T = req.shape[0]
    if act_offsets is None:
        return req.copy()
    if cu_seqlens is None:
        cu = np.array([0, T], dtype=np.int64)
    else:
        cu = np.asarray(cu_seqlens, dtype=np.int64)
    off = np.asarray(act_offsets, dtype=np.int64)
    out = np.zeros(T, dtype=np.int64)
    for s in range(cu.shape[0] - 1):
        lo, hi = int(cu[s]), int(cu[s + 1])
        if positions is None:
            q = np.arange(hi - lo, dtype=np.int64)
        else:
            q = np.asarray(positions, dtype=np.int64)[lo:hi]
        out[lo:hi] = np.where(q >= off[s], req[lo:hi], 0)
    return out


def build_adapter_kind_lut(adapter_kinds):
    """Bool table over adapter indices marking the probe slots, or None.

    Restates src/granite_switch/probe_routing.py:17-33: entry ``i`` is True
    when adapter index ``i`` (slot ``i - 1``) is a probe; index 0 (base) is
    always False; None when no slot is a probe (or no kinds are given).
    """
    if adapter_kinds is None or not any(k == "probe" for k in adapter_kinds):
        return None
    lut = np.zeros(len(adapter_kinds) + 1, dtype=bool)
    for slot, kind in enumerate(adapter_kinds):
        if kind == "probe":
            lut[slot + 1] = True
    return lut


def split_adapter_indices(kind_lut, ids):
    """Split one per-token index stream into (LoRA stream, probe stream).

    Restates src/granite_switch/probe_routing.py:36-58: where the LUT marks an
    index as a probe, the LoRA stream holds 0 and the probe stream the index;
    elsewhere the LoRA stream holds the index and the probe stream 0.  With no
    LUT the LoRA stream is the input and the probe stream all zeros.  Shapes
    are preserved.
    """
    ids = np.asarray(ids, dtype=np.int64)
    if kind_lut is None:
        return ids.copy(), np.zeros_like(ids)
    lut = np.asarray(kind_lut, dtype=bool)
    lora = np.empty_like(ids)
    probe = np.empty_like(ids)
    for pos in np.ndindex(ids.shape):
        v = int(ids[pos])
        is_probe = bool(lut[v])            # the reference indexes the LUT directly
        lora[pos] = 0 if is_probe else v
        probe[pos] = v if is_probe else 0
    return lora, probe


def build_remap(applicable, adapter_ranks) -> tuple[np.ndarray, list[int], list[int]]:
    """Remap table: global adapter id (1-based) -> kernel-local position.

    Restates src/granite_switch/vllm/core/lora.py:366-396: non-applicable
    adapters map to 0; applicable ones are promoted (lora.py:380) and ordered by
    a STABLE ascending sort on the promoted rank (lora.py:392), then numbered
    1.. in that order.

    Returns (remap[NA+1] int64, rank_order (0-based adapter idx), eff_ranks).
    """
    NA = len(adapter_ranks)
    eff = [promote_rank(int(r)) for r in adapter_ranks]
    applicable_adapters = [i for i in range(NA) if applicable[i]]
    # Python's sort is stable, exactly like the reference's ``sorted``.
    rank_order = sorted(applicable_adapters, key=lambda i: eff[i])
    remap = np.zeros(NA + 1, dtype=np.int64)
    for k, i in enumerate(rank_order):
        remap[i + 1] = k + 1
    return remap, rank_order, eff


def applicability(lora_A_slices, adapter_ranks) -> list[bool]:
    """An adapter applies to a module iff any of its first r rows of lora_A is
    nonzero in any slice (src/granite_switch/vllm/core/lora.py:353-362)."""
    NA = len(adapter_ranks)
    out = []
    for i in range(NA):
        r = int(adapter_ranks[i])
        nz = False
        for A in lora_A_slices:
            if r > 0 and np.any(np.asarray(A)[i, 0, :r, :] != 0):
                nz = True
        out.append(nz)
    return out


def finalize_tables(output_slices, rank_order, eff_ranks, block_n=32):
    """Per-module expand tables of the reference kernel.

    Restates src/granite_switch/vllm/core/lora.py:398-492 and :637-657:

      na[6]              count of applicable adapters per tier
      tile_to_slice[nT]  slice of each ``block_n``-wide output tile (lora.py:459-472)
      slice_col_r[S,6]   N_total + sum_{t'<t} n_t'*S*r_t' + s*r_t     (lora.py:474-492)
      tiers              OrderedDict rank -> [adapter idx] in kernel-local order
    """
    S = len(output_slices)
    N_total = int(sum(output_slices))
    for n_s in output_slices:
        if n_s % block_n != 0:
            raise AssertionError(f"block_n={block_n} must divide every output slice: {tuple(output_slices)}")
    tiers: dict[int, list[int]] = {}
    for i in rank_order:
        tiers.setdefault(eff_ranks[i], []).append(i)
    na = tuple(len(tiers.get(r, [])) for r in SUPPORTED_RANKS)
    num_tiles = (N_total + block_n - 1) // block_n
    cum = np.cumsum([0] + list(output_slices))
    tile_to_slice = np.zeros(num_tiles, dtype=np.int32)
    for t in range(num_tiles):
        c = t * block_n
        for s in range(S):
            if cum[s] <= c < cum[s + 1]:
                tile_to_slice[t] = s
                break
    bases, off = [], N_total
    for t, r in enumerate(SUPPORTED_RANKS):
        bases.append(off)
        off += na[t] * S * r
    slice_col_r = np.array([[bases[t] + s * SUPPORTED_RANKS[t] for t in range(6)] for s in range(S)], dtype=np.int32)
    return na, tile_to_slice, slice_col_r, tiers


def build_w_ext(W, lora_A_slices, tiers):
    """``cat([W] + [A rows in tier -> adapter -> slice -> rank order])``.

    Restates src/granite_switch/kernels/switch_lora_kernel.py:134-163 together
    with the per-tier stacking at src/granite_switch/vllm/core/lora.py:406-417.
    ``lora_A_slices[s]`` is [NA, 1, max_r, K] (zero-padded past the true rank).
    """
    parts = [np.asarray(W)]
    S = len(lora_A_slices)
    for r in SUPPORTED_RANKS:
        for i in tiers.get(r, []):
            for s in range(S):
                A = np.asarray(lora_A_slices[s])[i, 0]
                rows = A[:r] if A.shape[0] >= r else np.concatenate([A, np.zeros((r - A.shape[0], A.shape[1]), A.dtype)])
                parts.append(rows)
    return np.concatenate(parts, axis=0)


def build_lb_packed(lora_B_slices, tiers):
    """Single packed lora_B: tiers concatenated, each [n_r, N_total, r] row-major.

    Restates src/granite_switch/vllm/core/lora.py:435-448 and :649-657.
    ``lora_B_slices[s]`` is [NA, 1, N_s, max_r].
    """
    S = len(lora_B_slices)
    parts = []
    for r in SUPPORTED_RANKS:
        for i in tiers.get(r, []):
            cols = []
            for s in range(S):
                B = np.asarray(lora_B_slices[s])[i, 0]
                if B.shape[1] >= r:
                    cols.append(B[:, :r])
                else:
                    cols.append(np.concatenate([B, np.zeros((B.shape[0], r - B.shape[1]), B.dtype)], axis=1))
            parts.append(np.concatenate(cols, axis=0).reshape(-1))
    if not parts:
        return np.zeros(1, dtype=np.float32)
    return np.concatenate(parts)


def compute_bitmasks(adapter_indices, remap_tables_t, block_m: int = BLOCK_M) -> np.ndarray:
    """Per-module, per-tile int64 bitmask of present kernel-local adapters.

    Restates src/granite_switch/vllm/core/lora_kernel_meta.py:104-151 (and the
    Triton kernel :30-58): pad the tail tile with id 0, clamp ids to [0, NA],
    gather ``loc = remap_t[id, module]``, set bit ``loc-1`` when ``loc > 0``, OR
    over the tile.  Position 64 sets bit 63, i.e. the int64 sign bit.
    """
    ids = np.asarray(adapter_indices, dtype=np.int64)
    remap_t = np.asarray(remap_tables_t, dtype=np.int64)
    M = ids.shape[0]
    NA = remap_t.shape[0] - 1
    num_modules = remap_t.shape[1]
    num_tiles = (M + block_m - 1) // block_m
    out = np.zeros((num_modules, num_tiles), dtype=np.uint64)
    ids_c = np.clip(ids, 0, NA)
    for m in range(num_modules):
        loc = remap_t[ids_c, m]
        bits = np.where(loc > 0, np.left_shift(np.uint64(1), np.maximum(loc - 1, 0).astype(np.uint64)), np.uint64(0))
        for t in range(num_tiles):
            acc = np.uint64(0)
            for b in bits[t * block_m:(t + 1) * block_m]:
                acc |= b
            out[m, t] = acc
    return out.view(np.int64)


def remapped_indices(adapter_indices, remap_tables_t) -> np.ndarray:
    """``remap_t[ids].T`` -> [num_modules, M] kernel-local ids.

    Restates src/granite_switch/vllm/core/lora_kernel_meta.py:294 (the reference
    gathers without clamping; ids are in [0, NA] by contract).
    """
    ids = np.asarray(adapter_indices, dtype=np.int64)
    remap_t = np.asarray(remap_tables_t, dtype=np.int64)
    return np.ascontiguousarray(remap_t[ids].T)


def build_segments(eff_ids, num_adapters: int):
    """Adapter-sorted segments of the active tokens (stable counting sort).

    Not a reference function: the reference does this work implicitly, once per
    adapter, with ``torch.where(ids == a)`` (src/granite_switch/hf/core/lora.py:
    130-135, 321-325), which yields each adapter's tokens in ascending order and
    adapters in ascending id order (``unique`` is sorted).  The segments restate
    exactly that iteration order:

      seg_offsets[NA+1]: adapter g (1..NA) owns perm[seg_offsets[g-1]:seg_offsets[g]]
      perm[T_act]      : token indices, grouped by adapter, ascending within

    Ids outside [0, NA] are treated as base (the reference's bitmask clamps them
    away, lora_kernel_meta.py:46-47).
    """
    ids = np.asarray(eff_ids, dtype=np.int64)
    valid = (ids >= 1) & (ids <= num_adapters)
    counts = np.bincount(ids[valid], minlength=num_adapters + 1)[: num_adapters + 1]
    seg = np.zeros(num_adapters + 1, dtype=np.int64)
    seg[1:] = np.cumsum(counts[1:])
    perm = np.concatenate([np.nonzero(ids == g)[0] for g in range(1, num_adapters + 1)] + [np.zeros(0, np.int64)])
    return seg.astype(np.int32), perm.astype(np.int32)
