"""Per-token switched-LoRA on MI355X: segment metadata, packed adapters, apply.

This is the ``y``-given form of the reference's switched-LoRA math
(src/granite_switch/hf/core/lora.py:127-161 and :308-348):

    y[t, slice s] += (x[t] . lora_A[a-1, 0]^T) . lora_B[a-1, 0]^T   for id a > 0

with lora_B pre-scaled by alpha/r (src/granite_switch/composer/weight_transfer.py:
564-568).  Three device steps, all launched on torch's current stream with no
host synchronisation (so the whole thing can be captured in a HIP graph):

  1. ``build_segments``  per-token ids (+ aLoRA activation offsets on ragged
     packed batches) -> adapter-sorted token permutation and segment offsets;
  2. ``shrink``           z[slot] = x[perm[slot]] . A_g^T   (bf16/fp32 MFMA)
  3. ``expand_add``       y[perm[slot]] += z[slot] . B_g^T  (MFMA, in place)

Base rows are never written.  Nothing here falls back to the CPU: the HIP
library must be built.
"""

from __future__ import annotations

import ctypes
import dataclasses
import math
import os
from dataclasses import dataclass

import torch

from . import _lib

_DTYPES = {torch.bfloat16: _lib.GS_DTYPE_BF16, torch.float32: _lib.GS_DTYPE_FP32}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected bfloat16 or float32") from None


def _require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("switched-LoRA tensors must live on the GPU")


# ---------------------------------------------------------------------------
# Segments
# ---------------------------------------------------------------------------
@dataclass
class Segments:
    """Adapter-sorted segments of one batch (built once, reused by every module).

    eff_ids     [T] int32  effective per-token global id (0 = base)
    seg_offsets [NA+1] int32: adapter g owns perm[seg_offsets[g-1]:seg_offsets[g]]
    perm        [T] int32  token indices grouped by adapter, ascending within
    work        int32 per-chunk histograms of the builder's two-launch form
                (None: the one-launch form, which needs no workspace)
    """

    eff_ids: torch.Tensor
    seg_offsets: torch.Tensor
    perm: torch.Tensor
    num_tokens: int
    num_adapters: int
    work: torch.Tensor | None = None


def _as_i64(t, device):
    if t is None:
        return None
    if not isinstance(t, torch.Tensor):
        t = torch.as_tensor(t)
    return t.to(device=device, dtype=torch.int64).contiguous()


def _as_i32(t, device):
    if t is None:
        return None
    if not isinstance(t, torch.Tensor):
        t = torch.as_tensor(t)
    return t.to(device=device, dtype=torch.int32).contiguous()


def build_segments(adapter_ids: torch.Tensor, num_adapters: int, positions=None, cu_seqlens=None,
                   act_offsets=None, out: Segments | None = None) -> Segments:
    """Gate per-token ids by aLoRA activation offsets and sort tokens by adapter.

    adapter_ids: [T] requested adapter per token (0 = base, 1..num_adapters)
    positions:   [T] absolute positions (chunked prefill / decode), or None
                 (position = index inside the sequence)
    cu_seqlens:  [B+1] sequence boundaries of the packed batch, or None
    act_offsets: [B] activation offset per sequence: a token is adapted iff its
                 position >= the offset (tokens before the invocation point are
                 base only); None disables gating.
    Integer tensors must already be on the GPU for graph capture (conversions
    are skipped when dtypes already match).
    """
    _require_cuda(adapter_ids)
    dev = adapter_ids.device
    ids = _as_i64(adapter_ids.reshape(-1), dev)
    T = ids.shape[0]
    pos = _as_i64(positions, dev)
    cu = _as_i32(cu_seqlens, dev)
    off = _as_i64(act_offsets, dev)
    if pos is not None and pos.numel() != T:
        raise ValueError("positions must have one entry per token")
    num_seqs = 1
    if cu is not None:
        num_seqs = cu.numel() - 1
        if off is not None and off.numel() != num_seqs:
            raise ValueError("act_offsets must have one entry per sequence")
    elif off is not None and off.numel() != 1:
        raise ValueError("act_offsets without cu_seqlens describes one sequence")
    if out is None:
        ws = int(_lib.load().gs_build_segments_workspace_bytes(T, num_adapters))
        out = Segments(
            eff_ids=torch.empty(T, dtype=torch.int32, device=dev),
            seg_offsets=torch.empty(num_adapters + 1, dtype=torch.int32, device=dev),
            perm=torch.empty(max(T, 1), dtype=torch.int32, device=dev),
            num_tokens=T,
            num_adapters=num_adapters,
            work=torch.empty((ws + 3) // 4, dtype=torch.int32, device=dev) if ws > 0 else None,
        )
    else:
        _check_reused_segments(out, T, num_adapters, dev)
        out.num_tokens = T
    work = out.work
    _lib.call("gs_build_segments", ids.data_ptr(), _lib.ptr(pos), _lib.ptr(cu), _lib.ptr(off), T, num_seqs,
              num_adapters, out.eff_ids.data_ptr(), out.seg_offsets.data_ptr(), out.perm.data_ptr(),
              _lib.ptr(work), 0 if work is None else work.numel() * 4, _lib.stream_ptr(dev))
    return out


def _check_reused_segments(out: Segments, T: int, num_adapters: int, dev: torch.device) -> None:
    """``out`` is written in place by the builder: its buffers must hold this
    batch (T tokens, num_adapters adapters) before anything is launched."""
    bufs = (("eff_ids", out.eff_ids, T), ("perm", out.perm, max(T, 1)),
            ("seg_offsets", out.seg_offsets, num_adapters + 1))
    if out.num_adapters != num_adapters or out.seg_offsets.numel() != num_adapters + 1:
        raise ValueError(f"build_segments(out=...): the segments were allocated for {out.num_adapters} adapters, "
                         f"this call has {num_adapters}")
    for name, t, need in bufs:
        if t.dtype != torch.int32 or t.device != dev or not t.is_contiguous():
            raise ValueError(f"build_segments(out=...): {name} must be a contiguous int32 tensor on {dev}")
        if t.numel() < need:
            raise ValueError(f"build_segments(out=...): {name} holds {t.numel()} entries, this batch of {T} tokens "
                             f"needs {need}")
    if out.work is not None and (out.work.dtype != torch.int32 or out.work.device != dev):
        raise ValueError(f"build_segments(out=...): work must be an int32 tensor on {dev}")


def route_latest_wins(input_ids: torch.Tensor, control_tokens, id_offset: int = 1, cu_seqlens=None,
                      start_ids=None) -> torch.Tensor:
    """Latest-wins routing from control tokens (per sequence).

    Semantics of src/granite_switch/vllm/switch/multi.py:348-525 as pinned by
    tests/vllm/test_multi_switch_serving.py:141-153: a token equal to
    control_tokens[k] fires id k + id_offset (id_offset=1: no base slot;
    id_offset=0: slot 0 is a base-reset token); every position takes the id of
    the latest control token at or before it, else ``start_ids[s]`` (the state
    carried over from the sequence's cached prefix, 0 when None).
    """
    _require_cuda(input_ids)
    dev = input_ids.device
    ids = _as_i64(input_ids.reshape(-1), dev)
    T = ids.shape[0]
    ctl = _as_i64(control_tokens, dev)
    cu = _as_i32(cu_seqlens, dev)
    start = _as_i64(start_ids, dev)
    num_seqs = 1 if cu is None else cu.numel() - 1
    out = torch.empty(T, dtype=torch.int64, device=dev)
    _lib.call("gs_route_latest_wins", ids.data_ptr(), _lib.ptr(cu), T, num_seqs, ctl.data_ptr(), ctl.numel(),
              int(id_offset), _lib.ptr(start), out.data_ptr(), _lib.stream_ptr(dev))
    return out


# ---------------------------------------------------------------------------
# Packed adapters (load time)
# ---------------------------------------------------------------------------
def _round8(r: int) -> int:
    return ((r + 7) // 8) * 8


@dataclass
class PackedAdapters:
    """One module's adapters in the layout the kernels read.

    a_pack: rows of adapter g start at a_off[g] (elements): S*r_g rows of H,
            row s*r_g + j = lora_A slice s, rank row j.
    b_pack: adapter g at b_off[g]: [out_total, r_g] row-major, slices stacked
            along out, rank contiguous, pre-scaled.
    ranks[g]: r_g (true rank rounded up to a multiple of 8 with zero rows),
            0 for g = 0 and for adapters that are not applicable here.
    """

    a_pack: torch.Tensor
    b_pack: torch.Tensor
    a_off: torch.Tensor
    b_off: torch.Tensor
    ranks: torch.Tensor
    ranks_host: list
    output_slices: tuple
    hidden: int
    num_adapters: int
    max_rank: int
    a_off_host: list = None     # host copies of a_off / b_off (the small-batch path passes them by value)
    b_off_host: list = None

    @property
    def num_slices(self) -> int:
        return len(self.output_slices)

    @property
    def out_total(self) -> int:
        return int(sum(self.output_slices))

    @property
    def slice_bounds(self) -> list:
        b = [0]
        for s in self.output_slices:
            b.append(b[-1] + int(s))
        return b

    @property
    def dtype(self) -> torch.dtype:
        return self.a_pack.dtype

    def restricted(self, lo: int, hi: int) -> "PackedAdapters | None":
        """The same pack limited to the adapters whose rank lies in [lo, hi]:
        the others get rank 0 in the host tables, which the kernels skip (the
        device tensors are shared).  None when no adapter's rank is in range."""
        rk = [int(r) if lo <= int(r) <= hi else 0 for r in self.ranks_host]
        if not any(rk):
            return None
        return dataclasses.replace(self, ranks_host=rk, max_rank=max(rk))

    def rank_split(self) -> tuple:
        """(adapters of rank <= 64, adapters of larger rank) as restricted packs
        (either may be None).  The one-launch decode kernel takes the first;
        the segment kernels plan and launch each class for its own ranks."""
        cut = _lib.GS_RANK_CLASS_SPLIT
        return self.restricted(1, cut), self.restricted(cut + 1, _lib.GS_MAX_RANK)

    @staticmethod
    def from_slices(lora_A_slices, lora_B_slices, adapter_ranks=None, applicable=None) -> "PackedAdapters":
        """Pack checkpoint-layout adapters.

        lora_A_slices[s]: [NA, 1, max_r, H]; lora_B_slices[s]: [NA, 1, O_s, max_r]
        (the composed-checkpoint layout, src/granite_switch/composer/
        weight_transfer.py:547-622).  ``adapter_ranks`` gives each adapter's
        true rank (default max_r); only those rows/columns are packed, so the
        bytes the kernels read are the true-rank bytes.  ``applicable``
        defaults to the reference's rule: any nonzero lora_A value in the first
        r rows of any slice (src/granite_switch/vllm/core/lora.py:353-362).
        """
        S = len(lora_A_slices)
        if S != len(lora_B_slices) or S < 1 or S > _lib.GS_MAX_SLICES:
            raise ValueError("lora_A_slices and lora_B_slices must have the same 1..8 slices")
        A0 = lora_A_slices[0]
        NA, _, max_r, H = A0.shape
        dev, dt = A0.device, A0.dtype
        out_slices = tuple(int(B.shape[2]) for B in lora_B_slices)
        if adapter_ranks is None:
            adapter_ranks = [max_r] * NA
        if len(adapter_ranks) != NA:
            raise ValueError("adapter_ranks must have one entry per adapter")
        if applicable is None:
            flags = torch.zeros(NA, dtype=torch.bool, device=dev)
            rk = torch.tensor([int(r) for r in adapter_ranks], device=dev)
            mask = torch.arange(max_r, device=dev)[None, :] < rk[:, None]
            for A in lora_A_slices:
                flags |= (A[:, 0].ne(0).any(dim=-1) & mask).any(dim=1)
            applicable = flags.tolist()
        a_parts, b_parts = [], []
        a_off = [0] * (NA + 1)
        b_off = [0] * (NA + 1)
        ranks = [0] * (NA + 1)
        arow = 0
        belem = 0
        O = sum(out_slices)
        for a in range(NA):
            r_true = int(adapter_ranks[a])
            if not applicable[a] or r_true <= 0:
                continue
            if r_true > _lib.GS_MAX_RANK:
                raise ValueError(f"rank {r_true} exceeds {_lib.GS_MAX_RANK}")
            r = _round8(r_true)
            g = a + 1
            ranks[g] = r
            a_off[g] = arow * H
            b_off[g] = belem
            for s in range(S):
                A = lora_A_slices[s][a, 0, :min(r, r_true), :]
                if A.shape[0] < r:
                    A = torch.cat([A, torch.zeros(r - A.shape[0], H, dtype=dt, device=dev)])
                a_parts.append(A)
            Bs = []
            for s in range(S):
                B = lora_B_slices[s][a, 0, :, :min(r, r_true)]
                if B.shape[1] < r:
                    B = torch.cat([B, torch.zeros(B.shape[0], r - B.shape[1], dtype=dt, device=dev)], dim=1)
                Bs.append(B)
            b_parts.append(torch.cat(Bs, dim=0).reshape(-1))
            arow += S * r
            belem += O * r
        if a_parts:
            a_pack = torch.cat(a_parts).contiguous()
            b_pack = torch.cat(b_parts).contiguous()
        else:
            a_pack = torch.zeros(8, H, dtype=dt, device=dev)
            b_pack = torch.zeros(8 * O, dtype=dt, device=dev)
        max_rank = max([8] + ranks)
        return PackedAdapters(
            a_pack=a_pack,
            b_pack=b_pack,
            a_off=torch.tensor(a_off, dtype=torch.int64, device=dev),
            b_off=torch.tensor(b_off, dtype=torch.int64, device=dev),
            ranks=torch.tensor(ranks, dtype=torch.int32, device=dev),
            ranks_host=ranks,
            output_slices=out_slices,
            hidden=int(H),
            num_adapters=int(NA),
            max_rank=int(max_rank),
            a_off_host=list(a_off),
            b_off_host=list(b_off),
        )


# ---------------------------------------------------------------------------
# Workspace (split-K partial sums), cached per device
# ---------------------------------------------------------------------------
_workspaces: dict = {}
# Buffers replaced by a larger one.  They are never freed: a HIP graph captured
# while one was current still holds its address, and its replays keep using it
# (freed memory would go back to torch's allocator and could be handed to
# another tensor while a replay writes into it).
_retired: list = []


def _grow(table: dict, key, need: int, what: str, zero: bool = True) -> torch.Tensor:
    buf = table.get(key)
    if buf is None or buf.numel() < need:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"switched-LoRA {what} must be allocated before graph capture "
                               "(call reserve_workspace / reserve_small_workspace, or run once eagerly)")
        new = torch.zeros(max(need, 1 << 20), dtype=torch.uint8, device=torch.device(key[0], key[1]))
        if buf is not None:
            _retired.append(buf)
        table[key] = buf = new
    return buf


def _workspace(device: torch.device, need: int) -> torch.Tensor:
    return _grow(_workspaces, _dev_key(device), need, "workspace")


def shrink_workspace(num_tokens: int, hidden: int, num_slices: int, num_adapters: int, max_rank: int,
                     device: torch.device, ranks_host=None) -> torch.Tensor:
    """A workspace big enough for the split-K partials of one shrink of this shape.

    One buffer per device is reused by every call (stream order keeps calls on
    one stream apart); calls on different streams that may overlap in time
    must not share it.
    """
    need = int(_lib.load().gs_shrink_workspace_bytes(num_tokens, hidden, num_slices, num_adapters, max_rank,
                                                     None if ranks_host is None else _i32_array(ranks_host)))
    if need < 0:
        raise _lib.GraniteSwitchError("gs_shrink_workspace_bytes", _lib.GS_ERR_INVALID, _lib.last_error())
    return _workspace(device, need)


def shrink_ksplits(packed: "PackedAdapters", num_tokens: int) -> list:
    """The hidden-dimension split of each rank class of ``packed`` at this batch size."""
    out = (ctypes.c_int32 * 2)()
    n = int(_lib.load().gs_shrink_ksplits(_DTYPES[packed.dtype], int(num_tokens), packed.hidden, packed.num_slices,
                                          packed.num_adapters, packed.max_rank, _i32_array(packed.ranks_host), out))
    if n < 0:
        raise _lib.GraniteSwitchError("gs_shrink_ksplits", -n, _lib.last_error())
    return [int(out[i]) for i in range(n)]


def small_workspace_bytes(packed: "PackedAdapters", num_tokens: int) -> int:
    """Workspace bytes of the small-batch path for this module and batch size."""
    return int(_lib.load().gs_small_workspace_bytes(_DTYPES[packed.dtype], num_tokens, packed.hidden,
                                                    packed.num_slices, packed.num_adapters, packed.max_rank,
                                                    packed.out_total, _i32_array(packed.slice_bounds)))


def small_eligible(packed: "PackedAdapters", num_tokens: int, num_seqs: int = 1) -> bool:
    """True when the one-launch small-batch kernel can run this module and batch.

    It needs the adapters' host-side offset tables (``PackedAdapters.from_slices``
    keeps them) and decode-sized shapes: T <= 1024, <= 64 adapters, max rank
    <= 64, slice widths multiples of 128.
    """
    if packed.a_off_host is None or packed.b_off_host is None or not packed.ranks_host:
        return False
    return bool(_lib.load().gs_small_eligible(int(num_tokens), int(num_seqs), packed.num_slices,
                                              _i32_array(packed.slice_bounds), packed.num_adapters,
                                              packed.max_rank))


_cu_counts: dict = {}


def _device_cus(device: torch.device) -> int:
    key = _dev_key(device)
    n = _cu_counts.get(key)
    if n is None:
        n = int(torch.cuda.get_device_properties(device).multi_processor_count)
        _cu_counts[key] = n
    return n


def small_workgroups(packed: "PackedAdapters", num_tokens: int, row_split: int = 1) -> int:
    """Workgroups of one small-batch launch (producers + consumers)."""
    return int(_lib.load().gs_small_workgroups(_DTYPES[packed.dtype], int(num_tokens), packed.hidden,
                                               packed.num_slices, packed.num_adapters, packed.max_rank,
                                               packed.out_total, _i32_array(packed.slice_bounds), int(row_split)))


def _small_plan(packed: "PackedAdapters", num_tokens: int, num_seqs: int | None,
                largest_group: int | None = None) -> tuple[bool, int]:
    """(prefer the small-batch kernel, its row split) for this module and batch."""
    T = int(num_tokens)
    if packed.a_off_host is None or packed.b_off_host is None or not packed.ranks_host:
        return (False, 1)                             # no host tables: the small kernel cannot run
    key = (_dev_key(packed.a_pack.device), packed.dtype, packed.hidden, packed.num_slices, packed.num_adapters,
           packed.max_rank, tuple(packed.ranks_host), packed.out_total, tuple(packed.slice_bounds), T, num_seqs,
           largest_group)
    plan = _small_plans.get(key)
    if plan is not None:
        return plan
    if not small_eligible(packed, T, num_seqs or 1):
        plan = (False, 1)
    else:
        spread = packed.num_adapters if not num_seqs else min(packed.num_adapters, num_seqs)
        if largest_group is not None:
            largest = max(1, min(int(largest_group), T))
        elif num_seqs:
            largest = (T + spread - 1) // spread
        else:
            # ids drawn per token: at a mean of one chunk or less the largest
            # group runs over it by a few tokens (2 adapters, 64 tokens: 35
            # against 32), and the second chunk then doubles a workgroup's
            # walk, so a margin of two standard deviations is added there
            largest = (T + spread - 1) // spread
            if largest <= 32:
                largest = min(T, largest + int(2 * math.sqrt(largest)))
        chunks = (largest + 31) // 32                   # 32-token chunks in the estimated largest group
        cus = _device_cus(packed.a_pack.device)
        rs = 1
        while rs < chunks and rs * 2 <= 32 and small_workgroups(packed, T, rs * 2) <= 3 * cus:
            rs *= 2
        per_wg = -(-chunks // rs)
        fits = small_workgroups(packed, T, rs) <= (8 if T <= 256 else 4) * cus
        # the kernel streams lora_A through ~128 producer workgroups; past
        # ~28 MiB of it the segment shrink's wider grid is faster
        a_bytes = sum(int(r) for r in packed.ranks_host) * packed.num_slices * packed.hidden * \
            (4 if packed.dtype == torch.float32 else 2)
        plan = (fits and a_bytes <= _SMALL_MAX_A_BYTES and (per_wg <= 2 or (rs == 1 and chunks <= 3)), rs)
    if len(_small_plans) >= _SMALL_PLAN_CAP:     # batch sizes vary per step: keep the cache bounded
        _small_plans.clear()
    _small_plans[key] = plan
    return plan


_small_plans: dict = {}
_SMALL_PLAN_CAP = 4096
# lora_A bytes (all the module's adapters) past which the segment kernels are
# taken: measured 48 adapters of ranks 8-64 on a 12800-wide down projection
# (36.9 MB) 36-37 us one-launch against 27.3 us segments at 128-256 tokens;
# at 12.6-19.7 MB (gate_up, qkv at rank 64, down with 24 adapters) the
# one-launch kernel stays 20-40 % faster
_SMALL_MAX_A_BYTES = 28 << 20


def small_row_split(packed: "PackedAdapters", num_tokens: int, num_seqs: int | None = None,
                    largest_group: int | None = None) -> int:
    """Row split of the small-batch kernel for this batch (see ``small_preferred``)."""
    return _small_plan(packed, num_tokens, num_seqs, largest_group)[1]


def small_preferred(packed: "PackedAdapters", num_tokens: int, num_seqs: int | None = None,
                    largest_group: int | None = None) -> bool:
    """The ``auto`` path choice between the one-launch small-batch kernel and
    the segment kernels (build + shrink + expand), and with it the kernel's
    row split.

    A workgroup set of the one-launch kernel walks the 32-token chunks of its
    adapter's tokens one after another; a row split of RS gives chunks rs,
    rs + RS, ... to RS sets, multiplying the grid by about RS.  The host cannot
    see the groups without a synchronisation, so it estimates the largest one
    as ``T / min(adapters, sequences)`` (a sequence's tokens mostly share an
    adapter; ``num_seqs`` is the number of sequences when the caller knows
    them, ``None`` estimates ``T / adapters``).  A caller that knows the
    largest group (a serving scheduler assigns adapters per request on the
    host) passes it as ``largest_group`` and the estimate is not used.  The
    row split doubles while
    it is below the estimate's chunk count and the grid stays within 3
    workgroups per CU (the kernel holds 2 per CU at a time); the one-launch
    kernel is taken when it is eligible, its grid is within 4 workgroups per
    CU (8 for batches of up to 256 tokens), each workgroup is left with at
    most 2 chunks (3 without a split), and the module's lora_A is at most
    28 MiB (its ~128 producer workgroups stream it slower than the segment
    shrink's grid past that).  For per-token ids (no ``num_seqs``), an
    estimated group of one chunk or less gets a margin of two standard
    deviations, since one token over the chunk doubles a workgroup's walk.

    Measured on one MI355X (H = 2048..12800, 2..48 adapters, T = 64..1024):
    past these grids a second round of workgroups costs more than it saves
    (gate_up 4096 -> 25600 with 24 adapters: 2592 workgroups), and past two
    chunks per workgroup the segment kernels, which spread an adapter's tokens
    over row tiles, are faster.  Row splits took the 2048-wide 4-sequence
    aLoRA batch from 34.6 us (no split) to 14.3 us, against 17.8 us for the
    segment kernels.
    """
    return _small_plan(packed, num_tokens, num_seqs, largest_group)[0]


def reserve_workspace(device: torch.device, nbytes: int) -> None:
    """Pre-allocate the per-device shrink workspace (before graph capture)."""
    _workspace(device, nbytes)


# The small-batch kernel's state, one set per device: its sync buffer (the
# error word and each adapter's epoch and done count) and its workspace of
# epoch-tagged partials.  Both start zeroed; the workspace is used by nothing
# else, so it only ever holds tags of earlier epochs.
_sync_buffers: dict = {}
_small_workspaces: dict = {}
_ERR_WORD = 2
_SYNC_LINE = 32


def _dev_key(device: torch.device):
    return (device.type, device.index if device.index is not None else torch.cuda.current_device())


_side_streams: dict = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """The per-device stream on which the "split" path runs the large rank
    class's segment kernels beside the one-launch kernel (default priority)."""
    key = _dev_key(device)
    s = _side_streams.get(key)
    if s is None:
        s = _side_streams[key] = torch.cuda.Stream(device=torch.device(key[0], key[1]))
    return s


def _split_run(device: torch.device, large, small) -> None:
    """The "split" path: ``large()`` (the segment kernels of the adapters above
    rank 64) on the side stream, forked from the current stream, and
    ``small()`` (the one-launch kernel of the rest) on the current stream,
    then the current stream waits for the side stream.  The two touch disjoint
    rows of y and separate scratch buffers; the large class goes first, its
    kernels being the longer dependent chain.  Everything a later caller's
    work may reuse is released to the current stream only after the join."""
    cur = torch.cuda.current_stream(device)
    side = _side_stream(device)
    side.wait_stream(cur)
    try:
        with torch.cuda.stream(side):
            large()
        small()
    finally:
        cur.wait_stream(side)     # also when a call raised: nothing queued on the side stream outlives the join


def small_sync_buffer(device: torch.device) -> torch.Tensor:
    """The per-device sync buffer of the small-batch kernel (int32 words)."""
    key = _dev_key(device)
    buf = _sync_buffers.get(key)
    if buf is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("switched-LoRA sync buffer must be allocated before graph capture "
                               "(call reserve_small_workspace or run once eagerly)")
        buf = torch.zeros(int(_lib.load().gs_small_sync_bytes()) // 4, dtype=torch.int32, device=device)
        _sync_buffers[key] = buf
    return buf


def small_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """The per-device workspace of the small-batch kernel (at least ``nbytes``).

    A larger request replaces the buffer with a new zeroed one and retires the
    old one (never freed, see ``_retired``).  A graph captured earlier keeps
    the old buffer: its partials carry tags of the same per-adapter epochs as
    the new buffer's, and epochs only grow, so neither buffer ever holds a
    pair tagged with an epoch that has not started."""
    return _grow(_small_workspaces, _dev_key(device), nbytes, "small-batch workspace")


def reserve_small_workspace(device: torch.device, nbytes: int) -> None:
    """Pre-allocate the small-batch kernel's workspace and sync buffer (before graph capture)."""
    small_sync_buffer(device)
    small_workspace(device, nbytes)


def small_status(device: torch.device) -> int:
    """Error word of the small-batch kernel on ``device`` (synchronises).

    0 = every call so far handed off cleanly; bit 0 = an expand workgroup gave
    up waiting for its shrink partials, so that call's output was wrong.
    ``small_reset`` clears the state.
    """
    if _dev_key(device) not in _sync_buffers:
        return 0                       # no small-batch call has run on this device
    return int(small_sync_buffer(device)[_ERR_WORD].item())


class SmallPathError(_lib.GraniteSwitchError):
    """A one-launch decode call gave up waiting for its shrink partials: the
    output of that call (and of any call since the last check) is wrong."""


def check(device: torch.device | None = None) -> None:
    """Raise ``SmallPathError`` if a one-launch decode call on ``device`` has
    reported a failed hand-off since the last ``small_reset`` (synchronises).

    The kernel never stops the stream: a consumer whose wait runs out sets the
    error word and finishes, so the launch and every later one complete.  Call
    this at a point that synchronises anyway (end of a step, before returning
    results), or set ``GS_CHECK_EACH_CALL=1`` to check after every eager call.
    """
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    word = small_status(dev)
    if word:
        raise SmallPathError("gs_switched_lora_small", word,
                             f"error word {word:#x}: an expand workgroup gave up waiting for its shrink partials; "
                             "the affected outputs are wrong (small_reset() clears the state)")


def set_small_wait_limit(polls: int | None) -> int:
    """Bound the decode kernel's hand-off wait to ``polls`` looks (None restores
    the default); returns the previous bound.  0 makes every consumer give up
    at once and report it -- a test hook that still lets every launch end."""
    return int(_lib.load().gs_small_set_wait_limit(-1 if polls is None else int(polls)))


_CHECK_EACH_CALL = os.environ.get("GS_CHECK_EACH_CALL", "0") not in ("", "0")


_EPOCH_SHIFT = 20


def pending_from_counters(counters: torch.Tensor) -> int:
    """Weight of unfinished launches in the adapters' 64-bit launch counters.

    Every consumer of adapter g adds its share of 2^20 to g's counter, and the
    shares of one launch sum to exactly 2^20, so after complete launches the
    low 20 bits of every counter are 0 (the bits above count the epochs).
    Returns the sum of the low 20 bits: 0 iff no launch was half counted.
    """
    low = counters.to(torch.int64) & ((1 << _EPOCH_SHIFT) - 1)
    return int(low.sum().item())


def small_pending_count(device: torch.device) -> int:
    """Weight of unfinished small-batch launches on ``device`` (synchronises).

    Reads adapter g's launch counter, int32 words [32 g, 32 g + 1] of the
    sync buffer (one 128-byte line per adapter, g = 1..64), and returns
    ``pending_from_counters`` of them: 0 after every completed call."""
    return pending_from_sync(small_sync_buffer(device))


def pending_from_sync(sync: torch.Tensor) -> int:
    """``pending_from_counters`` of the counters held in a sync buffer
    (int32 words; adapter g's counter is the int64 at int32 word 32 g)."""
    words = sync.view(torch.int64)
    return pending_from_counters(words[_SYNC_LINE // 2::_SYNC_LINE // 2])


def small_reset(device: torch.device) -> None:
    """Zero the small-batch kernel's epoch, error word and partial workspace.

    The epoch restarts at 0, so the workspace must be cleared with it (a stale
    pair must never carry a tag the next epochs will use)."""
    small_sync_buffer(device).zero_()
    ws = _small_workspaces.get(_dev_key(device))
    if ws is not None:
        ws.zero_()


# ---------------------------------------------------------------------------
# Shrink / expand / fused apply
# ---------------------------------------------------------------------------
def shrink(x: torch.Tensor, segments: Segments, packed: PackedAdapters, z: torch.Tensor | None = None,
           partials_only: bool = False) -> torch.Tensor | None:
    """z[slot, s*r_g + j] = x[perm[slot]] . A_{g,s}[j] (compact, slot-major).

    ``partials_only``: when the module is one rank class whose hidden
    dimension is split (``shrink_ksplits``), write only the fp32 split-K
    partials to the per-device workspace (the shrink half of
    ``switched_lora_``) and return None; raises otherwise.
    """
    _require_cuda(x)
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    if x2.dtype != packed.dtype:
        raise TypeError("x and the packed adapters must share a dtype")
    T, H = x2.shape
    if H != packed.hidden or T != segments.num_tokens:
        raise ValueError("x shape does not match the segments / adapters")
    _check_segments(segments, packed)
    zw = packed.num_slices * packed.max_rank
    if partials_only:
        z = None
    elif z is None:
        z = torch.empty(max(T, 1), zw, dtype=x2.dtype, device=x2.device)
    elif z.dtype != x2.dtype or z.stride(-1) != 1 or z.dim() != 2 or z.shape[0] < T or z.shape[1] < zw:
        raise ValueError("z must be a [T, >= S*max_rank] buffer of x's dtype with unit column stride")
    ws = shrink_workspace(T, H, packed.num_slices, packed.num_adapters, packed.max_rank, x2.device, packed.ranks_host)
    _lib.call("gs_shrink", _dtype_code(x2), x2.data_ptr(), x2.stride(0), T, H, packed.a_pack.data_ptr(),
              packed.a_off.data_ptr(), packed.ranks.data_ptr(), packed.num_slices, packed.num_adapters,
              packed.max_rank, _i32_array(packed.ranks_host), segments.seg_offsets.data_ptr(),
              segments.perm.data_ptr(), _lib.ptr(z), zw if z is None else z.stride(0), ws.data_ptr(), ws.numel(),
              _lib.stream_ptr(x2.device))
    return z


def expand_add_(y: torch.Tensor, z: torch.Tensor, segments: Segments, packed: PackedAdapters) -> torch.Tensor:
    """y[perm[slot]] += z[slot] . B_g^T in place (rows of base tokens untouched)."""
    _require_cuda(y, z)
    if y.dtype != packed.dtype or z.dtype != packed.dtype:
        raise TypeError("y, z and the packed adapters must share a dtype")
    y2 = y.view(-1, y.shape[-1])
    if y2.stride(-1) != 1:
        raise ValueError("y must have unit column stride")
    T, O = y2.shape
    if O != packed.out_total or T != segments.num_tokens:
        raise ValueError("y shape does not match the segments / adapters")
    _check_segments(segments, packed)
    zw = packed.num_slices * packed.max_rank
    if z.dim() != 2 or z.stride(-1) != 1 or z.shape[0] < T or z.shape[1] < zw:
        raise ValueError("z must be a [T, >= S*max_rank] buffer with unit column stride")
    bounds = _i32_array(packed.slice_bounds)
    _lib.call("gs_expand_add", _dtype_code(y2), y2.data_ptr(), y2.stride(0), T, O, bounds, packed.num_slices,
              z.data_ptr(), z.stride(0), 0, None, packed.b_pack.data_ptr(), packed.b_off.data_ptr(),
              packed.ranks.data_ptr(), packed.num_adapters, packed.max_rank, _i32_array(packed.ranks_host),
              segments.seg_offsets.data_ptr(), segments.perm.data_ptr(), _lib.stream_ptr(y2.device))
    return y


def _xy2(x: torch.Tensor, y: torch.Tensor, packed: PackedAdapters):
    _require_cuda(x, y)
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    y2 = y.view(-1, y.shape[-1])
    if y2.stride(-1) != 1:
        raise ValueError("y must have unit column stride")
    if x2.dtype != packed.dtype or y2.dtype != packed.dtype:
        raise TypeError("x, y and the packed adapters must share a dtype")
    if x2.shape[1] != packed.hidden or y2.shape != (x2.shape[0], packed.out_total):
        raise ValueError("x / y shapes do not match the adapters")
    return x2, y2


def _call_small(x2, y2, packed, eff_ids=None, req=None, pos=None, cu=None, off=None, num_seqs=1, row_split=1):
    T = x2.shape[0]
    ws = small_workspace(x2.device, small_workspace_bytes(packed, T))
    sync = small_sync_buffer(x2.device)
    # issue every adapter's weight loads before the routing is known when most
    # adapters are likely to have tokens
    speculate = int(T >= 2 * packed.num_adapters)
    i64 = lambda v: (ctypes.c_int64 * len(v))(*[int(u) for u in v])
    _lib.call("gs_switched_lora_small", _dtype_code(x2), _lib.ptr(req), _lib.ptr(pos), _lib.ptr(cu), _lib.ptr(off),
              int(num_seqs), _lib.ptr(eff_ids), x2.data_ptr(), x2.stride(0), y2.data_ptr(), y2.stride(0), T,
              packed.hidden, packed.out_total, _i32_array(packed.slice_bounds), packed.num_slices,
              packed.a_pack.data_ptr(), i64(packed.a_off_host), packed.b_pack.data_ptr(), i64(packed.b_off_host),
              _i32_array(packed.ranks_host), packed.num_adapters, packed.max_rank, ws.data_ptr(), ws.numel(),
              sync.data_ptr(), sync.numel() * 4, int(row_split), speculate, _lib.stream_ptr(x2.device))
    if _CHECK_EACH_CALL and not torch.cuda.is_current_stream_capturing():
        check(x2.device)


def pair_launches(packed: PackedAdapters, num_tokens: int) -> bool:
    """True when gs_switched_lora runs this module's two rank classes in its
    pair launches (both classes in one shrink and one expand launch) for a
    batch of ``num_tokens``."""
    rc = _lib.load().gs_switched_lora_pair(_DTYPES[packed.dtype], int(num_tokens), packed.hidden,
                                           packed.out_total, _i32_array(packed.slice_bounds), packed.num_slices,
                                           packed.num_adapters, packed.max_rank, _i32_array(packed.ranks_host))
    if rc < 0:
        raise _lib.GraniteSwitchError("gs_switched_lora_pair", -rc, _lib.last_error())
    return rc == 1


def path_plan(packed: PackedAdapters, num_tokens: int, num_seqs: int | None = None,
              largest_group: int | None = None) -> str:
    """The kernels ``path="auto"`` runs for this module and batch: "small" (the
    one-launch kernel for every adapter), "split" (the one-launch kernel for
    the adapters of rank <= 64, the segment kernels for the larger ones) or
    "segments".  A module with a rank above 64 takes the segment kernels when
    they run its two classes in the pair launches (decode QKV with one
    rank-512 adapter among twelve rank-32 ones: 33.6 us against 39.5 us for
    "split")."""
    small_v, large_v = packed.rank_split()
    if small_v is None or not num_tokens or not small_preferred(small_v, num_tokens, num_seqs, largest_group):
        return "segments"
    if large_v is None:
        return "small"
    return "segments" if pair_launches(packed, num_tokens) else "split"


def switched_lora_routed_(y: torch.Tensor, x: torch.Tensor, adapter_ids: torch.Tensor, packed: PackedAdapters,
                          positions=None, cu_seqlens=None, act_offsets=None, path: str = "auto",
                          largest_group: int | None = None) -> torch.Tensor:
    """In place: y += switched-LoRA delta of x, routed straight from the per-token ids.

    ``adapter_ids`` / ``positions`` / ``cu_seqlens`` / ``act_offsets`` have the
    meaning of ``build_segments``.  ``path="auto"``: decode-sized batches
    (``small_preferred``) run in one launch that gates and groups the tokens
    itself; larger ones build segments first and run ``switched_lora_``.
    ``"small"`` / ``"segments"`` force one of the two.  The one-launch kernel
    takes the adapters of rank <= 64; a module that also holds larger ones
    runs those through segments built for them (``path_plan`` "split").
    ``largest_group`` (optional): the most tokens any one adapter has in the
    batch, when the caller knows it on the host; it replaces the path choice's
    estimate.
    """
    if path not in ("auto", "small", "segments"):
        raise ValueError(f"unknown path {path!r}")
    x2, y2 = _xy2(x, y, packed)
    dev = x2.device
    ids = _as_i64(adapter_ids.reshape(-1), dev)
    T = ids.shape[0]
    if T != x2.shape[0]:
        raise ValueError("adapter_ids must have one entry per token")
    pos = _as_i64(positions, dev)
    cu = _as_i32(cu_seqlens, dev)
    off = _as_i64(act_offsets, dev)
    if pos is not None and pos.numel() != T:
        raise ValueError("positions must have one entry per token")
    num_seqs = 1 if cu is None else cu.numel() - 1
    if off is not None and off.numel() != num_seqs:
        raise ValueError("act_offsets must have one entry per sequence")
    nseq_hint = num_seqs if cu is not None else None
    small_v, large_v = packed.rank_split()
    if path == "small" and small_v is None:
        raise ValueError("the one-launch kernel takes adapters of rank <= 64; this module has none")
    if path == "small" or (path == "auto" and path_plan(packed, T, nseq_hint, largest_group) != "segments"):
        if not small_eligible(small_v, T, num_seqs):
            raise ValueError("this module / batch is outside the small-batch kernel's limits")
        def small():
            _call_small(x2, y2, small_v, req=ids, pos=pos, cu=cu if off is not None else None, off=off,
                        num_seqs=num_seqs if off is not None else 1,
                        row_split=small_row_split(small_v, T, nseq_hint, largest_group))

        if large_v is None:
            small()
            return y

        def large():
            segs = build_segments(ids, packed.num_adapters, pos, cu, off)
            switched_lora_(y, x, segs, large_v, path="segments")

        _split_run(dev, large, small)
        return y
    segs = build_segments(ids, packed.num_adapters, pos, cu, off)
    return switched_lora_(y, x, segs, packed, path="segments")


def switched_lora_(y: torch.Tensor, x: torch.Tensor, segments: Segments, packed: PackedAdapters,
                   z: torch.Tensor | None = None, path: str = "auto", largest_group: int | None = None) -> torch.Tensor:
    """In place: y += switched-LoRA delta of x.

    ``path="auto"``: decode-sized batches (``small_preferred``) take the
    one-launch small-batch kernel, which groups tokens from
    ``segments.eff_ids`` itself; larger ones the two segment kernels.
    ``"small"`` / ``"segments"`` force one of the two.  The one-launch kernel
    takes the adapters of rank <= 64 and the segment kernels the rest
    (``path_plan`` "split").  The segment kernels run once per rank class
    (ranks <= 64 and above), each planned for its own largest rank.  On the
    segment path ``z`` is optional scratch [T, S*max_rank] of y's dtype
    (allocated when omitted) -- when the shrink is split over the hidden
    dimension the expand reads the fp32 partials from the workspace and z is
    not written.  ``largest_group`` as for ``switched_lora_routed_``.
    """
    if path not in ("auto", "small", "segments"):
        raise ValueError(f"unknown path {path!r}")
    x2, y2 = _xy2(x, y, packed)
    T, H = x2.shape
    if T != segments.num_tokens:
        raise ValueError("x / y shapes do not match the segments")
    _check_segments(segments, packed)
    if path != "segments" and T:
        small_v, large_v = packed.rank_split()
        if path == "small" and small_v is None:
            raise ValueError("the one-launch kernel takes adapters of rank <= 64; this module has none")
        if path == "small" or path_plan(packed, T, None, largest_group) != "segments":
            def small():
                _call_small(x2, y2, small_v, eff_ids=segments.eff_ids,
                            row_split=small_row_split(small_v, T, None, largest_group))

            if large_v is None:
                small()
                return y
            _split_run(x2.device, lambda: switched_lora_(y, x, segments, large_v, z, path="segments"), small)
            return y
    zw = packed.num_slices * packed.max_rank
    if z is None:
        z = torch.empty(max(T, 1), packed.num_slices * packed.max_rank, dtype=x2.dtype, device=x2.device)
    elif z.stride(-1) != 1 or z.shape[-1] < zw or (T and z.stride(0) != zw):
        raise ValueError("z must be a contiguous [T, S*max_rank] buffer")
    ws = shrink_workspace(T, H, packed.num_slices, packed.num_adapters, packed.max_rank, x2.device, packed.ranks_host)
    _lib.call("gs_switched_lora", _dtype_code(x2), x2.data_ptr(), x2.stride(0), y2.data_ptr(), y2.stride(0), T, H,
              packed.out_total, _i32_array(packed.slice_bounds), packed.num_slices, packed.a_pack.data_ptr(),
              packed.a_off.data_ptr(), packed.b_pack.data_ptr(), packed.b_off.data_ptr(), packed.ranks.data_ptr(),
              packed.num_adapters, packed.max_rank, _i32_array(packed.ranks_host), segments.seg_offsets.data_ptr(),
              segments.perm.data_ptr(), z.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(x2.device))
    return y


def switched_lora_noalloc_(y: torch.Tensor, x: torch.Tensor, segments: Segments, packed: PackedAdapters) -> torch.Tensor:
    """In place: y += switched-LoRA delta of x, allocating nothing.

    The segment path's two kernels (per rank class) with their scratch
    (split-K partials and the shrink output) in the library's static per-GPU
    array (``gs_switched_lora_noalloc``) -- for code that must not allocate,
    such as a region under HIP graph capture.  No tensor is created or copied
    here: x and y must already have unit column stride.  Shapes whose scratch
    would exceed the array (``_lib.GS_NOALLOC_SCRATCH_BYTES``) raise.  Calls
    that overlap in time on one GPU share the array and race.  The array is
    looked up on the first call on a device: make that call (or any call)
    eagerly before capturing one in a graph.
    """
    _require_cuda(x, y)
    if x.stride(-1) != 1 or y.stride(-1) != 1:
        raise ValueError("switched_lora_noalloc_: x and y need unit column stride (nothing is copied)")
    x2 = x.view(-1, x.shape[-1])
    y2 = y.view(-1, y.shape[-1])
    if x2.dtype != packed.dtype or y2.dtype != packed.dtype:
        raise TypeError("x, y and the packed adapters must share a dtype")
    if x2.shape[1] != packed.hidden or y2.shape != (x2.shape[0], packed.out_total):
        raise ValueError("x / y shapes do not match the adapters")
    T = x2.shape[0]
    if T != segments.num_tokens:
        raise ValueError("x / y shapes do not match the segments")
    _check_segments(segments, packed)
    _lib.call("gs_switched_lora_noalloc", _dtype_code(x2), x2.data_ptr(), x2.stride(0), y2.data_ptr(), y2.stride(0),
              T, packed.hidden, packed.out_total, _i32_array(packed.slice_bounds), packed.num_slices,
              packed.a_pack.data_ptr(), packed.a_off.data_ptr(), packed.b_pack.data_ptr(), packed.b_off.data_ptr(),
              packed.ranks.data_ptr(), packed.num_adapters, packed.max_rank, _i32_array(packed.ranks_host),
              segments.seg_offsets.data_ptr(), segments.perm.data_ptr(), _lib.stream_ptr(x2.device))
    return y


def _check_segments(segments: Segments, packed: PackedAdapters) -> None:
    """The kernels read seg_offsets[0..NA] and perm[0..T): both must match the pack."""
    if segments.num_adapters != packed.num_adapters or segments.seg_offsets.numel() != packed.num_adapters + 1:
        raise ValueError(f"segments were built for {segments.num_adapters} adapters, the pack holds "
                         f"{packed.num_adapters}")
    if segments.perm.numel() < segments.num_tokens:
        raise ValueError("segments.perm is shorter than the token count")


def _i32_array(vals):
    """Host int32 array for the C ABI's host-side table arguments."""
    return (ctypes.c_int32 * len(vals))(*[int(v) for v in vals])


def linear_bf16(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """out[M, N] = x[M, K] . w[N, K]^T in bf16 with fp32 accumulation (``gs_gemm_bf16_tn``).

    The vLLM layer's one GEMM, ``x_ext = x . w_ext^T``
    (src/granite_switch/vllm/core/lora.py:544).  ``x`` and ``w`` need
    unit-stride rows; ``out`` (allocated when omitted) may have a row stride.
    """
    _require_cuda(x, w)
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise ValueError("linear_bf16 takes bf16 operands")
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise ValueError(f"shapes {tuple(x.shape)} and {tuple(w.shape)} do not contract")
    if x.stride(1) != 1 or w.stride(1) != 1:
        raise ValueError("x and w need unit-stride rows")
    M, K = x.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=x.device)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (M, N) or (M and out.stride(1) != 1):
        raise ValueError("out must be a bf16 [M, N] tensor with unit-stride rows")
    _lib.call("gs_gemm_bf16_tn", x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), out.data_ptr(),
              out.stride(0) if M else N, M, N, K, _lib.stream_ptr(x.device))
    return out


def algorithmic_bytes(segments_host_ids, packed: PackedAdapters, true_ranks=None, elem_bytes: int = 2) -> int:
    """Bytes the op must move at minimum, for the roofline.

    x rows of active tokens + A and B of the adapters used (true rank) + read
    and write of the active y rows + 4 bytes per token id.  ``segments_host_ids``
    is the effective per-token id array on the host.
    """
    import numpy as np

    ids = np.asarray(segments_host_ids)
    S, H, O = packed.num_slices, packed.hidden, packed.out_total
    ranks = packed.ranks_host if true_ranks is None else [0] + list(true_ranks)
    act = ids[(ids > 0)]
    act = act[np.array([ranks[int(g)] > 0 for g in act], dtype=bool)] if act.size else act
    used = np.unique(act)
    rsum = sum(int(ranks[int(g)]) for g in used)
    t_act = int(act.size)
    return (t_act * H * elem_bytes + S * H * rsum * elem_bytes + O * rsum * elem_bytes
            + 2 * t_act * O * elem_bytes + 4 * ids.size)


def algorithmic_flops(segments_host_ids, packed: PackedAdapters, true_ranks=None) -> int:
    import numpy as np

    ids = np.asarray(segments_host_ids)
    S, H, O = packed.num_slices, packed.hidden, packed.out_total
    ranks = packed.ranks_host if true_ranks is None else [0] + list(true_ranks)
    tot = 0
    for g in ids[ids > 0]:
        r = int(ranks[int(g)])
        tot += 2 * H * S * r + 2 * r * O
    return int(tot)


__all__ = [
    "Segments",
    "PackedAdapters",
    "build_segments",
    "route_latest_wins",
    "shrink",
    "expand_add_",
    "switched_lora_",
    "switched_lora_routed_",
    "switched_lora_noalloc_",
    "small_eligible",
    "small_preferred",
    "path_plan",
    "shrink_ksplits",
    "small_workspace_bytes",
    "small_sync_buffer",
    "small_workspace",
    "reserve_small_workspace",
    "small_status",
    "SmallPathError",
    "check",
    "set_small_wait_limit",
    "pending_from_counters",
    "pending_from_sync",
    "small_pending_count",
    "small_reset",
    "shrink_workspace",
    "reserve_workspace",
    "algorithmic_bytes",
    "algorithmic_flops",
]
