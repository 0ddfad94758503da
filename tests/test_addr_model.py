"""CPU check of the segment kernels' memory accesses (no GPU needed).

Every hot loop of the kernels loads unconditionally from clamped addresses
and masks afterwards, so a wrong clamp is an out-of-bounds access.  The
library's address model (``gs_check_segment_addresses``) replays, on the host,
every global and LDS access of every launch a call makes -- every workgroup,
wave, lane and loop step -- with the launches' own plans and the kernels' own
address arithmetic (``csrc/gs_addr.h``, called by both), and reports any
access outside its buffer and any item a grid leaves uncovered.  This test
drives it at the benchmark shapes (the five workloads and the rank-512
population) and at the edge cases the GPU tests run: ragged and tiny
batches, one token, rank 8 to 512, odd hidden sizes, non-applicable
adapters, 64 and 256 adapters, and the vLLM layer's by-token form.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from granite_switch_amd import _lib, vllm_layers, workloads
from oracle import mapping as omap


def _pack_tables(ranks, S, H, O):
    """Host tables of PackedAdapters.from_slices: ranks rounded up to 8,
    adapter g's S*r rows of lora_A at a_off[g], its [O, r] lora_B at b_off[g]."""
    NA = len(ranks)
    r8 = [0] + [((int(r) + 7) // 8) * 8 if r > 0 else 0 for r in ranks]
    a_off, b_off = [0] * (NA + 1), [0] * (NA + 1)
    a = b = 0
    for g in range(1, NA + 1):
        if r8[g] == 0:
            continue
        a_off[g], b_off[g] = a, b
        a += S * r8[g] * H
        b += O * r8[g]
    return r8, a_off, b_off, max(a, 8 * H), max(b, 8 * O)


def _check(T, H, slices, ranks, eff, dtype=_lib.GS_DTYPE_BF16, ldx=None, ldy=None, z_off=None, z_ld=0, b_tables=None):
    NA = len(ranks)
    S, O = len(slices), int(sum(slices))
    r8, a_off, b_off, a_el, b_el = _pack_tables(ranks, S, H, O)
    if b_tables is not None:
        b_off, b_el = b_tables
    max_rank = max([8] + r8)
    seg, perm = omap.build_segments(np.asarray(eff, dtype=np.int64), NA)
    perm_full = np.zeros(max(T, 1), dtype=np.int32)
    perm_full[: len(perm)] = perm
    bounds = np.concatenate([[0], np.cumsum(slices)]).astype(np.int32)
    i32 = lambda v: (ctypes.c_int32 * len(v))(*[int(u) for u in v])
    i64 = lambda v: (ctypes.c_int64 * len(v))(*[int(u) for u in v])
    msg = ctypes.create_string_buffer(512)
    checked = ctypes.c_int64(0)
    bad = _lib.load().gs_check_segment_addresses(
        dtype, T, H, ldx or H, O, ldy or O, i32(bounds), S, i64(a_off), a_el, i64(b_off), b_el, i32(r8), NA, max_rank,
        i32(seg), i32(perm_full), None if z_off is None else i32(z_off), z_ld, msg, 512, ctypes.byref(checked))
    assert bad >= 0, f"bad arguments: {_lib.last_error()}"
    assert bad == 0, f"{bad} violations, first: {msg.value.decode()}"
    assert T == 0 or int((np.asarray(eff) > 0).sum()) == 0 or checked.value > 0
    return checked.value


def _eff(routing):
    return omap.alora_effective_ids(routing.req_ids, routing.positions, routing.cu_seqlens, routing.act_offsets)


@pytest.mark.parametrize("config", [0, 1, 2, 3, 4])
def test_benchmark_workloads(config):
    r = workloads.routing_for(config)
    eff = _eff(r)
    dt = _lib.GS_DTYPE_FP32 if config == 0 else _lib.GS_DTYPE_BF16
    for spec in workloads.module_specs(config):
        n = _check(r.num_tokens, spec.hidden, spec.output_slices, spec.ranks, eff, dt)
        print(f"config {config} {spec.name}: {n} accesses checked")


@pytest.mark.parametrize("config", [1, 4])
def test_rank512_population(config):
    r = workloads.population_routing(config, "r512")
    eff = _eff(r)
    for spec in workloads.population_specs(config, "r512"):
        _check(r.num_tokens, spec.hidden, spec.output_slices, spec.ranks, eff)


def test_rank512_population_with_a_prefill_chunk_on_the_large_adapter():
    """The large class holding far more tokens than expected: its looping
    grids must still cover every item."""
    r = workloads.population_routing(4, "r512")
    req = r.req_ids.copy()
    req[48:48 + 3 * 256] = 25                      # three prefill chunks on the rank-512 adapter
    eff = omap.alora_effective_ids(req, r.positions, r.cu_seqlens, r.act_offsets)
    for spec in workloads.population_specs(4, "r512"):
        _check(r.num_tokens, spec.hidden, spec.output_slices, spec.ranks, eff)


@pytest.mark.parametrize("large", [72, 96, 128, 200, 256, 512])
@pytest.mark.parametrize("T", [1, 64, 600, 4144])
def test_pair_launches_every_large_rank(large, T):
    """Two classes in the pair launches (gs_switched_lora_pair says so) at
    every k-group count of the large class's 64-column items (2, 4 and 8 per
    wave), odd large ranks, one token to a decoder-step batch: the replay of
    the pair shrink (large items on a stride of the small class's grid), the
    pair expand (claimed items) and the counter line."""
    slices = (2048, 1024, 1024)
    ranks = [32] * 24 + [large]                    # the large class sparse (its tokens expected: T / 26)
    rng = np.random.default_rng(large + T)
    eff = rng.integers(0, len(ranks) + 1, size=T)
    from test_library import _pair_query
    assert _pair_query(_lib.GS_DTYPE_BF16, T, 4096, slices, ranks) == 1
    _check(T, 4096, slices, ranks, eff)


EDGE = [
    # T, H, slices, ranks, seed, share of base tokens
    (1, 4096, (4096, 1024, 1024), [32] * 12, 0, 0.0),
    (7, 256, (128, 64), [8, 16, 32], 1, 0.2),
    (96, 256, (128, 64), [8, 16, 32], 2, 0.3),
    (300, 1000, (96, 32), [8, 24, 40], 3, 0.2),                  # H not a multiple of 64: register shrink
    (130, 520, (64,), [512, 8], 4, 0.1),
    (1100, 2048, (512, 256), [8, 16, 32, 64, 128, 16], 5, 0.2),
    (2048, 1024, (512, 256), [32, 8, 512, 64, 128, 16, 32, 256], 6, 0.1),
    (64, 4096, (4096,), [64] * 64, 7, 0.1),                       # every limit of the one-launch path
    (5000, 512, (256,), [8] * 256, 8, 0.0),                      # 256 adapters: the multi-pass tile lookup
    (4096, 12800, (4096,), [(8, 16, 32, 64)[a % 4] for a in range(48)], 9, 0.15),
    (200, 1024, (1024,), [128, 512], 10, 0.3),                    # large class only
    (400, 4096, (4096, 1024, 1024), [32] * 6 + [512], 11, 0.1),
]


@pytest.mark.parametrize("T,H,slices,ranks,seed,base", EDGE)
def test_edge_shapes(T, H, slices, ranks, seed, base):
    rng = np.random.default_rng(seed)
    NA = len(ranks)
    eff = rng.integers(1, NA + 1, size=T)
    eff[rng.random(T) < base] = 0
    for dt in (_lib.GS_DTYPE_BF16, _lib.GS_DTYPE_FP32):
        if dt == _lib.GS_DTYPE_FP32 and len(slices) * max(ranks) > 512:
            continue                                          # refused by the fp32 expand's LDS limit
        _check(T, H, slices, ranks, eff, dt)
    # a row stride wider than the row, and an all-base batch
    _check(T, H, slices, ranks, eff, ldx=H + 64, ldy=int(sum(slices)) + 32)
    _check(T, H, slices, ranks, np.zeros(T, dtype=np.int64))


def test_non_applicable_adapter_and_empty_batch():
    _check(0, 256, (128,), [16, 16], np.zeros(0, dtype=np.int64))
    eff = np.array([1, 2, 2, 0, 1, 3, 3, 3] * 20)
    _check(len(eff), 512, (256, 128), [32, 0, 16], eff)           # adapter 2 is not applicable here


def test_vllm_layer_reads_shrink_values_by_token():
    """The vLLM layer's segment expand reads each row's shrink values from
    x_ext by token, at the columns its fusion plan gives each adapter."""
    K, slices, ranks = 256, (256, 128, 128), [16, 512, 8, 32]
    base = torch.nn.Linear(K, sum(slices), bias=False)
    layer = vllm_layers.SwitchedLoRALinear(base, len(ranks), max(ranks), num_slices=3, output_slices=slices)
    with torch.no_grad():
        for A in layer.lora_A_slices:
            A.data.normal_()
    layer.finalize_weights(ranks)
    # the layer's own segment tables: promoted (tier) ranks, lora_B blocks in
    # lb_packed, first shrink column of each adapter in x_ext
    seg_rank = layer._seg_ranks.tolist()[1:]
    b_tables = (layer._seg_boff.tolist(), layer._lb_packed.numel())
    x_ext_cols = layer.w_ext.shape[0]
    rng = np.random.default_rng(3)
    for T in (100, 1500):
        eff = rng.integers(0, len(ranks) + 1, size=T)
        _check(T, K, slices, seg_rank, eff, z_off=layer._seg_zoff.tolist(), z_ld=x_ext_cols, b_tables=b_tables)


def test_model_catches_a_planted_out_of_range_table():
    """The model reports accesses outside their buffers: a lora_B offset that
    puts the last adapter's block past the end of the pack is caught."""
    T, H, slices, ranks = 64, 256, (128,), [16, 16]
    S, O = 1, 128
    r8, a_off, b_off, a_el, b_el = _pack_tables(ranks, S, H, O)
    eff = np.array([1, 2] * 32)
    seg, perm = omap.build_segments(eff, 2)
    i32 = lambda v: (ctypes.c_int32 * len(v))(*[int(u) for u in v])
    i64 = lambda v: (ctypes.c_int64 * len(v))(*[int(u) for u in v])
    msg = ctypes.create_string_buffer(512)
    checked = ctypes.c_int64(0)
    b_off_bad = list(b_off)
    b_off_bad[2] += O * 8                                          # half a block past the end
    bad = _lib.load().gs_check_segment_addresses(
        _lib.GS_DTYPE_BF16, T, H, H, O, O, i32([0, O]), S, i64(a_off), a_el, i64(b_off_bad), b_el, i32(r8), 2, 16,
        i32(seg), i32(perm), None, 0, msg, 512, ctypes.byref(checked))
    assert bad > 0 and "lora_B" in msg.value.decode()


# ---- the one-launch small-batch kernel (gs_check_small_addresses) ----------

def _check_small(T, H, slices, ranks, eff, dtype=_lib.GS_DTYPE_BF16, row_split=1, route_flags=1, num_seqs=1,
                 ldx=None, ldy=None):
    S, O = len(slices), int(sum(slices))
    r8, a_off, b_off, a_el, b_el = _pack_tables(ranks, S, H, O)
    NA = len(ranks)
    max_rank = max([8] + r8)
    bounds = np.concatenate([[0], np.cumsum(slices)]).astype(np.int32)
    i32 = lambda v: (ctypes.c_int32 * len(v))(*[int(u) for u in v])
    i64 = lambda v: (ctypes.c_int64 * len(v))(*[int(u) for u in v])
    msg = ctypes.create_string_buffer(512)
    checked = ctypes.c_int64(0)
    bad = _lib.load().gs_check_small_addresses(
        dtype, T, H, ldx or H, O, ldy or O, i32(bounds), S, i64(a_off), a_el, i64(b_off), b_el, i32(r8), NA, max_rank,
        i32(np.asarray(eff).tolist() or [0]), num_seqs, route_flags, row_split, msg, 512, ctypes.byref(checked))
    assert bad >= 0, f"bad arguments: {_lib.last_error()}"
    assert bad == 0, f"{bad} violations, first: {msg.value.decode()}"
    return checked.value


@pytest.mark.parametrize("config", [0, 1])
def test_small_kernel_benchmark_workloads(config):
    r = workloads.routing_for(config)
    eff = _eff(r)
    dt = _lib.GS_DTYPE_FP32 if config == 0 else _lib.GS_DTYPE_BF16
    for spec in workloads.module_specs(config):
        for flags in (1, 2 | 4 | 8):          # pre-gated ids; the request with positions, sequences, offsets
            n = _check_small(r.num_tokens, spec.hidden, spec.output_slices, spec.ranks, eff, dt, route_flags=flags,
                             num_seqs=len(r.cu_seqlens) - 1)
        print(f"small kernel, config {config} {spec.name}: {n} accesses checked")


SMALL = [
    # T, H, slices, ranks, seed, row splits
    (1000, 1024, (256, 128), [16, 64, 8], 1, (1, 2, 3, 8, 32)),
    (333, 1000, (128,), [8, 24, 40, 64, 16], 2, (1,)),
    (7, 4096, (128, 128, 256), [32, 32], 3, (1,)),
    (1024, 512, (256,), [32] * 64, 4, (1, 2, 32)),
    (512, 2048, (2048,), [8, 8, 8, 8], 62, (1, 4, 16)),
    (1024, 1024, (2560, 2560), [32] * 64, 70, (1, 2, 4)),           # tile groups
    (256, 4096, (4096, 1024, 1024), [32] * 12, 5, (1, 2)),          # decode QKV
    (1, 4096, (4096,), [64] * 3, 6, (1,)),
]


@pytest.mark.parametrize("T,H,slices,ranks,seed,splits", SMALL)
def test_small_kernel_shapes(T, H, slices, ranks, seed, splits):
    rng = np.random.default_rng(seed)
    NA = len(ranks)
    eff = rng.integers(0, NA + 1, size=T)
    if T >= 128:
        runs = np.repeat(rng.integers(0, NA + 1, size=T // 256 + 1), 128)      # runs of 128 tokens
        eff[: T // 2] = runs[: T // 2] if len(runs) >= T // 2 else np.resize(runs, T // 2)
    for dt in (_lib.GS_DTYPE_BF16, _lib.GS_DTYPE_FP32):
        for rs in splits:
            _check_small(T, H, slices, ranks, eff, dt, row_split=rs)
    _check_small(T, H, slices, ranks, eff, ldx=H + 64, ldy=int(sum(slices)) + 128)
    _check_small(T, H, slices, ranks, np.zeros(T, dtype=np.int64))
    if T > 1:
        _check_small(T, H, slices, ranks, eff, route_flags=2 | 4 | 8, num_seqs=min(T, 40))


def test_small_kernel_model_catches_a_short_lora_B_pack():
    """A lora_B pack one adapter block short is reported."""
    T, H, slices, ranks = 64, 256, (128,), [16, 16]
    S, O = 1, 128
    r8, a_off, b_off, a_el, b_el = _pack_tables(ranks, S, H, O)
    i32 = lambda v: (ctypes.c_int32 * len(v))(*[int(u) for u in v])
    i64 = lambda v: (ctypes.c_int64 * len(v))(*[int(u) for u in v])
    msg = ctypes.create_string_buffer(512)
    checked = ctypes.c_int64(0)
    eff = [1, 2] * 32
    bad = _lib.load().gs_check_small_addresses(
        _lib.GS_DTYPE_BF16, T, H, H, O, O, i32([0, O]), S, i64(a_off), a_el, i64(b_off), b_el - O * 16, i32(r8), 2, 16,
        i32(eff), 1, 1, 1, msg, 512, ctypes.byref(checked))
    assert bad > 0 and "lora_B" in msg.value.decode()


# ---- the segment builder (gs_check_build_addresses) ------------------------

def _check_build(req, NA, pos=None, cu=None, act=None, two_launch=False):
    T = len(req)
    arr = lambda a, dt: None if a is None else np.ascontiguousarray(a, dtype=dt)
    req_a, pos_a, cu_a, act_a = arr(req, np.int64), arr(pos, np.int64), arr(cu, np.int32), arr(act, np.int64)
    ptr = lambda a: None if a is None or a.size == 0 else a.ctypes.data
    msg = ctypes.create_string_buffer(512)
    checked = ctypes.c_int64(0)
    nseq = len(cu) - 1 if cu is not None else 1
    bad = _lib.load().gs_check_build_addresses(T, nseq, NA, ptr(req_a), ptr(pos_a), ptr(cu_a), ptr(act_a),
                                               int(two_launch), msg, 512, ctypes.byref(checked))
    assert bad >= 0, f"bad arguments: {_lib.last_error()}"
    assert bad == 0, f"{bad} violations, first: {msg.value.decode()}"
    return checked.value


@pytest.mark.parametrize("config", [0, 1, 2, 3, 4])
def test_builder_benchmark_workloads(config):
    r = workloads.routing_for(config)
    NA = workloads.num_adapters_for(config)
    for two in (False, True):
        _check_build(r.req_ids, NA, r.positions, r.cu_seqlens, r.act_offsets, two_launch=two)


@pytest.mark.parametrize("T,NA,seed", [(0, 4, 0), (1, 1, 1), (63, 3, 2), (1023, 7, 3), (1024, 64, 4), (1025, 255, 5),
                                       (5000, 256, 6), (65536, 24, 7)])
def test_builder_random_batches(T, NA, seed):
    """The GPU builder tests' batches: out-of-range ids, packed sequences with
    cached prefixes, activation offsets; with and without positions and
    sequences, both forms."""
    rng = np.random.default_rng(seed)
    req = rng.integers(-3, NA + 4, size=T)
    nseq = max(1, T // 50)
    cuts = np.sort(rng.choice(np.arange(1, T), size=min(nseq - 1, max(T - 1, 0)), replace=False)) if T > 1 else []
    cu = np.concatenate([[0], cuts, [T]]).astype(np.int32)
    lens = np.diff(cu)
    cached = rng.integers(0, 100, size=lens.size)
    pos = np.concatenate([c + np.arange(n) for c, n in zip(cached, lens)]) if T else np.zeros(0, np.int64)
    offs = rng.integers(0, 160, size=lens.size)
    for two in (False, True):
        _check_build(req, NA, pos, cu, offs, two_launch=two)
        _check_build(req, NA, None, cu, offs, two_launch=two)
        _check_build(req, NA, two_launch=two)
    if T > 1:                                     # more sequences than the LDS table holds
        cu2 = np.arange(0, T + 1, dtype=np.int32)
        _check_build(req, NA, None, cu2, rng.integers(0, 2, size=T), two_launch=T > 2048)


# ---- the layer GEMM (gs_check_gemm_addresses) -------------------------------

@pytest.mark.parametrize("M,N,K,pad", [
    (1, 7296, 4096, 0),            # one token
    (256, 7296, 4096, 0),          # decode QKV x . w_ext^T
    (300, 1000, 72, 0),            # K not a multiple of 64 (register-staged, zero-filled tail), ragged tiles
    (4144, 4864, 1024, 8),         # step down-projection shape at a shorter K, padded strides
    (257, 257, 512, 64),
    (1100, 3000, 8, 0),
])
def test_gemm_shapes(M, N, K, pad):
    msg = ctypes.create_string_buffer(512)
    checked = ctypes.c_int64(0)
    bad = _lib.load().gs_check_gemm_addresses(M, N, K, K + pad, K + pad, N + pad, msg, 512, ctypes.byref(checked))
    assert bad >= 0, f"bad arguments: {_lib.last_error()}"
    assert bad == 0, f"{bad} violations, first: {msg.value.decode()}"
    assert checked.value > 0


# ---- latest-wins routing, bitmasks, probe split (gs_check_token_addresses) ---

@pytest.mark.parametrize("T,nseq,NA,modules,block_m,seed", [
    (1, 1, 1, 1, 32, 0), (700, 40, 6, 4, 32, 1), (5000, 1, 64, 128, 32, 2), (333, 7, 10, 3, 24, 3),
    (1024, 1024, 255, 2, 1, 4), (4144, 304, 24, 128, 64, 5)])
def test_token_kernels(T, nseq, NA, modules, block_m, seed):
    rng = np.random.default_rng(seed)
    ids = rng.integers(-2, NA + 3, size=T).astype(np.int64)     # includes out-of-range ids
    cuts = np.sort(rng.choice(np.arange(1, T), size=min(nseq - 1, T - 1), replace=False)) if T > 1 else []
    cu = np.concatenate([[0], cuts, [T]]).astype(np.int32)
    msg = ctypes.create_string_buffer(512)
    checked = ctypes.c_int64(0)
    for with_cu in (True, False):
        bad = _lib.load().gs_check_token_addresses(
            T, len(cu) - 1, cu.ctypes.data if with_cu else None, min(NA + 1, 257), ids.ctypes.data, NA + 1, modules,
            block_m, min(NA + 1, 257), msg, 512, ctypes.byref(checked))
        assert bad == 0, f"{bad} violations, first: {msg.value.decode()}"
        assert checked.value > 0
