"""CPU check of the memory accesses of the reference-semantics ops over x_ext
(no GPU needed).

``gs_check_xext_addresses`` replays, on the host, every global and LDS access
of ``gs_switch_lora_expand`` (the column-block form the device would take,
every other column-block shape, and the per-tile forms),
``gs_switch_lora_shrink_expand`` (W-less, bf16 and fp32 output) and
``gs_switch_lora_expand_swiglu`` -- every workgroup, wave, lane and loop
step, with the kernels' own address arithmetic (``csrc/gs_addr.h``) -- and
reports any access outside its buffer.  The tables are the reference's, built
by the oracle's restatement of the layer's finalize step and of the bitmask
kernel (``finalize_tables``, ``compute_bitmasks``): the shapes of the GPU op
tests plus the decode and decoder-step projections.  The column-block
expand's idle waves once read past the end of x_ext on the GPU; its case (a
ragged last row group) is here.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from granite_switch_amd import _lib
from oracle import mapping as omap

RANKS = omap.SUPPORTED_RANKS


def _tables(slices, ranks, ids, block_n=32, wless=False):
    """The layer's tables for these adapters, and the per-token kernel-local
    ids and tile masks of the batch ``ids`` (global ids, 0 = base)."""
    NA = len(ranks)
    remap, order, eff = omap.build_remap([True] * NA, ranks)
    na, t2s, scr, _ = omap.finalize_tables(slices, order, eff, block_n)
    S, N = len(slices), int(sum(slices))
    shrink_cols = sum(na[t] * S * r for t, r in enumerate(RANKS))
    scr = np.asarray(scr, dtype=np.int32)
    if wless:                      # the cross weight has no base rows: shrink columns start at 0
        scr = scr - N
    x_cols = shrink_cols if wless else N + shrink_cols
    lb = sum(na[t] * N * r for t, r in enumerate(RANKS))
    loc = omap.remapped_indices(np.asarray(ids), remap[:, None])[0].astype(np.int64)
    bm = omap.compute_bitmasks(np.asarray(ids), remap[:, None])[0].astype(np.int64)
    return dict(na=np.asarray(na, dtype=np.int32), t2s=np.asarray(t2s, dtype=np.int32), scr=scr.reshape(-1),
                S=S, N=N, x_cols=x_cols, lb=max(lb, 8), loc=loc, bm=bm)


def _check(op, d, idx_bytes=8, H=0, stride_om=0, out_dtype=_lib.GS_DTYPE_BF16, stride_pad=0, block_n=32):
    M = len(d["loc"])
    msg = ctypes.create_string_buffer(512)
    checked = ctypes.c_int64(0)
    i64 = lambda a: np.ascontiguousarray(a, dtype=np.int64)
    loc, bm = i64(d["loc"]), i64(d["bm"])
    t2s, scr, na = (np.ascontiguousarray(d[k], dtype=np.int32) for k in ("t2s", "scr", "na"))
    bad = _lib.load().gs_check_xext_addresses(
        op, M, d["x_cols"] + stride_pad, d["x_cols"], loc.ctypes.data, idx_bytes, bm.ctypes.data, 1, len(bm), d["lb"],
        t2s.ctypes.data, len(t2s), scr.ctypes.data, na.ctypes.data, d["S"], block_n, d["N"], H, stride_om, out_dtype,
        msg, 512, ctypes.byref(checked))
    assert bad >= 0, f"bad arguments: {_lib.last_error()}"
    assert bad == 0, f"{bad} violations, first: {msg.value.decode()}"
    return checked.value


def _ids(T, NA, seed, base_run=True):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, NA + 1, size=T)
    if base_run:
        ids[T // 3: T // 3 + 40] = 0          # an all-base tile
    return ids


# the GPU op tests' shapes (slices, ranks, T) and the workload projections
EXPAND = [
    ((256, 128, 128), [16, 32, 16, 64, 8], 200),
    ((4096, 96), [32, 16, 32, 8], 1000),
    ((512,), [64, 16, 64], 700),
    ((4096, 1024, 1024), [32, 16, 32, 8], 300),
    ((4096, 2048), [64, 16, 8], 400),
    ((256, 128), [128, 16], 300),
    ((1024, 256), [32, 16, 8], 1500),
    ((1024, 32), [32, 16], 1100),
    ((1024, 32), [32, 16], 600),
    ((4096, 1024, 1024), [32] * 12, 256),              # decode QKV
    ((4096, 1024, 1024), [32] * 12 + [512], 256),      # decode QKV with a rank-512 adapter
    ((4096, 1024, 1024), [8, 16, 32, 64] * 6, 4144),    # decoder-step QKV
    ((4096,), [(8, 16, 32, 64)[a % 4] for a in range(48)], 4096),   # multi-switch down projection
    ((128,), [16, 16], 1),
    ((128,), [16, 16], 33),
]


@pytest.mark.parametrize("slices,ranks,T", EXPAND)
def test_expand_op(slices, ranks, T):
    d = _tables(slices, ranks, _ids(T, len(ranks), T))
    for idx_bytes in (8, 4):
        n = _check(0, d, idx_bytes)
    _check(0, d, 8, stride_pad=64)
    print(f"expand {slices} ranks {sorted(set(ranks))} T={T}: {n} accesses")


def test_expand_op_runs_of_adapters():
    """20 adapters in runs (more than one staging chunk of the column-block form)."""
    ranks = [16, 32] * 10
    order = [19, 3, 17, 0, 18, 20, 9, 16, 2, 20, 13, 1, 19, 18, 11, 17, 20, 4]
    for slices, T in (((4096, 96), 1000), ((512,), 700), ((2048, 1024), 500)):
        ids = np.array([order[(m // 57) % len(order)] for m in range(T)])
        _check(0, _tables(slices, ranks, ids))


def test_expand_op_64_adapters_and_all_base():
    ranks = [(16, 32, 64)[a % 3] for a in range(64)]
    _check(0, _tables((1024, 512), ranks, _ids(900, 64, 5)))
    _check(0, _tables((1024, 512), ranks, np.zeros(300, dtype=np.int64)))


WLESS = [
    ((64,), (16,), [0, 1] * 20),
    ((64,), (16,), [0] * 32),
    ((128,), (16, 32), [0, 1, 2, 2, 0, 1] * 8),
    ((4096,), (16, 32, 64, 128), [3] * 5 + [0] * 40 + [1, 2, 4] * 11),
    ((128,), (32, 64), [0, 1, 2, 2, 1, 0] * 8),
    ((128,), (16, 32), ([0, 1, 1, 2, 2, 2, 0] * 158)[:1100]),
]


@pytest.mark.parametrize("slices,ranks,ids", WLESS)
def test_shrink_expand_op(slices, ranks, ids):
    d = _tables(slices, list(ranks), np.asarray(ids), wless=True)
    N = d["N"]
    for out_dtype in (_lib.GS_DTYPE_BF16, _lib.GS_DTYPE_FP32):
        _check(1, d, stride_om=N, out_dtype=out_dtype)
    _check(1, d, stride_om=N + 32)                      # a wider output, as the tests' larger buffer


SWIGLU = [
    (128, [16, 32], 300),
    (128, [16, 32, 64], 1500),
    (256, [128, 16], 200),
    (12800, [8, 16, 32, 64] * 6, 256),                  # decode gate_up
    (12800, [8, 16, 32, 64] * 6, 2100),                 # past 1024 rows
]


@pytest.mark.parametrize("H,ranks,T", SWIGLU)
def test_swiglu_op(H, ranks, T):
    d = _tables((H, H), ranks, _ids(T, len(ranks), H + T))
    for idx_bytes in (8, 4):
        _check(2, d, idx_bytes, H=H, stride_om=H)


def test_model_catches_a_shrink_column_table_past_x_ext():
    """A slice table whose bases run past the end of x_ext is reported."""
    d = _tables((256,), [16, 32], _ids(200, 2, 1))
    d["scr"] = d["scr"] + 64
    msg = ctypes.create_string_buffer(512)
    checked = ctypes.c_int64(0)
    loc, bm = d["loc"].astype(np.int64), d["bm"].astype(np.int64)
    t2s, scr, na = (np.ascontiguousarray(d[k], dtype=np.int32) for k in ("t2s", "scr", "na"))
    bad = _lib.load().gs_check_xext_addresses(0, len(loc), d["x_cols"], d["x_cols"], loc.ctypes.data, 8,
                                              bm.ctypes.data, 1, len(bm), d["lb"], t2s.ctypes.data, len(t2s),
                                              scr.ctypes.data, na.ctypes.data, d["S"], 32, d["N"], 0, 0, 0, msg, 512,
                                              ctypes.byref(checked))
    assert bad > 0 and "x_ext" in msg.value.decode(), msg.value.decode()
