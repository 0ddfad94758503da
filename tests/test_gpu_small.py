"""GPU parity of the one-launch small-batch (decode) path.

The small path groups tokens inside its kernel, either from pre-gated ids
(``switched_lora_`` with segments) or from the raw routing
(``switched_lora_routed_``: requested ids + positions + sequence boundaries +
aLoRA offsets).  Checked against the CPU oracle at the target tolerance
(bf16 |got - ref| <= 2e-2 + 2e-2*|ref|, fp32 1e-5 + 1e-5*|ref|, ``ref`` the
float64 math rounded once), against the segment path, and for bit-identical
base rows.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from granite_switch_amd import switched, workloads
from oracle import lora as olora
from oracle import mapping as omap

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 2e-2, torch.float32: 1e-5}


def _say(msg):
    print(msg, flush=True)


def _np(t):
    return t.detach().float().cpu().numpy()


def _close(got, ref, tol, what):
    err = np.abs(np.asarray(got, np.float64) - ref)
    bad = err > tol + tol * np.abs(ref)
    assert not bad.any(), f"{what}: {int(bad.sum())} elements out of tolerance, max abs err {err.max():.3e}"


def _oracle(md, eff, dtype, mode="exact"):
    dt = "bf16" if dtype == torch.bfloat16 else "fp32"
    return olora.switched_lora_apply(_np(md.y), _np(md.x), eff, [_np(a) for a in md.lora_A_slices],
                                     [_np(b) for b in md.lora_B_slices], md.spec.output_slices, md.spec.ranks, dt,
                                     mode)


@pytest.fixture(autouse=True)
def _clean_handoff(dev):
    """Every test ends with the error word clear and no launch half-counted."""
    switched.small_reset(dev)
    yield
    torch.cuda.synchronize()
    assert switched.small_status(dev) == 0, f"small-path error word {switched.small_status(dev)}"
    assert switched.small_pending_count(dev) == 0, "a launch was left half counted in an adapter's launch counter"


def _check(md, y, eff, dtype):
    ref = _oracle(md, eff, dtype)
    _close(_np(y), ref, TOL[dtype], "small path vs oracle")
    base = eff == 0
    assert np.array_equal(_np(y)[base], _np(md.y)[base]), "base rows were modified"


@pytest.mark.parametrize("config", [0, 1])
def test_small_routed_configs(dev, config):
    """Configs 0 and 1 from the raw routing (gating inside the kernels)."""
    wl = workloads.make_workload(config, dev)
    md, r = wl.modules[0], wl.routing
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, md.spec.ranks)
    assert switched.small_eligible(pk, r.num_tokens, len(r.cu_seqlens) - 1)
    _say(f"small routed config={config} T={r.num_tokens}")
    y = md.y.clone()
    switched.switched_lora_routed_(y, md.x, torch.tensor(r.req_ids, device=dev), pk,
                                   torch.tensor(r.positions, device=dev), torch.tensor(r.cu_seqlens, device=dev),
                                   torch.tensor(r.act_offsets, device=dev), path="small")
    torch.cuda.synchronize()
    eff = omap.alora_effective_ids(r.req_ids, r.positions, r.cu_seqlens, r.act_offsets)
    _check(md, y, eff, wl.dtype)
    # the HF loop's own rounding sequence too
    _close(_np(y), _oracle(md, eff, wl.dtype, "hf"), TOL[wl.dtype], "small path vs HF-rounding oracle")


@pytest.mark.parametrize("config", [0, 1])
def test_small_matches_segment_path(dev, config):
    """Small path (eff ids from the builder) vs the segment path on the same inputs."""
    wl = workloads.make_workload(config, dev)
    md, r = wl.modules[0], wl.routing
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, md.spec.ranks)
    segs = switched.build_segments(torch.tensor(r.req_ids, device=dev), wl.num_adapters,
                                   torch.tensor(r.positions, device=dev), torch.tensor(r.cu_seqlens, device=dev),
                                   torch.tensor(r.act_offsets, device=dev))
    y_small = md.y.clone()
    y_seg = md.y.clone()
    switched.switched_lora_(y_small, md.x, segs, pk, path="small")
    switched.switched_lora_(y_seg, md.x, segs, pk, path="segments")
    torch.cuda.synchronize()
    eff = segs.eff_ids.cpu().numpy()
    _check(md, y_small, eff, wl.dtype)
    _check(md, y_seg, eff, wl.dtype)
    # both round one fp32 delta per element; split-K orders differ, so allow 1 ulp of the output
    d = (y_small.float() - y_seg.float()).abs()
    ulp = 2.0 ** -7 if wl.dtype == torch.bfloat16 else 2.0 ** -20
    assert bool((d <= ulp * y_seg.float().abs().clamp_min(1.0)).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,NA,ranks,slices,H,seed", [
    (1000, 3, [16, 64, 8], (256, 128), 1024, 1),        # ~250 tokens per adapter: 8 row tiles each
    (333, 5, [8, 24, 40, 64, 16], (128,), 1000, 2),     # ranks not multiples of 16, H not a k-chunk multiple
    (7, 2, [32, 32], (128, 128, 256), 4096, 3),         # tiny batch
    (1024, 64, [32] * 64, (256,), 512, 4),              # every limit at once
])
def test_small_shapes(dev, dtype, T, NA, ranks, slices, H, seed):
    spec = workloads.ModuleSpec("t", H, slices, ranks, max(ranks))
    md = workloads.make_module(spec, T, NA, dtype, dev, seed=seed)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, ranks)
    assert switched.small_eligible(pk, T)
    rng = np.random.default_rng(seed)
    ids = rng.integers(-1, NA + 2, size=T)           # includes out-of-range ids (-> base)
    _say(f"small shapes dtype={dtype} T={T} NA={NA} ranks={ranks[:6]} slices={slices} H={H}")
    y = md.y.clone()
    switched.switched_lora_routed_(y, md.x, torch.tensor(ids, device=dev), pk, path="small")
    torch.cuda.synchronize()
    eff = np.where((ids < 0) | (ids > NA), 0, ids)
    _check(md, y, eff, dtype)


def test_small_ragged_gating_and_nonapplicable(dev):
    """Packed ragged sequences, cached prefixes (absolute positions), an adapter that is not applicable."""
    T, NA = 700, 6
    spec = workloads.ModuleSpec("t", 768, (384, 128), [16, 32, 8, 64, 24, 40], 64)
    md = workloads.make_module(spec, T, NA, torch.bfloat16, dev, seed=21)
    for A in md.lora_A_slices:
        A[2].zero_()                                  # adapter 3 not applicable here
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks)
    assert pk.ranks_host[3] == 0
    rng = np.random.default_rng(21)
    cuts = np.sort(rng.choice(np.arange(1, T), size=39, replace=False))
    cu = np.concatenate([[0], cuts, [T]]).astype(np.int32)
    lens = np.diff(cu)
    cached = rng.integers(0, 300, size=lens.size)
    pos = np.concatenate([c + np.arange(n) for c, n in zip(cached, lens)]).astype(np.int64)
    offs = rng.integers(0, 400, size=lens.size).astype(np.int64)
    req = rng.integers(0, NA + 1, size=T)
    for with_pos in (True, False):
        y = md.y.clone()
        switched.switched_lora_routed_(y, md.x, torch.tensor(req, device=dev), pk,
                                       torch.tensor(pos, device=dev) if with_pos else None,
                                       torch.tensor(cu, device=dev), torch.tensor(offs, device=dev), path="small")
        torch.cuda.synchronize()
        eff = omap.alora_effective_ids(req, pos if with_pos else None, cu, offs)
        eff[eff == 3] = 0                             # non-applicable -> base, as the reference remaps it
        _say(f"ragged gating with_pos={with_pos}: active {int((eff > 0).sum())}")
        _check(md, y, eff, torch.bfloat16)


def test_small_all_base_and_no_tokens_for_some_adapters(dev):
    spec = workloads.ModuleSpec("t", 512, (256,), [16, 16, 16], 16)
    md = workloads.make_module(spec, 90, 3, torch.bfloat16, dev, seed=5)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks)
    y = md.y.clone()
    switched.switched_lora_routed_(y, md.x, torch.zeros(90, dtype=torch.int64, device=dev), pk, path="small")
    torch.cuda.synchronize()
    assert torch.equal(y, md.y)
    ids = np.where(np.arange(90) % 3 == 0, 2, 0)     # only adapter 2 present
    y = md.y.clone()
    switched.switched_lora_routed_(y, md.x, torch.tensor(ids, device=dev), pk, path="small")
    torch.cuda.synchronize()
    _check(md, y, ids, torch.bfloat16)
    # no tokens at all: nothing to do, no error
    y0 = md.y[:0].clone()
    switched.switched_lora_routed_(y0, md.x[:0], torch.zeros(0, dtype=torch.int64, device=dev), pk, path="small")
    torch.cuda.synchronize()
    assert y0.shape[0] == 0


def test_small_graph_replays(dev):
    """The routed one-launch op captured in a HIP graph; every replay equals eager, bit for bit."""
    wl = workloads.make_workload(1, dev)
    md, r = wl.modules[0], wl.routing
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, md.spec.ranks)
    args = (torch.tensor(r.req_ids, device=dev), pk, torch.tensor(r.positions, device=dev),
            torch.tensor(r.cu_seqlens, device=dev), torch.tensor(r.act_offsets, device=dev), "small")
    y_eager = md.y.clone()
    switched.switched_lora_routed_(y_eager, md.x, *args)
    torch.cuda.synchronize()
    y = md.y.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        switched.switched_lora_routed_(y, md.x, *args)
    for rep in range(3):
        y.copy_(md.y)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        _say(f"small graph replay {rep}")
        assert torch.equal(y, y_eager), f"replay {rep} differs from eager"


@pytest.mark.parametrize("speculate_tokens", [256, 8])
def test_small_back_to_back_calls(dev, speculate_tokens):
    """Many calls in a row on one stream (eager and in one graph), with and
    without speculative weight loads (T >= 2*NA or not): each reuses the
    counters the previous one left at zero; all outputs match the oracle."""
    T, NA = speculate_tokens, 12
    spec = workloads.ModuleSpec("t", 1024, (512, 256, 256), [32] * NA, 32)
    mods = [workloads.make_module(spec, T, NA, torch.bfloat16, dev, seed=40 + k) for k in range(3)]
    packs = [switched.PackedAdapters.from_slices(m.lora_A_slices, m.lora_B_slices, spec.ranks) for m in mods]
    rng = np.random.default_rng(9)
    ids = rng.integers(0, NA + 1, size=T)
    ids_d = torch.tensor(ids, device=dev)
    ys = [m.y.clone() for m in mods]
    for rep in range(4):
        for m, pk, y in zip(mods, packs, ys):
            prev = _np(y)
            switched.switched_lora_routed_(y, m.x, ids_d, pk, path="small")
            torch.cuda.synchronize()
            ref = olora.switched_lora_apply(prev, _np(m.x), ids, [_np(a) for a in m.lora_A_slices],
                                            [_np(b) for b in m.lora_B_slices], spec.output_slices, spec.ranks, "bf16")
            _close(_np(y), ref, 2e-2, f"chained small-path call {rep}")
    _say(f"back-to-back eager T={T}")
    ys2 = [m.y.clone() for m in mods]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for rep in range(4):
            for m, pk, y in zip(mods, packs, ys2):
                switched.switched_lora_routed_(y, m.x, ids_d, pk, path="small")
    for y, m in zip(ys2, mods):
        y.copy_(m.y)
    g.replay()
    torch.cuda.synchronize()
    _say(f"back-to-back graph T={T}")
    for y, y_e in zip(ys2, ys):
        assert torch.equal(y, y_e), "graph replay of chained calls differs from eager"


def _small_call(y, md, pk, ids, row_split):
    switched._call_small(md.x, y, pk, req=ids, row_split=row_split)


@pytest.mark.parametrize("dtype,T,NA,ranks,slices,H,splits,seed", [
    (torch.bfloat16, 1000, 3, [16, 64, 8], (256, 128), 1024, (2, 3, 8, 32), 61),   # ~330 tokens per adapter
    (torch.float32, 512, 4, [8, 8, 8, 8], (2048,), 2048, (4, 16), 62),             # one adapter with 256 tokens
    (torch.bfloat16, 1024, 64, [32] * 64, (256,), 512, (2, 32), 63),               # every limit at once
])
def test_small_row_split(dev, dtype, T, NA, ranks, slices, H, splits, seed):
    """Row splits spread an adapter's 32-token chunks over more workgroups.
    Every split matches the oracle, and row_split = 1 within one output ulp
    (a larger split may use fewer k-chunks, so the fp32 partials are added in
    another grouping)."""
    spec = workloads.ModuleSpec("t", H, slices, ranks, max(ranks))
    md = workloads.make_module(spec, T, NA, dtype, dev, seed=seed)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, ranks)
    rng = np.random.default_rng(seed)
    # long runs of one adapter, as sequences give them, plus base tokens
    cuts = np.sort(rng.choice(np.arange(1, T), size=max(1, NA // 2), replace=False))
    runs = np.split(np.arange(T), cuts)
    ids = np.zeros(T, np.int64)
    for run in runs:
        ids[run] = rng.integers(1, NA + 1)
    ids[rng.random(T) < 0.1] = 0
    ids_d = torch.tensor(ids, device=dev)
    y1 = md.y.clone()
    _small_call(y1, md, pk, ids_d, 1)
    torch.cuda.synchronize()
    _check(md, y1, ids, dtype)
    for rs in splits:
        _say(f"row split {rs}: dtype={dtype} T={T} NA={NA} largest group {int(np.bincount(ids)[1:].max())}")
        y = md.y.clone()
        _small_call(y, md, pk, ids_d, rs)
        torch.cuda.synchronize()
        _check(md, y, ids, dtype)
        d = (y.float() - y1.float()).abs()
        ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -20
        assert bool((d <= ulp * y1.float().abs().clamp_min(1.0)).all()), f"row_split={rs} vs row_split=1"


def test_small_row_split_changes_between_calls(dev):
    """Calls in a row on one stream with a different row split each (so a
    different number of consumers shares each adapter's epoch weight), eager
    and in one graph: every output matches the oracle."""
    T, NA = 640, 5
    spec = workloads.ModuleSpec("t", 1024, (256, 256), [16, 32, 8, 64, 24], 64)
    md = workloads.make_module(spec, T, NA, torch.bfloat16, dev, seed=64)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks)
    rng = np.random.default_rng(64)
    ids = np.repeat(rng.integers(0, NA + 1, size=T // 64), 64)
    ids_d = torch.tensor(ids, device=dev)
    order = (1, 4, 2, 20, 3, 1, 8)
    y = md.y.clone()
    for rs in order:
        prev = _np(y)
        _small_call(y, md, pk, ids_d, rs)
        torch.cuda.synchronize()
        ref = olora.switched_lora_apply(prev, _np(md.x), ids, [_np(a) for a in md.lora_A_slices],
                                        [_np(b) for b in md.lora_B_slices], spec.output_slices, spec.ranks, "bf16")
        _close(_np(y), ref, 2e-2, f"chained call with row_split={rs}")
    _say("row split chain eager")
    y2 = md.y.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for rs in order:
            _small_call(y2, md, pk, ids_d, rs)
    y2.copy_(md.y)
    g.replay()
    torch.cuda.synchronize()
    _say("row split chain graph")
    assert torch.equal(y2, y), "graph replay of the chain differs from eager"


def test_small_row_split_rejected_outside_limits(dev):
    spec = workloads.ModuleSpec("t", 512, (256,), [16, 16], 16)
    md = workloads.make_module(spec, 64, 2, torch.bfloat16, dev, seed=65)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks)
    ids_d = torch.ones(64, dtype=torch.int64, device=dev)
    for bad in (0, 33):
        with pytest.raises(Exception, match="row_split"):
            _small_call(md.y.clone(), md, pk, ids_d, bad)
    assert switched.small_workgroups(pk, 64, 0) == 0
    assert switched.small_workgroups(pk, 64, 2) > switched.small_workgroups(pk, 64, 1)


@pytest.mark.parametrize("row_split", [1, 2, 4])
def test_small_tile_groups(dev, row_split):
    """Consumers that walk several column tiles (64 adapters x 20 tiles puts
    them past 2 per CU, so the library groups 5 tiles each), with long runs of
    one adapter (several 32-token chunks per consumer, so the first tile's
    lora_B is reloaded) and row splits: oracle and the segment path agree."""
    T, NA = 1024, 64
    spec = workloads.ModuleSpec("t", 1024, (2560, 2560), [32] * NA, 32)
    md = workloads.make_module(spec, T, NA, torch.bfloat16, dev, seed=70 + row_split)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks)
    rng = np.random.default_rng(70)
    ids = np.repeat(rng.integers(0, NA + 1, size=T // 128), 128)   # 8 runs of 128 tokens
    ids[rng.random(T) < 0.05] = 0
    ids_d = torch.tensor(ids, device=dev)
    assert switched.small_workgroups(pk, T, row_split) < 8 * row_split * ((20 * NA + 7) // 8), "tile groups in use"
    _say(f"tile groups: row split {row_split}, grid {switched.small_workgroups(pk, T, row_split)}")
    y = md.y.clone()
    switched._call_small(md.x, y, pk, req=ids_d, row_split=row_split)
    y_seg = md.y.clone()
    switched.switched_lora_routed_(y_seg, md.x, ids_d, pk, path="segments")
    torch.cuda.synchronize()
    _check(md, y, ids, torch.bfloat16)
    d = (y.float() - y_seg.float()).abs()
    assert bool((d <= 2.0 ** -7 * y_seg.float().abs().clamp_min(1.0)).all()), "small path vs segment path"


def test_small_wait_limit_zero_reports_and_next_call_is_correct(dev):
    """With the wait bound at 0 looks every consumer gives up at once: the
    launch still ends, the error word is set and ``check`` raises.  After
    ``small_reset`` (and the default bound) the next call is correct."""
    wl = workloads.make_workload(1, dev)
    md, r = wl.modules[0], wl.routing
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, md.spec.ranks)
    args = (torch.tensor(r.req_ids, device=dev), pk, torch.tensor(r.positions, device=dev),
            torch.tensor(r.cu_seqlens, device=dev), torch.tensor(r.act_offsets, device=dev))
    _say("small path: wait bound 0 (forced give-up from the host)")
    prev = switched.set_small_wait_limit(0)
    try:
        y = md.y.clone()
        switched.switched_lora_routed_(y, md.x, *args, path="small")
        torch.cuda.synchronize()
    finally:
        switched.set_small_wait_limit(prev)
    assert switched.small_status(dev) & 1
    with pytest.raises(switched.SmallPathError):
        switched.check(dev)
    assert switched.small_pending_count(dev) == 0          # consumers still add their shares
    switched.small_reset(dev)
    switched.check(dev)
    _say("small path: default wait bound after reset")
    y = md.y.clone()
    switched.switched_lora_routed_(y, md.x, *args, path="small")
    torch.cuda.synchronize()
    switched.check(dev)
    eff = omap.alora_effective_ids(r.req_ids, r.positions, r.cu_seqlens, r.act_offsets)
    _check(md, y, eff, wl.dtype)
