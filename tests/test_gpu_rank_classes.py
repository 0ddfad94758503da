"""Modules whose adapters' ranks differ widely, on the GPU (rank classes).

The reference's imbalanced population -- N rank-32 adapters plus one rank-512
adapter, ids drawn over all of them (docs/SWITCH_KERNELS.md "Methodology";
"a rank-512 adapter costs rank-512 work only for the tokens that use it",
"Per-adapter rank tiers") -- and other mixes.  The segment kernels run once
per rank class (ranks <= 64 and above), each planned for its own ranks; the
one-launch decode kernel takes the rank <= 64 class and the segment kernels
the larger adapters.  Every path is checked against the oracle
(|got - ref| <= 2e-2 + 2e-2 |ref| in bf16, 1e-5 in fp32) with base rows
bit-identical.  gs_switched_lora runs a two-class module in the pair
launches (the small class's grid carries the sparse large class's items)
when its workspace holds both classes' partials and the pair's item counter
and the classes' forms allow; concurrently on two streams when it holds the
partials only; and in turn otherwise.  All three give the same bits.
"""

from __future__ import annotations

import ctypes

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


def _check(md, y, eff, dtype, what):
    dt = "bf16" if dtype == torch.bfloat16 else "fp32"
    ref = olora.switched_lora_apply(_np(md.y), _np(md.x), eff, [_np(a) for a in md.lora_A_slices],
                                    [_np(b) for b in md.lora_B_slices], md.spec.output_slices, md.spec.ranks, dt)
    got = _np(y).astype(np.float64)
    err = np.abs(got - ref)
    tol = TOL[dtype]
    bad = err > tol + tol * np.abs(ref)
    assert not bad.any(), f"{what}: {int(bad.sum())} out of tolerance, max abs err {err.max():.3e}"
    base = eff == 0
    assert np.array_equal(got[base], _np(md.y)[base]), f"{what}: base rows modified"
    return float(err.max())


@pytest.mark.parametrize("path", ["auto", "small", "segments"])
def test_decode_population_with_a_rank512_adapter(dev, path):
    """12 rank-32 adapters + 1 rank-512 on the decode QKV shape (T = 256)."""
    r = workloads.population_routing(1, "r512")
    NA = workloads.population_adapters(1, "r512")
    spec = workloads.population_specs(1, "r512")[0]
    md = workloads.make_module(spec, r.num_tokens, NA, torch.bfloat16, dev, seed=501)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks)
    assert pk.max_rank == 512 and pk.rank_split()[1].ranks_host[NA] == 512
    if path == "auto":
        # the segment kernels, both classes in the pair launches
        assert switched.pair_launches(pk, r.num_tokens)
        assert switched.path_plan(pk, r.num_tokens, r.num_tokens) == "segments"
    args = [torch.tensor(v, device=dev) for v in (r.req_ids, r.positions, r.cu_seqlens, r.act_offsets)]
    eff = omap.alora_effective_ids(r.req_ids, r.positions, r.cu_seqlens, r.act_offsets)
    assert (eff == NA).sum() > 0, "the rank-512 adapter has tokens"
    _say(f"decode r512 population, path={path}: {int((eff > 0).sum())} adapted, {int((eff == NA).sum())} on rank 512")
    y = md.y.clone()
    switched.switched_lora_routed_(y, md.x, args[0], pk, args[1], args[2], args[3], path=path)
    torch.cuda.synchronize()
    switched.check(dev)
    err = _check(md, y, eff, torch.bfloat16, f"routed path={path}")
    # with prebuilt segments (the one-launch kernel reads their effective ids)
    segs = switched.build_segments(args[0], NA, args[1], args[2], args[3])
    y2 = md.y.clone()
    switched.switched_lora_(y2, md.x, segs, pk, path=path)
    torch.cuda.synchronize()
    switched.check(dev)
    _check(md, y2, eff, torch.bfloat16, f"segments given, path={path}")
    _say(f"  max abs err {err:.3e}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("path", ["auto", "segments"])
def test_mixed_ranks_prefill_batch(dev, dtype, path):
    """Sequences of 256 tokens, one adapter each, over ranks 8..512; T = 2048
    (above the one-launch kernel's batch limit, so both rank classes run the
    segment kernels), and T = 512 (auto: the split, or the segment kernels
    when they run both classes in the pair launches)."""
    # (fp32 stages its shrink values in LDS at 4 bytes: 2 slices x rank 256 at most)
    top = 512 if dtype == torch.bfloat16 else 256
    ranks = [32, 8, top, 64, 128, 16, 32, 256]
    NA = len(ranks)
    H, slices = (1024, (512, 256)) if dtype == torch.bfloat16 else (512, (256, 128))
    spec = workloads.ModuleSpec("mixed", H, slices, ranks, top)
    for T in (2048, 512):
        L = 256
        nseq = T // L
        rng = np.random.default_rng(T)
        adapters = np.array([3, 1, 5, 8, 2, 4, 6, 7])[:nseq]           # the largest adapter (3) first
        req = np.repeat(adapters, L).astype(np.int64)
        req[rng.random(T) < 0.1] = 0
        md = workloads.make_module(spec, T, NA, dtype, dev, seed=600 + T)
        pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, ranks)
        _say(f"mixed ranks {ranks}, T={T}, {dtype}, path={path} (plan {switched.path_plan(pk, T)})")
        segs = switched.build_segments(torch.tensor(req, device=dev), NA)
        y = md.y.clone()
        switched.switched_lora_(y, md.x, segs, pk, path=path)
        torch.cuda.synchronize()
        switched.check(dev)
        _check(md, y, req, dtype, f"T={T} path={path}")


def test_shrink_materialises_z_per_class(dev):
    """gs_shrink with z requested on a two-class module whose hidden dimension
    is split in both classes: each class's partials are reduced into its own
    adapters' z rows only (the other class's rows are not overwritten), and
    the expand from that z matches the oracle."""
    ranks = [32, 256, 16, 32]
    NA = len(ranks)
    spec = workloads.ModuleSpec("two_class", 4096, (512, 512), ranks, 256)
    T = 300
    md = workloads.make_module(spec, T, NA, torch.bfloat16, dev, seed=77)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, ranks)
    ks = switched.shrink_ksplits(pk, T)
    assert len(ks) == 2 and min(ks) > 1, ks
    rng = np.random.default_rng(9)
    req = rng.integers(0, NA + 1, size=T)
    segs = switched.build_segments(torch.tensor(req, device=dev), NA)
    with pytest.raises(switched._lib.GraniteSwitchError, match="one rank class"):
        switched.shrink(md.x, segs, pk, partials_only=True)
    zw = pk.num_slices * pk.max_rank
    z = torch.full((T, zw), float("nan"), dtype=torch.bfloat16, device=dev)
    switched.shrink(md.x, segs, pk, z)
    torch.cuda.synchronize()
    seg_h, perm_h = segs.seg_offsets.cpu().numpy(), segs.perm.cpu().numpy()
    ref = olora.shrink_rows(_np(md.x), perm_h, seg_h, [_np(a) for a in md.lora_A_slices], ranks, zw)
    got = _np(z)
    for g in range(1, NA + 1):
        lo, hi = seg_h[g - 1], seg_h[g]
        cols = pk.num_slices * pk.ranks_host[g]
        err = np.abs(got[lo:hi, :cols] - olora.bf16_round(ref[lo:hi, :cols]))
        assert np.all(err <= 2e-2 + 2e-2 * np.abs(ref[lo:hi, :cols])), f"z of adapter {g}"
    y = md.y.clone()
    switched.expand_add_(y, z, segs, pk)
    torch.cuda.synchronize()
    _check(md, y, req, torch.bfloat16, "expand from the materialised z")


def test_noalloc_two_classes_equals_workspace_path(dev):
    """gs_switched_lora_noalloc on a two-class module: the same kernels per
    class, scratch in the static array, bit-identical to gs_switched_lora."""
    ranks = [32] * 6 + [512]
    NA = len(ranks)
    spec = workloads.ModuleSpec("qkv", 4096, (4096, 1024, 1024), ranks, 512)
    T = 400
    md = workloads.make_module(spec, T, NA, torch.bfloat16, dev, seed=88)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, ranks)
    req = np.random.default_rng(3).integers(0, NA + 1, size=T)
    segs = switched.build_segments(torch.tensor(req, device=dev), NA)
    y_ref = md.y.clone()
    switched.switched_lora_(y_ref, md.x, segs, pk, path="segments")
    y = md.y.clone()
    switched.switched_lora_noalloc_(y, md.x, segs, pk)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref), "noalloc differs from gs_switched_lora"
    _check(md, y, req, torch.bfloat16, "noalloc, two classes")


def test_only_large_adapters_and_no_applicable_adapter(dev):
    """A module whose every adapter is above rank 64 is one (large) class;
    one with no applicable adapter launches nothing and leaves y as it was."""
    ranks = [128, 512]
    spec = workloads.ModuleSpec("large", 1024, (1024,), ranks, 512)
    T = 200
    md = workloads.make_module(spec, T, 2, torch.bfloat16, dev, seed=5)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, ranks)
    assert pk.rank_split()[0] is None and switched.path_plan(pk, T) == "segments"
    req = np.random.default_rng(1).integers(0, 3, size=T)
    for path in ("auto", "segments"):
        y = md.y.clone()
        switched.switched_lora_routed_(y, md.x, torch.tensor(req, device=dev), pk, path=path)
        torch.cuda.synchronize()
        _check(md, y, req, torch.bfloat16, f"large only, path={path}")
    with pytest.raises(ValueError, match="rank <= 64"):
        switched.switched_lora_routed_(md.y.clone(), md.x, torch.tensor(req, device=dev), pk, path="small")
    none = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, ranks, applicable=[False, False])
    y = md.y.clone()
    switched.switched_lora_routed_(y, md.x, torch.tensor(req, device=dev), none, path="segments")
    torch.cuda.synchronize()
    assert torch.equal(y, md.y)


def _graph_replays_equal_eager(dev, run, restore, outputs, what):
    """Eager run, then the same run captured in a HIP graph and replayed three
    times (with eager work and synchronisations between), every replay
    bit-identical to the eager result."""
    run()
    torch.cuda.synchronize()
    ref = [o.clone() for o in outputs]
    restore()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for replay in range(3):
        restore()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        same = all(torch.equal(o, r) for o, r in zip(outputs, ref))
        _say(f"  {what}: replay {replay} {'bit-identical' if same else 'DIFFERS'}")
        assert same, f"{what}: graph replay {replay} differs from the eager run"
        _ = torch.ones(1024, device=dev).sum().item()     # eager work between replays
    return ref


def test_concurrent_classes_under_graph_capture(dev):
    """gs_switched_lora runs a two-class module (one rank-512 adapter among
    rank-32 ones) in the pair launches, whose item counter the shrink zeroes
    in every launch: captured into a graph, every replay equals the eager
    call.  The one-launch + segments "split" path forks a torch side stream,
    captured the same way."""
    ranks = [32] * 6 + [512]
    NA = len(ranks)
    spec = workloads.ModuleSpec("qkv", 4096, (4096, 1024, 1024), ranks, 512)
    T = 400
    md = workloads.make_module(spec, T, NA, torch.bfloat16, dev, seed=91)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, ranks)
    req = np.random.default_rng(4).integers(0, NA + 1, size=T)
    segs = switched.build_segments(torch.tensor(req, device=dev), NA)
    z = torch.empty(T, spec_zw(pk), dtype=torch.bfloat16, device=dev)
    y = md.y.clone()
    y0 = md.y.clone()
    ref = _graph_replays_equal_eager(dev, lambda: switched.switched_lora_(y, md.x, segs, pk, z, path="segments"),
                                     lambda: y.copy_(y0), [y], "two classes, segments")
    _check(md, ref[0], req, torch.bfloat16, "two classes, segments, eager")

    # fp32 (no pair launches; the fp32 expand stages S * max_rank <= 952
    # values per row): the large class on the library's side stream, forked
    # from and joined into the captured stream
    ranks_f = [32] * 6 + [256]
    spec_f = workloads.ModuleSpec("gate_up", 2048, (2048, 2048), ranks_f, 256)
    mdf = workloads.make_module(spec_f, T, NA, torch.float32, dev, seed=95)
    pkf = switched.PackedAdapters.from_slices(mdf.lora_A_slices, mdf.lora_B_slices, ranks_f)
    zf = torch.empty(T, spec_zw(pkf), dtype=torch.float32, device=dev)
    yf = mdf.y.clone()
    yf0 = mdf.y.clone()
    reff = _graph_replays_equal_eager(dev, lambda: switched.switched_lora_(yf, mdf.x, segs, pkf, zf, path="segments"),
                                      lambda: yf.copy_(yf0), [yf], "two classes, fp32, two streams")
    _check(mdf, reff[0], req, torch.float32, "two classes, fp32, two streams, eager")

    # decode-sized: the split path (one-launch kernel beside the segment
    # kernels), which path="small" forces for a module with a rank-512 adapter
    r = workloads.population_routing(1, "r512")
    NA1 = workloads.population_adapters(1, "r512")
    spec1 = workloads.population_specs(1, "r512")[0]
    md1 = workloads.make_module(spec1, r.num_tokens, NA1, torch.bfloat16, dev, seed=92)
    pk1 = switched.PackedAdapters.from_slices(md1.lora_A_slices, md1.lora_B_slices, spec1.ranks)
    assert switched.path_plan(pk1, r.num_tokens, r.num_tokens) == "segments"
    args = [torch.tensor(v, device=dev) for v in (r.req_ids, r.positions, r.cu_seqlens, r.act_offsets)]
    eff = omap.alora_effective_ids(r.req_ids, r.positions, r.cu_seqlens, r.act_offsets)
    segs1 = switched.build_segments(args[0], NA1, args[1], args[2], args[3])
    y1 = md1.y.clone()
    y10 = md1.y.clone()
    ref1 = _graph_replays_equal_eager(dev, lambda: switched.switched_lora_(y1, md1.x, segs1, pk1, path="small"),
                                      lambda: y1.copy_(y10), [y1], "split path")
    switched.check(dev)
    _check(md1, ref1[0], eff, torch.bfloat16, "split path, eager")


def spec_zw(pk):
    return pk.num_slices * pk.max_rank


def test_two_classes_in_a_one_class_workspace_run_in_turn(dev):
    """The workspace decides how gs_switched_lora runs a two-class module: the
    full size (gs_shrink_workspace_bytes) takes the pair launches, one
    256-byte line less (both classes' partials but no item counter) the two
    streams, one more line less (either class's partials, not both) the
    classes in turn.  The three results are bit-identical."""
    ranks = [32] * 8 + [256]
    NA = len(ranks)
    spec = workloads.ModuleSpec("gate_up", 4096, (2048, 2048), ranks, 256)
    T = 600
    md = workloads.make_module(spec, T, NA, torch.bfloat16, dev, seed=93)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, ranks)
    req = np.random.default_rng(5).integers(0, NA + 1, size=T)
    segs = switched.build_segments(torch.tensor(req, device=dev), NA)
    lib = switched._lib.load()

    def ws_bytes(p):
        return int(lib.gs_shrink_workspace_bytes(T, spec.hidden, pk.num_slices, NA, p.max_rank,
                                                  switched._i32_array(p.ranks_host)))

    # side by side the classes need align256(small) + large bytes, then one
    # 256-byte line for the pair's counter; a line fewer than both still
    # holds either class's partials
    full = ws_bytes(pk)
    both = full - 256
    one = both - 256
    _say(f"workspace: pair {full} B, two streams {both} B, in turn {one} B")
    outs = []
    for nbytes in (full, both, one):
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        z = torch.empty(T, spec_zw(pk), dtype=torch.bfloat16, device=dev)
        y = md.y.clone()
        switched._lib.call("gs_switched_lora", switched._dtype_code(md.x), md.x.data_ptr(), md.x.stride(0),
                           y.data_ptr(), y.stride(0), T, spec.hidden, pk.out_total,
                           switched._i32_array(pk.slice_bounds), pk.num_slices, pk.a_pack.data_ptr(),
                           pk.a_off.data_ptr(), pk.b_pack.data_ptr(), pk.b_off.data_ptr(), pk.ranks.data_ptr(), NA,
                           pk.max_rank, switched._i32_array(pk.ranks_host), segs.seg_offsets.data_ptr(),
                           segs.perm.data_ptr(), z.data_ptr(), ws.data_ptr(), nbytes,
                           switched._lib.stream_ptr(dev))
        torch.cuda.synchronize()
        outs.append(y)
    assert torch.equal(outs[0], outs[1]), "pair launches and two-stream run differ"
    assert torch.equal(outs[0], outs[2]), "pair launches and in-turn run differ"
    _check(md, outs[0], req, torch.bfloat16, "two classes")


def _run_with_workspace(md, pk, segs, T, spec, nbytes):
    lib = switched._lib
    ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=md.y.device)
    z = torch.empty(T, spec_zw(pk), dtype=md.y.dtype, device=md.y.device)
    y = md.y.clone()
    lib.call("gs_switched_lora", switched._dtype_code(md.x), md.x.data_ptr(), md.x.stride(0), y.data_ptr(),
             y.stride(0), T, spec.hidden, pk.out_total, switched._i32_array(pk.slice_bounds), pk.num_slices,
             pk.a_pack.data_ptr(), pk.a_off.data_ptr(), pk.b_pack.data_ptr(), pk.b_off.data_ptr(),
             pk.ranks.data_ptr(), pk.num_adapters, pk.max_rank, switched._i32_array(pk.ranks_host),
             segs.seg_offsets.data_ptr(), segs.perm.data_ptr(), z.data_ptr(), ws.data_ptr(), nbytes,
             lib.stream_ptr(md.y.device))
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("large", [72, 96, 128, 256, 512])
@pytest.mark.parametrize("T", [64, 600])
def test_pair_launches_every_large_rank(dev, large, T):
    """The pair launches at every k-group count of the large class's items
    (ranks 72..128: 2 per wave, ..256: 4, ..512: 8), odd ranks included:
    bit-identical to the two-stream and in-turn forms, and to the oracle."""
    ranks = [32] * 24 + [large]
    NA = len(ranks)
    spec = workloads.ModuleSpec("qkv", 4096, (2048, 1024, 1024), ranks, large)
    md = workloads.make_module(spec, T, NA, torch.bfloat16, dev, seed=700 + large + T)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, ranks)
    assert switched.pair_launches(pk, T)
    req = np.random.default_rng(large + T).integers(0, NA + 1, size=T)
    segs = switched.build_segments(torch.tensor(req, device=dev), NA)
    lib = switched._lib.load()
    full = int(lib.gs_shrink_workspace_bytes(T, spec.hidden, pk.num_slices, NA, pk.max_rank,
                                             switched._i32_array(pk.ranks_host)))
    # the small class's partials (KS x T x S*32 fp32 when split) come first,
    # the large class's from the next 256-byte boundary (planned at its
    # largest device k-split), then the counter line; the in-turn form needs
    # the larger of the two, and exists only when the small class has
    # partials too
    ks = (ctypes.c_int32 * 2)()
    assert lib.gs_shrink_ksplits(switched._lib.GS_DTYPE_BF16, T, spec.hidden, pk.num_slices, NA, pk.max_rank,
                                 switched._i32_array(pk.ranks_host), ks) == 2
    part0 = ks[0] * T * pk.num_slices * 32 * 4 if ks[0] > 1 else 0
    both = full - 256
    part1 = both - (part0 + 255) // 256 * 256
    sizes = [full, both] + ([max(part0, part1)] if part0 > 0 else [])
    outs = [_run_with_workspace(md, pk, segs, T, spec, n) for n in sizes]
    assert torch.equal(outs[0], outs[1]), "pair launches and two-stream run differ"
    if len(outs) > 2:
        assert torch.equal(outs[0], outs[2]), "pair launches and in-turn run differ"
    err = _check(md, outs[0], req, torch.bfloat16, f"pair launches, large rank {large}, T={T}")
    _say(f"pair launches, large rank {large}, T={T}: {int((req == NA).sum())} tokens on it, max abs err {err:.3e}")


@pytest.mark.parametrize("proj", [0, 1, 2, 3])
def test_step_population_with_a_rank512_adapter(dev, proj):
    """The decoder step's shape (T = 4144, chunked prefill plus decode rows)
    with the rank-512 population: each projection of one layer through the
    pair launches, every row against the oracle, base rows bit-identical."""
    r = workloads.population_routing(4, "r512")
    NA = workloads.population_adapters(4, "r512")
    spec = workloads.population_specs(4, "r512")[proj]
    md = workloads.make_module(spec, r.num_tokens, NA, torch.bfloat16, dev, seed=900 + proj)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks)
    assert switched.pair_launches(pk, r.num_tokens)
    eff = omap.alora_effective_ids(r.req_ids, r.positions, r.cu_seqlens, r.act_offsets)
    assert (eff == NA).sum() > 0, "the rank-512 adapter has tokens"
    _say(f"step r512 population, {spec.name}: {int((eff > 0).sum())} adapted, {int((eff == NA).sum())} on rank 512")
    args = [torch.tensor(v, device=dev) for v in (r.req_ids, r.positions, r.cu_seqlens, r.act_offsets)]
    segs = switched.build_segments(args[0], NA, args[1], args[2], args[3])
    y = md.y.clone()
    switched.switched_lora_(y, md.x, segs, pk)
    torch.cuda.synchronize()
    err = _check(md, y, eff, torch.bfloat16, f"step r512 {spec.name}")
    _say(f"  max abs err {err:.3e}")
