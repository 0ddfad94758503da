"""GPU parity of the switched-LoRA shrink / expand against the CPU oracle.

Tolerances (from the target): bf16 |got - ref| <= 2e-2 + 2e-2*|ref|; fp32
1e-5 + 1e-5*|ref|.  ``ref`` is the oracle's float64 math rounded once to the
output dtype; the HF loop's own rounding sequence is checked too.  Rows of
base tokens must come back bit-identical.
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
    bound = tol + tol * np.abs(ref)
    bad = err > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} elements out of tolerance, max abs err {err.max():.3e}"
    return float(err.max()) if err.size else 0.0


def _run_module(dev, md, routing, NA, rows_check=None):
    r = routing
    segs = switched.build_segments(torch.tensor(r.req_ids, device=dev), NA, torch.tensor(r.positions, device=dev),
                                   torch.tensor(r.cu_seqlens, device=dev),
                                   None if r.act_offsets is None else torch.tensor(r.act_offsets, device=dev))
    packed = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, md.spec.ranks)
    y = md.y.clone()
    switched.switched_lora_(y, md.x, segs, packed)
    torch.cuda.synchronize()
    return y, segs, packed


def _check_module(md, y, eff, rows, dtype, hf_too=True):
    tol = TOL[dtype]
    x, y0, yout = _np(md.x)[rows], _np(md.y)[rows], _np(y)[rows]
    A = [_np(a) for a in md.lora_A_slices]
    B = [_np(b) for b in md.lora_B_slices]
    dt = "bf16" if dtype == torch.bfloat16 else "fp32"
    ref = olora.switched_lora_apply(y0, x, eff[rows], A, B, md.spec.output_slices, md.spec.ranks, dt)
    e1 = _close(yout, ref, tol, "exact oracle")
    if hf_too:
        ref_hf = olora.switched_lora_apply(y0, x, eff[rows], A, B, md.spec.output_slices, md.spec.ranks, dt, "hf")
        _close(yout, ref_hf, tol, "HF rounding oracle")
    base = eff[rows] == 0
    assert np.array_equal(yout[base], y0[base]), "base rows were modified"
    return e1


@pytest.mark.parametrize("config", [0, 1, 3])
def test_switched_lora_full_config(dev, config):
    wl = workloads.make_workload(config, dev)
    md = wl.modules[0]
    _say(f"switched_lora config={config} T={wl.routing.num_tokens} slices={md.spec.output_slices}")
    y, segs, packed = _run_module(dev, md, wl.routing, wl.num_adapters)
    r = wl.routing
    eff = omap.alora_effective_ids(r.req_ids, r.positions, r.cu_seqlens, r.act_offsets)
    err = _check_module(md, y, eff, np.arange(r.num_tokens), wl.dtype)
    _say(f"  max abs err {err:.3e}")


def test_switched_lora_prefill_config2(dev):
    """Config 2 at full size: every row against the oracle, base rows' bits, B-linearity."""
    wl = workloads.make_workload(2, dev)
    md = wl.modules[0]
    r = wl.routing
    _say("switched_lora config=2 T=8192 O=25600")
    y, segs, packed = _run_module(dev, md, r, wl.num_adapters)
    eff = omap.alora_effective_ids(r.req_ids, r.positions, r.cu_seqlens, r.act_offsets)
    rng = np.random.default_rng(0)
    act = np.nonzero(eff > 0)[0]
    rows = np.sort(np.concatenate([rng.choice(act, 512, replace=False), rng.choice(np.nonzero(eff == 0)[0], 256,
                                                                                   replace=False)]))
    _check_module(md, y, eff, rows, wl.dtype, hf_too=False)
    base = torch.tensor(eff == 0, device=dev)
    assert torch.equal(y[base], md.y[base]), "base rows were modified"
    # every row against the oracle, in 1024-row blocks
    A = [_np(a) for a in md.lora_A_slices]
    B = [_np(b) for b in md.lora_B_slices]
    for r0 in range(0, r.num_tokens, 1024):
        blk = np.arange(r0, min(r.num_tokens, r0 + 1024))
        ref = olora.switched_lora_apply(_np(md.y[r0:r0 + 1024]), _np(md.x[r0:r0 + 1024]), eff[blk], A, B,
                                        md.spec.output_slices, md.spec.ranks, "bf16")
        _close(_np(y[r0:r0 + 1024]), ref, TOL[wl.dtype], f"config 2 rows {r0}..")
    # size-independent property: the delta is linear in B -> doubling B doubles y - y0 (to rounding)
    d1 = (y.float() - md.y.float())[torch.tensor(act[:256], device=dev)]
    packed2 = switched.PackedAdapters.from_slices(md.lora_A_slices, [2 * b for b in md.lora_B_slices], md.spec.ranks)
    y2 = md.y.clone()
    switched.switched_lora_(y2, md.x, segs, packed2)
    d2 = (y2.float() - md.y.float())[torch.tensor(act[:256], device=dev)]
    assert torch.allclose(d2, 2 * d1, atol=0.05, rtol=0.05)


def test_switched_lora_config4_one_layer_eager(dev):
    """One layer of the decoder step, eagerly, every projection on the shared
    segments (the full 32-layer graph-captured step: test_gpu_step.py)."""
    wl = workloads.make_workload(4, dev, layers=1)
    r = wl.routing
    eff = omap.alora_effective_ids(r.req_ids, r.positions, r.cu_seqlens, r.act_offsets)
    segs = switched.build_segments(torch.tensor(r.req_ids, device=dev), wl.num_adapters,
                                   torch.tensor(r.positions, device=dev), torch.tensor(r.cu_seqlens, device=dev),
                                   torch.tensor(r.act_offsets, device=dev))
    rng = np.random.default_rng(1)
    rows = np.sort(np.concatenate([np.arange(48), rng.choice(np.arange(48, r.num_tokens), 400, replace=False)]))
    for md in wl.modules:
        _say(f"config4 module {md.spec.name}")
        packed = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, md.spec.ranks)
        y = md.y.clone()
        switched.switched_lora_(y, md.x, segs, packed)     # segments reused across modules
        torch.cuda.synchronize()
        _check_module(md, y, eff, rows, wl.dtype, hf_too=False)


def test_shrink_matches_oracle(dev):
    wl = workloads.make_workload(3, dev)
    md = wl.modules[0]
    r = wl.routing
    segs = switched.build_segments(torch.tensor(r.req_ids, device=dev), wl.num_adapters)
    packed = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, md.spec.ranks)
    z = switched.shrink(md.x, segs, packed)
    torch.cuda.synchronize()
    seg_h, perm_h = segs.seg_offsets.cpu().numpy(), segs.perm.cpu().numpy()
    zw = packed.num_slices * packed.max_rank
    ref = olora.shrink_rows(_np(md.x), perm_h, seg_h, [_np(a) for a in md.lora_A_slices], md.spec.ranks, zw)
    got = _np(z)[: seg_h[-1]]
    # only the columns each adapter owns are defined
    for g in range(1, wl.num_adapters + 1):
        lo, hi = seg_h[g - 1], seg_h[g]
        rr = packed.ranks_host[g]
        _close(got[lo:hi, :rr], olora.bf16_round(ref[lo:hi, :rr]), 2e-2, f"z adapter {g}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_identity_known_answer(dev, dtype):
    """A_a = eye*0.1(a+1), B_a = eye*0.2(a+1) -> delta[:, j<r] = x[:, j] * 0.02(a+1)^2 (lora_cases.py:346-426)."""
    IN, OUT, R, NA = 256, 64, 8, 4
    A = torch.zeros(NA, 1, R, IN, dtype=dtype, device=dev)
    B = torch.zeros(NA, 1, OUT, R, dtype=dtype, device=dev)
    for a in range(NA):
        A[a, 0] = torch.eye(R, IN, device=dev) * 0.1 * (a + 1)
        B[a, 0] = torch.eye(OUT, R, device=dev) * 0.2 * (a + 1)
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(50, IN, generator=g, device=dev).to(dtype)
    y = torch.randn(50, OUT, generator=g, device=dev).to(dtype)
    ids = torch.tensor([a % (NA + 1) for a in range(50)], device=dev)
    segs = switched.build_segments(ids, NA)
    pk = switched.PackedAdapters.from_slices([A], [B], [R] * NA)
    out = y.clone()
    switched.switched_lora_(out, x, segs, pk)
    exp = y.double().clone()
    idc = ids.cpu()
    for t in range(50):
        a = int(idc[t])
        if a:
            # 0.1(a+1) and 0.2(a+1) as stored (rounded to dtype), then the closed form
            exp[t, :R] += x[t, :R].double() * float(A[a - 1, 0, 0, 0]) * float(B[a - 1, 0, 0, 0])
    tol = TOL[dtype]
    _close(_np(out), exp.cpu().numpy(), tol, "identity KAT")


def test_all_base_and_empty(dev):
    spec = workloads.ModuleSpec("t", 512, (256,), [16, 16], 16)
    md = workloads.make_module(spec, 70, 2, torch.bfloat16, dev, seed=2)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks)
    segs = switched.build_segments(torch.zeros(70, dtype=torch.int64, device=dev), 2)
    y = md.y.clone()
    switched.switched_lora_(y, md.x, segs, pk)
    torch.cuda.synchronize()
    assert torch.equal(y, md.y)
    # zero tokens
    segs0 = switched.build_segments(torch.zeros(0, dtype=torch.int64, device=dev), 2)
    y0 = torch.zeros(0, 256, dtype=torch.bfloat16, device=dev)
    switched.switched_lora_(y0, torch.zeros(0, 512, dtype=torch.bfloat16, device=dev), segs0, pk)
    torch.cuda.synchronize()


def test_non_applicable_adapter_leaves_rows(dev):
    spec = workloads.ModuleSpec("t", 256, (128, 64), [32, 32, 32], 32)
    md = workloads.make_module(spec, 90, 3, torch.bfloat16, dev, seed=4)
    for A in md.lora_A_slices:
        A[1].zero_()                                    # adapter 2 not applicable here
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks)
    assert pk.ranks_host[2] == 0
    ids = torch.tensor([t % 4 for t in range(90)], device=dev)
    segs = switched.build_segments(ids, 3)
    y = md.y.clone()
    switched.switched_lora_(y, md.x, segs, pk)
    torch.cuda.synchronize()
    two = ids == 2
    assert torch.equal(y[two], md.y[two])
    eff = ids.cpu().numpy().copy()
    eff[eff == 2] = 0          # the reference remaps a non-applicable adapter to base
    rows = np.arange(90)
    _check_module(md, y, eff, rows, torch.bfloat16)


@pytest.mark.parametrize("T", [1, 2, 7])
@pytest.mark.parametrize("path", ["segments", "small"])
def test_tiny_batches(dev, T, path):
    """Batches of 1, 2 and 7 tokens on both kernel paths (one tile, part-filled)."""
    ranks = [32] * 12
    NA = len(ranks)
    spec = workloads.ModuleSpec("qkv", 4096, (4096, 1024, 1024), ranks, 32)
    md = workloads.make_module(spec, T, NA, torch.bfloat16, dev, seed=40 + T)
    ids = ((np.arange(T) * 5 + 3) % (NA + 1)).astype(np.int64)
    _say(f"tiny batch T={T} path={path} ids={ids.tolist()}")
    segs = switched.build_segments(torch.tensor(ids, device=dev), NA)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, ranks)
    y = md.y.clone()
    switched.switched_lora_(y, md.x, segs, pk, path=path)
    torch.cuda.synchronize()
    if path == "small":
        switched.check(dev)
    _check_module(md, y, ids, np.arange(T), torch.bfloat16)


@pytest.mark.parametrize("dtype,T,ranks", [(torch.bfloat16, 5000, [8] * 180 + [32] * 76),
                                           (torch.float32, 1500, [16] * 100),
                                           (torch.bfloat16, 3000, [32] * 120 + [256] * 2)])
def test_more_than_64_adapters(dev, dtype, T, ranks):
    """Adapter tables past one wave (the kernels' multi-pass tile lookup), up
    to the builder's 256: every row against the oracle, base rows bit-identical."""
    NA = len(ranks)
    spec = workloads.ModuleSpec("t", 512, (256, 128), ranks, max(ranks))
    md = workloads.make_module(spec, T, NA, dtype, dev, seed=NA + T)
    ids = np.random.default_rng(NA).integers(0, NA + 1, size=T)
    _say(f"more than 64 adapters: NA={NA} T={T} {dtype}")
    segs = switched.build_segments(torch.tensor(ids, device=dev), NA)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, ranks)
    y = md.y.clone()
    switched.switched_lora_(y, md.x, segs, pk, path="segments")
    torch.cuda.synchronize()
    _check_module(md, y, ids, np.arange(T), dtype)


def test_one_adapter_past_2e18_slots(dev):
    """An adapter holding 2^18 or more tokens: its 32-slot expand tiles are cut
    with 64-bit products (tile jj * n passes 2^31 there).  Every row against
    the oracle; base rows bit-identical."""
    T = (1 << 18) + 4096
    spec = workloads.ModuleSpec("t", 128, (256,), [16, 16], 16)
    md = workloads.make_module(spec, T, 2, torch.bfloat16, dev, seed=11)
    ids = np.ones(T, dtype=np.int64)
    ids[::997] = 2
    ids[::1009] = 0
    assert int((ids == 1).sum()) >= (1 << 18)
    _say(f"one adapter past 2^18 slots: T={T} adapter-1 tokens={int((ids == 1).sum())}")
    segs = switched.build_segments(torch.tensor(ids, device=dev), 2)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks)
    y = md.y.clone()
    switched.switched_lora_(y, md.x, segs, pk, path="segments")
    torch.cuda.synchronize()
    _check_module(md, y, ids, np.arange(T), torch.bfloat16, hf_too=False)


@pytest.mark.parametrize("ranks,slices,H", [([8, 24, 40, 64], (96,), 1000), ([16, 512], (32, 64), 264),
                                            ([128, 8], (4096, 1024, 1024), 4096)])
def test_odd_shapes(dev, ranks, slices, H):
    """Ranks that are not multiples of 16, H not a multiple of the k-chunk, rank 512."""
    NA = len(ranks)
    spec = workloads.ModuleSpec("t", H, slices, ranks, max(ranks))
    T = 333
    md = workloads.make_module(spec, T, NA, torch.bfloat16, dev, seed=6)
    rng = np.random.default_rng(6)
    ids = rng.integers(0, NA + 1, size=T)
    segs = switched.build_segments(torch.tensor(ids, device=dev), NA)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, ranks)
    y = md.y.clone()
    _say(f"odd shape ranks={ranks} slices={slices} H={H}")
    switched.switched_lora_(y, md.x, segs, pk)
    torch.cuda.synchronize()
    _check_module(md, y, ids, np.arange(T), torch.bfloat16)


def test_graph_capture_replays(dev):
    """build_segments + shrink + expand captured in a HIP graph; every replay == eager."""
    wl = workloads.make_workload(1, dev)
    md = wl.modules[0]
    r = wl.routing
    ids = torch.tensor(r.req_ids, device=dev)
    pos = torch.tensor(r.positions, device=dev)
    cu = torch.tensor(r.cu_seqlens, device=dev)
    off = torch.tensor(r.act_offsets, device=dev)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, md.spec.ranks)
    y_eager = md.y.clone()
    segs = switched.build_segments(ids, wl.num_adapters, pos, cu, off)
    switched.switched_lora_(y_eager, md.x, segs, pk)
    torch.cuda.synchronize()
    y = md.y.clone()
    z = torch.empty(r.num_tokens, pk.num_slices * pk.max_rank, dtype=torch.bfloat16, device=dev)
    segs_g = switched.build_segments(ids, wl.num_adapters, pos, cu, off)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        switched.shrink(md.x, segs_g, pk, z)       # warm-up allocates the workspace
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        switched.build_segments(ids, wl.num_adapters, pos, cu, off, out=segs_g)
        switched.switched_lora_(y, md.x, segs_g, pk, z)
    for rep in range(3):
        y.copy_(md.y)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        _say(f"graph replay {rep}")
        assert torch.equal(y, y_eager), f"replay {rep} differs from eager"


@pytest.mark.parametrize("path", ["small", "segments"])
def test_graph_replay_after_workspace_growth(dev, path):
    """A graph captured at a small batch, then an eager call at a much larger
    batch that outgrows the per-device workspace, then replays: the replays
    still write into the captured (retired, kept alive) buffer and equal the
    eager result of the small batch."""
    NA = 6
    spec = workloads.ModuleSpec("t", 1024, (512, 256), [16, 32, 8, 32, 16, 32], 32)
    small = workloads.make_module(spec, 200, NA, torch.bfloat16, dev, seed=91)
    big = workloads.make_module(spec, 3000 if path == "segments" else 1000, NA, torch.bfloat16, dev, seed=92)
    pk_s = switched.PackedAdapters.from_slices(small.lora_A_slices, small.lora_B_slices, spec.ranks)
    pk_b = switched.PackedAdapters.from_slices(big.lora_A_slices, big.lora_B_slices, spec.ranks)
    g_ids = torch.Generator(device=dev).manual_seed(93)
    ids_s = torch.randint(0, NA + 1, (200,), generator=g_ids, device=dev)
    ids_b = torch.randint(0, NA + 1, (big.x.shape[0],), generator=g_ids, device=dev)
    y_eager = small.y.clone()
    switched.switched_lora_routed_(y_eager, small.x, ids_s, pk_s, path=path)
    torch.cuda.synchronize()
    y = small.y.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        switched.switched_lora_routed_(y, small.x, ids_s, pk_s, path=path)
    # an eager call whose workspace need exceeds the captured one
    _say(f"{path}: eager call at T={big.x.shape[0]} after capture")
    y_big = big.y.clone()
    switched.switched_lora_routed_(y_big, big.x, ids_b, pk_b, path=path)
    torch.cuda.synchronize()
    for rep in range(3):
        y.copy_(small.y)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        _say(f"{path}: replay {rep} after the workspace grew")
        assert torch.equal(y, y_eager), f"replay {rep} differs from eager"
    switched.check(dev)


@pytest.mark.parametrize("path", ["small", "segments"])
def test_slice_independence(dev, path):
    """LoRA weights on slice 0 only (reference tests/hf/test_lora.py:133-168):
    slice 0 changes, slices 1+ come back bit-identical, on both kernel paths."""
    T, NA = 96, 3
    spec = workloads.ModuleSpec("t", 512, (256, 128, 128), [16, 32, 8], 32)
    md = workloads.make_module(spec, T, NA, torch.bfloat16, dev, seed=81)
    for s in (1, 2):
        md.lora_A_slices[s].zero_()
        md.lora_B_slices[s].zero_()
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks)
    ids = torch.ones(T, dtype=torch.int64, device=dev)
    ids[::3] = 2
    y = md.y.clone()
    switched.switched_lora_routed_(y, md.x, ids, pk, path=path)
    torch.cuda.synchronize()
    print(f"slice independence path={path}", flush=True)
    assert not torch.equal(y[:, :256], md.y[:, :256]), "slice 0 should carry the delta"
    assert torch.equal(y[:, 256:], md.y[:, 256:]), "slices 1+ must stay bit-identical"
    ref = olora.switched_lora_apply(md.y.float().cpu().numpy(), md.x.float().cpu().numpy(), ids.cpu().numpy(),
                                    [a.float().cpu().numpy() for a in md.lora_A_slices],
                                    [b.float().cpu().numpy() for b in md.lora_B_slices], spec.output_slices,
                                    spec.ranks, "bf16")
    got = y.float().cpu().numpy()
    assert np.all(np.abs(got - ref) <= 2e-2 + 2e-2 * np.abs(ref))
