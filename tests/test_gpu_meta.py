"""GPU parity of the integer kernels: segment builder, routing, bitmasks.

Bit-exact against the CPU oracle (pinned in test_oracle.py) and against the
reference's known answers.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from granite_switch_amd import kernels, meta, ops, switched, workloads
from oracle import mapping as omap

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _check_segments(segs, eff, NA):
    seg_ref, perm_ref = omap.build_segments(eff, NA)
    got_eff = segs.eff_ids.cpu().numpy()
    assert np.array_equal(got_eff, eff), "effective ids differ"
    got_seg = segs.seg_offsets.cpu().numpy()
    assert np.array_equal(got_seg, seg_ref), "segment offsets differ"
    assert np.array_equal(segs.perm.cpu().numpy()[: seg_ref[-1]], perm_ref), "permutation differs"


@pytest.mark.parametrize("config", [0, 1, 2, 3, 4])
def test_build_segments_configs(dev, config):
    r = workloads.routing_for(config)
    NA = workloads.num_adapters_for(config)
    _say(f"build_segments config={config} T={r.num_tokens} NA={NA}")
    segs = switched.build_segments(torch.tensor(r.req_ids, device=dev), NA, torch.tensor(r.positions, device=dev),
                                   torch.tensor(r.cu_seqlens, device=dev),
                                   None if r.act_offsets is None else torch.tensor(r.act_offsets, device=dev))
    torch.cuda.synchronize()
    eff = omap.alora_effective_ids(r.req_ids, r.positions, r.cu_seqlens, r.act_offsets)
    _check_segments(segs, eff, NA)


@pytest.mark.parametrize("T,NA,seed", [(0, 4, 0), (1, 1, 1), (63, 3, 2), (1023, 7, 3), (1024, 64, 4), (1025, 255, 5),
                                       (5000, 256, 6), (65536, 24, 7)])
def test_build_segments_random(dev, T, NA, seed):
    rng = np.random.default_rng(seed)
    req = rng.integers(-3, NA + 4, size=T)           # includes out-of-range ids (-> base)
    nseq = max(1, T // 50)
    cuts = np.sort(rng.choice(np.arange(1, T), size=min(nseq - 1, max(T - 1, 0)), replace=False)) if T > 1 else []
    cu = np.concatenate([[0], cuts, [T]]).astype(np.int32)
    lens = np.diff(cu)
    cached = rng.integers(0, 100, size=lens.size)
    pos = np.concatenate([c + np.arange(l) for c, l in zip(cached, lens)]) if T else np.zeros(0, np.int64)
    offs = rng.integers(0, 160, size=lens.size)
    _say(f"build_segments random T={T} NA={NA} seqs={lens.size}")
    segs = switched.build_segments(torch.tensor(req, device=dev), NA, torch.tensor(pos, device=dev),
                                   torch.tensor(cu, device=dev), torch.tensor(offs, device=dev))
    torch.cuda.synchronize()
    eff = omap.alora_effective_ids(req, pos, cu, offs)
    eff = np.where((eff < 0) | (eff > NA), 0, eff)
    _check_segments(segs, eff, NA)


def _segments_buffers(T, NA, dev, two_launch):
    chunks = max(1, -(-T // 1024))
    return switched.Segments(
        eff_ids=torch.full((T,), -7, dtype=torch.int32, device=dev),
        seg_offsets=torch.full((NA + 1,), -7, dtype=torch.int32, device=dev),
        perm=torch.full((max(T, 1),), -7, dtype=torch.int32, device=dev),
        num_tokens=T, num_adapters=NA,
        # garbage in the histogram workspace: the count launch writes all of it
        work=torch.full((chunks * (NA + 1),), 12345, dtype=torch.int32, device=dev) if two_launch else None)


@pytest.mark.parametrize("T,NA,seed,gating", [(1, 1, 11, True), (1023, 7, 12, True), (1025, 255, 13, True),
                                              (4144, 24, 14, True), (9000, 256, 15, True), (20000, 24, 16, False),
                                              (65536, 24, 17, True), (131072, 3, 18, False)])
def test_build_segments_one_and_two_launch_forms(dev, T, NA, seed, gating):
    """The two-launch form (per-chunk histograms in a workspace) against the
    oracle and against the one-launch form, at batch sizes on both sides of
    the size from which the library recommends it."""
    rng = np.random.default_rng(seed)
    req = rng.integers(-2, NA + 3, size=T)
    cu = np.concatenate([[0], np.sort(rng.choice(np.arange(1, T), size=min(T - 1, max(1, T // 300)), replace=False))
                         if T > 1 else np.zeros(0, np.int64), [T]]).astype(np.int32)
    lens = np.diff(cu)
    pos = np.concatenate([c + np.arange(l) for c, l in zip(rng.integers(0, 64, size=lens.size), lens)])
    offs = rng.integers(0, 200, size=lens.size) if gating else None
    args = (torch.tensor(req, device=dev), NA, torch.tensor(pos, device=dev), torch.tensor(cu, device=dev),
            None if offs is None else torch.tensor(offs, device=dev))
    eff = omap.alora_effective_ids(req, pos, cu, offs) if gating else req
    eff = np.where((eff < 0) | (eff > NA), 0, eff)
    outs = []
    for two in (False, True):
        _say(f"build_segments {'two' if two else 'one'}-launch T={T} NA={NA} seqs={lens.size} gating={gating}")
        segs = switched.build_segments(*args, out=_segments_buffers(T, NA, dev, two))
        torch.cuda.synchronize()
        _check_segments(segs, eff, NA)
        outs.append(segs)
    assert torch.equal(outs[0].perm, outs[1].perm) and torch.equal(outs[0].seg_offsets, outs[1].seg_offsets)


def test_build_segments_no_gating_all_base_and_all_one(dev):
    for ids, NA in ((np.zeros(300, np.int64), 5), (np.ones(3000, np.int64), 5), (np.arange(2048) % 9, 8)):
        _say(f"build_segments plain T={ids.size}")
        segs = switched.build_segments(torch.tensor(ids, device=dev), NA)
        torch.cuda.synchronize()
        _check_segments(segs, ids, NA)


def _control_layout(kats, name):
    return kats["latest_wins"][name]


def test_route_latest_wins_kats(dev, kats):
    for case in kats["latest_wins"]["cases"]:
        atok = _control_layout(kats, case["layout"])
        _say(f"route {case['tokens']}")
        got = switched.route_latest_wins(torch.tensor(case["tokens"], device=dev), atok,
                                         id_offset=0 if case["layout"] == "base_reset" else 1)
        assert got.cpu().tolist() == case["expected"]


def test_route_latest_wins_chunked(dev, kats):
    for case in kats["latest_wins"]["chunked"]["cases"]:
        atok = _control_layout(kats, case["layout"])
        off, cur, out = 0, 0, []
        for n in case["chunks"]:
            part = switched.route_latest_wins(torch.tensor(case["tokens"][off:off + n], device=dev), atok,
                                              id_offset=0 if case["layout"] == "base_reset" else 1,
                                              start_ids=torch.tensor([cur], device=dev)).cpu().tolist()
            out += part
            cur = part[-1]
            off += n
        assert out == case["expected"], case


def test_route_latest_wins_packed_batch(dev):
    """Many sequences of random lengths in one launch, vs the oracle per sequence."""
    rng = np.random.default_rng(9)
    atok = [900 + k for k in range(13)]
    lens = rng.integers(1, 700, size=40)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    toks = rng.integers(0, 40, size=int(cu[-1]))
    ctl = rng.random(toks.size) < 0.02
    toks[ctl] = rng.choice(atok, size=int(ctl.sum()))
    start = rng.integers(0, 13, size=lens.size)
    got = switched.route_latest_wins(torch.tensor(toks, device=dev), atok, 0, torch.tensor(cu, device=dev),
                                     torch.tensor(start, device=dev)).cpu().numpy()
    for s in range(lens.size):
        exp = omap.latest_wins_ids(list(toks[cu[s]:cu[s + 1]]), atok, True, start[s])
        assert list(got[cu[s]:cu[s + 1]]) == exp, s


def test_bitmask_hand_derived(dev, kats):
    k = kats["bitmask"]
    ids = torch.tensor(k["adapter_indices"], device=dev)
    remap_t = torch.tensor(k["remap_tables"], dtype=torch.int64).T.contiguous().to(dev)
    for bm, expected in k["hand_derived"].items():
        got = kernels.compute_per_module_bitmasks(ids, remap_t, int(bm)).cpu().tolist()
        assert got == expected, bm
    for bm in (1, 3, 100):
        got = kernels.compute_per_module_bitmasks(ids.to(torch.int32), remap_t, bm).cpu().numpy()
        assert np.array_equal(got, omap.compute_bitmasks(k["adapter_indices"], remap_t.cpu().numpy(), bm))


def test_bitmask_op_and_facility(dev, kats):
    k = kats["bitmask"]
    ids = torch.tensor(k["adapter_indices"], device=dev)
    remap_t = torch.tensor(k["remap_tables"], dtype=torch.int64).T.contiguous().to(dev)
    got = ops.op("compute_per_module_bitmasks")(ids, remap_t).cpu().tolist()
    assert got == k["hand_derived"]["32"]
    fm = meta.FusedLoRAKernelMeta(dev)
    fm.register_remap_tables(torch.tensor(k["remap_tables"], dtype=torch.int64, device=dev), [(128, 128, 4)] * 3)
    ctx = meta.LoRAContext()
    fm.prepare_and_store(ids, ctx)
    assert ctx.per_module_bitmasks.cpu().tolist() == k["hand_derived"]["32"]
    tables = k["remap_tables"]
    assert ctx.remapped_indices.cpu().tolist() == [[tables[m][i] for i in k["adapter_indices"]] for m in range(3)]
    assert ctx.segments.seg_offsets.cpu().tolist()[-1] == sum(1 for i in k["adapter_indices"] if i > 0)


@pytest.mark.parametrize("block_m", [1, 8, 16, 32, 64])
def test_bitmask_random_equivalence(dev, block_m):
    for trial in range(40):
        rng = np.random.default_rng(7919 * block_m + trial)
        NA = int(rng.integers(1, 65))
        nm = int(rng.integers(1, 7))
        M = int(rng.integers(1, 301))
        ids = rng.integers(0, NA + 1, size=M)
        remap = rng.integers(0, NA + 1, size=(nm, NA + 1))
        remap[:, 0] = 0
        got = kernels.compute_per_module_bitmasks(torch.tensor(ids, device=dev),
                                                  torch.tensor(remap.T.copy(), device=dev), block_m).cpu().numpy()
        assert np.array_equal(got, omap.compute_bitmasks(ids, remap.T, block_m)), (trial, NA, nm, M)


def test_bitmask_sign_bit(dev):
    remap_t = torch.arange(65, dtype=torch.int64).reshape(1, 65).T.contiguous().to(dev)
    ids = torch.tensor([1, 32, 63, 64] + [0] * 126, device=dev)
    got = kernels.compute_per_module_bitmasks(ids, remap_t, 32).cpu().numpy()
    assert np.array_equal(got, omap.compute_bitmasks(ids.cpu().numpy(), remap_t.cpu().numpy(), 32))
    assert (got < 0).any()


def test_register_asserts_64_limit():
    fm = meta.FusedLoRAKernelMeta(torch.device("cpu"))
    with pytest.raises(AssertionError, match="at most 64"):
        fm.register_remap_tables(torch.tensor([[0, *range(1, 66)]]), [(256, 256, 65)])
