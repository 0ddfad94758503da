"""CPU tests: the C ABI library loads and exports its header, host-side logic.

No kernel is launched here: the only library calls are ones whose argument
validation rejects them before any HIP call.
"""

from __future__ import annotations

import ctypes
import glob
import os
import re

import numpy as np
import pytest
import torch

from granite_switch_amd import _lib, kernels, switched, vllm_layers, workloads
from oracle import mapping as omap

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        txt = open(h).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[\w\*\s]+?\b(gs_\w+)\s*\(", txt, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    names = _header_functions()
    assert len(names) >= 10
    for n in sorted(names):
        assert hasattr(lib, n), f"missing export {n}"
    assert set(_lib.SIGNATURES) == names, "ctypes signatures out of sync with the header"
    assert lib.gs_version() >= 100


def test_library_shares_torchs_hip_runtime():
    _lib.load()
    maps = open("/proc/self/maps").read()
    hip = {l.split()[-1] for l in maps.splitlines() if "libamdhip64" in l}
    assert len(hip) == 1, hip


def test_validation_errors_without_launch():
    with pytest.raises(_lib.GraniteSwitchError) as e:
        _lib.call("gs_build_segments", None, None, None, None, 4, 1, 0, None, None, None, None, 0, None)
    assert e.value.status == _lib.GS_ERR_INVALID and "num_adapters" in str(e.value)
    # the two-launch builder's workspace: 0 below the batch size where it pays,
    # ceil(T/1024) * (NA+1) int32 histograms from there
    lib = _lib.load()
    assert lib.gs_build_segments_workspace_bytes(0, 24) == 0
    assert lib.gs_build_segments_workspace_bytes(1024, 24) == 0
    assert lib.gs_build_segments_workspace_bytes(1025, 24) == 2 * 25 * 4
    assert lib.gs_build_segments_workspace_bytes(1 << 16, 24) == 64 * 25 * 4
    assert lib.gs_build_segments_workspace_bytes(1 << 16, 0) == 0
    # a workspace smaller than the histograms is refused before any launch
    fake = ctypes.c_void_p(256)
    with pytest.raises(_lib.GraniteSwitchError) as e:
        _lib.call("gs_build_segments", fake, None, None, None, 5000, 1, 24, fake, fake, fake, fake, 5 * 25 * 4 - 4,
                  None)
    assert e.value.status == _lib.GS_ERR_WORKSPACE and "workspace" in str(e.value)
    with pytest.raises(_lib.GraniteSwitchError) as e:
        _lib.call("gs_shrink", 0, None, 16, 4, 12, None, None, None, 1, 4, 16, None, None, None, None, 16, None, 0,
                  None)
    assert "hidden" in str(e.value)
    with pytest.raises(_lib.GraniteSwitchError) as e:
        _lib.call("gs_expand_add", 0, None, 64, 4, 48, (ctypes.c_int32 * 2)(0, 48), 1, None, 16, 0, None, None,
                  None, None, 4, 16, None, None, None, None)
    assert "multiple of 32" in str(e.value)
    na = (ctypes.c_int32 * 6)(65, 0, 0, 0, 0, 0)
    with pytest.raises(_lib.GraniteSwitchError) as e:
        _lib.call("gs_switch_lora_expand", None, 64, 1, 4, None, 8, None, 1, None, None, None, na, 1, 32, 32, None)
    assert "64-bit tile mask" in str(e.value)
    with pytest.raises(_lib.GraniteSwitchError) as e:
        _lib.call("gs_compute_bitmasks", None, 2, 4, None, 2, 1, 32, None, None, None)
    assert "idx_bytes" in str(e.value)
    with pytest.raises(_lib.GraniteSwitchError) as e:
        _lib.call("gs_gemm_bf16_tn", None, 12, None, 12, None, 8, 4, 8, 12, None)
    assert "multiple of 8" in str(e.value)
    with pytest.raises(_lib.GraniteSwitchError) as e:
        _lib.call("gs_gemm_bf16_tn", None, 8, None, 16, None, 4, 4, 8, 16, None)
    assert "lda" in str(e.value)


def test_workspace_plan_is_consistent():
    lib = _lib.load()
    small = lib.gs_shrink_workspace_bytes(256, 4096, 3, 12, 32, None)
    big = lib.gs_shrink_workspace_bytes(8192, 4096, 2, 12, 32, None)
    assert small > 0 and big > 0
    assert lib.gs_shrink_workspace_bytes(0, 4096, 3, 12, 32, None) == 256


def _ranks(vals):
    return (ctypes.c_int32 * len(vals))(*vals)


def test_rank_classes_plan_each_class_for_its_own_rank():
    """A module of rank-32 adapters plus one rank-512 adapter is planned as two
    rank classes.  The rank-32 class keeps the k-split and workspace of the
    module without the large adapter; the large class, expected to hold its
    adapter's share of the tokens, gets a deep k-split."""
    lib = _lib.load()
    ks = (ctypes.c_int32 * 2)()
    r32 = [0] + [32] * 12
    mixed = r32 + [512]
    bf16 = _lib.GS_DTYPE_BF16
    for T, H, S in ((256, 4096, 3), (4144, 4096, 3), (4144, 12800, 1), (4144, 4096, 2)):
        assert lib.gs_shrink_ksplits(bf16, T, H, S, 12, 32, _ranks(r32), ks) == 1
        ks_alone = ks[0]
        # the host-table class of a uniform module equals the table-less plan
        assert lib.gs_shrink_ksplits(bf16, T, H, S, 12, 32, None, ks) == 1 and ks[0] == ks_alone
        assert lib.gs_shrink_ksplits(bf16, T, H, S, 13, 512, _ranks(mixed), ks) == 2
        assert ks[0] == ks_alone, (T, H, S, ks[0], ks_alone)
        assert ks[1] >= 2, (T, H, S, ks[1])
        ws_mixed = lib.gs_shrink_workspace_bytes(T, H, S, 13, 512, _ranks(mixed))
        assert ws_mixed >= lib.gs_shrink_workspace_bytes(T, H, S, 12, 32, _ranks(r32))
    # no applicable adapter: no class, nothing to launch
    assert lib.gs_shrink_ksplits(bf16, 256, 4096, 1, 3, 32, _ranks([0, 0, 0, 0]), ks) == 0
    # a host table that disagrees with max_rank is refused
    assert lib.gs_shrink_ksplits(bf16, 256, 4096, 1, 2, 32, _ranks([0, 32, 64]), ks) == -_lib.GS_ERR_INVALID
    assert lib.gs_shrink_workspace_bytes(256, 4096, 1, 2, 32, _ranks([0, 32, 64])) < 0


def test_rank_split_views():
    """PackedAdapters.rank_split: the <= 64 view and the larger view share the
    device tensors and zero the other class's host ranks."""
    spec = workloads.ModuleSpec("m", 64, (64,), [16, 512, 64, 0], 512)
    md = workloads.make_module(spec, 4, 4, torch.float32, "cpu", seed=1)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks,
                                             applicable=[True, True, True, False])
    small, large = pk.rank_split()
    assert small.ranks_host == [0, 16, 0, 64, 0] and small.max_rank == 64
    assert large.ranks_host == [0, 0, 512, 0, 0] and large.max_rank == 512
    assert small.a_pack is pk.a_pack and large.b_off is pk.b_off
    only_small = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, [16, 0, 64, 0],
                                                     applicable=[True, False, True, False])
    assert only_small.rank_split()[1] is None


# -- host mirrors of the reference API ---------------------------------------
def test_kernels_promote_rank_matches_reference_table(kats):
    for rank, expected in kats["promote_rank"]["cases"]:
        assert kernels.promote_rank(rank) == expected
    for r in kats["promote_rank"]["raises"]:
        with pytest.raises(ValueError):
            kernels.promote_rank(r)
    assert kernels.get_switch_lora_expand_config() == {"block_m": 32, "block_n": 32, "num_warps": 4, "num_stages": 1}


def test_build_w_ext_row_order():
    W = torch.arange(6.0).reshape(2, 3)
    A16 = torch.arange(2 * 2 * 16 * 3, dtype=torch.float32).reshape(2, 2, 16, 3)
    A32 = -torch.arange(1 * 2 * 32 * 3, dtype=torch.float32).reshape(1, 2, 32, 3)
    w = kernels.build_w_ext(W, {32: A32, 16: A16})
    assert w.shape == (2 + 64 + 64, 3)
    assert torch.equal(w[:2], W)
    assert torch.equal(w[2:2 + 16], A16[0, 0])          # tier 16, adapter 0, slice 0
    assert torch.equal(w[2 + 16:2 + 32], A16[0, 1])     # ... slice 1
    assert torch.equal(w[2 + 32:2 + 48], A16[1, 0])     # adapter 1
    assert torch.equal(w[66:98], A32[0, 0])              # tier 32 after tier 16


def _fill(layer, ranks, seed=0, zero=()):
    g = torch.Generator().manual_seed(seed)
    A_sl = [layer.lora_A] if layer.num_slices == 1 else list(layer.lora_A_slices)
    B_sl = [layer.lora_B] if layer.num_slices == 1 else list(layer.lora_B_slices)
    with torch.no_grad():
        for s in range(layer.num_slices):
            for a, r in enumerate(ranks):
                if a in zero:
                    continue
                A_sl[s].data[a, 0, :r] = torch.randn(r, A_sl[s].shape[3], generator=g)
                B_sl[s].data[a, 0, :, :r] = torch.randn(B_sl[s].shape[2], r, generator=g)
    return [a.data.clone().numpy() for a in A_sl], [b.data.clone().numpy() for b in B_sl]


def test_vllm_finalize_tables_match_oracle():
    """finalize_weights on CPU tensors reproduces the reference's tables."""
    slices = (64, 32, 32)
    ranks = [32, 8, 16, 16, 32]
    base = torch.nn.Linear(48, sum(slices), bias=False)
    layer = vllm_layers.SwitchedLoRALinear(base, len(ranks), 32, num_slices=3, output_slices=slices)
    A, B = _fill(layer, ranks, zero=(4,))
    W = base.weight.data.clone().numpy()
    layer.finalize_weights(ranks)
    applicable = omap.applicability(A, ranks)
    remap, order, eff = omap.build_remap(applicable, ranks)
    na, tile_slice, scr, tiers = omap.finalize_tables(slices, order, eff, 32)
    assert layer.remap_table.tolist() == remap.tolist()
    assert layer._na == na
    assert layer.tile_to_slice.tolist() == tile_slice.tolist()
    assert layer.slice_col_r.tolist() == scr.tolist()
    np.testing.assert_array_equal(layer.w_ext.numpy(), omap.build_w_ext(W, A, tiers))
    np.testing.assert_array_equal(layer._lb_packed.numpy(), omap.build_lb_packed(B, tiers))
    # per-global-adapter tables of the segment path
    for g in range(1, len(ranks) + 1):
        if remap[g] == 0:
            assert layer._seg_ranks[g] == 0
        else:
            assert layer._seg_ranks[g] == eff[g - 1]
    # checkpoint tensors are released
    assert all(p.numel() == 0 for p in layer.lora_A_slices)


def test_vllm_finalize_pads_ranks_promoted_past_storage():
    """Stored rank 8 promotes to tier 16: the tier rows past the stored ones are zero."""
    slices = (32,)
    ranks = [8, 4, 8]
    base = torch.nn.Linear(24, 32, bias=False)
    layer = vllm_layers.SwitchedLoRALinear(base, 3, 8)
    A, B = _fill(layer, ranks, seed=3, zero=(1,))
    W = base.weight.data.clone().numpy()
    layer.finalize_weights(ranks)
    remap, order, eff = omap.build_remap(omap.applicability(A, ranks), ranks)
    na, tile_slice, scr, tiers = omap.finalize_tables(slices, order, eff, 32)
    assert layer.remap_table.tolist() == remap.tolist() == [0, 1, 0, 2]
    assert layer._na == na == (2, 0, 0, 0, 0, 0)
    np.testing.assert_array_equal(layer.w_ext.numpy(), omap.build_w_ext(W, A, tiers))
    np.testing.assert_array_equal(layer._lb_packed.numpy(), omap.build_lb_packed(B, tiers))
    assert layer.w_ext.shape == (32 + 2 * 16, 24)
    assert layer._seg_ranks.tolist() == [0, 16, 0, 16]
    assert layer._seg_zoff.tolist() == [0, 32, 0, 48]
    assert layer._seg_boff.tolist() == [0, 0, 0, 32 * 16]


def test_vllm_quantized_base_layer_is_refused_at_finalize():
    class QLinear(torch.nn.Module):
        input_size, output_size = 64, 32

        def __init__(self):
            super().__init__()
            self.qweight = torch.zeros(8, 32, dtype=torch.int32)

    layer = vllm_layers.SwitchedLoRALinear(QLinear(), 2, 16)
    assert (layer.in_features, layer.out_features) == (64, 32)
    assert layer.lora_A.dtype == torch.float16 and tuple(layer.lora_A.shape) == (2, 1, 16, 64)
    with pytest.raises(NotImplementedError, match="dequantize"):
        layer.finalize_weights([16, 16])
    with pytest.raises(ValueError, match="Unsupported base layer"):
        vllm_layers.SwitchedLoRALinear(torch.nn.ReLU(), 2, 16)


def test_vllm_block_n_alignment_assert():
    base = torch.nn.Linear(16, 96 + 65, bias=False)
    layer = vllm_layers.SwitchedLoRALinear(base, 1, 16, num_slices=2, output_slices=(96, 65))
    _fill(layer, [16])
    with pytest.raises(AssertionError, match="block_n=.*must divide"):
        layer.finalize_weights([16])


def test_packed_adapters_layout_cpu():
    slices = (32, 64)
    NA, H, maxr = 3, 24, 16
    ranks = [8, 16, 12]
    g = torch.Generator().manual_seed(1)
    A = [torch.randn(NA, 1, maxr, H, generator=g) for _ in slices]
    B = [torch.randn(NA, 1, o, maxr, generator=g) for o in slices]
    for s in range(2):
        for a, r in enumerate(ranks):
            A[s][a, 0, r:] = 0
            B[s][a, 0, :, r:] = 0
    pk = switched.PackedAdapters.from_slices(A, B, ranks)
    assert pk.ranks.tolist() == [0, 8, 16, 16]       # 12 rounded up to 16 with zero rows
    for a in range(NA):
        gi = a + 1
        r = pk.ranks_host[gi]
        rows = pk.a_pack.view(-1)[pk.a_off[gi]: pk.a_off[gi] + 2 * r * H].view(2 * r, H)
        for s in range(2):
            assert torch.equal(rows[s * r:(s + 1) * r, :], A[s][a, 0, :r])
        bm = pk.b_pack[pk.b_off[gi]: pk.b_off[gi] + 96 * r].view(96, r)
        assert torch.equal(bm, torch.cat([B[0][a, 0, :, :r], B[1][a, 0, :, :r]]))
    assert pk.slice_bounds == [0, 32, 96]


def test_non_applicable_adapter_is_skipped_in_pack():
    A = [torch.zeros(2, 1, 16, 8)]
    B = [torch.ones(2, 1, 32, 16)]
    A[0][0, 0, :16] = 1.0
    pk = switched.PackedAdapters.from_slices(A, B, [16, 16])
    assert pk.ranks.tolist() == [0, 16, 0]


# -- workloads ---------------------------------------------------------------
def test_workload_routing_shapes():
    r1 = workloads.routing_for(1)
    eff1 = omap.alora_effective_ids(r1.req_ids, r1.positions, r1.cu_seqlens, r1.act_offsets)
    assert r1.num_tokens == 256 and (eff1 == 0).sum() == round(0.2 * 256)
    r2 = workloads.routing_for(2)
    lens = np.diff(r2.cu_seqlens)
    assert r2.num_tokens == 8192 and lens.size == 16 and lens.min() >= 1
    r3 = workloads.routing_for(3)
    assert r3.num_tokens == 4096 and r3.act_offsets is None and r3.req_ids.max() <= 48
    r4 = workloads.routing_for(4)
    assert r4.num_tokens == 48 + 16 * 256
    r0 = workloads.routing_for(0)
    assert r0.num_tokens == 512


def test_workload_module_on_cpu():
    spec = workloads.ModuleSpec("t", 64, (32, 32), [8, 16], 16)
    md = workloads.make_module(spec, 10, 2, torch.float32, "cpu", seed=3)
    assert md.x.shape == (10, 64) and md.y.shape == (10, 64)
    # rows past the true rank are zero (stored padded to max_r)
    assert torch.all(md.lora_A_slices[0][0, 0, 8:] == 0) and torch.all(md.lora_B_slices[1][0, 0, :, 8:] == 0)
    # B is pre-scaled by alpha/r: std ~ 0.02 * 16/r
    assert md.lora_B_slices[0][1, 0].std().item() < 0.05


def _packed_stub(H, slices, NA, max_rank, dtype=torch.bfloat16):
    """The attributes the small-path plan reads, without device memory."""
    from types import SimpleNamespace

    bounds = [0]
    for w in slices:
        bounds.append(bounds[-1] + w)
    return SimpleNamespace(dtype=dtype, hidden=H, num_slices=len(slices), num_adapters=NA, max_rank=max_rank,
                           out_total=bounds[-1], slice_bounds=bounds, a_pack=SimpleNamespace(device=torch.device("cuda", 0)),
                           a_off_host=[0] * (NA + 1), b_off_host=[0] * (NA + 1), ranks_host=[0] + [max_rank] * NA)


@pytest.mark.parametrize("H,slices,NA,r,T,seqs,small,rs", [
    (4096, (4096, 1024, 1024), 12, 32, 256, 256, True, 1),     # decode QKV: one chunk per adapter
    (2048, (2048,), 4, 8, 512, 4, True, 4),                     # 4 sequences of 128 on 4 adapters
    (4096, (4096,), 2, 64, 512, None, True, 8),                 # ~256 tokens per adapter
    (4096, (12800, 12800), 24, 32, 128, None, True, 1),         # gate_up: tile groups of 5 bring the grid to 672
    (4096, (12800, 12800), 24, 64, 512, None, False, 1),        # rank 64 (no tile groups): grid past the GPU
    (12800, (4096,), 12, 16, 1024, 8, True, 2),                 # 128-token groups: split 2 fits 3 WG/CU
    (12800, (4096,), 12, 16, 1024, 4, False, 1),                # 256-token groups: 4 chunks per WG, segments
    (4096, (4096,), 4, 128, 64, None, False, 1),                # rank past the small kernel's limit
    (12800, (4096,), 48, 32, 128, None, False, 1),              # 48 adapters: 39 MB of lora_A, segments
    (12800, (4096,), 24, 32, 128, None, True, 1),               # 24 adapters: 19.7 MB, one launch
])
def test_small_path_plan(monkeypatch, H, slices, NA, r, T, seqs, small, rs):
    """The host's path choice and row split on a 256-CU part (the decisions
    measured on the GPU for these shapes)."""
    from granite_switch_amd import switched

    monkeypatch.setattr(switched, "_device_cus", lambda device: 256)
    monkeypatch.setattr(switched, "_small_plans", {})
    pk = _packed_stub(H, slices, NA, r)
    assert switched.small_preferred(pk, T, seqs) is small
    if small:
        assert switched.small_row_split(pk, T, seqs) == rs
        assert switched.small_workgroups(pk, T, rs) <= 4 * 256
    pk.a_off_host = None                                        # without host tables: never the small kernel
    assert switched.small_preferred(pk, T, seqs) is False


def test_small_path_plan_largest_group_hint(monkeypatch):
    """A known largest group replaces the estimate: 4 sequences of 128 tokens
    on 4 adapters with 3 of them on one adapter (384 tokens) go to the segment
    kernels, which measured faster there (gate_up 4096 -> 25600: 28.7 against
    34.5 us); without the hint the estimate (128) picks the one-launch kernel."""
    from granite_switch_amd import switched

    monkeypatch.setattr(switched, "_device_cus", lambda device: 256)
    monkeypatch.setattr(switched, "_small_plans", {})
    pk = _packed_stub(4096, (12800, 12800), 4, 32)
    assert switched.small_preferred(pk, 512, 4) is True
    assert switched.small_preferred(pk, 512, 4, largest_group=384) is False
    assert switched.small_preferred(pk, 512, 4, largest_group=128) is True
    # a hint larger than the batch is clamped to it
    assert switched.small_row_split(pk, 512, 4, largest_group=10 ** 6) == switched.small_row_split(pk, 512, 4, 512)


def test_pending_from_sync_reads_each_adapters_counter_low_bits():
    """Adapter g's 64-bit launch counter sits at int32 words [32 g, 32 g + 1]
    (low half first); an unfinished launch shows in its low 20 bits."""
    sync = torch.zeros(int(_lib.load().gs_small_sync_bytes()) // 4, dtype=torch.int32)
    counters = {1: 3 << 20,                       # three complete launches
                5: (7 << 32) | (1 << 20) | 17,    # a high epoch, one launch half counted (17)
                64: (2 << 20) | 5}                # last adapter line: 5 pending
    for g, c in counters.items():
        sync[32 * g] = np.int64(c & 0xFFFFFFFF).astype(np.uint32).view(np.int32)
        sync[32 * g + 1] = np.int32(c >> 32)
    sync[2] = 1                                   # the error word is not a counter
    sync[0] = 123                                 # nor is line 0
    assert switched.pending_from_sync(sync) == 17 + 5
    assert switched.pending_from_counters(torch.tensor([0, 1 << 20, (9 << 20) + 3])) == 3


def test_wait_limit_setter_round_trips():
    prev = switched.set_small_wait_limit(7)
    try:
        assert switched.set_small_wait_limit(0) == 7
        assert switched.set_small_wait_limit(None) == 0
        assert switched.set_small_wait_limit(None) == prev        # None restores the default
    finally:
        switched.set_small_wait_limit(prev)


def test_reused_segments_are_checked_before_any_launch():
    """build_segments(out=...) writes eff_ids / perm / seg_offsets in place: a
    Segments allocated for a smaller batch or another adapter count is refused
    before the builder runs (the kernels would write past its buffers)."""
    dev = torch.device("cpu")

    def segs(T, NA):
        return switched.Segments(eff_ids=torch.empty(T, dtype=torch.int32), seg_offsets=torch.empty(NA + 1, dtype=torch.int32),
                                 perm=torch.empty(max(T, 1), dtype=torch.int32), num_tokens=T, num_adapters=NA)

    switched._check_reused_segments(segs(64, 4), 64, 4, dev)
    switched._check_reused_segments(segs(64, 4), 10, 4, dev)       # a larger buffer holds a smaller batch
    with pytest.raises(ValueError, match="eff_ids holds 64"):
        switched._check_reused_segments(segs(64, 4), 65, 4, dev)
    with pytest.raises(ValueError, match="allocated for 4 adapters"):
        switched._check_reused_segments(segs(64, 4), 64, 5, dev)
    s = segs(64, 4)
    s.perm = torch.empty(32, dtype=torch.int32)
    with pytest.raises(ValueError, match="perm holds 32"):
        switched._check_reused_segments(s, 64, 4, dev)
    s = segs(64, 4)
    s.seg_offsets = torch.empty(5, dtype=torch.int64)
    with pytest.raises(ValueError, match="seg_offsets must be a contiguous int32"):
        switched._check_reused_segments(s, 64, 4, dev)
    with pytest.raises(ValueError, match="on cuda"):
        switched._check_reused_segments(segs(64, 4), 64, 4, torch.device("cuda", 0))


def test_population_workloads():
    """The bench's adapter populations: the rank-512 one adds adapter N+1 of
    rank 512 and draws ids over N+1; the idle one keeps the batch, all base."""
    for cfg in (1, 4):
        na = workloads.num_adapters_for(cfg)
        r = workloads.population_routing(cfg, "r512")
        assert workloads.population_adapters(cfg, "r512") == na + 1
        assert r.req_ids.max() == na + 1 and r.req_ids.min() >= 0
        assert r.num_tokens == workloads.routing_for(cfg).num_tokens
        for spec, base in zip(workloads.population_specs(cfg, "r512"), workloads.module_specs(cfg)):
            assert spec.ranks == list(base.ranks) + [512] and spec.max_rank == 512
        idle = workloads.population_routing(cfg, "all_base")
        assert not idle.req_ids.any()
        assert np.array_equal(idle.positions, workloads.routing_for(cfg).positions)
    assert workloads.population_specs(2, "balanced") == workloads.module_specs(2)


def _pair_query(dtype, T, H, slices, ranks):
    i32 = lambda v: (ctypes.c_int32 * len(v))(*[int(u) for u in v])
    r8 = [0] + [((int(r) + 7) // 8) * 8 if r > 0 else 0 for r in ranks]
    bounds = [0] + [int(b) for b in np.cumsum(slices)]
    return _lib.load().gs_switched_lora_pair(dtype, T, H, int(sum(slices)), i32(bounds), len(slices), len(ranks),
                                             max(r8), i32(r8))


def test_pair_launch_query():
    """gs_switched_lora_pair tells whether gs_switched_lora runs a module's two
    rank classes in its pair launches (on a 256-CU part; the host plan falls
    back to 256 without a GPU): the bench's rank-512 populations in bf16 do,
    their balanced ones (one class) and fp32 do not, nor a large class that
    holds a prefill batch's worth of tokens (not sparse).  Bad arguments give
    a negated status."""
    for cfg in (1, 4):
        for pop in ("balanced", "r512"):
            r = workloads.population_routing(cfg, pop)
            NA = workloads.population_adapters(cfg, pop)
            for spec in workloads.population_specs(cfg, pop):
                ranks = spec.ranks[:NA]
                want = 1 if pop == "r512" else 0
                assert _pair_query(_lib.GS_DTYPE_BF16, r.num_tokens, spec.hidden, spec.output_slices, ranks) == want
                assert _pair_query(_lib.GS_DTYPE_FP32, r.num_tokens, spec.hidden, spec.output_slices, ranks) == 0
    # two adapters, one of rank 512, 8192 tokens: ~4096 expected on it
    assert _pair_query(_lib.GS_DTYPE_BF16, 8192, 4096, (4096,), [32, 512]) == 0
    assert _pair_query(7, 256, 4096, (4096,), [32, 512]) < 0
