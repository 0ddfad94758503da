"""The 32-layer decoder step as the workload specifies it, on the GPU.

Granite-8B-shaped LoRA side: 32 layers x {qkv 4096->6144 (3 slices), o
4096->4096, gate_up 4096->25600 (2 slices), down 12800->4096}, T = 4144 (48
decode tokens + 16 prefill chunks of 256), 24 rank-32 adapters, aLoRA offsets.
The segments are built ONCE per step and reused by all 128 projections, and
the whole step (build + 128 shrink/expand pairs) is captured in one HIP graph
-- the metadata-once flow of src/granite_switch/vllm/granite_switch_model.py:
413-418, 458-460.

Checks: every replay equals the eager step bit for bit (replayed twice, with
eager work and synchronisations in between); every row of every projection of
the first and the last layer, and on the other layers all 48 decode rows and
256 prefill rows (16 per chunk, around each chunk's activation offset), is
within bf16 tolerance of the oracle (|got - ref| <= 2e-2 + 2e-2 |ref|); every
base row of every projection is bit-identical.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from granite_switch_amd import switched, workloads
from oracle import lora as olora
from oracle import mapping as omap

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _say(msg):
    print(msg, flush=True)


def _np(t):
    return t.detach().float().cpu().numpy()


def _sample_rows(r, eff):
    rows = list(range(48))                              # every decode token
    rng = np.random.default_rng(4)
    for c in range(16):
        lo = 48 + 256 * c
        act = np.nonzero(eff[lo:lo + 256] > 0)[0]
        first = int(act[0]) if act.size else 0           # the chunk's first adapted token
        near = [p for p in range(first - 3, first + 5) if 0 <= p < 256]
        rest = rng.choice(np.setdiff1d(np.arange(256), near), 16 - len(near), replace=False)
        rows += [lo + int(p) for p in near] + [lo + int(p) for p in rest]
    return np.unique(np.array(rows))


def test_decoder_step_32_layers_graph_captured(dev):
    wl = workloads.make_workload(4, dev)
    r = wl.routing
    NA, T = wl.num_adapters, r.num_tokens
    specs = workloads.module_specs(4)
    assert len(wl.modules) == 32 * 4 and T == 4144
    _say(f"decoder step: {len(wl.modules)} projections, T={T}, {NA} adapters")
    packs = [switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, md.spec.ranks)
             for md in wl.modules]
    ids = torch.tensor(r.req_ids, device=dev)
    pos = torch.tensor(r.positions, device=dev)
    cu = torch.tensor(r.cu_seqlens, device=dev)
    off = torch.tensor(r.act_offsets, device=dev)
    zbuf = [torch.empty(T, len(s.output_slices) * packs[k].max_rank, dtype=torch.bfloat16, device=dev)
            for k, s in enumerate(specs)]
    ws = max(int(switched._lib.load().gs_shrink_workspace_bytes(T, s.hidden, len(s.output_slices), NA,
                                                                  packs[k].max_rank,
                                                                  switched._i32_array(packs[k].ranks_host)))
             for k, s in enumerate(specs))
    switched.reserve_workspace(dev, ws)
    y0 = [md.y.clone() for md in wl.modules]
    segs = switched.build_segments(ids, NA, pos, cu, off)

    def step():
        switched.build_segments(ids, NA, pos, cu, off, out=segs)          # metadata once per step
        for j, (md, pk) in enumerate(zip(wl.modules, packs)):
            switched.switched_lora_(md.y, md.x, segs, pk, zbuf[j % 4], path="segments")

    def restore():
        for md, y in zip(wl.modules, y0):
            md.y.copy_(y)

    step()                                                                 # eager reference
    torch.cuda.synchronize()
    y_eager = [md.y.clone() for md in wl.modules]
    restore()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for replay in range(2):
        restore()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        same = all(torch.equal(md.y, ye) for md, ye in zip(wl.modules, y_eager))
        _say(f"  replay {replay}: {'bit-identical to eager' if same else 'DIFFERS from eager'}")
        assert same, f"graph replay {replay} differs from the eager step"
        # eager work between replays
        torch.cuda.synchronize()

    eff = omap.alora_effective_ids(r.req_ids, r.positions, r.cu_seqlens, r.act_offsets)
    assert np.array_equal(segs.eff_ids.cpu().numpy(), eff)
    sampled = _sample_rows(r, eff)
    every = np.arange(T)
    base_d = torch.tensor(eff == 0, device=dev)
    worst = 0.0
    for j, (md, y, yin) in enumerate(zip(wl.modules, y_eager, y0)):
        rows = every if j // 4 in (0, 31) else sampled
        rows_d = torch.tensor(rows, device=dev)
        if j % 4 == 0:
            _say(f"  layer {j // 4}: oracle on {rows.size} rows per projection")
        assert torch.equal(y[base_d], yin[base_d]), f"projection {j}: base rows were modified"
        A = [_np(a) for a in md.lora_A_slices]
        B = [_np(b) for b in md.lora_B_slices]
        ref = olora.switched_lora_apply(_np(yin[rows_d]), _np(md.x[rows_d]), eff[rows], A, B, md.spec.output_slices,
                                        md.spec.ranks, "bf16")
        got = _np(y[rows_d]).astype(np.float64)
        err = np.abs(got - ref)
        bad = err > TOL + TOL * np.abs(ref)
        assert not bad.any(), f"projection {j} ({md.spec.name}): {int(bad.sum())} out of tolerance"
        worst = max(worst, float(err.max()))
    _say(f"  all 128 projections within tolerance; max abs err {worst:.3e}")
