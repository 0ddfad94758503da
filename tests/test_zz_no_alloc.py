"""The allocation-free entry point ``gs_switched_lora_noalloc`` on the GPU.

It runs the segment path's kernels with their scratch in the library's
static per-GPU array.  Two calls in a row, the second on a smaller batch,
each checked bit for bit against ``gs_switched_lora`` (same kernels, caller
workspace) on the same inputs, and against the oracle at the bf16 tolerance
(|got - ref| <= 2e-2 + 2e-2 |ref|); base rows bit-identical.  Also: a shape
whose scratch exceeds the array is rejected, and a call inside a HIP graph
capture replays correctly.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from granite_switch_amd import _lib, switched, workloads
from oracle import lora as olora

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _np(t):
    return t.detach().float().cpu().numpy()


def _case(dev, spec, T, NA, seed):
    md = workloads.make_module(spec, T, NA, torch.bfloat16, dev, seed=seed)
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, NA + 1, size=T)
    segs = switched.build_segments(torch.tensor(ids, device=dev), NA)
    pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks)
    return md, ids, segs, pk


def _check(dev, md, ids, segs, pk, what):
    y_ref = md.y.clone()
    switched.switched_lora_(y_ref, md.x, segs, pk, path="segments")
    y = md.y.clone()
    switched.switched_lora_noalloc_(y, md.x, segs, pk)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref), f"{what}: differs from gs_switched_lora"
    ref = olora.switched_lora_apply(_np(md.y), _np(md.x), ids, [_np(a) for a in md.lora_A_slices],
                                    [_np(b) for b in md.lora_B_slices], md.spec.output_slices, md.spec.ranks, "bf16")
    got = _np(y).astype(np.float64)
    err = np.abs(got - ref)
    assert np.all(err <= 2e-2 + 2e-2 * np.abs(ref)), f"{what}: max abs err {err.max():.3e}"
    base = ids == 0
    assert np.array_equal(_np(y)[base], _np(md.y)[base]), f"{what}: base rows were modified"


def test_noalloc_two_calls_second_smaller(dev):
    NA = 24
    big = workloads.ModuleSpec("qkv", 4096, (4096, 1024, 1024), [32] * NA, 32)
    small = workloads.ModuleSpec("o", 2048, (2048,), [16, 32, 8] * 8, 32)
    _say("noalloc call 1: qkv 4096->6144, T=4144, 24 adapters")
    _check(dev, *_case(dev, big, 4144, NA, 1), "call 1")
    _say("noalloc call 2: 2048->2048, T=300, mixed ranks")
    _check(dev, *_case(dev, small, 300, NA, 2), "call 2")


def test_noalloc_under_graph_capture(dev):
    spec = workloads.ModuleSpec("gate_up", 4096, (12800, 12800), [32] * 12, 32)
    md, ids, segs, pk = _case(dev, spec, 1024, 12, 3)
    y_eager = md.y.clone()
    switched.switched_lora_(y_eager, md.x, segs, pk, path="segments")
    y = md.y.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        switched.switched_lora_noalloc_(y, md.x, segs, pk)
    for replay in range(3):
        y.copy_(md.y)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _say(f"noalloc graph replay {replay}")
        assert torch.equal(y, y_eager), f"replay {replay} differs from the eager call"


def test_noalloc_rejects_shapes_beyond_the_scratch(dev):
    T = 1 << 20
    with pytest.raises(_lib.GraniteSwitchError) as e:
        _lib.call("gs_switched_lora_noalloc", _lib.GS_DTYPE_BF16, None, 4096, None, 6144, T, 4096, 6144,
                  (_lib.c_i32 * 4)(0, 4096, 5120, 6144), 3, None, None, None, None, None, 24, 64, None, None, None,
                  None)
    assert e.value.status == _lib.GS_ERR_WORKSPACE and "static scratch" in str(e.value)
