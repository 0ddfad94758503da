"""GPU parity of the reference-form ops and layer wrappers.

* ``torch.ops.granite_switch.switch_lora_expand`` / ``..._swiglu`` vs the
  oracle's restatement of the reference kernels, on the same bf16 x_ext;
* vLLM-form ``SwitchedLoRALinear`` (fused w_ext GEMM + expand, segment path and
  op path) vs the switched-LoRA math;
* HF-form layers vs the HF loop restated in the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from granite_switch_amd import hf_layers, meta, ops, switched, vllm_layers
from oracle import lora as olora
from oracle import mapping as omap

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _np(t):
    return t.detach().float().cpu().numpy()


def _close(got, ref, tol, what):
    err = np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))
    bad = err > tol + tol * np.abs(ref)
    assert not bad.any(), f"{what}: {int(bad.sum())} bad, max abs err {err.max():.3e}"


def _make_vllm_layer(dev, K, slices, ranks, seed, fuse_swiglu=False, bias=False, zero=()):
    g = torch.Generator(device=dev).manual_seed(seed)
    base = torch.nn.Linear(K, sum(slices), bias=bias).to(device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        base.weight.copy_(torch.randn(sum(slices), K, generator=g, device=dev) / K ** 0.5)
    max_r = max(ranks)
    layer = vllm_layers.SwitchedLoRALinear(base, len(ranks), max_r, num_slices=len(slices),
                                           output_slices=slices if len(slices) > 1 else None, fuse_swiglu=fuse_swiglu)
    A_sl = [layer.lora_A] if len(slices) == 1 else list(layer.lora_A_slices)
    B_sl = [layer.lora_B] if len(slices) == 1 else list(layer.lora_B_slices)
    with torch.no_grad():
        for s in range(len(slices)):
            for a, r in enumerate(ranks):
                if a in zero:
                    continue
                A_sl[s].data[a, 0, :r] = (torch.randn(r, K, generator=g, device=dev) / K ** 0.5).to(torch.bfloat16)
                B_sl[s].data[a, 0, :, :r] = (torch.randn(slices[s], r, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    A_np = [_np(a) for a in A_sl]
    B_np = [_np(b) for b in B_sl]
    W = _np(base.weight)
    layer.finalize_weights(ranks)
    return layer, W, A_np, B_np


def _ctx_for(dev, layer, ids):
    fm = meta.FusedLoRAKernelMeta(dev)
    fm.register_remap_tables(layer.remap_table.unsqueeze(0), [(layer.in_features, layer._N_total, layer._num_applicable)])
    ctx = meta.LoRAContext()
    fm.prepare_and_store(ids, ctx)
    return ctx


@pytest.mark.parametrize("native_gemm", [False, True])
@pytest.mark.parametrize("slices,ranks", [((4096, 1024, 1024), [32] * 12), ((2048,), [8, 16, 32, 64, 128, 16]),
                                          ((512, 256), [16, 512, 8])])
def test_vllm_layer_segment_and_op_paths(dev, slices, ranks, native_gemm):
    K, T = 1024, 300
    _say(f"vllm layer slices={slices} ranks={ranks} native_gemm={native_gemm}")
    layer, W, A, B = _make_vllm_layer(dev, K, slices, ranks, seed=5, zero=(1,))
    layer.native_gemm = native_gemm
    g = torch.Generator(device=dev).manual_seed(8)
    x = torch.randn(T, K, generator=g, device=dev).to(torch.bfloat16)
    ids = torch.randint(0, len(ranks) + 1, (T,), generator=g, device=dev)
    ctx = _ctx_for(dev, layer, ids)
    layer._lora_ctx = ctx
    out_seg, _ = layer(x)                       # segment path
    out_seg = out_seg.clone()
    seg = ctx.segments
    ctx.segments = None
    out_op, _ = layer(x)                        # reference op path (bitmask tiles)
    ctx.segments = seg
    torch.cuda.synchronize()
    ids_h = ids.cpu().numpy()
    eff = ids_h.copy()
    eff[eff == 2] = 0                           # adapter 2 (index 1) is not applicable
    xb = _np(x)
    ref = olora.switched_lora_apply(xb @ W.T, xb, eff, A, B, slices, ranks, "f64")
    _close(_np(out_seg), ref, 2e-2, "segment path")
    _close(_np(out_op), ref, 2e-2, "op path")
    # both paths read the same bf16 shrink columns; they differ by at most 1 ulp of the output
    d = (out_seg.float() - out_op.float()).abs()
    assert (d <= 2 ** -7 * out_op.float().abs().clamp_min(1.0)).all()


def test_switch_lora_expand_op_matches_oracle(dev):
    """The op alone, on a fixed bf16 x_ext, vs the oracle's restatement of the Triton kernel."""
    slices, ranks, K, T = (256, 128, 128), [16, 32, 16, 64, 8], 512, 200
    layer, W, A, B = _make_vllm_layer(dev, K, slices, ranks, seed=9)
    g = torch.Generator(device=dev).manual_seed(10)
    x = torch.randn(T, K, generator=g, device=dev).to(torch.bfloat16)
    ids = torch.randint(0, len(ranks) + 1, (T,), generator=g, device=dev)
    ctx = _ctx_for(dev, layer, ids)
    x_ext = torch.mm(x, layer.w_ext.T)
    x_ext0 = _np(x_ext)
    loc = ctx.remapped_indices[0]
    for idx in (loc, loc.to(torch.int32)):
        xe = x_ext.clone()
        ops.op("switch_lora_expand")(xe, idx, ctx.per_module_bitmasks[0], layer._lb_packed, layer.tile_to_slice,
                                      layer.slice_col_r, *layer._na, layer._S, layer._block_n, layer._N_total)
        torch.cuda.synchronize()
        ref = olora.switch_lora_expand_xext(x_ext0, loc.cpu().numpy(), ctx.per_module_bitmasks[0].cpu().numpy(),
                                            _np(layer._lb_packed), layer.tile_to_slice.cpu().numpy(),
                                            layer.slice_col_r.cpu().numpy(), layer._na, layer._S, layer._block_n,
                                            layer._N_total)
        _close(_np(xe), ref, 2e-2, "switch_lora_expand")
        base = (loc == 0).cpu().numpy()
        assert np.array_equal(_np(xe)[base], x_ext0[base]), "base rows touched"
        # shrink columns are never written
        assert np.array_equal(_np(xe)[:, layer._N_total:], x_ext0[:, layer._N_total:])


@pytest.mark.parametrize("slices,ranks,T", [
    ((4096, 96), [32, 16, 32, 8], 1000),      # column blocks of 64 (a partial last one), ragged last row group
    ((512,), [64, 16, 64], 700),              # rank-64 tier, 32-column blocks
    ((4096, 1024, 1024), [32, 16, 32, 8], 300),   # 32-column blocks over eight row tiles, ragged last group
    ((4096, 2048), [64, 16, 8], 400),         # eight row tiles with a rank-64 tier
    ((256, 128), [128, 16], 300),             # a rank-128 tier: the per-tile kernel at decode sizes
    ((1024, 256), [32, 16, 8], 1500),         # past 1024 rows: the per-tile kernel
    ((1024, 32), [32, 16], 1100),             # per-tile kernel, last 128-column tile a quarter full
    ((1024, 32), [32, 16], 600),              # column-block kernel, N = 33 blocks of 32
])
def test_switch_lora_expand_op_kernel_forms(dev, slices, ranks, T):
    """Each kernel form of the reference op (column-block at decode batch
    sizes with 32- and 64-column blocks, over four or eight row tiles;
    per-tile past 1024 rows or with a tier
    above rank 64) vs the oracle, with int64 and int32 ids; base rows and the
    shrink columns are untouched."""
    K = 256
    layer, W, A, B = _make_vllm_layer(dev, K, slices, ranks, seed=31 + T)
    g = torch.Generator(device=dev).manual_seed(T)
    x = torch.randn(T, K, generator=g, device=dev).to(torch.bfloat16)
    ids = torch.randint(0, len(ranks) + 1, (T,), generator=g, device=dev)
    ids[T // 3: T // 3 + 40] = 0                     # a run of base rows (an all-base tile)
    ctx = _ctx_for(dev, layer, ids)
    x_ext = torch.mm(x, layer.w_ext.T)
    x_ext0 = _np(x_ext)
    loc = ctx.remapped_indices[0]
    ref = olora.switch_lora_expand_xext(x_ext0, loc.cpu().numpy(), ctx.per_module_bitmasks[0].cpu().numpy(),
                                        _np(layer._lb_packed), layer.tile_to_slice.cpu().numpy(),
                                        layer.slice_col_r.cpu().numpy(), layer._na, layer._S, layer._block_n,
                                        layer._N_total)
    base = (loc == 0).cpu().numpy()
    for idx in (loc, loc.to(torch.int32)):
        _say(f"expand op forms: slices={slices} ranks={ranks} T={T} ids={idx.dtype}")
        xe = x_ext.clone()
        ops.op("switch_lora_expand")(xe, idx, ctx.per_module_bitmasks[0], layer._lb_packed, layer.tile_to_slice,
                                      layer.slice_col_r, *layer._na, layer._S, layer._block_n, layer._N_total)
        torch.cuda.synchronize()
        got = _np(xe)
        _close(got, ref, 2e-2, "switch_lora_expand")
        assert np.array_equal(got[base], x_ext0[base]), "base rows touched"
        assert np.array_equal(got[:, layer._N_total:], x_ext0[:, layer._N_total:]), "shrink columns written"


@pytest.mark.parametrize("slices,T", [
    ((4096, 96), 1000),     # 64-column blocks
    ((512,), 700),          # 32-column blocks
    ((2048, 1024), 500),    # 32-column blocks over eight row tiles
])
def test_switch_lora_expand_op_runs_of_adapters(dev, slices, T):
    """The column-block form with 20 adapters (more than one staging chunk)
    and ids in runs, so a workgroup's tiles follow a few adapters, some past
    the first chunk, and tiles that follow none of the first ones; vs the
    oracle."""
    K, ranks = 256, [16, 32] * 10
    layer, W, A, B = _make_vllm_layer(dev, K, slices, ranks, seed=77 + T)
    g = torch.Generator(device=dev).manual_seed(5 + T)
    x = torch.randn(T, K, generator=g, device=dev).to(torch.bfloat16)
    order = [19, 3, 17, 0, 18, 20, 9, 16, 2, 20, 13, 1, 19, 18, 11, 17, 20, 4]
    ids = torch.tensor([order[(m // 57) % len(order)] for m in range(T)], device=dev)
    ctx = _ctx_for(dev, layer, ids)
    x_ext = torch.mm(x, layer.w_ext.T)
    x_ext0 = _np(x_ext)
    loc = ctx.remapped_indices[0]
    ref = olora.switch_lora_expand_xext(x_ext0, loc.cpu().numpy(), ctx.per_module_bitmasks[0].cpu().numpy(),
                                        _np(layer._lb_packed), layer.tile_to_slice.cpu().numpy(),
                                        layer.slice_col_r.cpu().numpy(), layer._na, layer._S, layer._block_n,
                                        layer._N_total)
    base = (loc == 0).cpu().numpy()
    _say(f"expand op runs of adapters: slices={slices} T={T}")
    xe = x_ext.clone()
    ops.op("switch_lora_expand")(xe, loc, ctx.per_module_bitmasks[0], layer._lb_packed, layer.tile_to_slice,
                                  layer.slice_col_r, *layer._na, layer._S, layer._block_n, layer._N_total)
    torch.cuda.synchronize()
    got = _np(xe)
    _close(got, ref, 2e-2, "switch_lora_expand")
    assert np.array_equal(got[base], x_ext0[base]), "base rows touched"


def test_switch_lora_expand_zero_bitmask_skips(dev):
    slices, ranks, K, T = (128,), [16, 16], 256, 64
    layer, W, A, B = _make_vllm_layer(dev, K, slices, ranks, seed=12)
    x = torch.randn(T, K, device=dev).to(torch.bfloat16)
    x_ext = torch.mm(x, layer.w_ext.T)
    ids = torch.ones(T, dtype=torch.int64, device=dev)
    bm = torch.zeros(2, dtype=torch.int64, device=dev)          # says: no adapter anywhere
    xe = x_ext.clone()
    ops.op("switch_lora_expand")(xe, ids, bm, layer._lb_packed, layer.tile_to_slice, layer.slice_col_r, *layer._na,
                                  layer._S, layer._block_n, layer._N_total)
    torch.cuda.synchronize()
    assert torch.equal(xe, x_ext)


def test_reference_ops_zero_rows(dev):
    """The reference ops on a batch of no rows return without a launch and
    leave their outputs as they were (the expand) or empty."""
    slices, ranks, K = (128,), [16, 16], 256
    layer, W, A, B = _make_vllm_layer(dev, K, slices, ranks, seed=21)
    x_ext = torch.zeros(0, layer.w_ext.shape[0], dtype=torch.bfloat16, device=dev)
    ids = torch.zeros(0, dtype=torch.int64, device=dev)
    bm = torch.zeros(0, dtype=torch.int64, device=dev)
    ops.op("switch_lora_expand")(x_ext, ids, bm, layer._lb_packed, layer.tile_to_slice, layer.slice_col_r, *layer._na,
                                  layer._S, layer._block_n, layer._N_total)
    H = 128
    lg, _, _, _ = _make_vllm_layer(dev, K, (H, H), [16, 32], seed=22, fuse_swiglu=True)
    xg = torch.zeros(0, lg.w_ext.shape[0], dtype=torch.bfloat16, device=dev)
    out = torch.empty(0, H, dtype=torch.bfloat16, device=dev)
    ops.op("switch_lora_expand_swiglu")(out, xg, ids, bm, lg._lb_packed, lg.slice_col_r, *lg._na, 2, 32, H, 2 * H)
    torch.cuda.synchronize()
    assert x_ext.shape[0] == 0 and out.shape == (0, H)


@pytest.mark.parametrize("with_ctx", [True, False])
def test_swiglu_path(dev, with_ctx):
    H, K, T = 1280, 512, 150
    ranks = [32, 16, 32]
    layer, W, A, B = _make_vllm_layer(dev, K, (H, H), ranks, seed=13, fuse_swiglu=True)
    g = torch.Generator(device=dev).manual_seed(14)
    x = torch.randn(T, K, generator=g, device=dev).to(torch.bfloat16)
    ids = torch.randint(0, 4, (T,), generator=g, device=dev)
    if with_ctx:
        layer._lora_ctx = _ctx_for(dev, layer, ids)
    else:
        layer._lora_ctx = None
    out, _ = layer(x)
    torch.cuda.synchronize()
    xb = _np(x)
    eff = ids.cpu().numpy() if with_ctx else np.zeros(T, np.int64)
    corr = olora.switched_lora_apply(xb @ W.T, xb, eff, A, B, (H, H), ranks, "f64")
    gte, up = corr[:, :H], corr[:, H:]
    ref = gte / (1 + np.exp(-gte)) * up
    _close(_np(out), ref, 3e-2, "swiglu")
    assert out.is_contiguous() and out.shape == (T, H)


def test_swiglu_op_matches_oracle(dev):
    H, K, T = 256, 256, 97
    ranks = [16, 64]
    layer, W, A, B = _make_vllm_layer(dev, K, (H, H), ranks, seed=15, fuse_swiglu=True)
    x = torch.randn(T, K, device=dev).to(torch.bfloat16)
    ids = torch.randint(0, 3, (T,), device=dev)
    ctx = _ctx_for(dev, layer, ids)
    x_ext = torch.mm(x, layer.w_ext.T)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    ops.op("switch_lora_expand_swiglu")(out, x_ext, ctx.remapped_indices[0], ctx.per_module_bitmasks[0],
                                         layer._lb_packed, layer.slice_col_r, *layer._na, 2, 32, H, 2 * H)
    torch.cuda.synchronize()
    ref = olora.expand_swiglu_xext(_np(x_ext), ctx.remapped_indices[0].cpu().numpy(),
                                   ctx.per_module_bitmasks[0].cpu().numpy(), _np(layer._lb_packed),
                                   layer.slice_col_r.cpu().numpy(), layer._na, 2, H, 2 * H)
    _close(_np(out), ref, 2e-2, "swiglu op")


def _runs_of_ids(T, NA, seed, max_run=300):
    """Per-token ids as runs (prefill sequences of one request each), with
    single tokens of random requests in between (decode rows): tiles holding
    one adapter, several, or only base rows."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < T:
        if rng.random() < 0.3:
            out.extend(rng.integers(0, NA + 1, size=int(rng.integers(1, 40))).tolist())
        else:
            out.extend([int(rng.integers(0, NA + 1))] * int(rng.integers(1, max_run)))
    return np.asarray(out[:T], np.int64)


@pytest.mark.parametrize("M,H,ranks,idx32", [(2000, 1376, [16, 32, 32, 16], False), (1500, 256, [64, 16, 8], True),
                                             (1100, 512, [128, 32], False), (1056, 640, [16] * 5, True),
                                             (1200, 384, [256, 16], False)])
def test_swiglu_op_large_batch_forms(dev, M, H, ranks, idx32):
    """The row-strip SwiGLU kernel (above 1024 rows, tiers up to rank 128:
    LDS shrink widths 32, 64 and 128, h not a multiple of 128, a partial last
    row tile, tiles of one, several or no adapters, int32 and int64 ids) and
    the per-tile kernel it leaves rank 256 to, against the oracle."""
    K = 256
    _say(f"swiglu op M={M} H={H} ranks={ranks} idx32={idx32}")
    layer, W, A, B = _make_vllm_layer(dev, K, (H, H), ranks, seed=17 + M, fuse_swiglu=True)
    g = torch.Generator(device=dev).manual_seed(M)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    ids = torch.tensor(_runs_of_ids(M, len(ranks), M), device=dev)
    ctx = _ctx_for(dev, layer, ids)
    x_ext = torch.mm(x, layer.w_ext.T)
    loc = ctx.remapped_indices[0]
    if idx32:
        loc = loc.to(torch.int32)
    out = torch.full((M, H), 7.0, dtype=torch.bfloat16, device=dev)
    ops.op("switch_lora_expand_swiglu")(out, x_ext, loc, ctx.per_module_bitmasks[0], layer._lb_packed,
                                         layer.slice_col_r, *layer._na, 2, 32, H, 2 * H)
    torch.cuda.synchronize()
    ref = olora.expand_swiglu_xext(_np(x_ext), ctx.remapped_indices[0].cpu().numpy(),
                                   ctx.per_module_bitmasks[0].cpu().numpy(), _np(layer._lb_packed),
                                   layer.slice_col_r.cpu().numpy(), layer._na, 2, H, 2 * H)
    _close(_np(out), ref, 2e-2, "swiglu op")


@pytest.mark.parametrize("M", [96, 1500])
def test_swiglu_op_extreme_gates(dev, M):
    """silu(g) * u for gates from -300 to 300 (e^-g overflowing and
    underflowing fp32), tiny gates and zero, on base rows (no delta), both
    kernel forms: every output within one bf16 ulp of the exact value, and
    the exact value's sign where it is zero."""
    H, K = 256, 128
    layer, W, A, B = _make_vllm_layer(dev, K, (H, H), [16], seed=31, fuse_swiglu=True)
    ids = torch.zeros(M, dtype=torch.int64, device=dev)
    ctx = _ctx_for(dev, layer, ids)
    x = torch.randn(M, K, device=dev).to(torch.bfloat16)
    x_ext = torch.mm(x, layer.w_ext.T)
    rng = np.random.default_rng(5)
    special = np.array([-300, -120, -89, -87, -20, -1, -1e-3, -1e-30, 0, 1e-30, 1e-3, 1, 20, 87, 89, 120, 300],
                       np.float64)
    g = np.concatenate([special, rng.uniform(-12, 12, size=M * H - special.size)]).reshape(M, H)
    u = rng.uniform(-4, 4, size=(M, H))
    x_ext[:, :H] = torch.tensor(g, dtype=torch.float32, device=dev).to(torch.bfloat16)
    x_ext[:, H:2 * H] = torch.tensor(u, dtype=torch.float32, device=dev).to(torch.bfloat16)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
    ops.op("switch_lora_expand_swiglu")(out, x_ext, ctx.remapped_indices[0], ctx.per_module_bitmasks[0],
                                         layer._lb_packed, layer.slice_col_r, *layer._na, 2, 32, H, 2 * H)
    torch.cuda.synchronize()
    gb = _np(x_ext[:, :H]).astype(np.float64)
    ub = _np(x_ext[:, H:2 * H]).astype(np.float64)
    with np.errstate(over="ignore"):
        exact = gb / (1.0 + np.exp(-gb)) * ub
    got = _np(out).astype(np.float64)
    # one bf16 ulp (or less) of the exact value; below 1e-30 (gates under
    # about -70, where fp32's e^-g overflows past -88.7 as in the reference's
    # own fp32 evaluation) any result of that size or zero
    ulp = np.maximum(np.abs(exact) * 2.0 ** -7, 1e-30)
    assert np.all(np.abs(got - exact) <= ulp), float(np.max(np.abs(got - exact) / ulp))
    assert np.array_equal(np.signbit(got[exact == 0]), np.signbit(exact[exact == 0]))


@pytest.mark.parametrize("merged", [False, True])
def test_hf_layers_match_hf_loop(dev, merged):
    K, NA, R = 384, 5, 16
    torch.manual_seed(0)
    if merged:
        slices = (256, 128, 128)
        layer = hf_layers.MergedSwitchedLoRALinear(K, slices, NA, R).to(dev)
        A_sl, B_sl = list(layer.lora_A_slices), list(layer.lora_B_slices)
    else:
        slices = (320,)
        layer = hf_layers.SwitchedLoRALinear(K, 320, NA, R).to(dev)
        A_sl, B_sl = [layer.lora_A], [layer.lora_B]
    with torch.no_grad():
        for B in B_sl:
            B.copy_(torch.randn_like(B) * 0.1)
    x = torch.randn(3, 40, K, device=dev)
    ids = torch.randint(0, NA + 1, (3, 40), device=dev)
    # the kernels compute no gradients: a forward autograd would track raises
    with pytest.raises(RuntimeError, match="no gradients"):
        layer(x, ids)
    with torch.no_grad():
        out = layer(x, ids)
        base = layer.base_layer(x)
    torch.cuda.synchronize()

    def ref_of(b_slices):
        return olora.switched_lora_apply(_np(base).reshape(-1, sum(slices)), _np(x).reshape(-1, K),
                                         ids.cpu().numpy().reshape(-1), [_np(a) for a in A_sl],
                                         [_np(b) for b in b_slices], slices, None, "fp32")

    _close(_np(out).reshape(-1, sum(slices)), ref_of(B_sl), 1e-4, "hf layer")
    # without freeze() the pack is cached until a weight changes
    pack = layer._auto_pack
    with torch.no_grad():
        layer(x, ids)
        assert layer._auto_pack is pack
        B_sl[0].mul_(2.0)                       # an in-place update moves the version counter
        out_b = layer(x, ids)
    assert layer._auto_pack is not pack
    torch.cuda.synchronize()
    _close(_np(out_b).reshape(-1, sum(slices)), ref_of(B_sl), 1e-4, "hf layer after a weight update")
    with torch.no_grad():
        B_sl[0].mul_(0.5)
    # frozen pack gives the same answer; context-passing indices too
    layer.freeze()
    layer._adapter_indices = ids
    with torch.no_grad():
        out2 = layer(x)
    torch.cuda.synchronize()
    assert torch.allclose(out2, out, atol=1e-6, rtol=1e-6)
    # all-base == base layer exactly
    with torch.no_grad():
        out3 = layer(x, torch.zeros_like(ids))
        assert torch.equal(out3, layer.base_layer(x))


def test_custom_ops_under_torch_compile(dev):
    remap_t = torch.tensor([[0, 1, 2, 3, 4], [0, 1, 0, 2, 0]], dtype=torch.int64, device=dev).T.contiguous()
    ids = torch.randint(0, 5, (200,), device=dev)

    def fn(a, r):
        return torch.ops.granite_switch.compute_per_module_bitmasks(a, r)

    eager = fn(ids, remap_t)
    compiled = torch.compile(fn, fullgraph=True, backend="aot_eager")(ids, remap_t)
    assert torch.equal(compiled, eager)
    assert np.array_equal(eager.cpu().numpy(), omap.compute_bitmasks(ids.cpu().numpy(), remap_t.cpu().numpy(), 32))


def test_segment_op_surface(dev):
    ids = torch.tensor([0, 2, 1, 2, 0, 1], device=dev)
    eff, seg, perm = ops.op("build_segments")(ids, 3, None, None, None)
    torch.cuda.synchronize()
    assert seg.cpu().tolist() == [0, 2, 4, 4]
    assert perm.cpu().tolist()[:4] == [2, 5, 1, 3]
    _ = switched


@pytest.mark.gpu
def test_hf_layer_path_and_check(dev):
    """The HF layer takes the segment kernels by default, which never wait
    across workgroups: with the one-launch kernel's wait bound forced to 0
    from the host its output stays right and check() passes.  With
    path = "auto" a decode-sized batch takes the one-launch kernel, and the
    forced give-up is reported by check()."""
    K, NA, R = 256, 3, 16
    torch.manual_seed(3)
    layer = hf_layers.MergedSwitchedLoRALinear(K, (256, 128), NA, R).to(dev).to(torch.bfloat16)
    with torch.no_grad():
        for B in layer.lora_B_slices:
            B.copy_(torch.randn_like(B) * 0.1)
    layer.freeze()
    x = torch.randn(64, K, device=dev, dtype=torch.bfloat16)
    ids = torch.randint(0, NA + 1, (64,), device=dev)
    assert layer.path == "segments"
    switched.small_reset(dev)
    prev = switched.set_small_wait_limit(0)
    try:
        with torch.no_grad():
            out = layer(x, ids)
            base = layer.base_layer(x)
        torch.cuda.synchronize()
        layer.check()                             # the segment kernels never wait
        ref = olora.switched_lora_apply(_np(base), _np(x), ids.cpu().numpy(),
                                        [_np(a) for a in layer.lora_A_slices], [_np(b) for b in layer.lora_B_slices],
                                        (256, 128), None, "bf16")
        _close(_np(out), ref, 2e-2, "hf layer, segment path")
        layer.path = "auto"
        assert switched.small_preferred(layer._packed, 64)
        with torch.no_grad():
            layer(x, ids)
        torch.cuda.synchronize()
    finally:
        switched.set_small_wait_limit(prev)
    with pytest.raises(switched.SmallPathError):
        layer.check()
    switched.small_reset(dev)
    with torch.no_grad():
        out_auto = layer(x, ids)
    torch.cuda.synchronize()
    layer.check()
    _close(_np(out_auto), ref, 2e-2, "hf layer, one-launch path")
