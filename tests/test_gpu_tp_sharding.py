"""Tensor-parallel sharding math of the vLLM-form layer, simulated on one GPU.

As tests/vllm/test_tp_sharding_math.py:235-325 of the reference: tp ranks run
one after another on the one GPU.  Each rank's layer gets its shard of the
base weight and loads the FULL checkpoint LoRA tensors through the layer's
weight_loader, which slices them for its rank (src/granite_switch/vllm/core/
lora.py:270-297): column-parallel layers (one slice, or QKV-like three) shard
lora_B along the output; row-parallel layers shard lora_A along the input and
all-reduce the partial output (LoRA delta included) before the bias.

Checks, for tp in {2, 4, 8} and both expand paths (segments, and the
reference op over bitmask tiles): every rank derives the same remap table;
column-parallel outputs concatenated slice by slice equal the tp = 1 output;
row-parallel partials summed through the layer's all_reduce hook, with the
bias added once after it, equal the tp = 1 output (|diff| <= 3e-2 + 3e-2
|ref|, the reference's bound for bf16 reductions over different splits).
"""

from __future__ import annotations

import pytest
import torch

from granite_switch_amd import meta, vllm_layers

pytestmark = pytest.mark.gpu

K, NS, NA, R, M = 512, 512, 3, 16, 96


def _say(msg):
    print(msg, flush=True)


def _case(dev, parallelism):
    g = torch.Generator(device=dev).manual_seed({"column": 1, "qkv": 2, "row": 3}[parallelism])
    slices = (NS, NS // 2, NS // 2) if parallelism == "qkv" else (NS,)
    bf = torch.bfloat16
    base_slices = [(torch.randn(n, K, generator=g, device=dev) / K ** 0.5).to(bf) for n in slices]
    biases = [(torch.randn(n, generator=g, device=dev) * 0.5).to(bf) for n in slices]
    lora_A = [(torch.randn(NA, 1, R, K, generator=g, device=dev) / K ** 0.5).to(bf) for _ in slices]
    lora_B = [(torch.randn(NA, 1, n, R, generator=g, device=dev) * 0.3).to(bf) for n in slices]
    x = torch.randn(M, K, generator=g, device=dev).to(bf)
    ids = torch.zeros(M, dtype=torch.long, device=dev)
    ids[10:30] = 1
    ids[30:50] = 2
    ids[50:70] = 3
    ids[70:] = torch.randint(0, NA + 1, (M - 70,), generator=g, device=dev)
    return slices, base_slices, biases, lora_A, lora_B, x, ids


def _layer(dev, slices, weight, bias, parallelism, tp, rank, lora_A, lora_B, all_reduce=None):
    out_f, in_f = weight.shape
    base = torch.nn.Linear(in_f, out_f, bias=True).to(device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        base.weight.copy_(weight)
        base.bias.copy_(bias)
    kind = None if tp == 1 else ("row" if parallelism == "row" else "column")
    layer = vllm_layers.SwitchedLoRALinear(base, NA, R, num_slices=len(slices),
                                           output_slices=slices if len(slices) > 1 else None, tp_size=tp,
                                           tp_rank=rank, parallel=kind, all_reduce=all_reduce)
    if len(slices) == 1:
        layer.lora_A.weight_loader(layer.lora_A, lora_A[0])
        layer.lora_B.weight_loader(layer.lora_B, lora_B[0])
    else:
        for i in range(len(slices)):
            layer.lora_A_slices[i].weight_loader(layer.lora_A_slices[i], lora_A[i])
            layer.lora_B_slices[i].weight_loader(layer.lora_B_slices[i], lora_B[i])
    layer.finalize_weights([R] * NA)
    return layer


def _forward(dev, layer, x, ids, segments):
    fm = meta.FusedLoRAKernelMeta(dev)
    fm.register_remap_tables(layer.remap_table.unsqueeze(0), [(layer.in_features, layer._N_total,
                                                                layer._num_applicable)])
    ctx = meta.LoRAContext()
    fm.prepare_and_store(ids, ctx)
    if not segments:
        ctx.segments = None                 # the reference op over bitmask tiles
    layer._lora_ctx = ctx
    with torch.no_grad():
        out, out_bias = layer(x)
    assert out_bias is None
    return out.float()


def _shard_rows(t, r, tp):
    n = t.shape[0] // tp
    return t[r * n:(r + 1) * n]


@pytest.mark.parametrize("segments", [True, False], ids=["segments", "op"])
@pytest.mark.parametrize("tp", [2, 4, 8])
@pytest.mark.parametrize("parallelism", ["column", "qkv", "row"])
def test_tp_ranks_combine_to_the_unsharded_layer(dev, parallelism, tp, segments):
    slices, base_slices, biases, lora_A, lora_B, x, ids = _case(dev, parallelism)
    W = torch.cat(base_slices)
    b = torch.cat(biases)
    ref_layer = _layer(dev, slices, W, b, parallelism, 1, 0, lora_A, lora_B)
    ref = _forward(dev, ref_layer, x, ids, segments)
    _say(f"tp={tp} {parallelism} ({'segment expand' if segments else 'reference op'}): ref |y| max "
         f"{ref.abs().max().item():.3f}")
    remaps = []
    if parallelism == "row":
        # two passes per rank: the first records each rank's partial (K
        # shard, LoRA delta included, no bias); the second hands every rank
        # the sum of the partials, as an all-reduce would, and the layer adds
        # its bias once after it
        partials = []

        def capture(t):
            partials.append(t.float().clone())
            return t

        kshard = K // tp
        for r in range(tp):
            layer = _layer(dev, slices, W[:, r * kshard:(r + 1) * kshard], b, parallelism, tp, r, lora_A, lora_B,
                           all_reduce=capture)
            remaps.append(layer.remap_table.clone())
            _forward(dev, layer, x[:, r * kshard:(r + 1) * kshard], ids, segments)
        assert len(partials) == tp
        reduced = torch.stack(partials).sum(0).to(torch.bfloat16)
        outs = []
        for r in range(tp):
            layer = _layer(dev, slices, W[:, r * kshard:(r + 1) * kshard], b, parallelism, tp, r, lora_A, lora_B,
                           all_reduce=lambda t: reduced.clone())
            outs.append(_forward(dev, layer, x[:, r * kshard:(r + 1) * kshard], ids, segments))
        for r in range(1, tp):
            assert torch.equal(outs[r], outs[0]), f"rank {r} differs from rank 0 after the reduce"
        combined = outs[0]
    else:
        rank_outs = []
        for r in range(tp):
            w_r = torch.cat([_shard_rows(w, r, tp) for w in base_slices])
            b_r = torch.cat([_shard_rows(v, r, tp) for v in biases])
            layer = _layer(dev, slices, w_r, b_r, parallelism, tp, r, lora_A, lora_B)
            remaps.append(layer.remap_table.clone())
            rank_outs.append(_forward(dev, layer, x, ids, segments))
        # each rank holds its shard of every slice: interleave them back
        parts = []
        for s, n in enumerate(slices):
            lo = sum(slices[:s]) // tp
            parts += [o[:, lo:lo + n // tp] for o in rank_outs]
        combined = torch.cat(parts, dim=1)
    for r in range(1, tp):
        assert torch.equal(remaps[r], remaps[0]), f"remap table of rank {r} differs"
    assert combined.shape == ref.shape
    err = (combined - ref).abs()
    bad = err > 3e-2 + 3e-2 * ref.abs()
    _say(f"  max abs diff {err.max().item():.3e}")
    assert not bad.any(), f"{int(bad.sum())} elements out of tolerance, max abs diff {err.max().item():.3e}"
