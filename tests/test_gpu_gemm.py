"""GPU parity of the bf16 GEMM x . w^T (the vLLM layer's x_ext = x . w_ext^T).

Reference: the same bf16 operands multiplied in fp32 by torch, rounded once to
bf16.  The kernel accumulates in fp32 in another order, so an element may land
one bf16 step away from the reference's rounding: tolerance 2^-7 relative plus
1e-5 absolute, far inside the 2e-2 bf16 parity bound.
"""

from __future__ import annotations

import pytest
import torch

from granite_switch_amd import switched

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _check(got, x, w):
    ref = (x.float() @ w.float().T)
    err = (got.float() - ref).abs()
    bad = err > 2.0 ** -7 * ref.abs() + 1e-5
    assert not bool(bad.any()), f"{int(bad.sum())} elements off, max abs err {float(err.max()):.3e}"


@pytest.mark.parametrize("M,N,K,seed", [
    (1, 32, 8, 1),              # one row, one partial tile, K below one k-tile
    (7, 300, 72, 2),            # ragged everything, K not a multiple of 64
    (256, 256, 64, 3),          # exactly one tile
    (513, 777, 520, 4),         # partial tiles on both sides
    (300, 7296, 4096, 5),       # decode-sized QKV w_ext (base 6144 + 12 adapters x 3 slices x 32)
    (2048, 4864, 12800, 6),     # down_proj w_ext shape at a prefill chunk
])
def test_gemm_matches_fp32_reference(dev, M, N, K, seed):
    _say(f"gemm M={M} N={N} K={K}")
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=dev) / K ** 0.5).to(torch.bfloat16)
    got = switched.linear_bf16(x, w)
    torch.cuda.synchronize()
    _check(got, x, w)


def test_gemm_strided_rows_and_output(dev):
    """x and out with row strides (a view into a wider buffer), as the layer's x_ext slices are."""
    g = torch.Generator(device=dev).manual_seed(11)
    M, N, K = 333, 520, 1024
    xb = torch.randn(M, K + 64, generator=g, device=dev).to(torch.bfloat16)
    x = xb[:, 32:32 + K]
    w = (torch.randn(N, K, generator=g, device=dev) / K ** 0.5).to(torch.bfloat16)
    outb = torch.full((M, N + 40), 7.0, dtype=torch.bfloat16, device=dev)
    out = outb[:, :N]
    switched.linear_bf16(x, w, out)
    torch.cuda.synchronize()
    _check(out, x, w)
    assert bool((outb[:, N:] == 7.0).all()), "columns past N were written"


def test_gemm_empty_and_graph(dev):
    g = torch.Generator(device=dev).manual_seed(12)
    w = torch.randn(64, 128, generator=g, device=dev).to(torch.bfloat16)
    assert switched.linear_bf16(torch.empty(0, 128, dtype=torch.bfloat16, device=dev), w).shape == (0, 64)
    x = torch.randn(300, 128, generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty(300, 64, dtype=torch.bfloat16, device=dev)
    eager = switched.linear_bf16(x, w).clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        switched.linear_bf16(x, w, out)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_vllm_layer_native_and_library_gemm_agree(dev):
    """The vLLM layer's x_ext GEMM through this library's kernel and through torch.mm."""
    from granite_switch_amd import vllm_layers

    K, slices, ranks, T = 1024, (2048, 512, 512), [32, 16, 64], 200
    g = torch.Generator(device=dev).manual_seed(21)
    base = torch.nn.Linear(K, sum(slices), bias=False).to(device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        base.weight.copy_(torch.randn(sum(slices), K, generator=g, device=dev) / K ** 0.5)
    layer = vllm_layers.SwitchedLoRALinear(base, len(ranks), max(ranks), num_slices=3, output_slices=slices)
    with torch.no_grad():
        for s in range(3):
            for a, r in enumerate(ranks):
                layer.lora_A_slices[s].data[a, 0, :r] = (torch.randn(r, K, generator=g, device=dev) / K ** 0.5).to(torch.bfloat16)
    layer.finalize_weights(ranks)
    x = torch.randn(T, K, generator=g, device=dev).to(torch.bfloat16)
    layer.native_gemm = True
    native = layer._gemm(x)
    layer.native_gemm = False
    library = layer._gemm(x)
    torch.cuda.synchronize()
    assert native.shape == library.shape == (T, layer.w_ext.shape[0])
    _check(native, x, layer.w_ext)
    d = (native.float() - library.float()).abs()
    assert bool((d <= 2.0 ** -7 * library.float().abs() + 1e-5).all())
