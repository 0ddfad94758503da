#!/usr/bin/env python3
"""Benchmark of the MI355X switched-LoRA path (one JSON line on stdout).

A step is one pass of the hot path over one batch: segment build (routing +
aLoRA gating + adapter sort), then shrink and expand-add for every projection
of the workload (one projection for the single-op shapes, 32 layers x 4 for
the decoder-step shape).  K steps are captured in one HIP graph and timed with
HIP events around its replay; inputs are resident in HBM and rotate over
enough independent buffer sets (x, y, adapters) to exceed twice the 256 MB
Infinity Cache, so every step reads from HBM.

The roofline object is for the dominant kernel, timed the same way (a graph of
K launches of that kernel alone, rotating buffers).  The CPU baseline is the
reference's HF loop restated on torch-CPU, timed on the host cores.

  python bench.py [--steps K] [--warmup W] [--no-cpu]
                                   # default: the 32-layer decoder step (config 4)
                                   # as the headline line; its "configs" key
                                   # holds every other workload (single op,
                                   # decode, prefill, multiswitch) and the
                                   # idle-batch and rank-512 populations on the
                                   # decode and decoder-step shapes, each with
                                   # its own step time, roofline, kernel times
                                   # and CPU baseline from this same run
  python bench.py --config N [--population {balanced,all_base,r512}]
                                   # one workload only
  python bench.py --config N --kernel-only KIND:PROJ
                                   # only one kernel's timing graph (e.g.
                                   # expand:gate_up_proj), so a rocprofv3
                                   # --stats summary of the run shows that
                                   # kernel's average alone
  python bench.py --config N --layer-gemm   # the vLLM layer's x . w_ext^T GEMM at
                                            # the workload's shapes, this library's
                                            # MFMA kernel and torch.mm, in TFLOP/s
  python bench.py --config N --xext   # the reference-semantics ops over x_ext
                                      # (switch_lora_expand, and the fused
                                      # SwiGLU expand for gate_up) at the
                                      # workload's shapes, in HBM GB/s
  python bench.py --copy-probe MIB   # a plain device copy of MIB MiB, the
                                     # reference for scaling rocprofv3's
                                     # FETCH_SIZE / WRITE_SIZE counters
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "switched-LoRA tokens/sec + achieved HBM GB/s (% of 8 TB/s) on 1 MI355X"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK = {"bf16": 2.5e15, "fp32": 157.3e12}
MALL_BYTES = 256 << 20
DEFAULT_STEPS = {0: 200, 1: 200, 2: 40, 3: 100, 4: 8}
# workload names used by the rocprofv3 summaries under profiles/
WORKLOAD_KEY = {0: "fp32_single_op_2048x2048_T512", 1: "decode_qkv_4096x6144_T256",
                2: "prefill_gate_up_4096x25600_T8192", 3: "multiswitch_down_12800x4096_T4096",
                4: "decoder_step_32_layers_T4144"}
TRAFFIC_TABLE = os.path.join(ROOT, "profiles", "hbm_traffic_pmc.md")


def measured_traffic(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` on `workload` from the rocprofv3 PMC summary, or None."""
    try:
        lines = open(TRAFFIC_TABLE).read().splitlines()
    except OSError:
        return None
    for line in lines:
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 6 and cells[0] == workload and cells[1] == kernel:
            try:
                return int(cells[5])
            except ValueError:
                return None
    return None


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def copy_probe(mib: int) -> None:
    """Five copies of `mib` MiB between fresh device buffers (torch's copy kernel)."""
    import torch

    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty(n, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(5):
        dst.copy_(src)
    end.record()
    end.synchronize()
    ms = start.elapsed_time(end) / 5
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "us_per_copy": ms * 1e3,
                      "gbs_read_plus_write": 2 * n / (ms * 1e-3) / 1e9}), flush=True)


def layer_gemm(cfg: int, n: int) -> None:
    """x . w_ext^T of every projection of the workload: w_ext stacks the base
    weight [O, H] with every adapter's lora_A rows at the reference's promoted
    tier ranks (src/granite_switch/vllm/core/lora.py:544, kernels/switch_lora_kernel.py:134-163)."""
    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from granite_switch_amd import switched, workloads
    from granite_switch_amd.kernels import promote_rank

    dev = torch.device("cuda:0")
    T = workloads.routing_for(cfg).num_tokens
    NA = workloads.num_adapters_for(cfg)
    rows = []
    for spec in workloads.module_specs(cfg):
        S, H, O = len(spec.output_slices), spec.hidden, sum(spec.output_slices)
        n_ext = O + S * sum(promote_rank(r) for r in spec.ranks[:NA])
        g = torch.Generator(device=dev).manual_seed(17)
        x = torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16)
        w = (torch.randn(n_ext, H, generator=g, device=dev) / H ** 0.5).to(torch.bfloat16)
        out = torch.empty(T, n_ext, dtype=torch.bfloat16, device=dev)
        flops = 2.0 * T * n_ext * H

        def timed(fn):
            fn()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(n):
                    fn()
            graph.replay()
            torch.cuda.synchronize()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            graph.replay()
            end.record()
            end.synchronize()
            return start.elapsed_time(end) * 1e3 / n

        t_native = timed(lambda: switched.linear_bf16(x, w, out))
        t_lib = timed(lambda: torch.mm(x, w.T, out=out))
        rows.append({"projection": spec.name, "M": T, "N": n_ext, "K": H,
                     "native_us": t_native, "native_tflops": flops / t_native / 1e6,
                     "native_mfma_frac": flops / t_native / 1e6 / (MFMA_PEAK["bf16"] / 1e12),
                     "torch_mm_us": t_lib, "torch_mm_tflops": flops / t_lib / 1e6,
                     "torch_mm_mfma_frac": flops / t_lib / 1e6 / (MFMA_PEAK["bf16"] / 1e12)})
        del x, w, out
    print(json.dumps({"workload": WORKLOAD_KEY[cfg], "gemm": "x . w_ext^T (bf16, fp32 accumulate)",
                      "peak_tflops": MFMA_PEAK["bf16"] / 1e12, "projections": rows}), flush=True)


def xext_ops(cfg: int, n: int) -> None:
    """The reference's own ops over x_ext = x . w_ext^T, as its vLLM layer calls
    them (src/granite_switch/vllm/core/lora.py:596-686): switch_lora_expand in
    place on x_ext[:, :N] (src/granite_switch/kernels/switch_lora_kernel.py:171-458)
    and, for gate_up, switch_lora_expand_swiglu into a [T, H] output (:668-857).
    For the in-place projections the vLLM layer's own expand when segments
    are built (gs_expand_add reading each row's shrink columns of x_ext by
    token) is timed beside the reference op, on the same inputs.
    x_ext is computed once per buffer set outside the timed region.  Algorithmic
    bytes: per adapted row its N output values read and written and its S*r
    shrink values read, each used adapter's lora_B tiers once, the ids; the
    SwiGLU form reads both halves of every row and writes every output row."""
    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from granite_switch_amd import meta, ops, switched, vllm_layers, workloads
    from granite_switch_amd.kernels import promote_rank

    dev = torch.device("cuda:0")
    routing = workloads.routing_for(cfg)
    NA = workloads.num_adapters_for(cfg)
    T = routing.num_tokens
    ids = torch.tensor(routing.req_ids, device=dev)
    segs = switched.build_segments(ids, NA, torch.tensor(routing.positions, device=dev),
                                   torch.tensor(routing.cu_seqlens, device=dev),
                                   torch.tensor(routing.act_offsets, device=dev) if routing.act_offsets is not None else None)
    eff = segs.eff_ids.to(torch.int64)              # 0 = base, a + 1 = adapter a (the reference's ids)
    eff_np = eff.cpu().numpy()
    rows = []
    for spec in workloads.module_specs(cfg):
        S, H = len(spec.output_slices), spec.hidden
        N = sum(spec.output_slices)
        fuse = spec.name == "gate_up_proj"
        ranks = list(spec.ranks[:NA])
        g = torch.Generator(device=dev).manual_seed(23)
        base = torch.nn.Linear(H, N, bias=False).to(device=dev, dtype=torch.bfloat16)
        with torch.no_grad():
            base.weight.copy_(torch.randn(N, H, generator=g, device=dev) / H ** 0.5)
        layer = vllm_layers.SwitchedLoRALinear(base, NA, max(ranks), num_slices=S,
                                               output_slices=tuple(spec.output_slices) if S > 1 else None,
                                               fuse_swiglu=fuse)
        A_sl = [layer.lora_A] if S == 1 else list(layer.lora_A_slices)
        B_sl = [layer.lora_B] if S == 1 else list(layer.lora_B_slices)
        with torch.no_grad():
            for s_ in range(S):
                for a, r in enumerate(ranks):
                    A_sl[s_].data[a, 0, :r] = (torch.randn(r, H, generator=g, device=dev) / H ** 0.5).to(torch.bfloat16)
                    B_sl[s_].data[a, 0, :, :r] = (torch.randn(spec.output_slices[s_], r, generator=g, device=dev)
                                                  * 0.02).to(torch.bfloat16)
        layer.finalize_weights(ranks)
        fm = meta.FusedLoRAKernelMeta(dev)
        fm.register_remap_tables(layer.remap_table.unsqueeze(0), [(H, layer._N_total, layer._num_applicable)])
        ctx = meta.LoRAContext()
        fm.prepare_and_store(eff, ctx)
        nsets = 2
        x_exts = []
        for _ in range(nsets):
            x = torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16)
            x_exts.append(torch.mm(x, layer.w_ext.T))
            del x
        out = torch.empty(T, N // 2 if fuse else 1, dtype=torch.bfloat16, device=dev)
        loc, bm = ctx.remapped_indices[0], ctx.per_module_bitmasks[0]
        if fuse:
            def call(i):
                ops.op("switch_lora_expand_swiglu")(out, x_exts[i % nsets], loc, bm, layer._lb_packed,
                                                     layer.slice_col_r, *layer._na, 2, layer._block_n, N // 2, N)
        else:
            def call(i):
                ops.op("switch_lora_expand")(x_exts[i % nsets], loc, bm, layer._lb_packed, layer.tile_to_slice,
                                              layer.slice_col_r, *layer._na, S, layer._block_n, N)
        def timed(fn):
            fn(0)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for i in range(n):
                    fn(i)
            graph.replay()
            torch.cuda.synchronize()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            graph.replay()
            end.record()
            end.synchronize()
            return start.elapsed_time(end) * 1e3 / n

        us = timed(call)
        # the layer's own expand over x_ext when segments are built: gs_expand_add
        # reading each row's shrink columns by token (vllm_layers._run_segment_expand)
        seg_us = None if fuse else timed(lambda i: layer._run_segment_expand(x_exts[i % nsets], segs))
        # adapted rows: an applicable adapter (a token of a non-applicable one stays base)
        rp = [promote_rank(r) for r in ranks]
        adapted = [a for a in range(NA) if ranks[a] > 0]
        act = np.isin(eff_np, [a + 1 for a in adapted])
        t_act = int(act.sum())
        used = sorted(set(int(v) - 1 for v in eff_np[act]))
        b_bytes = sum(N * rp[a] * 2 for a in used)
        shrink_bytes = sum(int((eff_np == a + 1).sum()) * S * rp[a] * 2 for a in used)
        if fuse:
            alg = T * N * 2 + T * (N // 2) * 2 + shrink_bytes + b_bytes + T * 8
        else:
            alg = 2 * t_act * N * 2 + shrink_bytes + b_bytes + T * 8
        rows.append({"projection": spec.name, "op": "switch_lora_expand_swiglu" if fuse else "switch_lora_expand",
                     "tokens": T, "adapted_tokens": t_act, "N": N, "us": us, "algorithmic_bytes": alg,
                     "hbm_gbs": alg / us / 1e3, "hbm_frac": alg / us / 1e3 / HBM_PEAK_GBS})
        if seg_us is not None:
            rows.append({"projection": spec.name, "op": "segment expand over x_ext (the vLLM layer's path)",
                         "tokens": T, "adapted_tokens": t_act, "N": N, "us": seg_us, "algorithmic_bytes": alg,
                         "hbm_gbs": alg / seg_us / 1e3, "hbm_frac": alg / seg_us / 1e3 / HBM_PEAK_GBS})
        del x_exts, out, layer, base
    print(json.dumps({"workload": WORKLOAD_KEY[cfg], "ops": "reference-semantics expand over x_ext (bf16)",
                      "peak_gbs": HBM_PEAK_GBS, "projections": rows}), flush=True)


def path_choice() -> None:
    """Both y-given paths on the same batches: the one-launch decode kernel
    (path="small") and build + shrink + expand (path="segments"), over
    projection shapes of 2048- to 12800-wide layers with 2-48 adapters at
    T = 64..1024 (ids uniform per token, 20 % of tokens on the base model),
    then batches of 4-8 sequences of 128-256 tokens that each hold one adapter
    (chunked-prefill mixes), and the 4-sequence aLoRA batch of the 2048-wide
    CPU-sized workload.  Each timing is one graph replay over rotating buffer
    sets (~250 MB, so weights come from HBM), divided by the calls.  "auto" is
    the path that switched.small_preferred picks (also with the batch's
    largest adapter group passed as a hint); the one-launch kernel runs with
    the row split switched.small_row_split picks."""
    import numpy as np
    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from granite_switch_amd import switched, workloads

    dev = torch.device("cuda:0")
    mixed = [8, 16, 32, 64] * 12
    shapes = (("proj2048", 2048, (2048,), 16, (2, 4, 8)), ("qkv", 4096, (4096, 1024, 1024), 16, (2, 4, 8, 12)),
              ("down", 12800, (4096,), 16, (2, 4, 8)), ("o_r64", 4096, (4096,), 64, (2, 4, 8)),
              ("qkv_r64", 4096, (4096, 1024, 1024), 64, (12,)), ("o", 4096, (4096,), 32, (24,)),
              ("down", 12800, (4096,), 32, (24,)), ("gate_up", 4096, (12800, 12800), 32, (24,)),
              ("down_mixed_rank", 12800, (4096,), None, (48,)))
    cases = []
    for name, H, sl, r, nas in shapes:
        for NA in nas:
            ranks = [r] * NA if r else mixed[:NA]
            spec = workloads.ModuleSpec(name=name, hidden=H, output_slices=sl, ranks=ranks, max_rank=max(ranks))
            for T in (64, 128, 256, 512, 1024):
                if T // NA <= 256 and (NA <= 8 or T >= 128):
                    g = torch.Generator(device="cpu").manual_seed(T)
                    ids = torch.randint(1, NA + 1, (T,), generator=g)
                    ids[torch.rand(T, generator=g) < 0.2] = 0
                    cases.append((spec, NA, T, ids, None, None, None, torch.bfloat16))
    for name, H, sl, r, NA, T, L in (("qkv", 4096, (4096, 1024, 1024), 16, 4, 512, 128),
                                     ("qkv", 4096, (4096, 1024, 1024), 16, 12, 512, 128),
                                     ("qkv", 4096, (4096, 1024, 1024), 16, 12, 1024, 128),
                                     ("qkv", 4096, (4096, 1024, 1024), 16, 24, 1024, 256),
                                     ("down", 12800, (4096,), 16, 4, 512, 128),
                                     ("down", 12800, (4096,), 16, 12, 512, 128),
                                     ("gate_up", 4096, (12800, 12800), 32, 4, 512, 128),
                                     ("gate_up", 4096, (12800, 12800), 32, 12, 1024, 128)):
        spec = workloads.ModuleSpec(name=name, hidden=H, output_slices=sl, ranks=[r] * NA, max_rank=r)
        g = np.random.default_rng(T + L + NA)
        ids = torch.tensor(np.repeat(g.integers(1, NA + 1, T // L), L))
        cases.append((spec, NA, T, ids, None, torch.arange(0, T + 1, L, dtype=torch.int32), None, torch.bfloat16))
    r0 = workloads.routing_for(0)
    spec0 = workloads.module_specs(0)[0]
    cases.append((spec0, workloads.num_adapters_for(0), r0.num_tokens, torch.tensor(r0.req_ids),
                   torch.tensor(r0.positions), torch.tensor(r0.cu_seqlens),
                   None if r0.act_offsets is None else torch.tensor(r0.act_offsets), workloads.dtype_for(0)))
    rows = []
    for spec, NA, T, ids, pos, cu, off, dtype in cases:
        H, sl = spec.hidden, spec.output_slices
        e = 4 if dtype == torch.float32 else 2
        per_call = NA * spec.max_rank * (len(sl) * H + sum(sl)) * e
        nsets = max(4, min(28, int(2.5e8 // (T * (H + sum(sl)) * e + per_call))))
        sets = []
        for i in range(nsets):
            md = workloads.make_module(spec, T, NA, dtype, dev, seed=50 + i)
            pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks)
            md.lora_A_slices = md.lora_B_slices = None
            sets.append((md, pk))
        ids_d = ids.to(dev)
        pos_d, cu_d, off_d = (None if t is None else t.to(dev) for t in (pos, cu, off))
        res = {}
        for path in ("small", "segments"):
            def call(i):
                md, pk = sets[i % nsets]
                switched.switched_lora_routed_(md.y, md.x, ids_d, pk, pos_d, cu_d, off_d, path=path)
            call(0)
            torch.cuda.synchronize()
            n = nsets * 2
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for i in range(n):
                    call(i)
            graph.replay()
            torch.cuda.synchronize()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            graph.replay()
            end.record()
            end.synchronize()
            res[path] = start.elapsed_time(end) * 1e3 / n
        nseq = None if cu is None else cu.numel() - 1
        largest = int(np.bincount(ids.numpy(), minlength=NA + 1)[1:].max())
        auto = "small" if switched.small_preferred(sets[0][1], T, nseq) else "segments"
        auto_hint = "small" if switched.small_preferred(sets[0][1], T, nseq, largest) else "segments"
        rs = switched.small_row_split(sets[0][1], T, nseq)
        rows.append({"projection": spec.name, "dtype": "fp32" if dtype == torch.float32 else "bf16",
                     "hidden": H, "output_slices": list(sl), "adapters": NA,
                     "ranks": sorted(set(spec.ranks)), "tokens": T, "sequences": nseq, "largest_group": largest,
                     "row_split": rs, "small_us": res["small"], "segments_us": res["segments"], "auto": auto,
                     "auto_with_largest_group": auto_hint})
        log(f"{spec.name} H={H} NA={NA} T={T} seqs={nseq} largest={largest} rs={rs}: small {res['small']:.2f} us, "
            f"segments {res['segments']:.2f} us, auto {auto}")
        del sets
    print(json.dumps({"comparison": "one-launch decode kernel vs segment kernels (bf16; the last row fp32)",
                      "rows": rows}), flush=True)


WL_NAMES = {0: "switched-LoRA single op fp32 2048->2048 T=512 (4x128) 4 adapters r8 aLoRA",
            1: "switched-LoRA decode QKV 4096->6144 T=256 12 adapters r32 (20% not yet activated)",
            2: "switched-LoRA chunked prefill gate_up 4096->25600 T=8192 (16 seqs) 12 adapters r32",
            3: "switched-LoRA multiswitch down 12800->4096 T=4096 (64x64) 48 adapters r8-64",
            4: "switched-LoRA side of a 32-layer Granite-8B-shaped step T=4144 24 adapters r32"}
POP_NAMES = {"balanced": "", "all_base": " -- idle batch: every token on the base model",
             "r512": " -- plus one rank-512 adapter (N+1 loaded, ids uniform over them)"}


def measure(cfg: int, population: str, K: int, W: int, nsets_arg=None, no_cpu=False, cpu_budget=12.0,
            only=None, kernels=True):
    """One workload (config ``cfg``, adapter ``population``): K graph-captured
    steps after W eager ones, per-kernel timings, algorithmic accounting and
    the CPU baseline.  Returns the result dict (the JSON line's fields)."""
    import torch

    from granite_switch_amd import _lib, switched, workloads

    dev = torch.device("cuda:0")
    routing = workloads.population_routing(cfg, population)
    NA = workloads.population_adapters(cfg, population)
    dtype = workloads.dtype_for(cfg)
    dname = "fp32" if dtype == torch.float32 else "bf16"
    e = 4 if dtype == torch.float32 else 2
    specs = workloads.population_specs(cfg, population)
    layers = 32 if cfg == 4 else 1
    T = routing.num_tokens
    tag = f"c{cfg}" + ("" if population == "balanced" else f"/{population}")

    # -- buffer sets ---------------------------------------------------------
    def module_bytes(spec):
        O = sum(spec.output_slices)
        rsum = sum(spec.ranks)
        return (T * spec.hidden + T * O + len(spec.output_slices) * rsum * spec.hidden + rsum * O) * e

    set_bytes = layers * sum(module_bytes(s) for s in specs)
    nsets = nsets_arg or max(1, min(64, math.ceil(2 * MALL_BYTES / set_bytes)))
    log(f"{tag}: {workloads.NAMES[cfg]}{POP_NAMES[population]}; T={T}; {nsets} buffer set(s) of "
        f"{set_bytes / 2**20:.1f} MiB")

    sets = []       # sets[i][layer*len(specs)+k] = (ModuleData without slices, PackedAdapters)
    cpu_sample = []
    for i in range(nsets):
        mods = []
        for layer in range(layers):
            for k, spec in enumerate(specs):
                md = workloads.make_module(spec, T, NA, dtype, dev, seed=7919 * (cfg + 1) + 101 * layer + k + 1000003 * i)
                pk = switched.PackedAdapters.from_slices(md.lora_A_slices, md.lora_B_slices, spec.ranks)
                if i == 0 and layer == 0 and not no_cpu:
                    cpu_sample.append((md.y.cpu(), md.x.cpu(), [a.cpu() for a in md.lora_A_slices],
                                       [b.cpu() for b in md.lora_B_slices], spec.output_slices))
                md.lora_A_slices = None
                md.lora_B_slices = None
                mods.append((md, pk))
        sets.append(mods)
    torch.cuda.synchronize()

    ids_d = torch.tensor(routing.req_ids, device=dev)
    pos_d = torch.tensor(routing.positions, device=dev)
    cu_d = torch.tensor(routing.cu_seqlens, device=dev)
    off_d = None if routing.act_offsets is None else torch.tensor(routing.act_offsets, device=dev)
    segs = switched.build_segments(ids_d, NA, pos_d, cu_d, off_d)
    zbuf = [torch.empty(max(T, 1), len(s.output_slices) * sets[0][k][1].max_rank, dtype=dtype, device=dev)
            for k, s in enumerate(specs)]
    ws_need = max(int(_lib.load().gs_shrink_workspace_bytes(T, s.hidden, len(s.output_slices), NA, sets[0][k][1].max_rank,
                                                            switched._i32_array(sets[0][k][1].ranks_host)))
                  for k, s in enumerate(specs))
    nseq_r = len(routing.cu_seqlens) - 1
    plans = {spec.name: switched.path_plan(sets[0][k][1], T, nseq_r) for k, spec in enumerate(specs)}
    small = all(p == "small" for p in plans.values()) and layers == 1
    split = any(p == "split" for p in plans.values())
    if small:
        switched.reserve_small_workspace(dev, max(switched.small_workspace_bytes(sets[0][k][1], T)
                                                  for k in range(len(specs))))
        switched.small_reset(dev)
    switched.reserve_workspace(dev, ws_need)
    path_name = ("small-batch" if small else
                 "split: one-launch kernel for ranks <= 64, segment kernels for larger ranks" if split else "segments")
    log(f"{tag} path: {path_name}")

    def build():
        switched.build_segments(ids_d, NA, pos_d, cu_d, off_d, out=segs)

    def pair(k, md, pk):
        if small:
            switched.switched_lora_routed_(md.y, md.x, ids_d, pk, pos_d, cu_d, off_d, path="small")
        else:
            switched.switched_lora_(md.y, md.x, segs, pk, zbuf[k], path="auto")

    # the shrink and expand kernels are timed alone for modules of one rank
    # class (a module with several runs each kernel once per class)
    ks_split = {}
    one_class = {}
    for k, spec in enumerate(specs):
        ksl = switched.shrink_ksplits(sets[0][k][1], T)
        one_class[spec.name] = len(ksl) == 1
        ks_split[spec.name] = len(ksl) == 1 and ksl[0] > 1

    def shrink(k, md, pk):
        # split hidden dimension: the shrink kernel alone (fp32 partials, what
        # switched_lora's expand reads); otherwise the kernel writing z
        switched.shrink(md.x, segs, pk, zbuf[k], partials_only=ks_split[specs[k].name])

    def expand(k, md, pk):
        switched.expand_add_(md.y, zbuf[k], segs, pk)

    def step(i):
        if not small:
            build()
        for j, (md, pk) in enumerate(sets[i % nsets]):
            pair(j % len(specs), md, pk)

    # -- warm-up, capture, timed replay ---------------------------------------
    if only is None:
        for i in range(W):
            step(i)
    else:
        build()
    torch.cuda.synchronize()

    def capture(fn):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        g.replay()                      # upload + one untimed run
        torch.cuda.synchronize()
        return g

    def timed(g, n):
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        g.replay()
        end.record()
        end.synchronize()
        return start.elapsed_time(end) / n       # ms per unit

    ms_per_step = None
    if only is None:
        g_steps = capture(lambda: [step(i) for i in range(K)])
        ms_per_step = timed(g_steps, K)
        del g_steps
        log(f"{tag} step: {ms_per_step * 1e3:.2f} us over {K} graph-captured steps")

    # -- host-side accounting --------------------------------------------------
    from granite_switch_amd.switched import algorithmic_bytes, algorithmic_flops

    eff = segs.eff_ids.cpu().numpy()
    op_bytes = 0
    op_flops = 0
    per_kernel_bytes = {}
    t_act = int((eff > 0).sum())
    for k, spec in enumerate(specs):
        pk = sets[0][k][1]
        b = algorithmic_bytes(eff, pk, spec.ranks, e)
        f = algorithmic_flops(eff, pk, spec.ranks)
        op_bytes += layers * b
        op_flops += layers * f
        S, H, O = len(spec.output_slices), spec.hidden, sum(spec.output_slices)
        used = np.unique(eff[eff > 0])
        rsum = sum(spec.ranks[g - 1] for g in used)
        zbytes = sum(S * spec.ranks[g - 1] for g in eff[eff > 0]) * e
        per_kernel_bytes[f"shrink:{spec.name}"] = t_act * H * e + S * H * rsum * e + zbytes + 4 * t_act
        per_kernel_bytes[f"expand:{spec.name}"] = O * rsum * e + 2 * t_act * O * e + zbytes + 4 * t_act
    nseq = len(routing.cu_seqlens) - 1
    per_kernel_bytes["build_segments"] = T * (8 + 8 + 4) + 4 * t_act + 12 * nseq + 4 * (NA + 1)

    # -- per-kernel timing (graphs of n launches of one kernel) -------------
    # Small path: the step is one fused kernel per projection.  Segment path:
    # switched_lora = the shrink and expand kernels of one projection (the
    # production pair); shrink alone also runs the split-K reduce when the
    # hidden dimension is split; expand alone reads a materialised z.
    kern_us = {}
    kern_launches = {}
    wanted = (lambda name: only is None or name == only)
    if kernels and not small and wanted("build_segments"):
        kern_launches["build_segments"] = 1
        g_b = capture(lambda: [build() for _ in range(K)])
        kern_us["build_segments"] = timed(g_b, K) * 1e3
    for k, spec in enumerate(specs):
        pk0 = sets[0][k][1]
        per_kernel_bytes[f"switched_lora:{spec.name}"] = (per_kernel_bytes[f"shrink:{spec.name}"]
                                                          + per_kernel_bytes[f"expand:{spec.name}"])
        per_kernel_bytes[f"small_fused:{spec.name}"] = algorithmic_bytes(eff, pk0, spec.ranks, e)
        if not kernels:
            continue
        mods = [sets[i][layer * len(specs) + k] for i in range(nsets) for layer in range(layers)]
        n = max(K, len(mods)) if cfg != 4 else len(mods)
        if small:
            kinds = (("small_fused", pair),)
        elif one_class[spec.name] and plans[spec.name] == "segments":
            kinds = (("switched_lora", pair), ("shrink", shrink), ("expand", expand))
        else:
            kinds = (("switched_lora", pair),)
        for kind, fn in kinds:
            name = f"{kind}:{spec.name}"
            if not wanted(name):
                continue
            if kind == "expand":          # the expand alone reads a materialised z
                switched.shrink(mods[0][0].x, segs, mods[0][1], zbuf[k])
            g_k = capture(lambda: [fn(k, *mods[j % len(mods)]) for j in range(n)])
            kern_us[name] = timed(g_k, n) * 1e3
            kern_launches[name] = layers
            del g_k
    if only is not None and not kern_us:
        raise SystemExit(f"--kernel-only {only}: no such kernel on this workload")
    switched.check(dev)
    for name, us in kern_us.items():
        log(f"{tag} kernel {name}: {us:.2f} us/launch, {per_kernel_bytes[name] / us / 1e3:.0f} GB/s algorithmic")
    roofline = None
    # every single kernel competes (the pair is two kernels): the split
    # shrinks are timed as the shrink kernel alone
    # (a module of several rank classes is timed as its pair only)
    singles = [n for n in kern_us
               if not n.startswith("switched_lora:") or f"shrink:{n.split(':', 1)[1]}" not in kern_us]
    if singles:
        dom = max(singles, key=lambda n: kern_us[n] * kern_launches[n])
        dom_gbs = per_kernel_bytes[dom] / (kern_us[dom] * 1e-6) / 1e9
        traffic = measured_traffic(WORKLOAD_KEY[cfg], dom) if population == "balanced" else None
        roofline = {"bound": "hbm", "kernel": dom, "achieved": dom_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": dom_gbs / HBM_PEAK_GBS, "traffic": traffic,
                    "algorithmic_bytes": per_kernel_bytes[dom], "avg_us": kern_us[dom]}

    # -- CPU baseline -----------------------------------------------------------
    cpu = None
    if not no_cpu and cpu_sample and only is None:
        from oracle import baseline

        ids_cpu = torch.tensor(eff.astype(np.int64))
        host = baseline.host_cpu()
        med, runs, threads = baseline.time_modules(cpu_sample, ids_cpu, budget_s=cpu_budget, min_runs=3)
        step_cpu = med * layers
        cpu = {
            "value": T / step_cpu if step_cpu > 0 else None,
            "unit": "tokens/s",
            "us_per_op": step_cpu * 1e6,
            "cores": threads,
            "kind": "port",
            "sample": (f"reference HF per-adapter loop (torch-CPU, {dname}) over "
                       f"{'one layer (4 projections), scaled x32' if cfg == 4 else 'the full op'}; "
                       f"median of {runs} runs on {threads} threads; host {host['model']}, "
                       f"{host.get('physical_cores')} physical cores / {host['logical_cpus']} threads "
                       f"({host['sockets']} sockets), {host['affinity']} CPUs in this process's affinity, "
                       f"cgroup quota {host['quota'] if host['quota'] is not None else 'none'}"),
        }
        log(f"{tag} cpu baseline: {med * 1e3:.3f} ms per sample pass on {threads} threads")

    us_op = None if ms_per_step is None else ms_per_step * 1e3
    value = None if ms_per_step is None else T / (ms_per_step * 1e-3)
    op_gbs = None if ms_per_step is None else op_bytes / (ms_per_step * 1e-3) / 1e9
    res = {
        "value": value,
        "unit": "tokens/s",
        "steps": K,
        "warmup": W,
        "ms_per_step": ms_per_step,
        "dtype": dname,
        "config": {"workload": WL_NAMES[cfg] + POP_NAMES[population], "population": population,
                   "tokens": T, "active_tokens": t_act, "adapters": NA,
                   "ranks": sorted(set(int(r) for r in specs[0].ranks)),
                   "projections": [f"{s.name} {s.hidden}->{sum(s.output_slices)}" for s in specs],
                   "layers": layers, "buffer_sets": nsets,
                   "path": path_name},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "us_per_op": us_op,
        "op_algorithmic_bytes": op_bytes,
        "op_hbm_gbs": op_gbs,
        "op_hbm_frac": None if op_gbs is None else op_gbs / HBM_PEAK_GBS,
        "op_mfma_frac": None if ms_per_step is None else op_flops / (ms_per_step * 1e-3) / MFMA_PEAK[dname],
        "kernels_us": kern_us,
    }
    del sets, zbuf, segs
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


# The other workloads and adapter populations measured by the default run
# (after the headline): (key, config, population).
EXTRAS = (("c0", 0, "balanced"), ("c1", 1, "balanced"), ("c2", 2, "balanced"), ("c3", 3, "balanced"),
          ("c1_all_base", 1, "all_base"), ("c1_r512", 1, "r512"),
          ("c4_all_base", 4, "all_base"), ("c4_r512", 4, "r512"))
EXTRA_CPU_BUDGET_S = 4.0


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=None, choices=[0, 1, 2, 3, 4],
                    help="measure only this workload (default: the decoder step as the headline line, with "
                         "every other workload and population under its 'configs' key)")
    ap.add_argument("--population", default="balanced", choices=["balanced", "all_base", "r512"],
                    help="adapter population of a --config run")
    ap.add_argument("--headline-only", action="store_true", help="default run without the 'configs' extras")
    ap.add_argument("--kernel-only", default=None, metavar="KIND:PROJ",
                    help="time only this kernel (build_segments, shrink:P, expand:P, switched_lora:P, "
                         "small_fused:P); no step, no CPU baseline")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--sets", type=int, default=None, help="buffer sets to rotate (default: > 2x MALL)")
    ap.add_argument("--copy-probe", type=int, default=None, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB five times (counter calibration)")
    ap.add_argument("--layer-gemm", action="store_true",
                    help="only time the vLLM layer's x . w_ext^T GEMM at the workload's shapes")
    ap.add_argument("--xext", action="store_true",
                    help="only time the reference-semantics expand ops over x_ext at the workload's shapes")
    ap.add_argument("--path-choice", action="store_true",
                    help="only time the one-launch decode kernel against the segment kernels over T = 128..1024")
    args = ap.parse_args()
    cfg_arg = args.config
    if args.copy_probe is not None:
        copy_probe(args.copy_probe)
        return
    if args.layer_gemm:
        layer_gemm(4 if cfg_arg is None else cfg_arg, args.steps or 10)
        return
    if args.xext:
        xext_ops(4 if cfg_arg is None else cfg_arg, args.steps or 20)
        return
    if args.path_choice:
        path_choice()
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU: the switched-LoRA kernels run on one MI355X; "
                                   "multi-GPU sharding is a design note only (run with --gpus 1)"}))
        sys.exit(2)

    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from granite_switch_amd import _lib

    _lib.load()
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    cfg = 4 if cfg_arg is None else cfg_arg
    K = args.steps if args.steps is not None else DEFAULT_STEPS[cfg]
    W = args.warmup
    res = measure(cfg, args.population, K, W, args.sets, args.no_cpu, 12.0, args.kernel_only)
    extras = None
    if cfg_arg is None and args.kernel_only is None and not args.headline_only:
        extras = {}
        for key, c, pop in EXTRAS:
            r = measure(c, pop, DEFAULT_STEPS[c], W, None, args.no_cpu, EXTRA_CPU_BUDGET_S)
            r.pop("unit", None)
            r["tokens_per_s"] = r.pop("value")
            extras[key] = r
    out = {
        "metric": METRIC,
        "value": res["value"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": res["dtype"],
        "data": "synthetic (seeded; random-init adapters in the composed-checkpoint layout)",
        "config": res["config"],
        "roofline": res["roofline"],
        "cpu_baseline": res["cpu_baseline"],
    }
    for k in ("us_per_op", "op_algorithmic_bytes", "op_hbm_gbs", "op_hbm_frac", "op_mfma_frac", "kernels_us"):
        out[k] = res[k]
    if extras is not None:
        out["configs"] = extras
    if args.kernel_only is not None:
        out["mode"] = f"kernel-only {args.kernel_only}: no step timed"
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
