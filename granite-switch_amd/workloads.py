"""Seeded synthetic switched-LoRA workloads (the five benchmark shapes).

Every workload is generated from a seed with torch generators on the target
device, in the reference's storage layout:

  lora_A_slices[s]: [NA, 1, max_r, H]   zero past each adapter's true rank
  lora_B_slices[s]: [NA, 1, O_s, max_r] pre-scaled by alpha/r (alpha = 16)

(src/granite_switch/composer/weight_transfer.py:547-622), x ~ N(0,1),
A ~ N(0, 1/H), B ~ N(0, 0.02^2) (0.02 read as a standard deviation) times
alpha/r, y ~ N(0,1).  Token ids follow the reference convention: 0 = base,
1..NA = adapters.  Routing is given as requested per-token ids plus optional
aLoRA activation offsets per sequence and absolute positions; the effective
ids are what ``switched.build_segments`` computes.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

ALPHA = 16.0

NAMES = {
    0: "c0 single-op fp32: 2048->2048, T=512 (4x128), 4 adapters r8, aLoRA offsets",
    1: "c1 decode bf16: T=256 (256x1), QKV 4096->6144, 12 adapters r32, 20% not yet activated",
    2: "c2 chunked prefill bf16: T=8192 (16 seqs log-uniform), gate_up 4096->25600, 12 adapters r32",
    3: "c3 multiswitch bf16: T=4096 (64x64), down 12800->4096, 48 adapters r{8,16,32,64} padded to 64",
    4: "c4 Granite-8B-shaped 32-layer LoRA side: T=4144 (48 decode + 16x256 prefill), 24 adapters r32",
}


@dataclass
class Routing:
    req_ids: np.ndarray              # [T] int64 requested adapter per token
    cu_seqlens: np.ndarray           # [B+1] int32
    positions: np.ndarray            # [T] int64 absolute positions
    act_offsets: np.ndarray | None   # [B] int64 or None

    @property
    def num_tokens(self) -> int:
        return int(self.req_ids.shape[0])


@dataclass
class ModuleSpec:
    name: str
    hidden: int
    output_slices: tuple
    ranks: list                      # true rank per adapter
    max_rank: int                    # storage rank (zero-padded)


@dataclass
class ModuleData:
    spec: ModuleSpec
    x: torch.Tensor
    y: torch.Tensor
    lora_A_slices: list
    lora_B_slices: list


@dataclass
class Workload:
    config: int
    name: str
    dtype: torch.dtype
    num_adapters: int
    routing: Routing
    modules: list = field(default_factory=list)   # list[ModuleData] (one per projection)


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def make_module(spec: ModuleSpec, T: int, num_adapters: int, dtype: torch.dtype, device, seed: int) -> ModuleData:
    g = _gen(device, seed)
    H = spec.hidden
    x = torch.randn(T, H, generator=g, device=device, dtype=torch.float32).to(dtype)
    y = torch.randn(T, sum(spec.output_slices), generator=g, device=device, dtype=torch.float32).to(dtype)
    A_sl, B_sl = [], []
    rk = torch.tensor(spec.ranks, device=device)
    rowmask = (torch.arange(spec.max_rank, device=device)[None, :] < rk[:, None]).to(torch.float32)
    scale = (ALPHA / rk.to(torch.float32))
    for o_s in spec.output_slices:
        A = torch.randn(num_adapters, 1, spec.max_rank, H, generator=g, device=device) / math.sqrt(H)
        A = A * rowmask[:, None, :, None]
        B = torch.randn(num_adapters, 1, o_s, spec.max_rank, generator=g, device=device) * 0.02
        B = B * rowmask[:, None, None, :] * scale[:, None, None, None]
        A_sl.append(A.to(dtype))
        B_sl.append(B.to(dtype))
    return ModuleData(spec=spec, x=x, y=y, lora_A_slices=A_sl, lora_B_slices=B_sl)


def _loguniform_lengths(rng, n, lo, hi, total):
    raw = np.exp(rng.uniform(math.log(lo), math.log(hi), size=n))
    lens = np.maximum(1, np.floor(raw / raw.sum() * total)).astype(np.int64)
    # fix the rounding so the lengths sum exactly to total
    diff = total - int(lens.sum())
    order = np.argsort(-raw)
    k = 0
    while diff != 0:
        j = order[k % n]
        step = 1 if diff > 0 else -1
        if lens[j] + step >= 1:
            lens[j] += step
            diff -= step
        k += 1
    return lens


def routing_for(config: int, seed: int = 0, num_adapters: int | None = None) -> Routing:
    """Seeded routing of one workload; ``num_adapters`` widens (or narrows)
    the range the adapter ids are drawn from (default: the workload's own)."""
    rng = np.random.default_rng(1000 + 17 * config + seed)
    na = num_adapters
    if config == 0:
        B, L, NA = 4, 128, na or 4
        lens = np.full(B, L)
        adapters = rng.integers(1, NA + 1, size=B)
        offsets = rng.integers(0, L, size=B)
        req = np.repeat(adapters, lens)
        pos = np.concatenate([np.arange(l) for l in lens])
        return Routing(req.astype(np.int64), np.concatenate([[0], np.cumsum(lens)]).astype(np.int32),
                       pos.astype(np.int64), offsets.astype(np.int64))
    if config == 1:
        T, NA = 256, na or 12
        req = rng.integers(1, NA + 1, size=T)
        ctx_len = rng.integers(16, 2048, size=T)           # decode position of each request
        inactive = np.zeros(T, dtype=bool)
        inactive[rng.permutation(T)[: int(round(0.2 * T))]] = True
        # activated requests have their invocation point at or before the decode
        # position, the 20% not yet activated have it after
        offsets = np.where(inactive, ctx_len + 1 + rng.integers(0, 16, size=T), ctx_len - rng.integers(0, 16, size=T))
        return Routing(req.astype(np.int64), np.arange(T + 1, dtype=np.int32), ctx_len.astype(np.int64),
                       offsets.astype(np.int64))
    if config == 2:
        B, T, NA = 16, 8192, na or 12
        lens = _loguniform_lengths(rng, B, 64, 2048, T)
        adapters = rng.integers(1, NA + 1, size=B)
        offsets = np.array([rng.integers(0, l) for l in lens])
        req = np.repeat(adapters, lens)
        pos = np.concatenate([np.arange(l) for l in lens])
        return Routing(req.astype(np.int64), np.concatenate([[0], np.cumsum(lens)]).astype(np.int32),
                       pos.astype(np.int64), offsets.astype(np.int64))
    if config == 3:
        B, L, NA = 64, 64, na or 48
        req = np.zeros(B * L, dtype=np.int64)
        for s in range(B):
            p = 0
            while p < L:
                run = int(rng.integers(4, 17))
                nid = 0 if rng.random() < 0.15 else int(rng.integers(1, NA + 1))
                req[s * L + p: s * L + min(L, p + run)] = nid
                p += run
        pos = np.tile(np.arange(L), B)
        return Routing(req, np.arange(0, B * L + 1, L).astype(np.int32), pos.astype(np.int64), None)
    if config == 4:
        NA, ND, NP, C = na or 24, 48, 16, 256
        dec_adapters = rng.integers(1, NA + 1, size=ND)
        dec_pos = rng.integers(16, 4096, size=ND)
        dec_off = np.array([rng.integers(0, p + 64) for p in dec_pos])   # some not yet activated
        pre_adapters = rng.integers(1, NA + 1, size=NP)
        chunk_idx = rng.integers(0, 8, size=NP)                        # cached prefix = chunk_idx * C
        pre_off = np.array([rng.integers(0, (ci + 1) * C) for ci in chunk_idx])
        req = np.concatenate([dec_adapters, np.repeat(pre_adapters, C)])
        pos = np.concatenate([dec_pos] + [ci * C + np.arange(C) for ci in chunk_idx])
        lens = np.concatenate([np.ones(ND, dtype=np.int64), np.full(NP, C)])
        return Routing(req.astype(np.int64), np.concatenate([[0], np.cumsum(lens)]).astype(np.int32),
                       pos.astype(np.int64), np.concatenate([dec_off, pre_off]).astype(np.int64))
    raise ValueError(f"unknown config {config}")


GRANITE_8B = dict(hidden=4096, heads=32, kv_heads=8, intermediate=12800)


def layer_specs(num_adapters: int, rank: int = 32) -> list:
    h, i = GRANITE_8B["hidden"], GRANITE_8B["intermediate"]
    hd = h // GRANITE_8B["heads"]
    kv = GRANITE_8B["kv_heads"] * hd
    ranks = [rank] * num_adapters
    return [
        ModuleSpec("qkv_proj", h, (h, kv, kv), ranks, rank),
        ModuleSpec("o_proj", h, (h,), ranks, rank),
        ModuleSpec("gate_up_proj", h, (i, i), ranks, rank),
        ModuleSpec("down_proj", i, (h,), ranks, rank),
    ]


def module_specs(config: int) -> list:
    if config == 0:
        return [ModuleSpec("proj", 2048, (2048,), [8] * 4, 8)]
    if config == 1:
        return [ModuleSpec("qkv_proj", 4096, (4096, 1024, 1024), [32] * 12, 32)]
    if config == 2:
        return [ModuleSpec("gate_up_proj", 4096, (12800, 12800), [32] * 12, 32)]
    if config == 3:
        return [ModuleSpec("down_proj", 12800, (4096,), [(8, 16, 32, 64)[a % 4] for a in range(48)], 64)]
    if config == 4:
        return layer_specs(24)
    raise ValueError(config)


def num_adapters_for(config: int) -> int:
    return {0: 4, 1: 12, 2: 12, 3: 48, 4: 24}[config]


def dtype_for(config: int) -> torch.dtype:
    return torch.float32 if config == 0 else torch.bfloat16


# Adapter populations on a workload's shapes (src/granite_switch docs/
# SWITCH_KERNELS.md "Methodology": balanced N x rank 32; imbalanced N x rank 32
# plus one larger adapter, N + 1 loaded, ids drawn uniformly over those
# loaded; and the idle batch, in which no token has an adapter).
POPULATIONS = ("balanced", "all_base", "r512")


def population_routing(config: int, population: str = "balanced") -> Routing:
    """Routing of ``population`` on workload ``config``'s shapes.

    balanced: the workload itself; all_base: the same batch with every token on
    the base model; r512: ids drawn over the workload's adapters plus one more
    (the rank-512 one), with the workload's activation offsets and positions.
    """
    if population == "balanced":
        return routing_for(config)
    if population == "all_base":
        r = routing_for(config)
        return Routing(np.zeros_like(r.req_ids), r.cu_seqlens, r.positions, r.act_offsets)
    if population == "r512":
        return routing_for(config, num_adapters=num_adapters_for(config) + 1)
    raise ValueError(f"unknown population {population!r}")


def population_adapters(config: int, population: str = "balanced") -> int:
    return num_adapters_for(config) + (1 if population == "r512" else 0)


def population_specs(config: int, population: str = "balanced") -> list:
    """Module specs of ``population``: r512 appends one adapter of rank 512 (storage rank 512)."""
    specs = module_specs(config)
    if population != "r512":
        return specs
    return [ModuleSpec(s.name, s.hidden, s.output_slices, list(s.ranks) + [512], 512) for s in specs]


def make_workload(config: int, device="cuda", seed: int = 0, layers: int | None = None) -> Workload:
    """Build a workload; for config 4, ``layers`` (default 32) layers x 4 modules."""
    routing = routing_for(config, seed)
    NA = num_adapters_for(config)
    dt = dtype_for(config)
    wl = Workload(config=config, name=NAMES[config], dtype=dt, num_adapters=NA, routing=routing)
    specs = module_specs(config)
    n_layers = (32 if layers is None else layers) if config == 4 else 1
    for layer in range(n_layers):
        for k, spec in enumerate(specs):
            wl.modules.append(make_module(spec, routing.num_tokens, NA, dt, device,
                                          seed=7919 * (config + 1) + 101 * layer + k + 1000003 * seed))
    return wl
