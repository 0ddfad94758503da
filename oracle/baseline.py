"""CPU baseline: the reference's HF switched-LoRA loop on torch-CPU.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): ``bench.py`` times it
as the ``cpu_baseline`` leg; the product never calls it.

Restates src/granite_switch/hf/core/lora.py:280-298 and :308-348 exactly: per
slice, for every active adapter (``unique`` of the positive ids), gather its
token rows, ``matmul`` with lora_A^T then with the pre-scaled lora_B^T, and
add into the output rows, in the tensors' own dtype.
"""

from __future__ import annotations

import os
import statistics
import subprocess
import time

import torch


def hf_loop(out: torch.Tensor, x: torch.Tensor, ids: torch.Tensor, lora_A_slices, lora_B_slices, output_slices):
    """In place on ``out`` [T, O]; ids [T] (0 = base)."""
    mask = ids > 0
    if not bool(mask.any()):
        return out
    active = ids[mask].unique()
    off = 0
    for s, o_s in enumerate(output_slices):
        A, B = lora_A_slices[s], lora_B_slices[s]
        out_slice = out[:, off:off + o_s]
        for a in active:
            idx = torch.where(ids == a)[0]
            if len(idx) == 0:
                continue
            lora = torch.matmul(x[idx], A[a - 1, 0].t())
            lora = torch.matmul(lora, B[a - 1, 0].t())
            out_slice[idx] += lora
        off += o_s
    return out


def _cgroup_cpu_quota() -> float | None:
    """CPUs granted by the cgroup v2 quota (``cpu.max``), or None when unlimited."""
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota == "max":
            return None
        return float(quota) / float(period)
    except (OSError, ValueError):
        return None


def host_cpu() -> dict:
    """The host's CPU as lscpu reports it, plus what this process may use.

    ``affinity``: CPUs in this process's affinity mask; ``quota``: CPUs its
    cgroup grants (None = no limit); ``threads``: the threads the baseline runs
    on -- every CPU it may run on, capped by the quota (more threads than the
    quota only queue for it).
    """
    info = {"model": "unknown", "sockets": None, "cores_per_socket": None, "threads_per_core": None,
            "logical_cpus": os.cpu_count()}
    try:
        out = subprocess.run(["lscpu"], stdout=subprocess.PIPE, stderr=subprocess.DEVNULL, text=True,
                             timeout=10).stdout
        keys = {"Model name": "model", "Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket",
                "Thread(s) per core": "threads_per_core", "CPU(s)": "logical_cpus"}
        for line in out.splitlines():
            k, _, v = line.partition(":")
            k = k.strip()
            if k in keys:
                v = v.strip()
                info[keys[k]] = v if keys[k] == "model" else int(v) if v.isdigit() else v
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    quota = _cgroup_cpu_quota()
    threads = affinity if quota is None else max(1, min(affinity, int(quota)))
    info.update(affinity=affinity, quota=quota, threads=threads)
    if isinstance(info["sockets"], int) and isinstance(info["cores_per_socket"], int):
        info["physical_cores"] = info["sockets"] * info["cores_per_socket"]
    return info


def cpu_threads() -> int:
    return host_cpu()["threads"]


def cpu_model() -> str:
    return str(host_cpu()["model"])


def time_modules(modules, ids: torch.Tensor, budget_s: float = 12.0, min_runs: int = 5):
    """Median seconds per pass of ``hf_loop`` over ``modules`` (CPU tensors).

    ``modules``: list of (y, x, lora_A_slices, lora_B_slices, output_slices).
    One warm-up pass, then passes until ``budget_s`` is spent (at least
    ``min_runs``).  Each pass works on a fresh copy of y.
    """
    threads = cpu_threads()
    torch.set_num_threads(threads)
    ys = [m[0].clone() for m in modules]

    def reset():
        for (y, *_), yb in zip(modules, ys):
            yb.copy_(y)

    def one_pass():
        for (y, x, A, B, sl), yb in zip(modules, ys):
            hf_loop(yb, x, ids, A, B, sl)

    reset()
    one_pass()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or time.perf_counter() < t_end:
        reset()
        t0 = time.perf_counter()
        one_pass()
        times.append(time.perf_counter() - t0)
        if len(times) >= 1000:
            break
    return statistics.median(times), len(times), threads
