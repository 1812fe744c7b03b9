"""CPU baseline for the decode GEMVs (test / benchmark infrastructure only).

Only ``bench.py``'s cpu_baseline leg imports this.  It restates, in torch on
the host CPU, the reference's dequantize-then-matmul definition of the decode
MLP linears (bench_gemv.py:30-53, models/int8_linear.py:50-53 for the
dequantize-per-forward pattern; the reference has no CPU int4 kernel, its
tinygemm path is GPU-only):

    x_hat = x * rsqrt(mean(x^2) + eps) * gamma           (fp32)
    W_eff = (q - 8) * s + z   per 128-k group           (fp32)
    h     = silu(x_hat @ Wg^T) * (x_hat @ Wu^T)          (gate | up)
    y     = h @ Wd^T                                     (down)

Each call dequantizes its weights, as a CPU int4 layer without a packed-int4
kernel must.  Weights rotate over several copies so the last-level cache
does not hold them.
"""

from __future__ import annotations

import os
import platform
import time

import torch


def host_threads() -> int:
    """Threads to use: the cores this process may run on, capped by
    OMP_NUM_THREADS when that is set."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def dequant_zp(packed: torch.Tensor, sz: torch.Tensor, group: int) -> torch.Tensor:
    """packed uint8 [N, K/2] (even k in the low nibble), scales_zeros bf16
    [K/group, N, 2] -> fp32 [N, K] with w = (q - 8) * s + z
    (models/int4_linear.py:61-63 storage, bench_gemv.py:51-52 dequant)."""
    n = packed.shape[0]
    q = torch.stack((packed & 15, packed >> 4), dim=-1).reshape(n, -1).float()
    s = sz[..., 0].float().t().repeat_interleave(group, dim=1)
    z = sz[..., 1].float().t().repeat_interleave(group, dim=1)
    return (q - 8.0) * s + z


def rmsnorm_f32(x: torch.Tensor, gamma: torch.Tensor, eps: float) -> torch.Tensor:
    x = x.float()
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * gamma.float()


def mlp_step(x, gamma, gu, down, group: int, eps: float = 1e-6) -> torch.Tensor:
    """One decode-MLP step: RMSNorm -> gate|up (SiLU-gate) -> down."""
    xn = rmsnorm_f32(x, gamma, eps)
    a = xn @ dequant_zp(gu[0], gu[1], group).t()
    half = a.shape[1] // 2
    h = torch.nn.functional.silu(a[:, :half]) * a[:, half:]
    return (h @ dequant_zp(down[0], down[1], group).t()).to(torch.bfloat16)


def time_mlp_steps(x, gamma, gu, down, group: int, algo_bytes: int, budget_s: float = 10.0,
                   copies: int = 24, max_steps: int = 1000) -> dict:
    """Time the decode-MLP step on the host CPU for about ``budget_s``
    seconds (at least one step) over ``copies`` rotated weight copies.
    Inputs are CPU tensors.  Returns µs per step and TB/s on the algorithmic
    bytes of one step."""
    threads = host_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        reps = [((gu[0].clone(), gu[1].clone()), (down[0].clone(), down[1].clone())) for _ in range(copies)]
        mlp_step(x, gamma, reps[0][0], reps[0][1], group)  # warm-up (allocator, thread pool)
        steps = 0
        t0 = time.perf_counter()
        while True:
            g, d = reps[steps % copies]
            mlp_step(x, gamma, g, d, group)
            steps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or steps >= max_steps:
                break
    finally:
        torch.set_num_threads(prev)
    us = el / steps * 1e6
    return {"us_per_step": us, "tbps": algo_bytes / (us * 1e-6) / 1e12, "steps": steps, "threads": threads,
            "cpu": cpu_model(), "seconds": el}


def time_mlp_steps_predequant(x, gamma, gu, down, group: int, algo_bytes: int, budget_s: float = 10.0,
                              min_rotation_bytes: int = 2 << 30, max_steps: int = 1000) -> dict:
    """The same step with the weights dequantized to fp32 once, before the
    timed loop (the bandwidth-bound CPU ceiling the reference computes in
    bench_cpu_bound.py:24-46, which streams plain float weights over rotated
    copies).  Copies are added until the rotation spans ``min_rotation_bytes``
    (2 GiB by default, beyond any host last-level cache)."""
    threads = host_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        wg = dequant_zp(gu[0], gu[1], group)
        wd = dequant_zp(down[0], down[1], group)
        per = (wg.numel() + wd.numel()) * 4
        copies = max(2, -(-min_rotation_bytes // per))
        reps = [(wg.clone(), wd.clone()) for _ in range(copies)]
        del wg, wd

        def step(g, d):
            xn = rmsnorm_f32(x, gamma, 1e-6)
            a = xn @ g.t()
            half = a.shape[1] // 2
            h = torch.nn.functional.silu(a[:, :half]) * a[:, half:]
            return (h @ d.t()).to(torch.bfloat16)

        step(*reps[0])  # warm-up
        steps = 0
        t0 = time.perf_counter()
        while True:
            step(*reps[steps % copies])
            steps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or steps >= max_steps:
                break
    finally:
        torch.set_num_threads(prev)
    us = el / steps * 1e6
    return {"us_per_step": us, "tbps": algo_bytes / (us * 1e-6) / 1e12, "steps": steps, "threads": threads,
            "cpu": cpu_model(), "seconds": el, "copies": copies, "fp32_bytes_per_step": per}
