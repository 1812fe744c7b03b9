#!/usr/bin/env python3
"""Decode-GEMV benchmark on one MI355X.

Workload (the int4 decoder-MLP GEMVs at M = 1): every step runs
  gate|up  RMSNorm -> int4 group-128 GEMV K=2560, N=2x10240 -> SiLU(gate)*up
  down     int4 group-128 GEMV K=10240, N=2560
on synthetic weights N(0, 0.02) quantized symmetric int4 (bf16 scales), bf16
activations N(0, 1), gamma = 1 + N(0, 0.1), eps 1e-6, seed 0, held in the
decode layout the modules use (16-row tiled blocks; gate|up paired for the
SiLU-gate epilogue).  The weights rotate over copies spanning >= 1 GiB so
every step streams them from HBM, and the K timed steps are one HIP-graph
replay.

value = algorithmic bytes of K steps / their GPU time, in TB/s, where one
call's algorithmic bytes are packed weights + scales + x + gamma + output
(each byte once, no re-reads).  Also reported:
  roofline     the gate|up GEMV alone (the dominant kernel): its average
               launch duration from HIP events on its launch stream, and the
               HBM bytes per launch measured by rocprofv3 counters when a
               committed summary holds them;
  cpu_baseline the same MLP step as dequantize-then-matmul in torch on the
               host cores (a bounded sample of steps), and the same step on
               weights dequantized once;
  detail       per-kernel times in both weight layouts, the launch and
               streaming-read floors, the full synthetic decode step (26 int4
               decoder layers + bf16 head) in µs against its bytes-moved
               roofline, the C1-C4 GEMV table, torch's bf16 linear at the
               C2/C3 shapes, the fused attention step and the fp32 heads,
               each against its HBM roofline.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-step]

Counter runs (HBM bytes per launch of the PROFILE_CASES GEMVs -- the M=1
decode GEMVs and the C4 split-K tile GEMV -- scaled by what the same counter
reads for a plain 256 MiB elementwise copy):
  rocprofv3 --pmc FETCH_SIZE --output-format csv -d D1 -o run -- python3 bench.py --profile-gemvs
  rocprofv3 --pmc WRITE_SIZE --output-format csv -d D2 -o run -- python3 bench.py --profile-gemvs
  python3 bench.py --pmc-summary D1 D2      (prints the traffic summary)

Matrix-core use of the several-row tile GEMVs (C4 shapes at M = 16 and 32):
  rocprofv3 --kernel-trace --output-format csv -d T -o run -- python3 bench.py --profile-tiles
  rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA SQ_INSTS_VALU --output-format csv -d P -o run \
      -- python3 bench.py --profile-tiles
  python3 bench.py --mfma-summary T P
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "breeze-tts-2_amd"))

HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16 matrix-core peak of MI355X
MI355X_SIMDS = 256 * 4
MI355X_CLOCK_GHZ = 2.4
GROUP = 128
EPS = 1e-6
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_decode_traffic.txt")
COPY_BYTES = 256 << 20


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algo_bytes(wbits: int, n: int, k: int, m: int, norm: bool, epi: int) -> int:
    """Algorithmic bytes of one GEMV call: weights + scales + x (+ gamma)
    + output (+ residual); SiLU-gate halves the output."""
    if wbits == 4:
        w = n * k // 2 + (k // GROUP) * n * 4
    elif wbits == 8:
        w = n * k + 4 * n
    else:
        w = 2 * n * k
    n_out = n // 2 if epi == 1 else n
    return w + 2 * m * k + (2 * k if norm else 0) + 2 * m * n_out + (2 * m * n_out if epi == 2 else 0)


def read_traffic():
    """HBM bytes per launch of the gate|up GEMV (the first PROFILE_CASES
    entry) from the committed rocprofv3 counter summary (line
    'traffic_bytes_per_launch[<case>]: <int>'), else None."""
    want = PROFILE_CASES[0][0]
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                m = re.match(r"\s*traffic_bytes_per_launch\[(.*)\]:\s*(\d+)", line)
                if m and m.group(1) == want:
                    return int(m.group(2))
    except OSError:
        pass
    return None


# (name, format "int4"/"fp8", layout, N, K, M, epilogue, RMSNorm): the GEMVs
# whose HBM traffic the counter runs measure, launched PROFILE_REPS times
# each (after one warm-up launch) in this order by --profile-gemvs.
PROFILE_CASES = [
    ("int4 gate|up K2560 N20480 M1", "int4", "tiled", 20480, 2560, 1, 1, True),
    ("int4 down K10240 N2560 M1", "int4", "tiled", 2560, 10240, 1, 0, False),
    ("fp8 gate|up K2560 N20480 M1", "fp8", "tiled", 20480, 2560, 1, 1, True),
    ("fp8 down K10240 N2560 M1", "fp8", "tiled", 2560, 10240, 1, 0, False),
    ("int4 qkv K2560 N6144 M1", "int4", "tiled", 6144, 2560, 1, 0, True),
    ("int4 o_proj K4096 N2560 M1", "int4", "tiled", 2560, 4096, 1, 2, False),
    ("fp8 qkv K2560 N4096 M1", "fp8", "tiled", 4096, 2560, 1, 0, True),
    ("fp8 o_proj K4096 N2560 M1", "fp8", "tiled", 2560, 4096, 1, 2, False),
    ("int4 C4 K10240 N2560 M32 (row-major, split-K tile)", "int4", "rowmajor", 2560, 10240, 32, 0, False),
    ("int4 C4 K10240 N2560 M32 (tiled, panel, 3 K slices)", "int4", "tiled", 2560, 10240, 32, 0, False),
    ("fp8 C4 K10240 N2560 M32 (tiled, panel, 4 K slices)", "fp8", "tiled", 2560, 10240, 32, 0, False),
    ("int4 C4 K2560 N20480 M32 (tiled, panel)", "int4", "tiled", 20480, 2560, 32, 0, False),
    ("fp8 C4 K2560 N20480 M32 (tiled, panel)", "fp8", "tiled", 20480, 2560, 32, 0, False),
]
PROFILE_REPS = 12

# Shader clock cycles of the device-side wait ahead of a timed graph replay
# (about 200 us at 2.4 GHz): longer than the host's submission of the
# graph, so the first step starts on an already submitted graph.
LAUNCH_COVER_CYCLES = 480_000


def profile_gemvs(torch, G, dev) -> int:
    """Launch each PROFILE_CASES GEMV 1 + PROFILE_REPS times, rotating over
    copies that span >= 1 GiB, then a 256 MiB elementwise copy three times,
    for rocprofv3 counter runs; --pmc-summary reads them back."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    for name, fmt, layout, N, K, M, epi, norm in PROFILE_CASES:
        w = torch.randn(N, K, device=dev, generator=gen) * 0.02
        base, wfmt, _ = _weights(torch, G, fmt, N, K, epi, w, layout)
        del w
        wbytes = sum(t.numel() * t.element_size() for t in base)
        ncopy = max(2, -(-(1 << 30) // wbytes))
        copies = [tuple(t.clone() for t in base) for _ in range(ncopy)]
        x = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
        gamma = (1 + 0.1 * torch.randn(K, device=dev, generator=gen)).to(torch.bfloat16) if norm else None
        n_out = N // 2 if epi == 1 else N
        res = torch.randn(M, n_out, device=dev, generator=gen).to(torch.bfloat16) if epi == 2 else None
        out = torch.empty(M, n_out, device=dev, dtype=torch.bfloat16)
        for i in range(1 + PROFILE_REPS):
            c = copies[i % ncopy]
            G.gemv(x, c[0], wfmt, N, sc0=c[1] if len(c) > 1 else None, group=GROUP, gamma=gamma, eps=EPS,
                   epilogue=epi, residual=res, out=out)
        torch.cuda.synchronize()
        log(f"{name}: {1 + PROFILE_REPS} launches")
        del copies, base
        torch.cuda.empty_cache()
    a_cp = torch.ones(COPY_BYTES // 4, device=dev)
    b_cp = torch.empty_like(a_cp)
    for _ in range(3):
        torch.mul(a_cp, 1.0, out=b_cp)
    torch.cuda.synchronize()
    log(f"3 copies of {COPY_BYTES} bytes")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-step", action="store_true", help="skip the 26-layer decode step detail")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-config GEMV table (C1-C4)")
    ap.add_argument("--no-floors", action="store_true", help="skip the launch and streaming-read floors")
    ap.add_argument("--detail-out", metavar="FILE",
                    help="also write the full record (every table) as one JSON line to FILE")
    ap.add_argument("--profile-gemvs", action="store_true",
                    help="only launch the PROFILE_CASES GEMVs (eagerly) and a 256 MiB copy, for counter runs")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarize two rocprofv3 --pmc runs of --profile-gemvs")
    ap.add_argument("--config-summary", metavar="DETAIL_FILE",
                    help="print the C1-C4 configuration table, the floors, the decode steps and the library "
                         "comparator from a --detail-out file")
    ap.add_argument("--sq-summary", metavar="PMC_DIR",
                    help="per-tile instruction and wait counters of the PROFILE_CASES GEMVs from a rocprofv3 "
                         "--pmc run (SQ_ counters) of --profile-gemvs")
    ap.add_argument("--profile-tiles", action="store_true",
                    help="only launch the several-row (C4, M = 16 and 32) GEMVs eagerly, for counter runs")
    ap.add_argument("--profile-depth", action="store_true",
                    help="only build and time the depth-decoder frame graph, for kernel-trace runs")
    ap.add_argument("--mfma-summary", nargs=2, metavar=("TRACE_DIR", "PMC_DIR"),
                    help="summarize a rocprofv3 --kernel-trace run and a --pmc run of --profile-tiles")
    ap.add_argument("--profile-step", type=int, metavar="M",
                    help="only build the 26-layer decode step at M rows (tiled layout) and replay its graph, "
                         "for kernel-trace runs")
    ap.add_argument("--step-summary", metavar="TRACE_DIR",
                    help="per-kernel breakdown of the decode-step replays in a rocprofv3 --kernel-trace run of "
                         "--profile-step")
    args = ap.parse_args()
    if args.pmc_summary:
        return pmc_summary(*args.pmc_summary)
    if args.mfma_summary:
        return mfma_summary(*args.mfma_summary)
    if args.sq_summary:
        return sq_summary(args.sq_summary)
    if args.config_summary:
        return config_summary(args.config_summary)
    if args.step_summary:
        return step_summary(args.step_summary)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the decode GEMVs here run "
              "on a single MI355X and no multi-GPU path is built).", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2

    import torch

    from breeze_amd import gemv as G
    from breeze_amd import _lib

    _lib.lib()  # fails loudly when the HIP library is missing
    if not torch.cuda.is_available():
        print("bench.py needs a GPU (torch.cuda.is_available() is False)", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"device {torch.cuda.get_device_name(0)}")
    if args.profile_tiles:
        return profile_tiles(torch, G, dev)
    if args.profile_gemvs:
        return profile_gemvs(torch, G, dev)
    if args.profile_step:
        print(json.dumps({"decode_step": decode_step(torch, G, dev, log, args.profile_step, reps=STEP_REPS)}),
              flush=True)
        return 0
    if args.profile_depth:
        print(json.dumps({"depth_frame": depth_frame(torch, dev, log)}), flush=True)
        return 0

    # ---- synthetic C2 weights (seed 0: W, then gamma, then x, on the CPU)
    K1, N1, K2, N2, M = 2560, 20480, 10240, 2560, 1
    torch.manual_seed(0)
    w_gu = torch.randn(N1, K1) * 0.02
    w_dn = torch.randn(N2, K2) * 0.02
    gamma = (1 + 0.1 * torch.randn(K1)).to(torch.bfloat16)
    x = torch.randn(M, K1).to(torch.bfloat16)
    gu_p, gu_sz, _ = G.quantize_int4_device(w_gu.to(dev), GROUP, True, G.W_INT4_ZP)
    dn_p, dn_sz, _ = G.quantize_int4_device(w_dn.to(dev), GROUP, True, G.W_INT4_ZP)
    del w_gu, w_dn
    # the decode layout: gate|up tiled paired (8 gate + 8 up rows per block), down tiled
    gu_t = G.pack_tiled(G.W_INT4_ZP, gu_p, K1, G.W_INT4_TILED_PAIRED, sc0=gu_sz)
    dn_t = G.pack_tiled(G.W_INT4_ZP, dn_p, K2, G.W_INT4_TILED, sc0=dn_sz)
    gamma_d, x_d = gamma.to(dev), x.to(dev)
    b_gu = algo_bytes(4, N1, K1, M, True, 1)
    b_dn = algo_bytes(4, N2, K2, M, False, 0)
    step_bytes = b_gu + b_dn
    wbytes = gu_t.numel() + dn_t.numel()
    # enough (gate|up, down) pairs that each weight ALONE spans >= 1 GiB: the
    # per-kernel legs below rotate through one of the two only
    ncopy = max(2, -(-(1 << 30) // min(gu_t.numel(), dn_t.numel())))
    copies = [(gu_t.clone(), dn_t.clone()) for _ in range(ncopy)]
    h = torch.empty(M, N1 // 2, device=dev, dtype=torch.bfloat16)
    y = torch.empty(M, N2, device=dev, dtype=torch.bfloat16)
    log(f"C2 M={M}: {ncopy} weight copies ({ncopy * wbytes / 2**30:.2f} GiB), {step_bytes} algorithmic bytes/step")

    def gate_up(c):
        G.gemv(x_d, c[0], G.W_INT4_TILED_PAIRED, N1, gamma=gamma_d, eps=EPS, epilogue=G.EPI_SILU_GATE, out=h)

    def down(c):
        G.gemv(h, c[1], G.W_INT4_TILED, N2, out=y)

    def step(i):
        c = copies[i % ncopy]
        gate_up(c)
        down(c)

    def capture(fn, n):
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(st):
            with torch.cuda.graph(g, stream=st):
                for i in range(n):
                    fn(i)
        torch.cuda.current_stream().wait_stream(st)
        torch.cuda.synchronize()
        return g

    def timed(g):
        """Replay g once between synchronizations; returns (event ms, wall s).

        A short device-side wait goes ahead of the start event, so the host's
        submission of the graph (tens of us for a graph of K steps, the GPU
        idle meanwhile) overlaps it: the events bracket exactly the K steps
        on the GPU, not the host's launch latency in front of the first."""
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        if hasattr(torch.cuda, "_sleep"):
            torch.cuda._sleep(LAUNCH_COVER_CYCLES)
        s_ev.record()
        g.replay()
        e_ev.record()
        torch.cuda.synchronize()
        return s_ev.elapsed_time(e_ev), time.perf_counter() - t0

    # ---- eager check of one step against a dequantize-then-matmul on the GPU
    step(0)
    torch.cuda.synchronize()
    xn = x_d.float() * torch.rsqrt(x_d.float().pow(2).mean(-1, keepdim=True) + EPS) * gamma_d.float()
    a = xn @ G.dequant(G.W_INT4_ZP, gu_p, N1, K1, sc0=gu_sz, group=GROUP).float().t()
    ref_h = torch.nn.functional.silu(a[:, : N1 // 2]) * a[:, N1 // 2:]
    err_h = ((h.float() - ref_h).abs().max() / ref_h.abs().max()).item()
    ref_y = h.float() @ G.dequant(G.W_INT4_ZP, dn_p, N2, K2, sc0=dn_sz, group=GROUP).float().t()
    err_y = ((y.float() - ref_y).abs().max() / ref_y.abs().max()).item()
    del a, ref_h, ref_y, xn
    log(f"parity vs dequantize-then-matmul: gate|up {err_h:.2e}, down {err_y:.2e}")
    if not (err_h <= 1e-2 and err_y <= 1e-2):
        print(f"parity check failed: gate|up {err_h}, down {err_y}", file=sys.stderr)
        return 1

    # ---- warm-up W steps, then exactly K timed steps (one graph replay each)
    if args.warmup:
        gw = capture(step, args.warmup)
        timed(gw)
        del gw
    log(f"capturing {args.steps} steps")
    gk = capture(step, args.steps)
    # the first replay of a freshly instantiated graph also uploads it to the
    # device (a fixed ~30 us, 2 us per step at 20 steps): that replay is
    # set-up, untimed; the timed replay then runs exactly the K steps
    gk.replay()
    torch.cuda.synchronize()
    ms, wall = timed(gk)
    log(f"{args.steps} steps: {ms:.3f} ms (events), {wall * 1e3:.3f} ms (wall)")
    del gk
    value_tbps = step_bytes * args.steps / (ms * 1e-3) / 1e12

    # ---- dominant kernel alone: gate|up, back-to-back launches on one stream;
    #      the median of three replays (one replay disturbed by, e.g., a
    #      profiler's buffer flush does not move it)
    reps = 2 * ncopy

    def per_launch_us(g):
        timed(g)
        return statistics.median(timed(g)[0] for _ in range(3)) * 1e3 / reps

    g_gu = capture(lambda i: gate_up(copies[i % ncopy]), reps)
    us_gu = per_launch_us(g_gu)
    del g_gu
    g_dn = capture(lambda i: down(copies[i % ncopy]), reps)
    us_dn = per_launch_us(g_dn)
    del g_dn
    achieved = b_gu / (us_gu * 1e-6) / 1e9
    traffic = read_traffic()
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                "kernel": "gemv_wide int4 tiled-paired SiLU-gate K2560 N20480 M1 (+RMSNorm), 5 row blocks "
                          "per workgroup",
                "algorithmic_bytes": b_gu, "avg_launch_us": round(us_gu, 3)}
    log(f"gate|up {us_gu:.2f} us ({achieved:.0f} GB/s), down {us_dn:.2f} us "
        f"({b_dn / us_dn / 1e3:.0f} GB/s)")
    del copies

    # ---- the same two GEMVs over the row-major layout (the other kernels)
    rm = [(gu_p.clone(), gu_sz.clone(), dn_p.clone(), dn_sz.clone()) for _ in range(ncopy)]  # >= 1 GiB each
    g_rm = capture(lambda i: G.gemv(x_d, rm[i % ncopy][0], G.W_INT4_ZP, N1, sc0=rm[i % ncopy][1], group=GROUP,
                                    gamma=gamma_d, eps=EPS, epilogue=G.EPI_SILU_GATE, out=h), reps)
    us_gu_rm = per_launch_us(g_rm)
    del g_rm
    g_rm = capture(lambda i: G.gemv(h, rm[i % ncopy][2], G.W_INT4_ZP, N2, sc0=rm[i % ncopy][3], group=GROUP,
                                    out=y), reps)
    us_dn_rm = per_launch_us(g_rm)
    del g_rm, rm
    torch.cuda.empty_cache()
    log(f"row-major layout: gate|up {us_gu_rm:.2f} us, down {us_dn_rm:.2f} us")

    detail = {
        "gate_up_us": round(us_gu, 3), "down_us": round(us_dn, 3),
        "down_gbps": round(b_dn / us_dn / 1e3, 1),
        "rowmajor_gate_up_us": round(us_gu_rm, 3), "rowmajor_down_us": round(us_dn_rm, 3),
        "step_roofline_us": round(step_bytes / HBM_PEAK_GBPS / 1e3, 3),
        "parity_rel_err": {"gate_up": err_h, "down": err_y},
    }
    if not args.no_floors:
        detail["floors"] = floors(torch, G, dev, log)

    # ---- full synthetic decode step (26 int4 layers + bf16 head), M = 1
    if not args.no_step:
        detail["decode_step"] = decode_step(torch, G, dev, log, 1)
        detail["decode_step_m2"] = decode_step(torch, G, dev, log, 2)
        detail["decode_step_rowmajor"] = decode_step(torch, G, dev, log, 1, layout="rowmajor")
        detail["decode_step_attn"] = decode_step(torch, G, dev, log, 2, attn_pos=1023, cache_len=1024)
        detail["depth_frame"] = depth_frame(torch, dev, log)
    if not args.no_configs:
        detail["configs"] = config_table(torch, G, dev, log)
        detail["modules"] = module_table(torch, dev, log)
        detail["library_bf16_linear"] = library_table(torch, dev, log)
        detail["attention"] = attention_table(torch, dev, log)
        detail["fp32_heads"] = heads_table(torch, dev, log)

    # ---- CPU baseline: same MLP step on the host cores (bounded sample)
    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, ROOT)
        from oracle.cpu_baseline import time_mlp_steps

        log(f"CPU baseline: about {args.cpu_seconds:.0f} s of host work")
        r = time_mlp_steps(x, gamma, (gu_p.cpu(), gu_sz.cpu()), (dn_p.cpu(), dn_sz.cpu()), GROUP, step_bytes,
                           budget_s=args.cpu_seconds)
        cpu = {"value": r["tbps"], "unit": "TB/s", "cores": r["threads"], "kind": "port",
               "sample": f"{r['steps']} full C2 M=1 MLP steps (RMSNorm, int4 gate|up dequant+matmul, SiLU, "
                         f"int4 down dequant+matmul) in torch fp32 on {r['threads']} threads of {r['cpu']}, "
                         f"24 rotated weight copies",
               "us_per_step": round(r["us_per_step"], 1)}
        log(f"CPU: {r['us_per_step']:.0f} us/step on {r['threads']} threads")
        from oracle.cpu_baseline import time_mlp_steps_predequant

        r2 = time_mlp_steps_predequant(x, gamma, (gu_p.cpu(), gu_sz.cpu()), (dn_p.cpu(), dn_sz.cpu()), GROUP,
                                       step_bytes, budget_s=args.cpu_seconds)
        cpu["predequantized"] = {
            "value": r2["tbps"], "unit": "TB/s", "cores": r2["threads"], "us_per_step": round(r2["us_per_step"], 1),
            "sample": f"{r2['steps']} of the same steps with the weights dequantized to fp32 once "
                      f"({r2['fp32_bytes_per_step']} fp32 weight bytes per step, {r2['copies']} rotated copies)"}
        log(f"CPU, pre-dequantized fp32 weights: {r2['us_per_step']:.0f} us/step")

    out = {
        "metric": "int4/fp8 GEMV achieved HBM TB/s at M=1; µs per decoder-layer decode step",
        "value": round(value_tbps, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "int4 group-128 decoder-MLP GEMVs, M=1: RMSNorm->gate|up K2560 N2x10240 "
                               "SiLU-gate, then down K10240 N2560",
                   "weights": "int4 symmetric g128 (bf16 scales) in the 16-row tiled layout (gate|up paired), "
                              "bf16 activations, fp32 accumulate",
                   "M": 1, "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "detail": detail,
    }
    # the full record (every table) goes to stderr and, with --detail-out, to
    # a file; the last stdout line is the compact summary a driver parses
    full = json.dumps(out)
    log(f"full record: {full}")
    if args.detail_out:
        with open(args.detail_out, "w") as f:
            f.write(full + "\n")
    print(json.dumps(compact(out)), flush=True)
    return 0


SUMMARY_MAX_CHARS = 4000


def _pick(d, *keys):
    return {k: d[k] for k in keys if isinstance(d, dict) and k in d}


def compact(out: dict) -> dict:
    """The one-line summary of a full bench record: the contract keys,
    `roofline`, `cpu_baseline` (without its nested second leg's sample) and
    a `summary` of the per-kernel µs, the decode steps against their
    roofline and the C3 fp8 decode GEMVs.  Stays under SUMMARY_MAX_CHARS."""
    head = {k: out[k] for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config")}
    head["roofline"] = out.get("roofline")
    cpu = out.get("cpu_baseline")
    if cpu:
        cpu = _pick(cpu, "value", "unit", "cores", "kind", "sample", "us_per_step")
        pre = out["cpu_baseline"].get("predequantized")
        if pre:
            cpu["predequantized_us_per_step"] = pre.get("us_per_step")
    head["cpu_baseline"] = cpu
    d = out.get("detail", {})
    s = _pick(d, "gate_up_us", "down_us", "rowmajor_gate_up_us", "rowmajor_down_us", "step_roofline_us")
    steps = {}
    for key, name in (("decode_step", "c5_m1"), ("decode_step_m2", "c5_m2"),
                      ("decode_step_rowmajor", "c5_m1_rowmajor"), ("decode_step_attn", "c5_m2_attn_pos1023"),
                      ("depth_frame", "depth_frame_fp8")):
        if key in d:
            steps[name] = _pick(d[key], "us", "roofline_us", "x_roofline", "replay_matches_eager")
    if steps:
        s["decode_steps"] = steps
    fl = d.get("floors")
    if fl:
        s["floors"] = {"empty_node_us": fl.get("empty_node_us"), "read_fit": fl.get("read_fit")}
    gemvs = {}
    for r in d.get("configs", []):
        if r.get("layout") == "tiled" and r.get("M") in (1, 2) and r["config"].startswith(("C1", "C2", "C3")):
            gemvs[f"{r['config'].split(' ')[0]} {r['config'].split(' ', 1)[1]} M{r['M']}"] = [r["us"], r["frac"]]
    if gemvs:
        s["gemv_us_frac"] = gemvs
    mods = {f"{r['module']} M{r['M']}": [r["us"], r["frac"]] for r in d.get("modules", [])}
    if mods:
        s["module_us_frac"] = mods
    head["summary"] = s
    if len(json.dumps(head)) > SUMMARY_MAX_CHARS:  # never: trimmed from the largest optional part first
        s.pop("gemv_us_frac", None)
    return head


# The several-row GEMVs whose matrix-core use is reported (C4 at M = 16, 32,
# tile_cases() in launch order), each launched TILE_REPS times (after one
# sizing launch) by --profile-tiles.
TILE_REPS = 20


def tile_cases() -> list:
    return [(name, fmt, N, K, M, layout) for name, fmt, N, K, _, _, _ in CONFIG_SHAPES if name.startswith("C4")
            for layout in ("rowmajor", "tiled") for M in (16, 32)]


SEVERAL_ROW_KERNELS = ("gemv_tile", "gemv_panel")


def profile_tiles(torch, G, dev) -> int:
    """Launch each tile_cases() GEMV TILE_REPS times (launch shape from the
    static table or the built-in rule, as in the config table) for
    rocprofv3 counter and trace runs; --mfma-summary reads them back."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    for name, fmt, N, K, M, layout in tile_cases():
        w = torch.randn(N, K, device=dev, generator=gen) * 0.02
        base, wfmt, _ = _weights(torch, G, fmt, N, K, 0, w, layout)
        del w
        p, sc = base[0], (base[1] if len(base) > 1 else None)
        x = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
        out = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
        G.gemv(x, p, wfmt, N, sc0=sc, group=GROUP, out=out)  # sizes the workspace (one extra launch)
        torch.cuda.synchronize()
        for _ in range(TILE_REPS):
            G.gemv(x, p, wfmt, N, sc0=sc, group=GROUP, out=out)
        torch.cuda.synchronize()
        log(f"{name} {layout} M={M}: {TILE_REPS + 1} launches")
    return 0


def mfma_summary(trace_dir: str, pmc_dir: str) -> int:
    """Matrix-core utilisation of the several-row tile GEMVs: per launch,
    SQ_VALU_MFMA_BUSY_CYCLES (summed over all SIMDs) / (SIMDs x launch
    duration x peak engine clock), with the duration from the kernel trace
    of the same command.  At a lower actual clock the utilisation is higher,
    so this is a lower bound."""
    import csv
    import glob
    import statistics

    def rows(d, pattern):
        paths = glob.glob(os.path.join(d, "**", pattern), recursive=True)
        if not paths:
            raise SystemExit(f"no {pattern} under {d}")
        return list(csv.DictReader(open(paths[0])))

    cases = tile_cases()

    def groups(seq):
        # launches of the several-row kernels in launch order, split into the tile_cases() runs
        n = TILE_REPS + 1
        if len(seq) != n * len(cases):
            raise SystemExit(f"{len(seq)} tile dispatches, expected {n * len(cases)}")
        return [seq[i * n + 1:(i + 1) * n] for i in range(len(cases))]

    def several(kname):
        return any(k in kname for k in SEVERAL_ROW_KERNELS)

    tr = sorted((int(r["Dispatch_Id"]), int(r["End_Timestamp"]) - int(r["Start_Timestamp"]), r["Kernel_Name"])
                for r in rows(trace_dir, "*kernel_trace.csv") if several(r["Kernel_Name"]))
    per = {}
    for r in rows(pmc_dir, "*counter_collection.csv"):
        if not several(r["Kernel_Name"]):
            continue
        per.setdefault(int(r["Dispatch_Id"]), {}).setdefault(r["Counter_Name"], 0.0)
        per[int(r["Dispatch_Id"])][r["Counter_Name"]] += float(r["Counter_Value"])
    pm = [per[k] for k in sorted(per)]
    print(f"matrix-core use of the several-row tile GEMVs, MI355X ({MI355X_SIMDS} SIMDs, "
          f"{MI355X_CLOCK_GHZ} GHz peak engine clock); median of {TILE_REPS} launches each")
    print(f"{'config':28s} {'layout':8s} {'M':>3s} {'us':>7s} {'TFLOP/s':>8s} {'MFMA busy':>10s} {'util':>7s} "
          f"{'MFMA instr':>10s} {'VALU instr':>11s}  kernel")
    for (name, fmt, N, K, M, layout), t, c in zip(cases, groups(tr), groups(pm)):
        us = statistics.median(d for _, d, _ in t) / 1e3
        busy = statistics.median(x.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) for x in c)
        util = busy / (MI355X_SIMDS * us * 1e-6 * MI355X_CLOCK_GHZ * 1e9)
        kern = re.search(r"gemv_(tile|panel)<[^>]*>", t[0][2])
        print(f"{name:28s} {layout:8s} {M:3d} {us:7.2f} {2.0 * M * N * K / us / 1e6:8.1f} {busy:10.0f} {100 * util:6.2f}% "
              f"{statistics.median(x.get('SQ_INSTS_MFMA', 0.0) for x in c):10.0f} "
              f"{statistics.median(x.get('SQ_INSTS_VALU', 0.0) for x in c):11.0f}  {kern.group(0) if kern else ''}")
    return 0


def pmc_summary(fetch_dir: str, write_dir: str) -> int:
    """Per-launch FETCH_SIZE / WRITE_SIZE (KiB) of each PROFILE_CASES GEMV
    from two rocprofv3 counter runs of --profile-gemvs, each scaled by the
    ratio of the known bytes of the 256 MiB copy to what the counter read for
    it; the median over each case's PROFILE_REPS launches (the warm-up
    launch dropped)."""
    import csv
    import glob
    import statistics

    n = 1 + PROFILE_REPS

    def load(d, counter):
        paths = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if not paths:
            raise SystemExit(f"no counter_collection.csv under {d}")
        per = {}
        for row in csv.DictReader(open(paths[0])):
            if row["Counter_Name"] != counter:
                continue
            key = int(row["Dispatch_Id"])
            per.setdefault(key, [row["Kernel_Name"], 0.0])[1] += float(row["Counter_Value"])
        seq = [per[k] for k in sorted(per)]
        gemv = [(name, v) for name, v in seq if "gemv_" in name]
        # the copies are the last three elementwise multiplies (earlier ones scale the synthetic weights)
        copy = [v for name, v in seq if "elementwise" in name.lower() and "mul" in name.lower()][-3:]
        if len(gemv) != n * len(PROFILE_CASES) or not copy:
            raise SystemExit(f"{d}: {len(gemv)} GEMV dispatches (expected {n * len(PROFILE_CASES)}), "
                             f"{len(copy)} copy dispatches")
        cases = [gemv[i * n + 1:(i + 1) * n] for i in range(len(PROFILE_CASES))]
        return [(c[0][0], statistics.median(v for _, v in c)) for c in cases], statistics.median(copy)

    fetch, f_copy = load(fetch_dir, "FETCH_SIZE")
    write, w_copy = load(write_dir, "WRITE_SIZE")
    kib = COPY_BYTES / 1024
    fr, wr = kib / f_copy, kib / w_copy
    print(f"HBM traffic per launch, median of {PROFILE_REPS} launches per case; counters scaled by a "
          f"{COPY_BYTES}-byte copy: FETCH_SIZE {f_copy:.1f} KiB -> read scale {fr:.4f}, "
          f"WRITE_SIZE {w_copy:.1f} KiB -> write scale {wr:.4f}")
    print(f"{'case':56s} {'algorithmic B':>13s} {'fetch B':>11s} {'write B':>9s} {'traffic B':>11s} "
          f"{'traffic/algo':>12s}  kernel")
    lines = []
    for case, (kname, f), (_, w) in zip(PROFILE_CASES, fetch, write):
        name, fmt, layout, N, K, M, epi, norm = case
        algo = algo_bytes(4 if fmt == "int4" else 8, N, K, M, norm, epi)
        fb, wb = int(round(f * fr * 1024)), int(round(w * wr * 1024))
        kern = re.search(r"gemv_\w+<[^>]*>", kname)
        print(f"{name:56s} {algo:13d} {fb:11d} {wb:9d} {fb + wb:11d} {(fb + wb) / algo:12.4f}  "
              f"{kern.group(0) if kern else kname[:60]}")
        lines.append(f"traffic_bytes_per_launch[{name}]: {fb + wb}")
    for line in lines:
        print(line)
    return 0


def config_summary(path: str) -> int:
    """The configuration table and its context (floors, decode steps, torch's
    bf16 linear) from the full record bench.py wrote with --detail-out."""
    rec = json.loads(open(path).read().strip().splitlines()[-1])
    det = rec["detail"]
    fl = det["floors"]
    reads = ", ".join(f"{r['mib']} MiB {r['us']} us ({r['gbps']} GB/s)" for r in fl["read"])
    line = (f"floors: empty graph node {fl['empty_node_us']} us; read-only kernel {reads}; fit "
            f"{fl['read_fit']['fixed_us']} us + bytes at {fl['read_fit']['gbps']} GB/s")
    cp = fl.get("copy_1gib") or {}
    if cp:
        line += f"; 1 GiB device copy {cp.get('us')} us ({cp.get('gbps_read_plus_write')} GB/s read+write)"
    print(line)
    for c in fl.get("chunks", []):
        print(f"  read with a GEMV's decomposition: {c['what']}: {c['us']} us ({c['gbps']} GB/s)")
    for c in fl.get("shared_x", []):
        print(f"  whole-K read, x shared by all workgroups (bz_shared_read): {c['what']}, {c['workgroups']} x "
              f"({c['x_bytes']} B of x + {c['w_bytes_per_workgroup']} B own): {c['us']} us "
              f"({c['gbps_per_workgroup']} GB/s per workgroup)")
    for key, what in (("decode_step", "tiled, M=1, copy for attention"), ("decode_step_m2", "tiled, M=2, copy for attention"),
                      ("decode_step_rowmajor", "rowmajor, M=1, copy for attention"),
                      ("decode_step_attn", "tiled, M=2, attention at 1023 of 1024")):
        st = det.get(key)
        if st:
            print(f"26-layer decode step ({what}): {st['us']} us, roofline {st['roofline_us']} us ({st['x_roofline']}x)")
    print()
    print(f"{'config':52s} {'layout':8s} {'M':>3s} {'us':>8s} {'GB/s':>8s} {'roof_us':>8s} {'frac':>6s} {'TFLOP/s':>8s}  launch")
    for r in det["configs"]:
        print(f"{r['config']:52s} {r['layout']:8s} {r['M']:3d} {r['us']:8.2f} {r['gbps']:8.1f} {r['roofline_us']:8.2f} "
              f"{r['frac']:6.3f} {r['tflops']:8.2f}  {r['launch']}")
    print()
    print("torch bf16 linear (hipBLASLt), cold weight copies (the reference's library comparator, bench_gemv.py:36-42)")
    print(f"{'shape':32s} {'M':>2s} {'us':>8s} {'GB/s':>8s} {'roof_us':>8s} {'frac':>6s}")
    for r in det["library_bf16_linear"]:
        print(f"{r['shape']:32s} {r['M']:2d} {r['us']:8.2f} {r['gbps']:8.1f} {r['roofline_us']:8.2f} {r['frac']:6.3f}")
    return 0


# The SQ counters of one --pmc pass for sq_summary (at most 8 SQ_ counters in
# a pass on this part).
SQ_COUNTERS = ("SQ_WAVES", "SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_WAVE_CYCLES",
               "SQ_WAIT_INST_ANY", "SQ_BUSY_CYCLES")


def sq_summary(pmc_dir: str) -> int:
    """Per launch of each PROFILE_CASES GEMV (median of its PROFILE_REPS
    launches, the warm-up dropped), from a rocprofv3 --pmc run of
    --profile-gemvs with SQ_COUNTERS: wave instructions per 1 KiB weight tile
    by kind (VALU, MFMA, SALU, LDS), the waves, and the share of the waves'
    cycles spent waiting for an instruction's operands or memory
    (SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES)."""
    import csv
    import glob
    import statistics

    paths = glob.glob(os.path.join(pmc_dir, "**", "*counter_collection.csv"), recursive=True)
    if not paths:
        raise SystemExit(f"no counter_collection.csv under {pmc_dir}")
    per = {}
    for row in csv.DictReader(open(paths[0])):
        if "gemv_" not in row["Kernel_Name"]:
            continue
        d = per.setdefault(int(row["Dispatch_Id"]), {"kernel": row["Kernel_Name"]})
        d[row["Counter_Name"]] = d.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
    seq = [per[k] for k in sorted(per)]
    n = 1 + PROFILE_REPS
    if len(seq) != n * len(PROFILE_CASES):
        raise SystemExit(f"{len(seq)} GEMV dispatches, expected {n * len(PROFILE_CASES)}")
    print(f"wave instructions per 1 KiB weight tile and wait share, median of {PROFILE_REPS} launches per case")
    print(f"{'case':56s} {'tiles':>7s} {'VALU/t':>7s} {'MFMA/t':>7s} {'SALU/t':>7s} {'LDS/t':>6s} {'waves':>6s} "
          f"{'wait':>6s}  kernel")
    for i, (name, fmt, layout, N, K, M, epi, norm) in enumerate(PROFILE_CASES):
        c = seq[i * n + 1:(i + 1) * n]
        med = {k: statistics.median(x.get(k, 0.0) for x in c) for k in SQ_COUNTERS}
        tiles = N * K // (2048 if fmt == "int4" else 1024)  # 1 KiB of weight bytes per tile
        wait = med["SQ_WAIT_INST_ANY"] / med["SQ_WAVE_CYCLES"] if med["SQ_WAVE_CYCLES"] else 0.0
        kern = re.search(r"gemv_\w+<[^>]*>", c[0]["kernel"])
        print(f"{name:56s} {tiles:7d} {med['SQ_INSTS_VALU'] / tiles:7.1f} {med['SQ_INSTS_MFMA'] / tiles:7.1f} "
              f"{med['SQ_INSTS_SALU'] / tiles:7.1f} {med['SQ_INSTS_LDS'] / tiles:6.1f} {med['SQ_WAVES']:6.0f} "
              f"{100 * wait:5.1f}%  {kern.group(0) if kern else ''}")
    return 0


FLOOR_MIB = (13, 26, 52)
# (label, bytes, bytes per workgroup): the tiled decode weights read with
# their own kernel's decomposition (one workgroup per 16-row block) and with
# more, smaller chunks per workgroup
FLOOR_CHUNKS = [
    ("int4 down K10240 N2560, 160 blocks", 13926400, 87040),
    ("int4 down bytes, 320 workgroups", 13926400, 43520),
    ("int4 down bytes, 850 workgroups", 13926400, 16384),
    ("int4 gate|up K2560 N20480, 1280 blocks", 27852800, 21760),
    ("fp8 down K10240 N2560, 160 blocks", 26234880, 163968),
    ("fp8 down bytes, 640 workgroups", 26234880, 40992),
]
# Whole-K floors of the several-row GEMVs (bz_shared_read): every workgroup
# reads all of x (bf16, M rows) beside its own weight bytes.
FLOOR_SHARED = [
    ("int4 K10240 N2560 M=32, one 16-row block per workgroup", 32 * 10240 * 2, 87040, 160),
    ("int4 K10240 N2560 M=16, one 16-row block per workgroup", 16 * 10240 * 2, 87040, 160),
    ("int4 K2560 N20480 M=32, five 16-row blocks per workgroup", 32 * 2560 * 2, 5 * 21760, 256),
]


def floors(torch, G, dev, log) -> dict:
    """What any launch costs and what streaming can reach on this GPU, as
    HIP-graph replays:
      empty_node_us  one empty workgroup (bz_stream_read with no bytes),
                     launched back to back in a graph;
      read           bz_stream_read (non-temporal 16-byte loads, nothing
                     written, 16 KiB per workgroup) over 13, 26 and 52 MiB --
                     the sizes of the int4 down, int4 gate|up and fp8 gate|up
                     weights -- rotating through >= 1 GiB, with the line
                     t = fixed + bytes / rate fitted through the three points;
      chunks         the same read with the decode GEMVs' own decomposition
                     (one workgroup per 16-row block of a tiled weight) and
                     with more workgroups, at their byte counts;
      shared_x       bz_shared_read: each workgroup reads all of x and its
                     own weight bytes, the floor of a several-row GEMV that
                     gives every workgroup the whole K (weights rotating
                     through >= 1 GiB, x the same for every call);
      copy_1gib      torch's device-to-device copy of 1 GiB (read + write)."""
    from breeze_amd.fused.kernels import graph_time_us

    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    empty = graph_time_us(lambda: G.stream_read(None, sink), iters=256)

    def timed_read(size, chunk, x=None, workgroups=0):
        ncopy = max(2, -(-(1 << 30) // size))
        pool = torch.randint(0, 1 << 30, (ncopy * size // 4,), dtype=torch.int32, device=dev)
        bufs = [pool[i * size // 4:(i + 1) * size // 4] for i in range(ncopy)]
        st = {"i": 0}

        def fn():
            if x is None:
                G.stream_read(bufs[st["i"] % ncopy], sink, chunk=chunk)
            else:
                G.shared_read(x, bufs[st["i"] % ncopy], chunk, workgroups, sink)
            st["i"] += 1

        us = graph_time_us(fn, iters=min(2 * ncopy, 256))
        del pool, bufs
        return us

    reads = []
    for mib in FLOOR_MIB:
        size = mib << 20
        us = timed_read(size, 16384)
        reads.append({"mib": mib, "bytes": size, "us": round(us, 3), "gbps": round(size / us / 1e3, 1)})
        log(f"read floor {mib} MiB: {us:.2f} us ({size / us / 1e3:.0f} GB/s)")
    chunks = []
    for label, size, chunk in FLOOR_CHUNKS:
        us = timed_read(size, chunk)
        chunks.append({"what": label, "bytes": size, "chunk": chunk, "workgroups": size // chunk, "us": round(us, 3),
                       "gbps": round(size / us / 1e3, 1)})
        log(f"read {label} ({size // chunk} x {chunk} B): {us:.2f} us ({size / us / 1e3:.0f} GB/s)")
    shared = []
    for label, xbytes, wchunk, wgs in FLOOR_SHARED:
        x = torch.randint(0, 1 << 30, (xbytes // 4,), dtype=torch.int32, device=dev)
        us = timed_read(wchunk * wgs, wchunk, x=x, workgroups=wgs)
        per_wg = xbytes + wchunk
        shared.append({"what": label, "x_bytes": xbytes, "w_bytes_per_workgroup": wchunk, "workgroups": wgs,
                       "us": round(us, 3), "gbps_per_workgroup": round(per_wg / us / 1e3, 1)})
        log(f"shared-x read {label} ({wgs} x ({xbytes} + {wchunk}) B): {us:.2f} us")
        del x
    xs = [r["bytes"] for r in reads]
    ys = [r["us"] for r in reads]
    xm, ym = sum(xs) / len(xs), sum(ys) / len(ys)
    slope = sum((a - xm) * (b - ym) for a, b in zip(xs, ys)) / sum((a - xm) ** 2 for a in xs)
    fixed = ym - slope * xm
    a = torch.empty(1 << 28, dtype=torch.int32, device=dev)
    b = torch.empty_like(a)
    a.fill_(1)
    b.copy_(a)
    torch.cuda.synchronize()
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_ev.record()
    for _ in range(5):
        b.copy_(a)
    e_ev.record()
    torch.cuda.synchronize()
    copy_us = s_ev.elapsed_time(e_ev) * 1e3 / 5
    del a, b
    torch.cuda.empty_cache()
    log(f"empty node {empty:.2f} us; read line {fixed:.2f} us + bytes at {1 / slope / 1e3:.0f} GB/s; "
        f"1 GiB copy {copy_us:.0f} us ({2 * (1 << 30) / copy_us / 1e3:.0f} GB/s read+write)")
    return {"empty_node_us": round(empty, 3), "read": reads,
            "read_fit": {"fixed_us": round(fixed, 3), "gbps": round(1 / slope / 1e3, 1)}, "chunks": chunks,
            "shared_x": shared,
            "copy_1gib": {"us": round(copy_us, 1), "gbps_read_plus_write": round(2 * (1 << 30) / copy_us / 1e3, 1)}}


# The library comparator of the reference (bench_gemv.py:36-42): cuBLAS bf16
# F.linear on cold weight copies; here torch's bf16 linear (hipBLASLt).
LIBRARY_SHAPES = [
    ("gate|up K2560 N20480", 20480, 2560),
    ("down K10240 N2560", 2560, 10240),
    ("qkv K2560 N4096", 4096, 2560),
    ("o_proj K4096 N2560", 2560, 4096),
]


def library_table(torch, dev, log) -> list:
    """bf16 torch.nn.functional.linear (hipBLASLt) at the C2/C3 GEMV shapes,
    M = 1 and 2, weights N(0, 0.02) in bf16 rotating through >= 1 GiB, timed
    as graph replays.  Roofline bytes: bf16 weights + x + output."""
    from breeze_amd.fused.kernels import graph_time_us

    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    rows = []
    for name, N, K in LIBRARY_SHAPES:
        w = (torch.randn(N, K, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        ncopy = max(2, -(-(1 << 30) // (2 * N * K)))
        ws = [w.clone() for _ in range(ncopy)]
        for M in (1, 2):
            x = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
            st = {"i": 0}

            def fn():
                torch.nn.functional.linear(x, ws[st["i"] % ncopy])
                st["i"] += 1

            us = graph_time_us(fn, iters=min(2 * ncopy, 128))
            nbytes = 2 * N * K + 2 * M * K + 2 * M * N
            roof = nbytes / HBM_PEAK_GBPS / 1e3
            rows.append({"shape": name, "M": M, "us": round(us, 2), "gbps": round(nbytes / us / 1e3, 1),
                         "roofline_us": round(roof, 2), "frac": round(roof / us, 3)})
            log(f"bf16 F.linear {name} M={M}: {us:6.2f} us ({nbytes / us / 1e3:5.0f} GB/s)")
        del ws, w
        torch.cuda.empty_cache()
    return rows


# (name, weight format, N, K, epilogue, RMSNorm prologue, M values): the
# GEMV shapes of the benchmark configurations C1-C4
CONFIG_SHAPES = [
    ("C1 rms->int4 K2048 N2048", "int4", 2048, 2048, 0, True, (1, 2)),
    # one GPU's share of an 8-way tensor-parallel layer (column-parallel
    # gate|up [gate_i; up_i], row-parallel down): the same kernels at the shard shape
    ("E 1/8 shard rms->int4 gate|up K2560 N2x1280 silu", "int4", 2560, 2560, 1, True, (1, 2)),
    ("E 1/8 shard int4 down K1280 N2560", "int4", 2560, 1280, 0, False, (1, 2)),
    ("C2 rms->int4 gate|up K2560 N2x10240 silu", "int4", 20480, 2560, 1, True, (1, 2)),
    ("C2 int4 down K10240 N2560", "int4", 2560, 10240, 0, False, (1, 2)),
    ("C3 rms->fp8 qkv K2560 N4096", "fp8", 4096, 2560, 0, True, (1, 2)),
    ("C3 fp8 o_proj K4096 N2560", "fp8", 2560, 4096, 0, False, (1, 2)),
    ("C3 rms->fp8 gate|up K2560 N2x10240 silu", "fp8", 20480, 2560, 1, True, (1, 2)),
    ("C3 fp8 down K10240 N2560", "fp8", 2560, 10240, 0, False, (1, 2)),
    ("C4 int4 K2560 N20480", "int4", 20480, 2560, 0, False, (4, 8, 16, 32)),
    ("C4 int4 K10240 N2560", "int4", 2560, 10240, 0, False, (4, 8, 16, 32)),
    ("C4 fp8 K2560 N20480", "fp8", 20480, 2560, 0, False, (4, 8, 16, 32)),
    ("C4 fp8 K10240 N2560", "fp8", 2560, 10240, 0, False, (4, 8, 16, 32)),
]


def _weights(torch, G, fmt, N, K, epi, w, layout):
    """(buffers, format, bits, gemv kwargs) of a synthetic weight in the
    tiled decode layout (paired for SiLU-gate) or the row-major one."""
    if fmt == "int4":
        p, sz, _ = G.quantize_int4_device(w, GROUP, True, G.W_INT4_ZP)
        if layout == "tiled":
            wfmt = G.W_INT4_TILED_PAIRED if epi == 1 else G.W_INT4_TILED
            return (G.pack_tiled(G.W_INT4_ZP, p, K, wfmt, sc0=sz),), wfmt, 4
        return (p, sz), G.W_INT4_ZP, 4
    c, sc = G.quantize_fp8_device(w, 1e-12)
    if layout == "tiled":
        wfmt = G.W_FP8_TILED_PAIRED if epi == 1 else G.W_FP8_TILED
        return (G.pack_tiled(G.W_FP8, c.view(torch.uint8), K, wfmt, sc0=sc),), wfmt, 8
    return (c.view(torch.uint8), sc), G.W_FP8, 8


def config_table(torch, G, dev, log) -> list:
    """Each GEMV of C1-C4 (synthetic weights N(0, 0.02), int4 symmetric g128
    or fp8 e4m3 per-row, bf16 x N(0, 1)) in both layouts -- "tiled" (the
    decode layout the modules hold: the streaming kernel, and for several
    rows the panel or tile kernel) and "rowmajor" (the other kernels:
    row-sliced paths, and the several-row tile kernel from M = 5) -- timed
    as HIP-graph replays over weight copies
    rotating through >= 1 GiB: µs per call, algorithmic GB/s and the fraction
    of the 8 TB/s bytes-moved roofline."""
    from breeze_amd import tuning
    from breeze_amd.fused.kernels import graph_time_us

    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    rows = []
    for name, fmt, N, K, epi, norm, Ms in CONFIG_SHAPES:
        w = torch.randn(N, K, device=dev, generator=gen) * 0.02
        gamma = (1 + 0.1 * torch.randn(K, device=dev, generator=gen)).to(torch.bfloat16) if norm else None
        xs = {M: torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16) for M in Ms}
        n_out = N // 2 if epi == 1 else N
        for layout in ("tiled", "rowmajor"):
            base, wfmt, bits = _weights(torch, G, fmt, N, K, epi, w, layout)
            wbytes = sum(t.numel() * t.element_size() for t in base)
            ncopy = max(2, -(-(1 << 30) // wbytes))
            copies = [tuple(t.clone() for t in base) for _ in range(ncopy)]
            del base
            for M in Ms:
                x = xs[M]
                out = torch.empty(M, n_out, device=dev, dtype=torch.bfloat16)
                st = {"i": 0}

                def call():
                    c = copies[st["i"] % ncopy]
                    st["i"] += 1
                    sc = c[1] if len(c) > 1 else None
                    G.gemv(x, c[0], wfmt, N, sc0=sc, group=GROUP, gamma=gamma, eps=EPS, epilogue=epi, out=out)

                if M == Ms[0]:  # the first timing of a freshly copied weight set reads high: one untimed pass
                    graph_time_us(call, iters=2 * ncopy)  # of the timed graph's own length
                us = graph_time_us(call, iters=2 * ncopy)
                nbytes = algo_bytes(bits, N, K, M, norm, epi)
                roof = nbytes / HBM_PEAK_GBPS / 1e3
                tflops = 2.0 * M * N * K / us / 1e6
                launch = tuning.lookup(dev, N, K, wfmt, epi, norm, M)
                rows.append({"config": name, "layout": layout, "M": M, "us": round(us, 2),
                             "gbps": round(nbytes / us / 1e3, 1), "roofline_us": round(roof, 2),
                             "frac": round(roof / us, 3), "tflops": round(tflops, 2),
                             "mfma_peak_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 5),
                             "launch": list(launch) if launch else "rule"})
                log(f"{name:42s} {layout:8s} M={M:2d}: {us:7.2f} us  {nbytes / us / 1e3:6.0f} GB/s  "
                    f"({roof / us * 100:4.1f}% of roofline)")
            del copies
            torch.cuda.empty_cache()
        del w
    return rows


# (module class, name, N, K): the reference-named Linear modules at the
# decode shapes, called as a model calls them (forward on [M, K] bf16).
MODULE_SHAPES = [
    ("Int4Linear", "down K10240 N2560", 2560, 10240),
    ("Fp8Linear", "down K10240 N2560", 2560, 10240),
    ("Fp8Linear", "gate K2560 N10240", 10240, 2560),
]


def module_table(torch, dev, log) -> list:
    """Int4Linear / Fp8Linear forward (models/int4_linear.py:99-109,
    models/fp8_linear.py:68-84) at M = 1 and 2 on N(0, 0.02) weights (int4
    with the reference's asymmetric quantizer, group 128), timed as HIP-graph
    replays over module copies whose buffers span >= 1 GiB.  Roofline bytes:
    the buffers the forward reads (the tiled weight with its scales) + x +
    output."""
    import copy

    from breeze_amd.fp8_linear import Fp8Linear
    from breeze_amd.fused.kernels import graph_time_us
    from breeze_amd.int4_linear import Int4Linear

    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    rows = []
    for cls_name, name, N, K in MODULE_SHAPES:
        lin = torch.nn.Linear(K, N, bias=False, device=dev)
        with torch.no_grad():
            lin.weight.copy_(torch.randn(N, K, device=dev, generator=gen) * 0.02)
        mod = Int4Linear(lin) if cls_name == "Int4Linear" else Fp8Linear(lin)
        del lin
        buf = mod.weight_int4 if cls_name == "Int4Linear" else mod.weight_fp8
        wbytes = buf.numel() * buf.element_size()
        mods = [copy.deepcopy(mod) for _ in range(max(2, -(-(1 << 30) // wbytes)))]
        for M in (1, 2):
            x = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
            st = {"i": 0}

            def call():
                mods[st["i"] % len(mods)](x)
                st["i"] += 1

            if M == 1:
                graph_time_us(call, iters=2 * len(mods))
            us = graph_time_us(call, iters=2 * len(mods))
            nbytes = wbytes + 2 * M * K + 2 * M * N
            roof = nbytes / HBM_PEAK_GBPS / 1e3
            rows.append({"module": f"{cls_name} {name}", "M": M, "us": round(us, 2),
                         "gbps": round(nbytes / us / 1e3, 1), "roofline_us": round(roof, 2),
                         "frac": round(roof / us, 3)})
            log(f"{cls_name} {name} M={M}: {us:6.2f} us ({nbytes / us / 1e3:5.0f} GB/s, "
                f"{roof / us * 100:4.1f}% of roofline)")
        del mods, mod
        torch.cuda.empty_cache()
    return rows


def attention_table(torch, dev, log) -> list:
    """The fused decode-attention step alone (q/k RMSNorm + RoPE + cache
    write + attention over cache positions [0, pos] + split combine) of the
    C5 geometry: 16 query heads and 4 KV heads of 256, bf16 caches of 1024 /
    2048 positions, M = 1 and 2, the library's default split.  Timed as HIP-
    graph replays over caches rotating through >= 1 GiB, so the keys and
    values stream from HBM.  Roofline bytes: keys and values over [0, pos]
    read once, the token's qkv row, norm weights, cos/sin, the new key and
    value written, the mask row and the output."""
    from breeze_amd import attention as AT
    from breeze_amd.fused.kernels import graph_time_us

    HQ, HKV, D = 16, 4, 256
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    rows = []
    for S in (1024, 2048):
        for M in (1, 2):
            per = 2 * 2 * M * HKV * S * D  # one cache pair
            ncopy = max(2, -(-(1 << 30) // per))
            caches = [(torch.randn(M, HKV, S, D, device=dev, generator=gen).to(torch.bfloat16),
                       torch.randn(M, HKV, S, D, device=dev, generator=gen).to(torch.bfloat16)) for _ in range(ncopy)]
            qkv = torch.randn(M, (HQ + 2 * HKV) * D, device=dev, generator=gen).to(torch.bfloat16)
            th = torch.rand(M, D // 2, device=dev, generator=gen) * 6
            cos = torch.cat([th.cos(), th.cos()], -1).to(torch.bfloat16)
            sin = torch.cat([th.sin(), th.sin()], -1).to(torch.bfloat16)
            qn = (1 + 0.1 * torch.randn(D, device=dev, generator=gen)).to(torch.bfloat16)
            kn = (1 + 0.1 * torch.randn(D, device=dev, generator=gen)).to(torch.bfloat16)
            mask = torch.zeros(M, 1, 1, S, device=dev, dtype=torch.bfloat16)
            out = torch.empty(M, HQ * D, device=dev, dtype=torch.bfloat16)
            split = AT.default_split(S)
            for p in (127, S - 1):
                pos = torch.tensor([p], device=dev)
                st = {"i": 0}

                def fn():
                    k, v = caches[st["i"] % ncopy]
                    st["i"] += 1
                    AT.attention_step(qkv, cos, sin, pos, k, v, mask, qn, kn, EPS, out, split=split)

                if p == 127:  # the first timing of a freshly made cache set reads high: one untimed pass
                    graph_time_us(fn, iters=min(2 * ncopy, 64))
                us = graph_time_us(fn, iters=min(2 * ncopy, 128))
                nbytes = (2 * 2 * M * HKV * (p + 1) * D + 2 * M * (HQ + 2 * HKV) * D + 2 * 2 * D + 2 * 2 * M * D
                          + 2 * 2 * M * HKV * D + 2 * M * S + 2 * M * HQ * D)
                roof = nbytes / HBM_PEAK_GBPS / 1e3
                rows.append({"cache": S, "M": M, "pos": p, "split": split, "us": round(us, 2),
                             "gbps": round(nbytes / us / 1e3, 1), "roofline_us": round(roof, 3),
                             "frac": round(roof / us, 3)})
                log(f"attention step S={S} M={M} pos={p:4d} split={split}: {us:6.2f} us "
                    f"({nbytes / us / 1e3:5.0f} GB/s, {roof / us * 100:4.1f}% of roofline)")
            del caches
            torch.cuda.empty_cache()
    return rows


def heads_table(torch, dev, log) -> list:
    """The fp32 heads the reference keeps unquantized: the backbone lm_head
    2052 x 2048 at M = 1, 2 (CFG) and one depth codebook head 2051 x 1024
    (picked from 15 by a device index), each as fp32 weights rotating through
    >= 1 GiB.  Roofline bytes: the fp32 weight matrix + x + output."""
    from breeze_amd.fused.kernels import graph_time_us
    from breeze_amd.heads import head_f32

    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    rows = []
    for name, N, K, C, Ms in (("backbone lm_head", 2052, 2048, 1, (1, 2)), ("depth codebook head", 2051, 1024, 15, (1,))):
        w = (torch.randn(C, N, K, device=dev, generator=gen) * 0.02) if C > 1 else \
            (torch.randn(N, K, device=dev, generator=gen) * 0.02)
        per = w.numel() * 4
        ncopy = max(2, -(-(1 << 30) // per))
        ws = [w.clone() for _ in range(ncopy)]
        index = torch.tensor([7], device=dev, dtype=torch.int64)
        for M in Ms:
            x = torch.randn(M, K, device=dev, generator=gen)
            out = torch.empty(M, N, device=dev)
            st = {"i": 0}

            def fn():
                wi = ws[st["i"] % ncopy]
                st["i"] += 1
                head_f32(x, wi, index=index if C > 1 else None, out=out)

            us = graph_time_us(fn, iters=min(2 * ncopy, 128))
            nbytes = 4 * N * K + 4 * M * K + 4 * M * N
            roof = nbytes / HBM_PEAK_GBPS / 1e3
            rows.append({"head": f"{name} {N}x{K} fp32" + (f" (1 of {C}, device index)" if C > 1 else ""),
                         "M": M, "us": round(us, 2), "gbps": round(nbytes / us / 1e3, 1),
                         "roofline_us": round(roof, 3), "frac": round(roof / us, 3)})
            log(f"fp32 head {name} {N}x{K} M={M}: {us:6.2f} us ({nbytes / us / 1e3:5.0f} GB/s, "
                f"{roof / us * 100:4.1f}% of roofline)")
        del ws, w
        torch.cuda.empty_cache()
    return rows


# Timed replays of the decode-step graph (the last STEP_REPS x STEP_KERNELS
# GEMV dispatches of a --profile-step run); 26 layers x 4 GEMVs + the head.
STEP_REPS = 20
STEP_KERNELS = 26 * 4 + 1


def step_summary(trace_dir: str) -> int:
    """Where a decode step's time goes, from a rocprofv3 --kernel-trace run
    of --profile-step: the last STEP_REPS replays of the graph (STEP_KERNELS
    GEMV launches each), per kernel the calls per step, the average and the
    sum of their durations, then the gaps between the end of one launch and
    the start of the next and the step's span from the first start to the
    last end (medians over the replays)."""
    import csv
    import glob
    import statistics

    paths = glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not paths:
        raise SystemExit(f"no kernel_trace.csv under {trace_dir}")
    rows = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"])
                  for r in csv.DictReader(open(paths[0])) if "gemv_" in r["Kernel_Name"])
    need = STEP_REPS * STEP_KERNELS
    if len(rows) < need:
        raise SystemExit(f"{len(rows)} GEMV dispatches, fewer than {need}")
    steps = [rows[len(rows) - need + i * STEP_KERNELS:len(rows) - need + (i + 1) * STEP_KERNELS]
             for i in range(STEP_REPS)]

    def short(name):
        m = re.search(r"(gemv_\w+<[^>]*>)", name)
        return m.group(1) if m else name[:60]

    per = {}
    for st in steps:
        seen = {}
        for t0, t1, name in st:
            seen.setdefault(short(name), []).append((t1 - t0) / 1e3)
        for k, v in seen.items():
            per.setdefault(k, []).append(v)
    spans = [(st[-1][1] - st[0][0]) / 1e3 for st in steps]
    busy = [sum(t1 - t0 for t0, t1, _ in st) / 1e3 for st in steps]
    gaps = [[(st[i + 1][0] - st[i][1]) / 1e3 for i in range(len(st) - 1)] for st in steps]
    print(f"decode step: {STEP_KERNELS} GEMV launches per step, median over {STEP_REPS} graph replays")
    print(f"{'kernel':40s} {'calls':>5s} {'avg us':>8s} {'sum us':>8s}")
    for k, v in sorted(per.items(), key=lambda kv: -statistics.median(sum(x) for x in kv[1])):
        calls = len(v[0])
        print(f"{k:40s} {calls:5d} {statistics.median(statistics.mean(x) for x in v):8.2f} "
              f"{statistics.median(sum(x) for x in v):8.1f}")
    flat = sorted(g for gs in gaps for g in gs)
    print(f"kernel time per step {statistics.median(busy):.1f} us; gaps between launches: median "
          f"{statistics.median(flat):.2f} us, 90th percentile {flat[int(0.9 * len(flat))]:.2f} us, "
          f"sum per step {statistics.median(sum(g) for g in gaps):.1f} us; span first start to last end "
          f"{statistics.median(spans):.1f} us")
    return 0


def decode_step(torch, G, dev, log, M: int = 1, attn_pos: int | None = None, cache_len: int = 1024,
                layout: str = "tiled", reps: int = 20) -> dict:
    """26 decoder layers (hidden 2560, 16x256 q heads, 4 KV heads, MLP 10240)
    of int4 group-128 weights: RMSNorm->QKV, attention replaced by a copy of
    the [M, 4096] query part, o_proj + residual, RMSNorm->gate|up SiLU-gate,
    down + residual; then a final RMSNorm -> bf16 head K2560 N8192.  One HIP
    graph per step.

    layout "tiled" (the decode layout): the QKV GEMV stores its first 4096
    columns a second time into the attention-output buffer (the copy, done
    by the same launch), and the first layer reads the step's input directly,
    so the graph holds GEMV launches only.  layout "rowmajor": the row-major
    kernels, the copy as a device copy node.

    With ``attn_pos`` the copy is replaced by the real decode attention step
    (q/k RMSNorm + RoPE + cache write, attention over cache positions
    [0, attn_pos] of a bf16 cache of ``cache_len`` positions per layer); its
    algorithmic bytes (keys and values read once) join the roofline.

    Returns µs per step against the bytes-moved roofline, and a checksum of
    the logits (float64 sum) for comparison across layouts and runs."""
    H, QKV, ATT, MLP, LAYERS, VOCAB = 2560, 6144, 4096, 10240, 26, 8192
    HQ, HKV, D = 16, 4, 256
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    tiled = layout == "tiled"

    def q4(n, k, paired=False):
        w = torch.randn(n, k, device=dev, generator=gen) * 0.02
        p, sz, _ = G.quantize_int4_device(w, GROUP, True, G.W_INT4_ZP)
        if not tiled:
            return {"w": p, "sc0": sz, "wfmt": G.W_INT4_ZP, "group": GROUP}
        wfmt = G.W_INT4_TILED_PAIRED if paired else G.W_INT4_TILED
        return {"w": G.pack_tiled(G.W_INT4_ZP, p, k, wfmt, sc0=sz), "wfmt": wfmt}

    def gam(k):
        return (1 + 0.1 * torch.randn(k, device=dev, generator=gen)).to(torch.bfloat16)

    layers = [dict(qkv=q4(QKV, H), o=q4(H, ATT), gu=q4(2 * MLP, H, paired=True), dn=q4(H, MLP), g1=gam(H),
                   g2=gam(H)) for _ in range(LAYERS)]
    head = (torch.randn(VOCAB, H, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
    gf = gam(H)
    h0 = torch.randn(M, H, device=dev, generator=gen).to(torch.bfloat16)
    hs = torch.empty_like(h0)
    qkv = torch.empty(M, QKV, device=dev, dtype=torch.bfloat16)
    att = torch.empty(M, ATT, device=dev, dtype=torch.bfloat16)
    mid = torch.empty(M, MLP, device=dev, dtype=torch.bfloat16)
    logits = torch.empty(M, VOCAB, device=dev, dtype=torch.bfloat16)
    if attn_pos is not None:
        from breeze_amd import attention as AT

        for L in layers:
            L["k"] = torch.randn(M, HKV, cache_len, D, device=dev, generator=gen).to(torch.bfloat16)
            L["v"] = torch.randn(M, HKV, cache_len, D, device=dev, generator=gen).to(torch.bfloat16)
            L["qn"], L["kn"] = gam(D), gam(D)
        th = torch.rand(M, D // 2, device=dev, generator=gen) * 6
        cos = torch.cat([th.cos(), th.cos()], -1).to(torch.bfloat16)
        sin = torch.cat([th.sin(), th.sin()], -1).to(torch.bfloat16)
        pos = torch.tensor([attn_pos], device=dev)
        mask = torch.zeros(M, 1, 1, cache_len, device=dev, dtype=torch.bfloat16)
        split = AT.default_split(cache_len)

    def gemv(x, wt, n, **kw):
        G.gemv(x, n=n, **wt, **kw)

    def run():
        if not tiled:
            hs.copy_(h0)
        for i, L in enumerate(layers):
            x_in = h0 if (tiled and i == 0) else hs
            second = {"out2": att} if (tiled and attn_pos is None) else {}
            gemv(x_in, L["qkv"], QKV, gamma=L["g1"], eps=EPS, out=qkv, **second)
            if attn_pos is None:
                if not tiled:
                    att.copy_(qkv[:, :ATT])
            else:
                AT.attention_step(qkv, cos, sin, pos, L["k"], L["v"], mask, L["qn"], L["kn"], EPS, att, split=split)
            gemv(att, L["o"], H, epilogue=G.EPI_RESIDUAL, residual=x_in, out=hs)
            gemv(hs, L["gu"], 2 * MLP, gamma=L["g2"], eps=EPS, epilogue=G.EPI_SILU_GATE, out=mid)
            gemv(mid, L["dn"], H, epilogue=G.EPI_RESIDUAL, residual=hs, out=hs)
        G.gemv(hs, head, G.W_BF16, VOCAB, gamma=gf, eps=EPS, out=logits)

    mid_bytes = 2 * 2 * M * ATT  # the copy: read and write [M, 4096] bf16
    if attn_pos is not None:
        # qkv in, q/k norm weights, cos/sin, the new k/v written, keys and values
        # over [0, pos] read once, the mask row, attention out
        mid_bytes = (2 * M * QKV + 2 * 2 * D + 2 * 2 * M * D + 2 * 2 * M * HKV * D
                     + 2 * 2 * M * HKV * (attn_pos + 1) * D + 2 * M * (attn_pos + 1) + 2 * M * ATT)
    nbytes = LAYERS * (algo_bytes(4, QKV, H, M, True, 0) + mid_bytes + algo_bytes(4, H, ATT, M, False, 2)
                       + algo_bytes(4, 2 * MLP, H, M, True, 1) + algo_bytes(4, H, MLP, M, False, 2)) \
        + algo_bytes(16, VOCAB, H, M, True, 0)
    run()
    torch.cuda.synchronize()
    checksum = float(logits.double().sum().item())
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            run()
    torch.cuda.current_stream().wait_stream(st)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    replay_checksum = float(logits.double().sum().item())
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_ev.record()
    for _ in range(reps):
        g.replay()
    e_ev.record()
    torch.cuda.synchronize()
    us = s_ev.elapsed_time(e_ev) * 1e3 / reps
    roof = nbytes / HBM_PEAK_GBPS / 1e3
    what = "copy for attention" if attn_pos is None else f"attention at position {attn_pos} of {cache_len}"
    log(f"decode step ({layout}, 26 layers + head, M={M}, {what}): {us:.1f} us, roofline {roof:.1f} us "
        f"({us / roof:.2f}x), logits checksum {checksum:.6e}")
    del g, layers, head
    torch.cuda.empty_cache()
    res = {"us": round(us, 2), "algorithmic_bytes": nbytes, "roofline_us": round(roof, 2),
           "x_roofline": round(us / roof, 3), "M": M, "layout": layout, "logits_checksum": checksum,
           "replay_matches_eager": replay_checksum == checksum}
    if attn_pos is not None:
        res.update(attn_pos=attn_pos, cache_len=cache_len)
    return res


def depth_frame(torch, dev, log) -> dict:
    """One depth-decoder frame at the reference's depth shape: 12 decoder
    layers (hidden 1024, MLP 8192, 8 q / 2 kv heads of 128), 16 codebooks of
    2051 tokens, embeddings of width 2048, fp8 layers (the service's
    `--fp8 depth`), CFG batch 2, greedy; random weights.  The whole frame --
    the 2-position start and 14 single-token steps through the fused layers,
    the fp32 codebook heads and the sampling -- is one DepthDecodeGraph
    replay.  Roofline bytes: per position every layer's fp8 weights and row
    scales and the inputs projector (bf16) once, plus each step's fp32
    codebook head matrix."""
    import types

    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3Model

    from breeze_amd.fused.depth_graph import DepthDecodeGraph
    from breeze_amd.fused.install import install_fused_depth

    H, I, L, HQ, HKV, D, C, V, E = 1024, 8192, 12, 8, 2, 128, 16, 2051, 2048
    cfg = Qwen3Config(hidden_size=H, intermediate_size=I, num_attention_heads=HQ, num_key_value_heads=HKV,
                      head_dim=D, num_hidden_layers=L, rms_norm_eps=1e-6, max_position_embeddings=64, vocab_size=V)
    cfg._attn_implementation = "eager"
    cfg.num_codebooks = C
    cfg.backbone_hidden_size = E
    torch.manual_seed(0)
    with torch.device(dev):
        m = Qwen3Model(cfg).to(torch.bfloat16).eval()
        m.embed_tokens = torch.nn.Embedding(C * V, E, dtype=torch.bfloat16)
        m.inputs_embeds_projector = torch.nn.Linear(E, H, bias=False, dtype=torch.bfloat16)
        m.backbone_hidden_state_projector = None
        with torch.no_grad():
            for prm in m.parameters():
                if prm.dim() == 2:
                    prm.normal_(0, 0.02)
        head = types.SimpleNamespace(weight=torch.randn(C - 1, H, V) * 0.02, num_codebooks=C)
    install_fused_depth(types.SimpleNamespace(depth_decoder=types.SimpleNamespace(model=m)), batch_size=2,
                        mlp_bits=8, attn_bits=8)
    g = DepthDecodeGraph(types.SimpleNamespace(model=m, codebooks_head=head), batch_size=2, do_sample=False,
                         guidance_scale=3.0)
    bh = torch.randn(2, E, device=dev).to(torch.bfloat16)
    first = torch.tensor([5, 5], device=dev)
    g.run(bh, first)  # stages the inputs; the eager frame also warms the allocator
    g.capture(num_warmup=2)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    reps = 20
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_ev.record()
    for _ in range(reps):
        g.replay()
    e_ev.record()
    torch.cuda.synchronize()
    us = s_ev.elapsed_time(e_ev) * 1e3 / reps
    qkv = (HQ + 2 * HKV) * D
    layer = (H * qkv + HQ * D * H + 2 * I * H + I * H) + 4 * (qkv + H + 2 * I + H)
    positions = 2 + (C - 2)
    nbytes = positions * (L * layer + 2 * E * H) + (C - 1) * V * H * 4
    roof = nbytes / HBM_PEAK_GBPS / 1e3
    log(f"depth frame (12 fp8 layers, 16 positions, 15 fp32 codebook heads, CFG 2, greedy): {us:.1f} us, "
        f"roofline {roof:.1f} us ({us / roof:.1f}x)")
    res = {"us": round(us, 1), "algorithmic_bytes": nbytes, "roofline_us": round(roof, 2),
           "x_roofline": round(us / roof, 2), "positions": positions, "layers": L, "batch": 2,
           "weights": "fp8 e4m3 per-row (layers), fp32 (codebook heads)"}
    del g, m, head
    torch.cuda.empty_cache()
    return res


if __name__ == "__main__":
    sys.exit(main())
