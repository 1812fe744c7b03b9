"""bench.py's last stdout line: the compact summary of a full record stays a
few KB (a driver keeps only the tail of stdout) and carries the contract
keys, `roofline` and `cpu_baseline` (CPU; no GPU run)."""

from __future__ import annotations

import importlib.util
import json
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _full_record(b) -> dict:
    """A record with every optional table present and long labels, shaped
    as main() writes it."""
    step = {"us": 565.19, "algorithmic_bytes": 1493403648, "roofline_us": 186.68, "x_roofline": 3.028, "M": 1,
            "layout": "tiled", "logits_checksum": -1.234567890123e3, "replay_matches_eager": True}
    configs = []
    for name, fmt, N, K, epi, norm, Ms in b.CONFIG_SHAPES:
        for layout in ("tiled", "rowmajor"):
            for M in Ms:
                configs.append({"config": name, "layout": layout, "M": M, "us": 123.45, "gbps": 1234.5,
                                "roofline_us": 12.34, "frac": 0.123, "tflops": 12.34, "mfma_peak_frac": 0.01234,
                                "launch": [3, 5, 4, 5, 0]})
    detail = {
        "gate_up_us": 7.374, "down_us": 5.349, "down_gbps": 2608.3, "rowmajor_gate_up_us": 8.676,
        "rowmajor_down_us": 7.339, "step_roofline_us": 5.229, "parity_rel_err": {"gate_up": 1e-3, "down": 2e-3},
        "floors": {"empty_node_us": 1.556, "read": [{"mib": 13, "bytes": 1, "us": 1.0, "gbps": 1.0}] * 3,
                   "read_fit": {"fixed_us": 1.677, "gbps": 7430.3}, "chunks": [{"what": "x" * 60}] * 6,
                   "shared_x": [{"what": "y" * 60}] * 3, "copy_1gib": {"us": 413.0, "gbps_read_plus_write": 5200.0}},
        "decode_step": step, "decode_step_m2": dict(step, M=2), "decode_step_rowmajor": dict(step, layout="rowmajor"),
        "decode_step_attn": dict(step, attn_pos=1023, cache_len=1024),
        "depth_frame": {"us": 4917.6, "algorithmic_bytes": 5543600000, "roofline_us": 692.95, "x_roofline": 7.1,
                        "positions": 16, "layers": 12, "batch": 2, "weights": "fp8"},
        "configs": configs,
        "modules": [{"module": f"{c} {n}", "M": m, "us": 7.41, "gbps": 3554.0, "roofline_us": 3.28, "frac": 0.443}
                    for c, n, _, _ in b.MODULE_SHAPES for m in (1, 2)],
        "library_bf16_linear": [{"shape": "gate|up K2560 N20480", "M": 1, "us": 47.3}] * 8,
        "attention": [{"what": "z" * 80}] * 12, "fp32_heads": [{"head": "h" * 60}] * 6,
    }
    return {
        "metric": "int4/fp8 GEMV achieved HBM TB/s at M=1; µs per decoder-layer decode step", "value": 3.2735,
        "unit": "TB/s", "n_gpus": 1, "steps": 20, "warmup": 5, "ms_per_step": 0.01278, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "w" * 110, "weights": "v" * 110, "M": 1, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": 3781.5, "peak": 8000.0, "unit": "GB/s", "frac": 0.4727,
                     "traffic": 28049916, "kernel": "k" * 70, "algorithmic_bytes": 27883520, "avg_launch_us": 7.374},
        "cpu_baseline": {"value": 0.000353, "unit": "TB/s", "cores": 16, "kind": "port", "sample": "s" * 200,
                         "us_per_step": 118459.2,
                         "predequantized": {"value": 0.004, "unit": "TB/s", "cores": 16, "us_per_step": 10530.9,
                                            "sample": "p" * 150}},
        "detail": detail,
    }


def test_summary_line_is_short_and_complete():
    b = _bench()
    full = _full_record(b)
    assert len(json.dumps(full)) > 8000  # the full record would not survive an 8,000-character tail
    line = json.dumps(b.compact(full))
    assert len(line) <= b.SUMMARY_MAX_CHARS
    got = json.loads(line)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in got, key
    assert got["roofline"]["frac"] == 0.4727 and got["roofline"]["traffic"] == 28049916
    assert got["cpu_baseline"]["cores"] == 16 and got["cpu_baseline"]["kind"] == "port"
    steps = got["summary"]["decode_steps"]
    assert steps["c5_m1"]["us"] == 565.19 and steps["c5_m2"]["x_roofline"] == 3.028
    # the C1-C3 tiled decode GEMVs at M = 1 and 2: 14 rows
    assert len(got["summary"]["gemv_us_frac"]) == 14
    assert len(got["summary"]["module_us_frac"]) == 2 * len(b.MODULE_SHAPES)


def test_summary_without_optional_parts():
    b = _bench()
    full = _full_record(b)
    full["cpu_baseline"] = None
    full["detail"] = {"gate_up_us": 7.0, "down_us": 5.0}
    got = json.loads(json.dumps(b.compact(full)))
    assert got["cpu_baseline"] is None
    assert got["summary"] == {"gate_up_us": 7.0, "down_us": 5.0}


def test_step_summary_reads_a_kernel_trace(tmp_path, capsys):
    """--step-summary over a synthetic kernel trace: the last STEP_REPS x
    STEP_KERNELS GEMV dispatches are the timed replays; per-kernel calls and
    sums, gaps and span come out of their timestamps."""
    b = _bench()
    lines = ["Kernel_Name,Start_Timestamp,End_Timestamp"]
    t = 0
    lines.append(f'"void bz::quantize_int4_kernel(int)",{t},{t + 500}')   # not a GEMV: ignored
    t += 1000
    for rep in range(b.STEP_REPS + 2):       # two untimed replays first
        for i in range(b.STEP_KERNELS):
            name = "void bz::gemv_stream<5, 1, 4>(bz::StreamParams)" if i % 4 == 2 else \
                "void bz::gemv_stream<4, 1, 5>(bz::StreamParams)"
            lines.append(f'"{name}",{t},{t + 4000}')
            t += 4000 + 1500                 # 4 us kernels, 1.5 us gaps
    d = tmp_path / "trace" / "host"
    d.mkdir(parents=True)
    (d / "run_kernel_trace.csv").write_text("\n".join(lines) + "\n")
    assert b.step_summary(str(tmp_path / "trace")) == 0
    out = capsys.readouterr().out
    assert "gemv_stream<5, 1, 4>" in out and "gemv_stream<4, 1, 5>" in out
    assert "gaps between launches: median 1.50 us" in out
    span = b.STEP_KERNELS * 4.0 + (b.STEP_KERNELS - 1) * 1.5
    assert f"span first start to last end {span:.1f} us" in out
