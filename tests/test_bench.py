"""bench.py's driver-facing contract, on the CPU (no GPU work): the refusal of
more than one GPU, the default line's table of BASELINE rows, the counter
records it reads into roofline.traffic, and the kernel-trace summary."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def test_table_rows_are_workloads():
    known = set(bench.WORKLOADS) | set(bench.PREFILL) | set(bench.DECODE) | set(bench.PROJ)
    assert bench.TABLE and all(name in known for name in bench.TABLE)
    assert "int4_g32_gemv_m1" not in bench.TABLE      # the headline itself is the line's value
    assert len(set(bench.TABLE)) == len(bench.TABLE)


def test_fp32_prefill_workloads_mirror_the_bf16_ones():
    # every bf16 prefill workload has an fp32-entry twin of the same product,
    # whose algorithmic bytes count 4-byte x
    assert {k.replace("prefill_f32_", "prefill_") for k in bench.PREFILL_F32} == set(bench.PREFILL)
    for name, (prec, gs, (N, K), M) in bench.PREFILL_F32.items():
        assert bench.PREFILL[name.replace("prefill_f32_", "prefill_")] == (prec, gs, (N, K), M)
        assert bench.prefill_bytes(prec, gs, N, K, M, 4) - bench.prefill_bytes(prec, gs, N, K, M) == 2 * M * K
    assert bench.profiled_traffic("int8", 5632, 2048, 512, "prefill_f32") is None   # no counter record


@pytest.mark.parametrize("prec,N,K,M,kind", [
    ("int4", 32000, 2048, 1, ""),            # the headline's dominant launch
    ("int8", 5632, 2048, 1, ""),             # configs[0]
    ("int4", 32000, 2048, 8, ""),            # configs[1] at M = 8
    ("int8", 5632, 2048, 2048, "prefill"),   # configs[3]
    ("int4", 2048, 5632, 512, "prefill"),
])
def test_traffic_records_parse(prec, N, K, M, kind):
    t = bench.profiled_traffic(prec, N, K, M, kind)
    alg = bench.alg_bytes(prec, 32 if prec == "int4" else 0, N, K, M) if not kind else \
        bench.prefill_bytes(prec, 32 if prec == "int4" else 0, N, K, M)
    assert t is not None and 0.9 * alg < t < 10 * alg


@pytest.mark.parametrize("workload", ["decode_1p1b_int8", "decode_7b_int4", "proj_7b_int4_m1", "proj_7b_int4_m8"])
def test_step_traffic_records_parse(workload):
    t = bench.profiled_step_traffic(workload)
    assert t is not None and t > 1e9


def test_algorithmic_bytes_closed_forms():
    # INT4 g32: K N / 2 weight bytes + 4 K N / 32 scale bytes + x and y
    assert bench.alg_bytes("int4", 32, 32000, 2048, 1) == 41096192
    # INT8 per-channel: K N + 4 N + x and y
    assert bench.alg_bytes("int8", 0, 5632, 2048, 1) == 11587584
    # prefill: bf16 x
    assert bench.prefill_bytes("int8", 0, 5632, 2048, 512) == 5632 * 2048 + 4 * 5632 + 2 * 512 * 2048 + 4 * 512 * 5632


def test_trace_summary(tmp_path, capsys):
    csv = tmp_path / "trace.csv"
    rows = ["Kernel_Name,Start_Timestamp,End_Timestamp"]
    t = 0
    for i in range(10):
        for name, dur in (("gemv_burst<4, 1, 4, 1, 0, 0, 0>", 9000 + 10 * i), ("other", 1000)):
            rows.append(f'"{name}",{t},{t + dur}')
            t += dur + 100
    csv.write_text("\n".join(rows) + "\n")
    bench.trace_summary(str(csv), "gemv_burst<4, 1, 4, 1", 4)
    out = capsys.readouterr().out
    assert "| `gemv_burst<4, 1, 4, 1, 0, 0, 0>` | 10 |" in out
    # the last 4 launches: 9060, 9070, 9080, 9090 ns
    assert "Last 4 of 10 dispatches" in out and "avg 9.075 us" in out
