"""CPU checks of bench.py's host logic: the algorithmic bytes behind the
roofline figures, the rocprofv3 summary (durations -> GB/s, PMC counters ->
HBM traffic through the copy-probe calibration), and the one-GPU contract."""
import csv
import importlib
import importlib.util
import re
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _by_label(bench, label):
    return next(v for v in bench.KNOWN_LAUNCHES.values() if v[0] == label)


def test_algorithmic_bytes_are_the_surveyed_per_call_figures(bench):
    # (2 M N + N) s for RMSNorm and 3 M I s for SiLU-and-mul at the configs
    # the metric is quoted on (C1, C2, C4)
    assert _by_label(bench, "C1 RMSNorm [2048,1536] fp16")[1] == 12_585_984
    assert _by_label(bench, "C2 SiLU-and-mul [2048,8960] fp16")[1] == 110_100_480
    assert _by_label(bench, "C4 RMSNorm [16384,3584] bf16")[1] == 234_888_192
    assert _by_label(bench, "C4 SiLU-and-mul [16384,18944] bf16")[1] == 1_862_270_976


def test_every_prefill_gemm_launch_carries_its_flops(bench):
    for (frag, grid), v in bench.KNOWN_LAUNCHES.items():
        if frag.startswith("tiled_gemm<"):
            assert len(v) == 3 and v[2] > 0, frag


def test_tiled_gemm_fragments_name_every_template_argument(bench):
    # the trace matches a fragment as a substring of the demangled kernel name,
    # which lists every template argument, defaulted ones included: a fragment
    # short of the kernel's arity matches nothing
    src = (ROOT / "llm-inference-optimizer_amd" / "csrc" / "tiled_gemm.h").read_text()
    decl = re.search(r"template <([^>]*)>\s*__global__[^\n]*\n[^\n]*tiled_gemm\(", src)
    assert decl, "tiled_gemm kernel declaration not found"
    arity = len(decl.group(1).split(","))
    frags = [frag for frag, _ in bench.KNOWN_LAUNCHES if frag.startswith("tiled_gemm<")]
    assert frags
    for frag in frags:
        assert len(frag[len("tiled_gemm<"):-1].split(",")) == arity, frag


def test_stream_kernel_fragments_name_every_template_argument(bench):
    # as above, for the weight-streaming decode kernel
    src = (ROOT / "llm-inference-optimizer_amd" / "csrc" / "w8a16_stream.h").read_text()
    decl = re.search(r"template <([^>]*)>\s*__global__[^\n]*w8a16_stream\(", src)
    assert decl, "w8a16_stream kernel declaration not found"
    arity = len(decl.group(1).split(","))
    frags = [frag for frag, _ in bench.KNOWN_LAUNCHES if frag.startswith("w8a16_stream<")]
    assert frags
    for frag in frags:
        assert len(frag[len("w8a16_stream<"):-1].split(",")) == arity, frag


def _write(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def test_rocprof_summary_turns_traces_and_counters_into_rates(bench, tmp_path):
    c2 = "void mi355::silu_mul_chunks<mi355::F16, mi355::F16, 512, 2>(void const*, void const*, void*, long)"
    copy = "stream_copy(unsigned int const*, unsigned int*, unsigned long)"
    _write(tmp_path / "run_kernel_trace.csv", [
        {"Kernel_Name": c2, "Grid_Size_X": 1146880, "Grid_Size_Y": 1, "Grid_Size_Z": 1,
         "Start_Timestamp": 1000, "End_Timestamp": 1000 + 18_000},
        {"Kernel_Name": c2, "Grid_Size_X": 1146880, "Grid_Size_Y": 1, "Grid_Size_Z": 1,
         "Start_Timestamp": 50_000, "End_Timestamp": 50_000 + 18_400},
        {"Kernel_Name": "unrelated_kernel", "Grid_Size_X": 64, "Grid_Size_Y": 1, "Grid_Size_Z": 1,
         "Start_Timestamp": 0, "End_Timestamp": 5},
    ])
    # the copy probe moves exactly 1 GiB each way; the counters read 2% low,
    # so both scales are 1 / 0.98
    gib_kib = (1 << 30) / 1024
    counters = []
    for name, grid, fetch, write in ((copy, 67108864, 0.98 * gib_kib, 0.98 * gib_kib),
                                     (c2, 1146880, 0.98 * 2 * 2048 * 8960 * 2 / 1024,
                                      0.98 * 2048 * 8960 * 2 / 1024)):
        counters.append({"Kernel_Name": name, "Grid_Size": grid, "Counter_Name": "FETCH_SIZE", "Counter_Value": fetch})
        counters.append({"Kernel_Name": name, "Grid_Size": grid, "Counter_Name": "WRITE_SIZE", "Counter_Value": write})
    _write(tmp_path / "run_counter_collection.csv", counters)

    text, traffic = bench.rocprof_summary([str(tmp_path)])
    row = next(line for line in text.splitlines() if line.startswith("| silu_mul_chunks"))
    cells = [c.strip() for c in row.split("|")[1:-1]]
    assert cells[1] == "1146880" and cells[2] == "2"        # grid, launches
    assert cells[3] == "18.200"                              # mean of 18.0 and 18.4 us
    assert int(cells[6]) == round(110_100_480 / 18.2 / 1e3)  # GB/s
    t = traffic["C2 SiLU-and-mul [2048,8960] fp16"]
    assert t["algorithmic_bytes"] == 110_100_480
    assert abs(t["traffic_bytes"] - 110_100_480) <= 2       # calibrated back to the ideal
    assert "unrelated_kernel" not in text

    # a second call in the same process sees only its own directory
    empty = tmp_path / "empty"
    empty.mkdir()
    text2, traffic2 = bench.rocprof_summary([str(empty)])
    assert traffic2 == {} and "silu_mul_chunks" not in text2


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       cwd=str(ROOT), timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def _kernel(bench, nbytes, us):
    return bench.kernel_entry("k", nbytes, us)


def test_per_config_block_carries_every_config_and_decode_latency(bench):
    # the compact block the driver keeps inside `roofline`: C1 / C2 / C4
    # fractions, same-size probe times, and the C3 decode latencies per M
    k = {"c1_rmsnorm_f16_2048x1536": _kernel(bench, 12_585_984, 4.0),
         "c1_rmsnorm_f16_2048x1536_graph": _kernel(bench, 12_585_984, 3.5),
         "c1_rmsnorm_f16_2048x1536_api": _kernel(bench, 12_585_984, 3.7),
         "empty_kernel_eager_us": 1.5,
         "c2_silu_mul_f16_2048x8960": _kernel(bench, 110_100_480, 18.0)}
    c4 = {"c4_rmsnorm_bf16_16384x3584": _kernel(bench, 234_888_192, 39.5),
          "c4_silu_mul_bf16_16384x18944": _kernel(bench, 1_862_270_976, 286.0)}
    dec = {f"M={m}": {"rmsnorm_api_us": 15.0, "silu_mul_api_us": 15.5, "rmsnorm_call_us": 7.2,
                      "silu_mul_call_us": 7.4, "rmsnorm_device_us": 3.9,
                      "silu_mul_device_us": 4.1, "graph_per_kernel_us": 1.7 + m / 100,
                      "graph_replay_us": 84 * (1.7 + m / 100)} for m in (1, 2, 4, 8, 32)}
    dec["floor"] = {"empty_kernel_graph_node_us": 1.6, "row_copy_graph_node_us": 1.6}
    ceil = {lab: {"us": 1.0} for lab, _, _ in bench.CEILING_SHAPES}
    pc = bench.per_config({"kernels": k, "c4": c4, "decode": dec, "ceilings": ceil,
                           "copy_ceiling": {"frac_of_peak": 0.82}})
    assert pc["C1_rmsnorm_f16_2048x1536"]["frac"] == round(12_585_984 / 4.0 / 1e3 / 8000, 4)
    assert pc["C1_rmsnorm_f16_2048x1536"]["graph_us"] == 3.5
    assert pc["C1_rmsnorm_f16_2048x1536"]["api_us"] == 3.7
    assert pc["C1_rmsnorm_f16_2048x1536"]["empty_kernel_eager_us"] == 1.5
    assert pc["C4_silu_mul_bf16_16384x18944"]["frac"] == round(1_862_270_976 / 286.0 / 1e3 / 8000, 4)
    assert set(pc["C3_decode_f16_latency"]) == {"M1", "M2", "M4", "M8", "M32"}
    assert pc["C3_decode_f16_latency"]["M8"]["graph_node_us"] == 1.78
    assert pc["C3_decode_f16_latency"]["M8"]["rms_call_us"] == 7.2
    assert all("probe_us" in pc[c] for c in ("C1_rmsnorm_f16_2048x1536", "C2_silu_mul_f16_2048x8960",
                                             "C4_rmsnorm_bf16_16384x3584", "C4_silu_mul_bf16_16384x18944"))
    import json
    assert len(json.dumps(pc)) < 2500  # the whole stdout line stays far below the driver's 16 KB tail
