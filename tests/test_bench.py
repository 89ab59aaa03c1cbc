"""bench.py's output contract: one JSON line with the metric, throughput, roofline and CPU
baseline fields, and a refusal of more than one GPU."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


@pytest.mark.gpu
def test_bench_json_line():
    """A small workload through the whole bench: every field of the line, the roofline and
    CPU-baseline objects, and the row-sample check of the timed kernel's output."""
    print("[case] bench.py --config 1 --size 1024", flush=True)
    r = subprocess.run([sys.executable, "-u", BENCH, "--config", "1", "--size", "1024",
                        "--steps", "5", "--warmup", "2", "--cpu-seconds", "0.5"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [l for l in r.stdout.splitlines() if l.strip()]
    assert len(lines) == 1, r.stdout
    d = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline", "parity_row_sample", "kernel_ms"):
        assert key in d, key
    assert d["n_gpus"] == 1 and d["steps"] == 5 and d["warmup"] == 2
    assert d["unit"] == "GFLOP/s" and d["higher_is_better"] is True and d["value"] > 0
    assert d["dtype"] == "f32" and d["data"] == "synthetic" and d["vs_baseline"] is None
    assert "workload" in d["config"] and "model" not in d["config"]
    roof = d["roofline"]
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    assert roof["traffic"] is None  # measured for the full workload only
    cpu = d["cpu_baseline"]
    assert cpu["kind"] == "port" and cpu["cores"] == 1 and cpu["value"] > 0 and cpu["sample"]
    assert d["parity_row_sample"] is True
    (p,) = d["per_config"]
    assert p["config"] == 1 and p["O"] == 128 and p["precision"] == "fp32"
    lay = p["layout"]
    assert 0 < lay["num_panels"] <= lay["num_units"] <= lay["num_chunks"]
    assert lay["num_heavy"] <= lay["num_units"] and lay["row_grouped"] in (0, 1)
    assert lay["num_row_step_batches"] > 0  # uniform random FP32 panels take row steps
    for mode in ("accumulate", "overwrite"):
        m = p[mode]
        assert m["parity_row_sample"] is True
        assert m["kernel_ms"] > 0 and m["single_launch_median_ms"] > 0
        assert abs(m["roofline"]["achieved"] - p["bytes_alg"] / m["kernel_ms"] / 1e6) < \
            1e-3 * m["roofline"]["achieved"] + 0.1
        assert m["speedup_vs_rocsparse_fp32"] > 0
        rf = m["roofline"]
        # the schedule's floor holds at least C and every distinct B row once
        assert rf["floor_bytes"] >= rf["floor"]["c_bytes"] + rf["floor"]["b_once_bytes"] > 0
        assert rf["frac_ceiling"] == round(p["bytes_alg"] / rf["floor_bytes"], 4)
    assert d["value"] == p["accumulate"]["gflops"]
    # the summary closes both the JSON line and stderr, where a kept tail of either holds it
    keys = list(d)
    assert keys.index("summary") > keys.index("per_config")
    assert [r["mode"] for r in d["summary"]] == ["acc", "ove"]
    assert r.stderr.rstrip().splitlines()[-1].startswith("[summary]")


def test_traffic_stamp_matches_sources():
    """The measured HBM traffic in profiles/ is stamped with the hash of the kernel and layout
    sources it was profiled at; bench.py reports it only while that hash is current."""
    sys.path.insert(0, ROOT)
    import bench
    import json
    d = json.load(open(os.path.join(ROOT, "profiles", "hbm_traffic.json")))
    assert set(d) >= {"sources_sha256_16", "launches"}
    for key, e in d["launches"].items():
        assert e["bytes"] > 0 and e["fetch_kib"] > 0 and e["write_kib"] >= 0, key
    got, stamp = bench.measured_traffic("config2-fp16-accumulate")
    if d["sources_sha256_16"] == bench.traffic_source_hash():
        assert got == d["launches"]["config2-fp16-accumulate"]["bytes"]
    else:
        assert got is None and stamp.startswith("stale")
