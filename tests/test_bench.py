"""bench.py's output contract: one JSON line with the headline rate, its roofline and the
CPU baseline; one GPU only; the rocprofv3 counter summary's normalisation."""
import csv
import json
import os
import subprocess
import sys

import pytest

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args, timeout=300, env=None):
    return subprocess.run([sys.executable, "-u", os.path.join(ROOT, "bench.py"), *args], capture_output=True,
                          text=True, timeout=timeout, env=env)


def test_refuses_more_than_one_gpu():
    r = run_bench("--gpus", "2", timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr, (r.returncode, r.stderr)
    r = run_bench(timeout=120, env=dict(os.environ, WORLD_SIZE="2"))
    assert r.returncode == 2 and "one GPU" in r.stderr, (r.returncode, r.stderr)


def test_counter_summary(tmp_path):
    """Averages over the last dispatches of each kernel and the derived utilisations, on
    made-up counter values whose quotients are known."""
    fwd = "_ZN7onionop20attn_fwd_pipe_kernelIDF16bLi64ELb1ELb0ELi2ELi2EEEvPKT_S3_S3_PKhPS1_PfS7_iiiiifNS_6VarLenEi"
    rows = []
    for i, gui in enumerate([8000.0, 16000.0, 16000.0]):  # the first dispatch falls outside last=2
        rows += [(fwd, "GRBM_GUI_ACTIVE", gui), (fwd, "SQ_VALU_MFMA_BUSY_CYCLES", 512000.0 + i),
                 (fwd, "SQ_ACTIVE_INST_VALU", 128000.0), (fwd, "SQ_VALU_MFMA_COEXEC_CYCLES", 204800.0),
                 (fwd, "SQ_LDS_IDX_ACTIVE", 100000.0), (fwd, "SQ_LDS_BANK_CONFLICT", 25000.0),
                 (fwd, "SQ_INSTS_MFMA", 1000.0), (fwd, "SQ_INSTS_VALU", 9950.0),
                 ("at::native::vectorized_elementwise_kernel<4>", "GRBM_GUI_ACTIVE", 5.0)]
    path = tmp_path / "pmc.csv"
    with open(path, "w", newline="") as f:
        wr = csv.writer(f)
        wr.writerow(["Kernel_Name", "Counter_Name", "Counter_Value"])
        wr.writerows(rows)
    out = bench.counter_summary([str(path)], last=2)
    assert list(out) == ["attn_fwd_pipe_kernel<DF16bLi64ELb1ELb0ELi2ELi2>"], out.keys()
    d = next(iter(out.values()))
    simd = 16000.0 / 8 * 1024  # GUI is summed over 8 XCDs; 1024 SIMDs
    assert d["GRBM_GUI_ACTIVE"] == 16000.0
    assert d["mfma_busy"] == round(512001.5 / simd, 4)
    assert d["valu_busy"] == round(4 * 128000.0 / simd, 4)
    assert d["coexec"] == round(204800.0 / simd, 4)
    assert d["lds_active"] == round(100000.0 / (16000.0 / 8 * 256), 4)
    assert d["bank_conflict_share"] == 0.25
    assert d["valu_per_mfma"] == 9.95


def test_measured_traffic():
    with open(os.path.join(ROOT, "profiles", "hbm_traffic.json")) as f:
        rec = json.load(f)["kernels"]
    assert bench.measured_traffic("attn_bwd_dkdv") == int(rec["attn_bwd_dkdv"]["bytes"])
    assert bench.measured_traffic("no_such_kernel") is None


def test_cpu_baseline_record():
    """The CPU leg's record on a tiny case: the oracle's float32 tile algorithm, timed."""
    r = bench.cpu_baseline(E=16, L=64, H=1, B=1, threads=1)
    assert r["kind"] == "port" and r["unit"] == "TFLOP/s" and r["cores"] == 1
    assert r["value"] > 0 and r["nproc"] == os.cpu_count()
    assert "(E,L,H,B)=(16,64,1,1)" in r["sample"]


@pytest.mark.gpu
def test_bench_json_line():
    """A short run of the headline: every field of the contract, and the figures agree with
    one another (value from ms_per_step, roofline fraction from achieved / peak)."""
    r = run_bench("--steps", "3", "--warmup", "1", "--no-cpu", "--no-memory", "--no-workloads")
    assert r.returncode == 0, r.stderr[-2000:]
    line = json.loads(r.stdout.strip().splitlines()[-1])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "settle_ms"):
        assert key in line, key
    assert line["n_gpus"] == 1 and line["steps"] == 3 and line["warmup"] == 1
    assert line["unit"] == "TFLOP/s" and line["higher_is_better"] is True and line["vs_baseline"] is None
    assert line["dtype"] == "bf16" and "workload" in line["config"]
    flops = line["config"]["flops_per_step"]
    assert flops == 14 * 4 * 4 * 4096 * 4096 * 64 / 2
    assert line["value"] == pytest.approx(flops / (line["ms_per_step"] * 1e-3) / 1e12, rel=1e-3)
    rf = line["roofline"]
    assert rf["bound"] == "mfma" and rf["unit"] == "TFLOP/s" and rf["peak"] == 2500.0
    assert rf["frac"] == pytest.approx(rf["achieved"] / rf["peak"], abs=1e-4)
    assert rf["kernel"] in rf["kernel_us"] and rf["avg_us"] == rf["kernel_us"][rf["kernel"]]
    assert rf["kernel_us"][rf["kernel"]] == max(t for n, t in rf["kernel_us"].items() if n != "attn_bwd_pre")
    assert 0 < rf["frac"] < 1 and line["value"] > 0
