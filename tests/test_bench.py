"""bench.py's contract: one JSON line with the headline metric, the roofline and
the CPU baseline; more than one GPU is refused with a message."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def run_bench(*args: str, timeout: int = 240) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=timeout, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    res = run_bench("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert res.returncode == 2
    assert "one GPU" in res.stderr
    assert res.stdout.strip() == ""


@pytest.mark.gpu
def test_default_line_carries_the_contract(device, capsys, monkeypatch):
    # in this process (the test process already holds the GPU: no child process)
    print("[case] bench.py default config, short run", flush=True)
    sys.path.insert(0, str(ROOT))
    import bench

    monkeypatch.setattr(sys, "argv", ["bench.py", "--steps", "5", "--warmup", "2", "--cpu-seconds", "1",
                                      "--no-other-configs"])
    assert bench.main() == 0
    out = capsys.readouterr().out
    lines = [l for l in out.splitlines() if l.startswith("{")]
    assert len(lines) == 1
    line = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
                "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in line, key
    assert line["n_gpus"] == 1 and line["steps"] == 5 and line["warmup"] == 2
    assert line["unit"] == "GB/s" and line["higher_is_better"] is True and line["dtype"] == "bf16"
    assert line["config"]["workload"].startswith("cfg2_qwen3_8b")
    assert "one allocation" in line["config"]["kv_layout"]  # the default: alloc_kv_pools
    roof = line["roofline"]
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    assert 0 < roof["frac"] < 1 and abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    # the step's throughput (both kernels) is below the main kernel's alone; a
    # 5-step run times each within a few percent (event overhead, clocks)
    assert 0 < line["value"] <= 1.05 * roof["achieved"]
    cpu = line["cpu_baseline"]
    assert cpu["kind"] in ("port", "reference") and cpu["cores"] >= 1 and cpu["value"] > 0 and cpu["sample"]


@pytest.mark.gpu
def test_other_configs_are_timed_in_the_same_run(device, monkeypatch):
    # the default run's "other_configs" figures, on two small configs
    print("[case] bench.other_configs on cfg1_small + cfg5_verify", flush=True)
    sys.path.insert(0, str(ROOT))
    import bench
    from simpler_amd import workloads

    keep = {k: workloads.CONFIGS[k] for k in ("cfg1_small", "cfg2_qwen3_8b", "cfg5_verify")}
    monkeypatch.setattr(workloads, "CONFIGS", keep)
    monkeypatch.setattr(sys, "argv", ["bench.py", "--steps", "3", "--warmup", "1"])
    res = bench.other_configs(bench.parse(), device, skip="cfg2_qwen3_8b")
    assert sorted(res) == ["cfg1_small", "cfg5_verify"]
    for r in res.values():
        assert r["main_us"] > 0 and r["step_us"] >= 0.9 * r["main_us"] and 0 < r["frac"] < 1
        assert r["kernel"].startswith("pa_") and r["workers"] >= 1


def test_shape_variants_keep_the_configs_draws():
    # --q-len / --num-heads / --causal change the shape, keep the seed (so the
    # context lengths and block table), and name the variant
    sys.path.insert(0, str(ROOT))
    import argparse

    import bench
    from simpler_amd.workloads import CONFIGS, make_case

    base = CONFIGS["cfg5_verify"]
    ns = argparse.Namespace(q_len=1, num_heads=0, causal=-1)
    v = bench.variant_config(base, ns)
    assert v.name == "cfg5_verify[q_len=1]" and v.q_len == 1 and v.num_heads == base.num_heads and v.causal
    assert v.index == base.index
    a, b = make_case(base), make_case(v)
    assert a.seed == b.seed
    assert a.context_lens.tolist() == b.context_lens.tolist() and a.block_table.equal(b.block_table)
    same = bench.variant_config(base, argparse.Namespace(q_len=0, num_heads=0, causal=-1))
    assert same is base
