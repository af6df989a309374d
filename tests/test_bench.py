"""CPU checks of bench.py's driver contract: the JSON line assembled from the workloads' raw
measurements, the single-GPU guard, and a failing workload ending the run with its status."""
import argparse
import json
import os
import subprocess
import sys

import pytest

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _args(**kw):
    base = dict(gpus=1, steps=50, warmup=5, decode_steps=1000, no_cpu_baseline=True, settle_ms=bench.SETTLE_MS)
    base.update(kw)
    return argparse.Namespace(**base)


def _fake_parts():
    pct = {"p10_ms": 0.16, "median_ms": 0.17, "p90_ms": 0.18}
    return {
        "prefill": {"B": 4, "T": 4096, "H": 16, "K": 128, "ms_step": 0.17, "ms_launch": 0.168, "wall_ms": 0.2,
                    "pct": pct, "ms_step_cache_resident": 0.15, "ms_launch_cache_resident": 0.148,
                    "pct_cache_resident": pct, "input_sets": 2, "min_bytes": 278921216, "cold_ms_step": 0.2,
                    "settle": {"calls": 640, "ms": 100.2}},
        "decode": {"us_step": 25.0, "rot_us_step": 32.0, "eager_us_step": 40.0, "per_graph": 50},
        "varlen": {"ms_step": 0.4, "ms_launch": 0.39, "pct": pct, "lens": [4096] * 8, "input_sets": 2},
        "varlen_docs": {"ms_step": 0.5, "ms_launch": 0.49, "pct": pct, "lens": [100, 4000, 28668]},
        "train": {"fwd_ms": 0.28, "bwd_ms": 0.6},
        "block_pair": {"gdn_layer_ms": 1.0, "attn_layer_ms": 1.0},
    }


def test_assembled_line_keeps_the_driver_contract():
    res = bench.assemble(_fake_parts(), _args(), {"value": 1.0, "unit": "tokens/s", "cores": 16, "kind": "port",
                                                  "sample": "s"})
    line = json.loads(json.dumps(res))  # one JSON-serialisable object
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
                "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in line, key
    assert line["n_gpus"] == 1 and line["higher_is_better"] is True and line["vs_baseline"] is None
    assert line["value"] == pytest.approx(4 * 4096 / 0.17e-3, rel=1e-6)
    # the first K steps without the settle phase are reported beside the headline
    assert line["cold_ms_per_step"] == 0.2 and line["cold_value"] == pytest.approx(4 * 4096 / 0.2e-3, rel=1e-6)
    assert line["settle"]["prefill_calls"] == 640 and line["settle"]["ms_per_workload"] == bench.SETTLE_MS
    rf = line["roofline"]
    assert set(("bound", "achieved", "peak", "unit", "frac", "traffic")) <= set(rf)
    assert rf["achieved"] == pytest.approx(47_244_640_256 / 0.168e-3 / 1e12, rel=1e-3)
    assert rf["frac"] == pytest.approx(rf["achieved"] / bench.BF16_PEAK_TFLOPS, rel=1e-3)
    assert rf["flops_causal_halved"] == 36_507_222_016 and rf["flops_reference_flops_py"] == 17_179_869_184
    # the headline rotates over two input sets (DRAM-served); the one-set rate is reported beside it
    assert rf["input_sets"] == 2 and line["varlen"]["input_sets"] == 2
    assert line["cache_resident_value"] == pytest.approx(4 * 4096 / 0.15e-3, rel=1e-6)
    assert rf["cache_resident_frac"] == pytest.approx(47_244_640_256 / 0.148e-3 / 1e12 / bench.BF16_PEAK_TFLOPS,
                                                      rel=1e-3)
    # the decode headline is the DRAM-served (rotating) step; the cache-resident one is reported beside it
    assert line["decode"]["us_per_step"] == 32.0
    assert line["decode"]["frac_hbm_peak"] == pytest.approx(bench.decode_bytes() / 32e-6 / 8e12, rel=1e-3)
    assert line["decode"]["cache_resident_frac_hbm_peak"] == pytest.approx(bench.decode_bytes() / 25e-6 / 8e12, rel=1e-3)
    vd = line["varlen_docs"]
    assert vd["tokens_per_s"] == pytest.approx(32768 / 0.5e-3, rel=1e-6) and vd["longest_doc_chunks"] == 448


def test_doc_length_fixture_fills_every_window():
    """The committed lengths of the real-distribution leg: 8 windows of exactly 4,096 tokens, every
    document at least one token, drawn from a pool with the reference sample's statistics."""
    windows = bench.doc_length_windows()
    assert len(windows) == 8 and all(sum(w) == 4096 for w in windows)
    assert all(n >= 1 for w in windows for n in w)
    with open(bench.DOC_LENGTHS) as f:
        rec = json.load(f)
    assert rec["source_stats"]["n"] == 100_000 and rec["source_stats"]["median"] == 454.0


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 2 and "one GPU" in res.stderr


@pytest.mark.skipif(__import__("torch").cuda.is_available(), reason="checks the no-GPU failure path")
def test_a_failing_workload_ends_the_run_with_its_status():
    with pytest.raises(SystemExit) as ei:
        bench.run_part("prefill", _args(steps=1, warmup=1, decode_steps=1))
    assert ei.value.code == 1
