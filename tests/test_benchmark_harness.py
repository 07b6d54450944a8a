"""The benchmark harness (gqa-flash-attn-rtx3060_amd/benchmark/run.py): row
schema, median aggregation and work counts on the CPU; its correctness gate's
fp32 reference against the oracle; a quick GPU run."""
from __future__ import annotations

import importlib.util
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

REPO = Path(__file__).resolve().parent.parent
_spec = importlib.util.spec_from_file_location(
    "gqa_bench_run", REPO / "gqa-flash-attn-rtx3060_amd" / "benchmark" / "run.py")
run = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(run)

# Row keys of the reference's results JSON (benchmark/run.py:181-188).
REF_ROW_KEYS = {"workload", "seq_kv", "ours_ms", "fa2_ms", "sdpa_ms", "tok_s", "speedup_vs_fa2",
                "speedup_vs_sdpa", "peak_mem_gb"}


def test_row_schema_and_speedups():
    r = run.make_row("prefill", 16384, 2.0, float("nan"), 6.0, 0.8)
    assert REF_ROW_KEYS <= set(r)
    assert r["tok_s"] == 16384 * 1000.0 / 2.0
    assert r["speedup_vs_sdpa"] == 3.0 and math.isnan(r["speedup_vs_fa2"])
    flops, nbytes = run.work("prefill", 16384)
    assert flops == 2199157473280  # 4*D*Hq*S(S+1)/2
    assert abs(r["tflops"] - flops / 2e-3 / 1e12) < 1e-9
    d = run.make_row("decode", 131072, 0.1, 0.2, 0.5, 1.0)
    assert d["tok_s"] == 1000.0 / 0.1
    assert run.work("decode", 131072)[1] == 536887296


def test_median_aggregation():
    mk = lambda ms: [run.make_row("decode", 2048, ms, float("nan"), 2 * ms, 0.1)]
    agg = run.aggregate_median([mk(1.0), mk(3.0), mk(2.0)])
    assert len(agg) == 1 and agg[0]["ours_ms"] == 2.0 and agg[0]["sdpa_ms"] == 4.0


def test_markdown_table_has_every_row():
    rows = [run.make_row("prefill", L, 1.0, float("nan"), 2.0, 0.1) for L in (2048, 4096)]
    t = run.markdown_table(rows).splitlines()
    assert len(t) == 2 + 2 and "| prefill | 4096 |" in t[3]


def test_reference_attention_matches_oracle():
    # The harness's fp32 gate reference (torch, run here on the CPU) against
    # the pinned oracle: bottom-right causal, G = 4, Sq < Skv.
    from oracle import gqa_oracle
    g = torch.Generator().manual_seed(3)
    q = (torch.randn(1, 8, 5, 64, generator=g) * 0.5).to(torch.bfloat16)
    k = (torch.randn(1, 2, 9, 64, generator=g) * 0.5).to(torch.bfloat16)
    v = (torch.randn(1, 2, 9, 64, generator=g) * 0.5).to(torch.bfloat16)
    got = run.reference_attention(torch, q, k, v, causal=True).numpy()
    want = gqa_oracle.gqa_reference(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal=True,
                                    dtype=np.float64)
    assert np.abs(got - want).max() < 1e-5


@pytest.mark.gpu
def test_quick_run_writes_reference_schema(tmp_path):
    assert run.main(["--quick", "--out", str(tmp_path)]) == 0
    files = list(tmp_path.glob("*.json"))
    assert len(files) == 1
    data = json.loads(files[0].read_text())
    assert {"commit", "device", "dtype", "trials", "config", "rows"} <= set(data)
    assert [(r["workload"], r["seq_kv"]) for r in data["rows"]] == [("prefill", 8192), ("decode", 8192)]
    for r in data["rows"]:
        assert REF_ROW_KEYS <= set(r) and r["ours_ms"] > 0
