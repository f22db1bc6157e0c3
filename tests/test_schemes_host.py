"""Host logic of the scheme plugin and the microbench counterparts (no GPU).

Restates the reference's contract tests: tunable validation
(schemes/base.py:48-62), registry lookup (schemes/__init__.py:32-36), the
worker's FP8 contract (worker.py:117-121), and the microbench dry-run plan
(tests/test_microbench_dry_run.py:7-30)."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path
from types import SimpleNamespace

import pytest

from td_benchmark_amd import schemes
from td_benchmark_amd.microbench import SCRIPTS

ROOT = Path(__file__).resolve().parents[1]


def test_m1_spec_meets_worker_fp8_contract():
    spec, builder = schemes.REGISTRY["m1"]
    assert spec.weight_dtype == "fp8" and spec.act_quant == "group128"
    assert spec.requires_nvshmem is False
    assert builder is schemes.build
    assert set(spec.tunables_schema) == {"block_m", "n_chunks", "n_streams", "n_chunks_gateup", "n_chunks_down",
                                         "exact_dot"}


def test_validate_tunables_defaults_and_errors():
    spec = schemes.SPEC
    assert schemes.validate_tunables(spec, {}) == {"block_m": 0, "n_chunks": 1, "n_streams": 1,
                                                   "n_chunks_gateup": 0, "n_chunks_down": 0, "exact_dot": False}
    assert schemes.validate_tunables(spec, {"exact_dot": True})["exact_dot"] is True
    with pytest.raises(schemes.SchemeConfigError, match="expected bool"):
        schemes.validate_tunables(spec, {"exact_dot": 1})
    assert schemes.validate_tunables(spec, {"n_chunks": 4})["n_chunks"] == 4
    with pytest.raises(schemes.SchemeConfigError, match="violate schema"):
        schemes.validate_tunables(spec, {"bogus": 1})
    with pytest.raises(schemes.SchemeConfigError, match="expected int"):
        schemes.validate_tunables(spec, {"block_m": "64"})
    with pytest.raises(schemes.SchemeConfigError, match="expected int"):
        schemes.validate_tunables(spec, {"n_streams": True})


def test_build_scheme_rejects_unknown_code_bad_context_and_missing_data():
    with pytest.raises(schemes.SchemeConfigError, match="not registered"):
        schemes.build_scheme(None, None, None, SimpleNamespace(code="zz", tunables={}))
    with pytest.raises(schemes.SchemeConfigError, match="one GPU"):
        schemes.build_scheme(None, SimpleNamespace(world_size=2), object(), SimpleNamespace(code="m1", tunables={}))
    with pytest.raises(RuntimeError, match="DataBundle"):
        schemes.build_scheme(None, SimpleNamespace(world_size=1), None, SimpleNamespace(code="m1", tunables={}))
    with pytest.raises(schemes.SchemeConfigError, match="block_m"):
        schemes.build_scheme(None, SimpleNamespace(world_size=1), object(),
                             SimpleNamespace(code="m1", tunables={"block_m": 48}))
    # the b schemes' K/N chunk counts (configs/run_v1.yaml: n_chunks_gateup 2, n_chunks_down 4)
    for bad in ({"n_chunks_gateup": 2}, {"n_chunks_down": 4}, {"n_chunks_gateup": -1, "n_chunks_down": 2},
                {"n_chunks_gateup": 2, "n_chunks_down": 4, "n_chunks": 2}):
        with pytest.raises(schemes.SchemeConfigError, match="n_chunks"):
            schemes.build_scheme(None, SimpleNamespace(world_size=1), object(),
                                 SimpleNamespace(code="m1", tunables=bad))
    # the exact-dot mode belongs to the fused W13, which the K-split structure does not run
    with pytest.raises(schemes.SchemeConfigError, match="exact_dot"):
        schemes.build_scheme(None, SimpleNamespace(world_size=1), object(),
                             SimpleNamespace(code="m1", tunables={"n_chunks_gateup": 2, "n_chunks_down": 4,
                                                                  "exact_dot": True}))


@pytest.mark.parametrize("name", SCRIPTS)
def test_microbench_dry_run_plan(name):
    r = subprocess.run([sys.executable, "-m", f"td_benchmark_amd.microbench.{name}", "--dry-run"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 0, r.stderr
    plan = json.loads(r.stdout)
    assert plan["kind"] == "microbench"
    assert plan["script"] == f"{name}.py"
    assert plan["server_verify"] is True
    assert plan["sweep"] and plan["metrics"] and plan["metrics"][0] == "latency_ms"
    assert plan["exp_id"].startswith("EXP-")
    assert plan["result_schema"]["kind"] == "microbench"
    assert {"metric", "unit", "aggregation"} <= set(plan["result_schema"])
    assert plan["recommended_command"][0] == "torchrun"
    assert {"purpose", "warmup", "repeat", "output", "server_verify_detail"} <= set(plan)


def test_microbench_exp_ids_match_reference_scripts():
    ids = {}
    for name in SCRIPTS:
        r = subprocess.run([sys.executable, "-m", f"td_benchmark_amd.microbench.{name}", "--dry-run"],
                           capture_output=True, text=True, timeout=120, cwd=ROOT)
        ids[name] = json.loads(r.stdout)["exp_id"]
    assert ids == {"mb_moe_align": "EXP-010", "mb_dispatch_prep": "EXP-011", "mb_tile_order_groupgemm": "EXP-012",
                   "mb_group_gemm": "EXP-014", "mb_quant_kernels": "EXP-015", "mb_chunk_overlap": "EXP-016"}


def test_microbench_sweeps_match_reference():
    from td_benchmark_amd.microbench import (mb_chunk_overlap, mb_dispatch_prep, mb_group_gemm, mb_moe_align,
                                             mb_quant_kernels, mb_tile_order_groupgemm)
    from td_benchmark_amd.microbench.common import iter_cases

    assert mb_moe_align.SWEEP == {"M": [1024, 2048, 4096, 6647], "E": [64, 128], "top_k": [8, 16]}
    assert mb_quant_kernels.SWEEP["kernel"] == ["group128", "swiglu_group128"]
    assert mb_group_gemm.SWEEP["tile"] == [64, 128, 256]
    assert mb_tile_order_groupgemm.SWEEP["order"] == ["expert_major", "phase_major", "half_phase"]
    assert mb_dispatch_prep.SWEEP["M"] == [1024, 2048, 4096, 6647]
    # microbench/mb_chunk_overlap.py sweep, with M of REWORK-B.md:960
    assert mb_chunk_overlap.SWEEP == {"M": [1024, 5120], "scheme": ["b1", "b2", "b3"],
                                      "n_chunks": [1, 2, 4, 8, 16]}
    assert len(list(iter_cases(mb_moe_align.SWEEP, 0))) == 16
    assert len(list(iter_cases(mb_moe_align.SWEEP, 3))) == 3


def test_tile_order_l2_hit_rate_reads_rocprof_counter_rows(tmp_path):
    """The l2_hit_rate of the tile-order microbench: TCC hits over hits plus
    misses, summed over the grouped GEMM's dispatches only."""
    from td_benchmark_amd.microbench.mb_tile_order_groupgemm import l2_hit_rate_from_csv

    cols = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    rows = [(1, "void moe::grouped_gemm_kernel<64, false>(moe::GemmArgs)", "TCC_HIT_sum", 300.0),
            (1, "void moe::grouped_gemm_kernel<64, false>(moe::GemmArgs)", "TCC_MISS_sum", 100.0),
            (2, "void moe::grouped_gemm_kernel<64, false>(moe::GemmArgs)", "TCC_HIT_sum", 500.0),
            (2, "void moe::grouped_gemm_kernel<64, false>(moe::GemmArgs)", "TCC_MISS_sum", 100.0),
            (3, "void moe::quant_group128_kernel<false>(...)", "TCC_HIT_sum", 0.0),
            (3, "void moe::quant_group128_kernel<false>(...)", "TCC_MISS_sum", 1e9)]
    path = tmp_path / "l2_counter_collection.csv"
    with path.open("w", newline="") as fh:
        w = __import__("csv").writer(fh, quoting=__import__("csv").QUOTE_NONNUMERIC)
        w.writerow(cols)
        w.writerows(rows)
    assert l2_hit_rate_from_csv([path]) == 800.0 / 1000.0
    assert l2_hit_rate_from_csv([path], kernel_substr="no_such_kernel") is None
