"""Host-side logic that runs without a GPU: the tile configuration heuristic
(A4), the workload table, the bench contract's CPU parts."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle

ROOT = Path(__file__).resolve().parents[1]


def test_moe_config_block_m_tracks_rows_per_expert():
    from td_benchmark_amd import ops

    # DeepSeek-V3 prefill: 8192*8/256 = 256 rows per expert -> 128
    assert ops.get_moe_config(8192, 256, 8)["BLOCK_SIZE_M"] == 128
    # decode: 128*8/256 = 4 rows per expert -> 32 (its weight stream is faster than 16's)
    assert ops.get_moe_config(128, 256, 8)["BLOCK_SIZE_M"] == 32
    assert ops.get_moe_config(48, 4, 2)["BLOCK_SIZE_M"] == 32   # 24 rows per expert
    assert ops.get_moe_config(64, 4, 2)["BLOCK_SIZE_M"] == 64   # 32 rows per expert
    assert ops.get_moe_config(1280, 256, 8)["BLOCK_SIZE_M"] == 64  # 40 rows per expert (DeepSeek-V3 shape)
    assert ops.get_moe_config(1536, 256, 8)["BLOCK_SIZE_M"] == 128  # 48
    assert ops.get_moe_config(512, 64, 8)["BLOCK_SIZE_M"] == 128  # 64 rows per expert
    assert ops.get_moe_config(1024, 64, 8)["BLOCK_SIZE_M"] == 256  # 128: one tile per expert
    assert ops.get_moe_config(2560, 64, 8)["BLOCK_SIZE_M"] == 256  # 320
    assert ops.get_moe_config(16384, 128, 8)["BLOCK_SIZE_M"] == 256  # Qwen3 one pass: 1024
    for T in (1, 7, 100, 4096, 65536):
        cfg = ops.get_moe_config(T, 128, 8)
        assert cfg["BLOCK_SIZE_M"] in ops.SUPPORTED_BLOCK_M
        assert cfg["BLOCK_SIZE_K"] == 128


def test_workload_table_matches_benchmark_configs():
    from td_benchmark_amd import workloads

    c = workloads.CONFIGS
    assert (c["dsv3"].T, c["dsv3"].H, c["dsv3"].I, c["dsv3"].E, c["dsv3"].top_k) == (8192, 7168, 2048, 256, 8)
    assert (c["tiny"].T, c["tiny"].H, c["tiny"].I, c["tiny"].E, c["tiny"].top_k) == (64, 256, 512, 8, 2)
    assert c["dsv3"].gemm_flop == 6 * 8192 * 8 * 7168 * 2048
    for wl in c.values():
        assert wl.H % 128 == 0 and wl.I % 128 == 0
        assert wl.block_m in (16, 32, 64, 128, 256)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_bench_stage_bytes_and_traffic_lookup():
    sys.path.insert(0, str(ROOT))
    import bench
    from td_benchmark_amd import workloads

    wl = workloads.CONFIGS["dsv3"]
    b = bench.stage_bytes(wl, ntpp=81024, active=256)
    # W13 weights dominate: 256 experts x 2I x H bytes
    assert b["w13"] > 256 * 2 * 2048 * 7168
    assert b["reduce"] == 2 * wl.S * wl.H + 2 * wl.T * wl.H
    # the committed PMC summary holds the W13 launch's traffic at DSv3 (256-row tiles)
    traffic, src = bench.measured_traffic("dsv3", "grouped_gemm_kernel<256,true>")
    assert src == "moe_layer_dsv3_hbm_traffic.md"
    assert b["w13"] < traffic < 1.5 * b["w13"]
    assert bench.measured_traffic("no_such_workload", "x") == (None, None)


def test_bench_metric_is_baseline_metric():
    sys.path.insert(0, str(ROOT))
    import bench

    base = json.loads((ROOT / "BASELINE.json").read_text())
    assert bench.METRIC == base["metric"]


def test_ops_fail_loudly_without_library(monkeypatch, tmp_path):
    from td_benchmark_amd import _lib

    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "missing.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="no fallback"):
        _lib.lib()


def test_gemm_tile_rows_rule():
    from td_benchmark_amd import ops
    assert ops.gemm_tile_rows(128, 65536, 256) == 256      # DSv3: 256 slots per expert
    assert ops.gemm_tile_rows(16, 1024, 256) == 16         # decode
    assert ops.gemm_tile_rows(64, 160 * 8, 8) == 256       # the threshold itself
    assert ops.gemm_tile_rows(64, 160 * 8 - 1, 8) == 64
    assert ops.gemm_tile_rows(64, 16, 8, tile_m=128) == 128


@pytest.mark.parametrize("T,E,k,BM,tile_m,n_tiles,routing", [
    (8192, 256, 8, 128, 256, 16, "sigmoid"),   # DSv3 W13
    (8192, 256, 8, 128, 256, 28, "sigmoid"),   # DSv3 W2
    (4096, 8, 2, 128, 256, 112, "softmax"),    # Mixtral W13
    (128, 256, 8, 32, 32, 16, "zipf"),         # decode
    (4096, 2, 1, 16, 256, 1, "softmax"),       # runs longer than 65 blocks
])
def test_tile_map_covers_every_position_once(T, E, k, BM, tile_m, n_tiles, routing):
    """The host restatement of the GEMM's tile mapping (tests/tile_map.py)
    partitions the sorted positions x n-tiles: every (position, n-tile) of the
    padded order lies in exactly one active tile, tiles stay inside one run,
    and each XCD range is contiguous."""
    from moe_cases import route
    from tile_map import XCDS, pick_tiles, tile_map
    rng = np.random.default_rng(T + E)
    ids, _ = route(rng.standard_normal((T, E), dtype=np.float32), k, routing, rng)
    srt, eids, ntpp = oracle.moe_align(ids, E, BM)
    for col_major in (False, True):  # the group orders of short-K and long-K plain launches
        tiles = tile_map(eids, ntpp, BM, tile_m, n_tiles, col_major=col_major)
        cov = np.zeros((ntpp, n_tiles), np.int32)
        for ti in tiles:
            assert ti.rows % BM == 0 and 0 < ti.rows <= max(tile_m, BM)
            assert len(set(eids[ti.pos0 // BM:(ti.pos0 + ti.rows) // BM].tolist())) == 1
            cov[ti.pos0:ti.pos0 + ti.rows, ti.j] += 1
        assert cov.min() == 1 and cov.max() == 1
        ts = sorted(t.t for t in tiles)
        assert len(set(ts)) == len(ts) and max(t.xcd for t in tiles) < XCDS
    picked = pick_tiles(tiles, srt, T * k)
    assert {f"xcd{x}_first" for x in {t.xcd for t in tiles}} <= set(picked)


def test_bench_summarize_samples_follows_reference_statistics():
    """avg/min/med/p95/std as moe_bench/timing.py:23-34 defines them (p95 at
    index int(0.95 * (n - 1)) of the sorted samples, population std)."""
    sys.path.insert(0, str(ROOT))
    import bench
    s = bench.summarize_samples([5.0, 1.0, 3.0, 2.0, 4.0])
    assert s["avg"] == 3.0 and s["min"] == 1.0 and s["med"] == 3.0
    assert s["p95"] == 4.0  # sorted[int(0.95 * 4)] = sorted[3]
    assert abs(s["std"] - 2.0 ** 0.5) < 1e-12
    assert bench.summarize_samples([])["n"] == 0


def test_bench_cpu_baseline_runs_the_torch_golden_on_all_cores():
    """The CPU baseline leg on the tiny configuration, with CPU tensors in
    place of the GPU workload: torch threads = os.cpu_count(), the lscpu model
    name, and the stage timings of the torch ops."""
    import os

    import torch

    from moe_cases import make_case
    sys.path.insert(0, str(ROOT))
    import bench
    from td_benchmark_amd import workloads
    wl = workloads.CONFIGS["tiny"]
    c = make_case(wl.T, wl.H, wl.I, wl.E, wl.top_k, wl.block_m, seed=0)
    f8 = lambda a: torch.from_numpy(a).view(torch.float8_e4m3fn)  # noqa: E731
    data = workloads.LayerData(torch.from_numpy(c.x.view(np.int16)).view(torch.bfloat16),
                               torch.from_numpy(c.topk_ids), torch.from_numpy(c.topk_w),
                               f8(c.w13_q), torch.from_numpy(c.w13_s), f8(c.w2_q), torch.from_numpy(c.w2_s))
    cb = bench.cpu_baseline(data, wl, budget_s=0.2)
    assert cb["value"] > 0 and cb["cores"] == os.cpu_count() and cb["kind"] == "port"
    assert cb["cpu_model"]
    D = torch.zeros((wl.S, wl.H), dtype=torch.bfloat16)
    st = bench.cpu_stage_times(data, wl, D, wl.block_m)
    assert st["quant_us"] > 0 and st["align_us"] > 0 and st["reduce_us"] > 0


def test_split_bounds_are_whole_128_blocks_covering_the_range():
    from td_benchmark_amd.ops import _split_bounds

    assert _split_bounds(2048, 4) == [(0, 512), (512, 1024), (1024, 1536), (1536, 2048)]
    assert _split_bounds(640, 4) == [(0, 256), (256, 384), (384, 512), (512, 640)]
    assert _split_bounds(256, 4) == [(0, 128), (128, 256)]   # never an empty chunk
    for total in (128, 384, 7168):
        for n in (1, 2, 3, 5):
            b = _split_bounds(total, n)
            assert b[0][0] == 0 and b[-1][1] == total
            assert all(k0 < k1 and k0 % 128 == 0 and k1 % 128 == 0 for k0, k1 in b)
            assert all(b[i][1] == b[i + 1][0] for i in range(len(b) - 1))
