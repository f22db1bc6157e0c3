"""GPU: whole output tiles of the full-size DeepSeek-V3, Mixtral, Qwen3 and
DeepSeek-V3 decode layers against the CPU oracle.

The layers are too large for the oracle to run whole, so the check picks
complete workgroup tiles of each grouped GEMM launch (tests/tile_map.py):
the first and last active tile of every XCD's range of the expert-major
order, both parts of a run split unevenly over its row tiles (a one-block
tile and the larger last tile holding the run's padding), a tile of an expert
with a single row tile (at the decode layer's 32-row tiles, two workgroups
per CU, the weights of such an expert stream with the non-temporal hint), a
256-row tile run by the 128-row body, and the first and last row tiles of the
expert with the most blocks.  For each picked
tile every valid row and every column of its n-tile is compared:
* W13 as a plain GEMM (C13 bf16 by slot) within the GEMM tests' bound, one
  bf16 step plus the oracle's matrix-core bound (overlap/kernels.py:95-214);
* the fused W13 epilogue's FP8 codes and scales of the same rows and group
  against the oracle chain (silu_and_mul + 1x128 quant of the oracle's C13,
  overlap_forward.py:277-284): each differing code traced to a differing h or
  scale of the GPU's own chain and from there to a C13 flip inside the MFMA
  accumulation bound, at the measured rate of that cause;
* W2 with routed weights (D bf16 by slot, A rows and scales by sorted
  position) on its own tile map, same bound (overlap_forward.py:289-302).
The oracle runs on the tile's expert and columns only: the other positions of
the sorted order are set to the pad value S, so the oracle skips them.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moe_cases import A7_MAX_FRAC, A7_MAX_ULP, a7_account, a7_assert, bf16_bits, count_bar, e4m3_ulp_diff, u8_bits
from tile_map import COL_MAJOR_K, pick_tiles, tile_map, tile_positions

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", params=["dsv3", "mixtral", "qwen3", "dsv3_decode"])
def layer(request):
    from td_benchmark_amd import ops, workloads
    wl = workloads.CONFIGS[request.param]
    print(f"case: full-size tiles {wl.name}", flush=True)
    d = workloads.generate(wl, "cuda")
    runner = ops.FusedExpertsRunner(d.w13, d.w13_s, d.w2, d.w2_s, wl.T, wl.top_k, wl.block_m)
    runner.run(d.x, d.topk_w, d.topk_ids)
    a = runner.align
    # W13 as a plain GEMM, and the GPU's own unfused chain, for tracing
    C13 = torch.empty((wl.S, 2 * wl.I), dtype=torch.bfloat16, device="cuda")
    ops.dispatch_fused_moe_kernel(runner.q1, d.w13, C13, runner.s1, d.w13_s, None, None, a.sorted_ids, a.expert_ids,
                                  a.ntpp, False, wl.top_k, {"BLOCK_SIZE_M": wl.block_m})
    h = torch.empty((wl.S, wl.I), dtype=torch.bfloat16, device="cuda")
    ops.silu_and_mul(h, C13)
    torch.cuda.synchronize()
    ntpp = int(a.ntpp.item())
    host = dict(
        sorted=a.sorted_ids.cpu().numpy(), eids=a.expert_ids.cpu().numpy(), ntpp=ntpp,
        q1=u8_bits(runner.q1), s1=runner.s1.cpu().numpy(),
        hq=u8_bits(runner.hq), hs=np.ascontiguousarray(runner.hs.cpu().numpy()),
        topk_w=d.topk_w.cpu().numpy().ravel())
    tile_m = ops.gemm_tile_rows(runner.BM, runner.S, runner.E, runner.tile_m)
    print(f"  ntpp {ntpp}, tile height {tile_m}", flush=True)
    return wl, d, runner, C13, h, host, tile_m


def _expert_cols(w: torch.Tensor, ws: torch.Tensor, e: int, groups: list[int]):
    """Expert e's weight rows of the given 128-row scale groups, as a
    one-expert operand for the oracle: (fp8 [1, 128*len(groups), K], scales)."""
    q = torch.cat([w[e, g * 128:(g + 1) * 128] for g in groups]).view(torch.uint8).cpu().numpy()[None]
    s = ws[e, groups].cpu().numpy()[None]
    return np.ascontiguousarray(q), np.ascontiguousarray(s)


def _only(host, ti, BM):
    """The sorted order with every position outside the tile set to the pad
    value, and the block ids with the tile's blocks on (local) expert 0."""
    S = host["topk_w"].size
    srt = np.full_like(host["sorted"], S)
    p = np.arange(ti.pos0, ti.pos0 + ti.rows)
    srt[p] = host["sorted"][p]
    eids = np.full_like(host["eids"], -1)
    eids[ti.pos0 // BM:(ti.pos0 + ti.rows) // BM] = 0
    return srt, eids


def _fused_ref(layer, name, ti):
    """The oracle chain of a picked tile's fused outputs (C13 of gate group j
    and up group I/128 + j by slot, with its fp32 value and bound, then h, the
    codes and the scale), computed once per layer and tile."""
    wl, d, runner, C13, h, host, tile_m = layer
    cache = host.setdefault("fused_ref", {})
    if name not in cache:
        S, I, BM = wl.S, wl.I, wl.block_m
        pos = tile_positions(ti, host["sorted"], S)
        slots = host["sorted"][pos]
        srt, eids = _only(host, ti, BM)
        B, Bs = _expert_cols(d.w13, d.w13_s, ti.expert, [ti.j, I // 128 + ti.j])
        cref, cf32, cbnd = oracle.grouped_gemm(host["q1"], host["s1"], B, Bs, srt, eids, host["ntpp"], BM, S,
                                               wl.top_k, with_f32=True, with_bound=True)
        cref, cf32, cbnd = cref[slots], cf32[slots], cbnd[slots]
        href = oracle.silu_and_mul(cref)
        qref, sref = oracle.quant_group128(href)
        cache[name] = (cref, cf32, cbnd, href, qref, sref)
    return cache[name]


def test_w13_whole_tiles(layer):
    wl, d, runner, C13, h, host, tile_m = layer
    S, I, BM = wl.S, wl.I, wl.block_m
    tiles = tile_map(host["eids"], host["ntpp"], BM, tile_m, I // 128)
    picked = pick_tiles(tiles, host["sorted"], S)
    c13 = bf16_bits(C13)
    h_gpu = bf16_bits(h)
    for name, ti in picked.items():
        pos = tile_positions(ti, host["sorted"], S)
        slots = host["sorted"][pos]
        srt, eids = _only(host, ti, BM)
        # plain W13: scale groups 2j and 2j+1
        groups = [2 * ti.j, 2 * ti.j + 1]
        B, Bs = _expert_cols(d.w13, d.w13_s, ti.expert, groups)
        ref, bnd = oracle.grouped_gemm(host["q1"], host["s1"], B, Bs, srt, eids, host["ntpp"], BM, S, wl.top_k,
                                       with_bound=True)
        got = c13[slots][:, 256 * ti.j:256 * ti.j + 256]
        bad = oracle.gemm_close(got, ref[slots], bnd[slots])
        print(f"  W13 {name}: {ti} rows {pos.size}, outside bound {int(bad.sum())}", flush=True)
        assert not bad.any(), f"W13 tile {name}: {int(bad.sum())} of {bad.size} outside the bound"
        # fused codes of group j: gate group j and up group I/128 + j
        cref, cf32, cbnd, href, qref, sref = _fused_ref(layer, name, ti)
        cols = np.r_[128 * ti.j:128 * ti.j + 128]
        c_gpu = np.concatenate([c13[slots][:, cols], c13[slots][:, I + cols]], axis=1)
        rep = a7_account(host["hq"][pos][:, cols], host["hs"][pos][:, ti.j:ti.j + 1], h_gpu[slots][:, cols], c_gpu,
                         qref, sref, href, cref, cf32, cbnd)
        a7_assert(rep, f"{wl.name} fused W13 tile {name}")


def test_w2_whole_tiles(layer):
    wl, d, runner, C13, h, host, tile_m = layer
    S, H, BM = wl.S, wl.H, wl.block_m
    n_tiles = (H // 128 + 1) // 2
    tiles = tile_map(host["eids"], host["ntpp"], BM, tile_m, n_tiles, col_major=wl.I >= COL_MAJOR_K)
    picked = pick_tiles(tiles, host["sorted"], S)
    D = bf16_bits(runner.D[:S])
    for name, ti in picked.items():
        pos = tile_positions(ti, host["sorted"], S)
        slots = host["sorted"][pos]
        srt, eids = _only(host, ti, BM)
        groups = [g for g in (2 * ti.j, 2 * ti.j + 1) if g < H // 128]
        B, Bs = _expert_cols(d.w2, d.w2_s, ti.expert, groups)
        ref, bnd = oracle.grouped_gemm(host["hq"], host["hs"], B, Bs, srt, eids, host["ntpp"], BM, S, 1,
                                       a_row_by_pos=True, topk_w=host["topk_w"], with_bound=True)
        got = D[slots][:, 256 * ti.j:256 * ti.j + 128 * len(groups)]
        bad = oracle.gemm_close(got, ref[slots], bnd[slots])
        print(f"  W2 {name}: {ti} rows {pos.size}, outside bound {int(bad.sum())}", flush=True)
        assert not bad.any(), f"W2 tile {name}: {int(bad.sum())} of {bad.size} outside the bound"


def test_w13_exact_whole_tiles(layer):
    """The exact-dot W13 on the same full-size layer: every picked tile's codes
    within the north-star bar (<= 1 ULP on <= 0.1 % of codes) of the oracle
    chain, its scales likewise, and no more differing codes than the FP8 form."""
    wl, d, runner, C13, h, host, tile_m = layer
    S, I, BM = wl.S, wl.I, wl.block_m
    runner.exact_dot = True
    try:
        runner.stage_w13()
        torch.cuda.synchronize()
        hq_x = u8_bits(runner.hq)
        hs_x = np.ascontiguousarray(runner.hs.cpu().numpy())
    finally:
        runner.exact_dot = False
    tiles = tile_map(host["eids"], host["ntpp"], BM, tile_m, I // 128)
    picked = pick_tiles(tiles, host["sorted"], S)
    n = nd = nd_fp8 = 0
    for name, ti in picked.items():
        pos = tile_positions(ti, host["sorted"], S)
        _, _, _, _, qref, sref = _fused_ref(layer, name, ti)
        cols = np.r_[128 * ti.j:128 * ti.j + 128]
        dx = e4m3_ulp_diff(hq_x[pos][:, cols], qref)
        df = e4m3_ulp_diff(host["hq"][pos][:, cols], qref)
        s_diff = hs_x[pos][:, ti.j:ti.j + 1] != sref
        print(f"  exact W13 {name}: {int((dx > 0).sum())} of {dx.size} codes differ (max {int(dx.max())} ulp), "
              f"{int(s_diff.sum())} scales; FP8 form {int((df > 0).sum())}", flush=True)
        assert dx.max() <= A7_MAX_ULP, f"exact W13 tile {name}: a code {int(dx.max())} ulp off"
        assert s_diff.sum() <= count_bar(A7_MAX_FRAC, s_diff.size), \
            f"exact W13 tile {name}: {int(s_diff.sum())} scales differ"
        n += dx.size
        nd += int((dx > 0).sum())
        nd_fp8 += int((df > 0).sum())
    assert nd <= A7_MAX_FRAC * n, f"{wl.name}: {nd} of {n} exact-mode codes differ"
    assert nd <= nd_fp8
