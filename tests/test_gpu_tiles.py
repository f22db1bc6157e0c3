"""GPU: the GEMM's workgroup tile height never changes a result.

A tile of tile_m rows spans tile_m / block_size_m consecutive align blocks of
one expert (the reference's fused_moe_kernel runs one align block per program,
overlap/kernels.py:95-126).  Each output element is the same sequence of MFMAs
and scale FMAs whichever tile computes it, so the fused W13 outputs (hq, hs by
sorted position), the W2 rows (D by slot) and the layer output must be bit for
bit those of tile_m = block_size_m, including the zero rows of expert -1
blocks under an expert map.  The oracle checks of the 256-row tiles themselves
are in test_gpu_kernels.py (block size 256 and the automatic choice)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moe_cases import bf16_bits, make_case, to_gpu, u8_bits

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

TILE_CASES = [
    # (T, H, I, E, k, BM, routing, local experts or None)
    (300, 256, 256, 4, 2, 16, "softmax", None),     # 16-row blocks in tiles of up to 16 blocks
    (500, 384, 256, 6, 3, 64, "zipf", None),        # skewed: long and short runs
    (600, 256, 384, 3, 2, 128, "softmax", None),    # pairs of 128-row blocks
    (400, 256, 256, 8, 2, 32, "softmax", [1, 4, 6]),  # expert map: runs of -1 blocks
]


def _run(c, g, BM, tile_m, local):
    from td_benchmark_amd import ops
    if local is None:
        w = (g["w13"], g["w13_s"], g["w2"], g["w2_s"])
        kw = {}
    else:
        w = tuple(g[n][local].contiguous() for n in ("w13", "w13_s", "w2", "w2_s"))
        emap = np.full(c.E, -1, np.int32)
        emap[local] = np.arange(len(local), dtype=np.int32)
        kw = {"global_num_experts": c.E, "expert_map": torch.from_numpy(emap).cuda()}
    r = ops.FusedExpertsRunner(*w, c.T, c.k, BM, tile_m=tile_m, **kw)
    r.D.zero_()
    y = r.run(g["x"], g["topk_w"].view(-1), g["topk_ids"].view(-1))
    torch.cuda.synchronize()
    ntpp = int(r.align.ntpp.item())
    srt = r.align.sorted_ids.cpu().numpy()[:ntpp]
    slots = srt[srt < c.S]
    return {"ntpp": ntpp, "hq": u8_bits(r.hq)[:ntpp], "hs": r.hs.cpu().numpy()[:ntpp],
            "D": bf16_bits(r.D)[slots], "y": bf16_bits(y), "slots": slots}


@pytest.mark.parametrize("T,H,I,E,k,BM,routing,local", TILE_CASES)
def test_tile_height_does_not_change_results(T, H, I, E, k, BM, routing, local):
    c = make_case(T, H, I, E, k, BM, seed=T + BM, routing=routing)
    g = to_gpu(c)
    heights = [t for t in (16, 32, 64, 128, 256) if t >= BM]
    print(f"case: tiles T={T} E={E} k={k} BM={BM} {routing} local={local} heights={heights}", flush=True)
    base = _run(c, g, BM, BM, local)
    # the runs really span several blocks, so the larger tiles group blocks
    _, eids, _ = oracle.moe_align(c.topk_ids, E, BM)
    nb = base["ntpp"] // BM
    assert np.any(eids[1:nb] == eids[:nb - 1])
    for tm in heights[1:] + [0]:
        got = _run(c, g, BM, tm, local)
        assert got["ntpp"] == base["ntpp"]
        for key in ("hq", "hs", "D", "y"):
            assert np.array_equal(got[key], base[key]), f"tile_m={tm}: {key} differs"


def test_tile_height_rejects_bad_values():
    from td_benchmark_amd import MoeKernelError, ops
    c = make_case(64, 256, 256, 4, 2, 64, seed=1)
    g = to_gpu(c)
    with pytest.raises(ValueError):
        ops.FusedExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], c.T, c.k, 64, tile_m=32)
    q1, s1 = ops.per_token_group_quant_fp8(g["x"])
    sorted_ids, eids, ntpp = ops.moe_align_block_size(g["topk_ids"], 64, c.E)
    with pytest.raises(MoeKernelError):
        ops.gemm_w13_silu_quant(q1, s1, g["w13"], g["w13_s"], sorted_ids, eids, ntpp, c.S, c.k, 64, tile_m=96)
