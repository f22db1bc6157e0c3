"""GPU: activation scales K-major by sorted position.

The prebuilt layer can pass the 1x128 activation scales between its kernels
K-major by sorted position (moe_gather_scales_by_position, then the _pos
GEMMs), so a GEMM step reads its tile's scales as one contiguous run.  This is
a layout between the build's own kernels with no counterpart in the
reference; every output of the layer must be bit-identical to the row-major
path, which the other GPU tests hold to the oracle -- at padding positions
too, where both read A row 0."""
from __future__ import annotations

import numpy as np
import pytest

from moe_cases import bf16_bits, make_case, to_gpu, u8_bits

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.mark.parametrize("E,BM", [(6, 32), (5, 16)])  # max_padded 456 (16 B rows) and 345 (unaligned rows)
@pytest.mark.parametrize("H", [512, 384])  # 4 groups (vector loads) and 3 (scalar loads)
def test_gather_matches_numpy(H, E, BM):
    from td_benchmark_amd import ops
    c = make_case(90, H, 256, E, 3, BM, seed=H + E)
    g = to_gpu(c)
    print(f"case: gather scales H={H} E={E} BM={BM}", flush=True)
    _, s = ops.per_token_group_quant_fp8(g["x"])
    sorted_ids, _, ntpp = ops.moe_align_block_size(g["topk_ids"], c.BM, c.E)
    out = torch.full((H // 128, sorted_ids.numel()), 5.0, device="cuda")
    ops.gather_scales_by_position(s, sorted_ids, ntpp, c.S, c.k, out=out)
    torch.cuda.synchronize()
    s_np, srt, n = s.cpu().numpy(), sorted_ids.cpu().numpy(), int(ntpp.item())
    want = np.repeat(s_np[:1].T, out.shape[1], axis=1)  # padding and past ntpp: row 0
    for p in range(n):
        if srt[p] < c.S:
            want[:, p] = s_np[srt[p] // c.k]
    assert np.array_equal(out.cpu().numpy(), want)


POS_CASES = [
    # (T, H, I, E, k, BM, routing, local experts or None)
    (64, 256, 512, 8, 2, 64, "softmax", None),     # tiny
    (700, 512, 256, 4, 2, 64, "softmax", None),    # 256-row tiles over 64-row blocks, 64-row tail body
    (128, 384, 256, 16, 8, 16, "zipf", None),      # 16-row tiles, 3 scale groups of H
    (200, 256, 384, 8, 2, 32, "softmax", [0, 3, 5]),  # expert map: zero blocks
]


@pytest.mark.parametrize("T,H,I,E,k,BM,routing,local", POS_CASES)
def test_position_major_scales_give_identical_layers(T, H, I, E, k, BM, routing, local):
    from td_benchmark_amd import ops
    c = make_case(T, H, I, E, k, BM, seed=T + E, routing=routing)
    g = to_gpu(c)
    print(f"case: scales by position T={T} H={H} I={I} E={E} k={k} BM={BM} local={local}", flush=True)
    if local is None:
        w, kw = (g["w13"], g["w13_s"], g["w2"], g["w2_s"]), {}
    else:
        w = tuple(g[n][local].contiguous() for n in ("w13", "w13_s", "w2", "w2_s"))
        emap = np.full(E, -1, np.int32)
        emap[local] = np.arange(len(local), dtype=np.int32)
        kw = {"global_num_experts": E, "expert_map": torch.from_numpy(emap).cuda()}
    outs = []
    for by_pos in (False, True):
        r = ops.FusedExpertsRunner(*w, c.T, c.k, BM, scales_by_position=by_pos, **kw)
        r.D.zero_()
        y = r.run(g["x"], g["topk_w"].view(-1), g["topk_ids"].view(-1))
        torch.cuda.synchronize()
        ntpp = int(r.align.ntpp.item())
        srt = r.align.sorted_ids.cpu().numpy()[:ntpp]
        slots = srt[srt < c.S]
        outs.append({"hq": u8_bits(r.hq)[:ntpp], "hs": r.hs.cpu().numpy()[:ntpp],
                     "D": bf16_bits(r.D)[slots], "y": bf16_bits(y)})
    for key in ("hq", "hs", "D", "y"):
        assert np.array_equal(outs[0][key], outs[1][key]), f"{key} differs between the scale layouts"
