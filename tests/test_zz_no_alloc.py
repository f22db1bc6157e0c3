"""GPU: the allocation-free align entry point (moe_align_block_size_noalloc,
workspace in a static device array) against the existing entry point
(moe_align_block_size with a caller workspace), through the C ABI, bit for
bit: two calls in a row, the second with a smaller input, so the second call
runs over a scratch array that still holds the first call's larger contents;
and the limit check.  No counterpart in the reference (its align always takes
caller memory)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _align_both(ids_np: np.ndarray, E: int, BM: int):
    from td_benchmark_amd import ops
    from td_benchmark_amd._lib import check, lib
    L = lib()
    S = ids_np.size
    ids = torch.from_numpy(ids_np.ravel().astype(np.int32)).cuda()
    ref = ops.AlignBuffers(S, E, BM, ids.device)
    ref.run(ids)
    mp = ref.max_padded
    sorted_ids = torch.full((max(mp, 1),), -7, dtype=torch.int32, device="cuda")
    eids = torch.full((max(ref.max_blocks, 1),), -7, dtype=torch.int32, device="cuda")
    ntpp = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    before = torch.cuda.memory_stats().get("allocation.all.allocated", 0)
    check(L.moe_align_block_size_noalloc(_p(ids), S, E, BM, _p(sorted_ids), _p(eids), _p(ntpp), mp, stream),
          "moe_align_block_size_noalloc")
    torch.cuda.synchronize()
    assert torch.cuda.memory_stats().get("allocation.all.allocated", 0) == before
    assert int(ntpp.item()) == int(ref.ntpp.item())
    assert torch.equal(sorted_ids[:mp], ref.sorted_ids[:mp])
    assert torch.equal(eids[: ref.max_blocks], ref.expert_ids[: ref.max_blocks])
    return int(ntpp.item())


@pytest.mark.parametrize("first,second", [
    ((8192, 8, 256, 128, "sigmoid"), (2048, 8, 256, 128, "sigmoid")),   # DSv3 then a smaller batch
    ((4096, 8, 128, 64, "softmax"), (100, 8, 128, 64, "softmax")),      # three-launch then one-launch path
    ((16384, 8, 512, 128, "softmax"), (3000, 4, 512, 32, "zipf")),      # chunk counts past the LDS stage
])
def test_noalloc_align_equals_align_on_two_calls(first, second):
    from moe_cases import route
    for i, (T, k, E, BM, routing) in enumerate((first, second)):
        rng = np.random.default_rng(T + E + i)
        ids, _ = route(rng.standard_normal((T, E), dtype=np.float32), k, routing, rng)
        print(f"case: noalloc align call {i + 1}: T={T} k={k} E={E} BM={BM} {routing}", flush=True)
        _align_both(ids, E, BM)


def test_noalloc_align_rejects_sizes_beyond_its_scratch():
    from td_benchmark_amd._lib import STATUS, lib
    L = lib()
    limit = 4 * 1024 * 1024
    S, E = 1 << 20, 1024
    assert L.moe_align_workspace_bytes(S, E) > limit
    dummy = torch.zeros(1, dtype=torch.int32, device="cuda")
    rc = L.moe_align_block_size_noalloc(_p(dummy), S, E, 128, _p(dummy), _p(dummy), _p(dummy),
                                        L.moe_align_max_padded(S, E, 128), None)
    assert STATUS[rc] == "MOE_ERR_CAPACITY"
