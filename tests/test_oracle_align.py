"""Pins the oracle's moe_align_block_size (A3).

The reference calls vLLM's ``moe_align_block_size`` (overlap/overlap_forward.py:
165-169), which is not vendored; its padded-cumsum layout is restated in-repo
at tdx/kernels/moe_utils.py:168-217.  The oracle is held to
  * a brute-force construction on tiny inputs (Python sort + per-expert
    chunking, no cumsum arithmetic shared with the C code),
  * invariants on larger random inputs: every valid slot appears exactly once,
    blocks are expert-homogeneous and ascending in expert id, padding equals
    S, ntpp = sum ceil(c_e/BM)*BM, expert_ids is -1 past ntpp,
  * the edge cases the reference's inputs have: empty experts, all slots on
    one expert, ids outside [0, E) (an expert map's -1) dropped, a capacity
    that is too small.
The within-expert order (ascending slot) is this build's choice where vLLM's
order is unpinned; the GEMM results do not depend on it.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle


def brute_force_align(ids: list[int], E: int, BM: int, max_padded: int):
    S = len(ids)
    order = sorted((e, s) for s, e in enumerate(ids) if 0 <= e < E)
    sorted_ids: list[int] = []
    eids: list[int] = []
    for e in range(E):
        mine = [s for (ee, s) in order if ee == e]
        while mine:
            chunk, mine = mine[:BM], mine[BM:]
            sorted_ids += chunk + [S] * (BM - len(chunk))
            eids.append(e)
    ntpp = len(sorted_ids)
    sorted_ids += [S] * (max_padded - ntpp)
    eids += [-1] * ((max_padded + BM - 1) // BM - len(eids))
    return sorted_ids, eids, ntpp


@pytest.mark.parametrize("S,E,BM,seed", [(1, 1, 16, 0), (7, 3, 4, 1), (40, 5, 16, 2), (64, 8, 16, 3),
                                         (33, 4, 32, 4), (100, 16, 8, 5)])
def test_align_matches_brute_force(S, E, BM, seed):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, E, S).astype(np.int32)
    mp = oracle.max_padded_size(S, E, BM)
    got = oracle.moe_align(ids, E, BM, mp)
    ref = brute_force_align(ids.tolist(), E, BM, mp)
    assert got[0].tolist() == ref[0]
    assert got[1].tolist() == ref[1]
    assert got[2] == ref[2]


def test_align_drops_out_of_range_ids_and_handles_empty_experts():
    ids = np.array([2, -1, 2, 9, 0, 2, -1], np.int32)
    E, BM = 4, 2
    mp = oracle.max_padded_size(ids.size, E, BM)
    sorted_ids, eids, ntpp = oracle.moe_align(ids, E, BM, mp)
    ref = brute_force_align(ids.tolist(), E, BM, mp)
    assert (sorted_ids.tolist(), eids.tolist(), ntpp) == ref
    assert ntpp == 2 + 4            # expert 0: 1 slot -> 2; expert 2: 3 slots -> 4; 1, 3 empty
    assert eids[:3].tolist() == [0, 2, 2]


def check_invariants(ids: np.ndarray, E: int, BM: int):
    S = ids.size
    mp = oracle.max_padded_size(S, E, BM)
    sorted_ids, eids, ntpp = oracle.moe_align(ids, E, BM, mp)
    counts = np.bincount(ids[(ids >= 0) & (ids < E)], minlength=E)
    assert ntpp == int(((counts + BM - 1) // BM * BM).sum())
    assert ntpp <= mp
    body = sorted_ids[:ntpp]
    valid = body[body < S]
    assert np.array_equal(np.sort(valid), np.nonzero((ids >= 0) & (ids < E))[0])
    assert np.all(sorted_ids[ntpp:] == S)
    assert np.all(body[body >= S] == S)
    nb = ntpp // BM
    assert np.all(eids[nb:] == -1)
    assert np.all(np.diff(eids[:nb]) >= 0)
    for b in range(nb):
        blk = sorted_ids[b * BM:(b + 1) * BM]
        v = blk[blk < S]
        assert v.size > 0                          # no all-padding block
        assert np.all(ids[v] == eids[b])
        assert np.all(np.diff(v) > 0)              # stable (ascending slot) order
        n_valid = v.size
        assert np.all(blk[:n_valid] < S) and np.all(blk[n_valid:] == S)  # valid rows form a prefix
    return sorted_ids, eids, ntpp


@pytest.mark.parametrize("T,k,E,BM,kind", [(512, 8, 256, 128, "uniform"), (300, 2, 8, 64, "zipf"),
                                           (128, 8, 256, 16, "uniform"), (1000, 1, 1, 128, "one"),
                                           (257, 4, 64, 32, "hot")])
def test_align_invariants(T, k, E, BM, kind):
    rng = np.random.default_rng(T + E)
    if kind == "uniform":
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
    elif kind == "zipf":
        p = np.arange(1, E + 1, dtype=np.float64) ** -1.2
        ids = np.stack([rng.choice(E, k, replace=False, p=p / p.sum()) for _ in range(T)])
    elif kind == "one":
        ids = np.zeros((T, k), np.int64)
    else:  # half the slots on expert 3
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
        ids[: T // 2, 0] = 3
    check_invariants(ids.astype(np.int32).ravel(), E, BM)


def test_align_capacity_formula_and_error():
    # max_padded = S + E*(BM-1), capped at S*BM when S < E
    assert oracle.max_padded_size(65536, 256, 128) == 65536 + 256 * 127
    assert oracle.max_padded_size(3, 256, 16) == 48
    ids = np.arange(4, dtype=np.int32)   # 4 experts, one slot each -> ntpp = 4*BM
    with pytest.raises(ValueError):
        oracle.moe_align(ids, 4, 16, max_padded=63)
    _, _, ntpp = oracle.moe_align(ids, 4, 16, max_padded=64)
    assert ntpp == 64
