"""The C ABI without a GPU: the library loads, exports every entry point the
header declares with the argument count the ctypes binding uses, its status
codes match the header, and argument validation rejects bad calls before any
device work (no kernel is launched here)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from td_benchmark_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "moe_mi355x.h"


def header_decls() -> dict[str, int]:
    """name -> parameter count for every function the header declares."""
    text = re.sub(r"/\*.*?\*/|//[^\n]*", "", HEADER.read_text(), flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:int|int64_t)\s+(moe_\w+)\s*\(([^)]*)\)\s*;", text):
        args = [a for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        decls[m.group(1)] = len(args)
    return decls


@pytest.fixture(scope="module")
def L():
    if not _lib.LIB_PATH.exists():
        pytest.skip("native library not built")
    return _lib.lib()


def test_header_and_binding_agree():
    decls = header_decls()
    assert decls, "no declarations parsed"
    assert set(decls) == set(_lib.SIGNATURES)
    for name, n in decls.items():
        assert len(_lib.SIGNATURES[name][1]) == n, name


def test_library_exports_every_declared_symbol(L):
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in header_decls():
        assert hasattr(handle, name), name


def test_status_codes_match_header():
    text = HEADER.read_text()
    codes = {m.group(1): int(m.group(2)) for m in re.finditer(r"#define\s+(MOE_\w+)\s+\(?(-?\d+)\)?", text)}
    for value, name in _lib.STATUS.items():
        assert codes[name] == value


def test_host_only_sizing_functions(L):
    assert L.moe_align_max_padded(65536, 256, 128) == 65536 + 256 * 127
    assert L.moe_align_max_padded(3, 256, 16) == 48
    assert L.moe_align_max_padded(10, 4, 0) < 0
    assert L.moe_align_workspace_bytes(65536, 256) >= 4 * 65536
    assert L.moe_align_workspace_bytes(10, 0) < 0


def test_validation_rejects_bad_arguments_without_device_work(L):
    E = {name: code for code, name in _lib.STATUS.items()}
    buf = (ctypes.c_int32 * 64)()          # host memory: only ever passed to a rejected call
    dummy = ctypes.cast(buf, ctypes.c_void_p)
    # null pointers on a non-empty problem
    assert L.moe_quant_group128(None, 4, 128, None, None, None) == E["MOE_ERR_NULL_POINTER"]
    assert L.moe_grouped_gemm(None, None, None, None, None, None, None, None, 10, 2, 0, 256, 256,
                              4, 64, 100, None, None) == E["MOE_ERR_NULL_POINTER"]
    # shapes that are not multiples of 128, bad block sizes, bad top-k, bad expert counts
    odd = ctypes.c_void_p(ctypes.addressof(buf) + 1)  # a bf16 row start that is not 2-byte aligned
    assert L.moe_quant_group128(odd, 4, 100, dummy, dummy, None) == E["MOE_ERR_BAD_SHAPE"]
    assert L.moe_quant_group128_padded(dummy, 4, 100, dummy, 100, dummy, None) == E["MOE_ERR_BAD_SHAPE"]
    assert L.moe_quant_group128_padded(odd, 4, 100, dummy, 128, dummy, None) == E["MOE_ERR_BAD_SHAPE"]
    assert L.moe_quant_group128_padded(None, 4, 100, None, 128, None, None) == E["MOE_ERR_NULL_POINTER"]
    assert L.moe_quant_group128(None, -1, 128, None, None, None) == E["MOE_ERR_BAD_SHAPE"]
    assert L.moe_grouped_gemm(None, None, None, None, None, None, None, None, 10, 2, 0, 200, 256,
                              4, 64, 100, None, None) == E["MOE_ERR_BAD_SHAPE"]
    assert L.moe_grouped_gemm(None, None, None, None, None, None, None, None, 10, 2, 0, 256, 256,
                              4, 48, 100, None, None) == E["MOE_ERR_BAD_BLOCK_SIZE"]
    assert L.moe_grouped_gemm(None, None, None, None, None, None, None, None, 10, 0, 0, 256, 256,
                              4, 64, 100, None, None) == E["MOE_ERR_BAD_TOPK"]
    assert L.moe_gemm_w13_silu_quant(None, None, None, None, None, None, None, 10, 2, 256, 256,
                                     0, 64, 100, None, None, None) == E["MOE_ERR_BAD_EXPERTS"]
    assert L.moe_gemm_w13_silu_quant_exact(None, None, None, None, None, None, None, 10, 2, 256, 256, 4, 64, 100,
                                           0, 1, None, None, None) == E["MOE_ERR_NULL_POINTER"]
    assert L.moe_gemm_w13_silu_quant_exact(None, None, None, None, None, None, None, 10, 2, 256, 256, 4, 48, 100,
                                           0, 0, None, None, None) == E["MOE_ERR_BAD_BLOCK_SIZE"]
    assert L.moe_gemm_w13_silu_quant_exact(None, None, None, None, None, None, None, 10, 2, 200, 256, 4, 64, 100,
                                           0, 0, None, None, None) == E["MOE_ERR_BAD_SHAPE"]
    assert L.moe_align_block_size(None, 10, 4, 16, None, None, None, 100, None, None) == \
        E["MOE_ERR_NULL_POINTER"]
    assert L.moe_align_block_size(dummy, 10, 4, 16, dummy, dummy, dummy, 10, dummy, None) == \
        E["MOE_ERR_CAPACITY"]
    assert L.moe_align_block_size(dummy, 10, 2000, 16, dummy, dummy, dummy, 10 ** 6, dummy, None) == \
        E["MOE_ERR_BAD_EXPERTS"]
    assert L.moe_reduce_topk(None, 4, 0, 128, None, None) == E["MOE_ERR_BAD_TOPK"]
    assert L.moe_silu_and_mul(None, 4, 12, None, None) == E["MOE_ERR_NULL_POINTER"]
    # empty problems are a no-op success
    assert L.moe_reduce_topk(None, 0, 8, 128, None, None) == 0
    assert L.moe_quant_group128(None, 0, 128, None, None, None) == 0


def test_chunked_and_mapped_entry_points_validate_arguments(L):
    E = {name: code for code, name in _lib.STATUS.items()}
    buf = (ctypes.c_int32 * 64)()          # host memory: only ever passed to a rejected call
    d = ctypes.cast(buf, ctypes.c_void_p)
    # N-split: the window must lie inside full_N and start on a 128 boundary
    args = [d, d, d, d, d, d, d, None, 10, 2, 0]
    assert L.moe_grouped_gemm_n_split(*args, 512, 384, 256, 256, 4, 64, 100, d, None) == E["MOE_ERR_BAD_SHAPE"]
    assert L.moe_grouped_gemm_n_split(*args, 512, 64, 128, 256, 4, 64, 100, d, None) == E["MOE_ERR_BAD_SHAPE"]
    assert L.moe_grouped_gemm_n_split(None, None, None, None, None, None, None, None, 10, 2, 0, 512, 128, 128,
                                      256, 4, 64, 100, None, None) == E["MOE_ERR_NULL_POINTER"]
    assert L.moe_grouped_gemm_n_split(*args, 512, 128, 128, 256, 4, 48, 100, d, None) == E["MOE_ERR_BAD_BLOCK_SIZE"]
    # K-split: the K window must lie inside both A and B
    kargs = [d, d, 512, 0, d, d, d, d, d, None, 10, 2, 0, 256]
    assert L.moe_grouped_gemm_k_split(*kargs, 512, 384, 256, 4, 64, 100, 1, d, None) == E["MOE_ERR_BAD_SHAPE"]
    assert L.moe_grouped_gemm_k_split(d, d, 256, 128, d, d, d, d, d, None, 10, 2, 0, 256, 512, 0, 256, 4, 64,
                                      100, 1, d, None) == E["MOE_ERR_BAD_SHAPE"]
    assert L.moe_grouped_gemm_k_split(*kargs, 512, 64, 128, 4, 64, 100, 1, d, None) == E["MOE_ERR_BAD_SHAPE"]
    # mapped align needs its map
    assert L.moe_align_block_size_mapped(d, 10, 4, 16, None, d, d, d, 100, d, None) == E["MOE_ERR_NULL_POINTER"]
    assert L.moe_align_block_size_mapped(d, 10, 4, 16, d, d, d, d, 10, d, None) == E["MOE_ERR_CAPACITY"]
    # tile order out of range
    assert L.moe_grouped_gemm_ordered(d, d, d, d, d, d, d, None, 10, 2, 0, 256, 256, 4, 64, 100, 3, d,
                                      None) == E["MOE_ERR_BAD_SHAPE"]


def test_noalloc_align_checks_its_limit_before_any_device_call(L):
    """The allocation-free align rejects a problem whose workspace exceeds its
    static array (MOE_ALIGN_NOALLOC_SCRATCH_BYTES), bad sizes, expert counts,
    block sizes, null pointers and short outputs before it touches a device,
    so these calls are safe without a GPU."""
    text = HEADER.read_text()
    limit = int(eval(re.search(r"#define\s+MOE_ALIGN_NOALLOC_SCRATCH_BYTES\s+(\([^)]*\))", text).group(1)))
    assert limit == 4 * 1024 * 1024
    S, E = 1 << 20, 1024
    assert L.moe_align_workspace_bytes(S, E) > limit
    p = ctypes.c_void_p(16)
    assert _lib.STATUS[L.moe_align_block_size_noalloc(p, S, E, 128, p, p, p, 1 << 30, None)] == "MOE_ERR_CAPACITY"
    assert _lib.STATUS[L.moe_align_block_size_noalloc(p, -1, E, 128, p, p, p, 1 << 30, None)] == "MOE_ERR_BAD_SHAPE"
    assert _lib.STATUS[L.moe_align_block_size_noalloc(p, 64, 0, 128, p, p, p, 1 << 30, None)] == "MOE_ERR_BAD_EXPERTS"
    # the remaining argument checks also run before the symbol lookup
    assert _lib.STATUS[L.moe_align_block_size_noalloc(p, 64, 2000, 128, p, p, p, 1 << 30, None)] == \
        "MOE_ERR_BAD_EXPERTS"
    assert _lib.STATUS[L.moe_align_block_size_noalloc(p, 64, 8, 48, p, p, p, 1 << 30, None)] == \
        "MOE_ERR_BAD_BLOCK_SIZE"
    for nulls in ((None, p, p, p), (p, None, p, p), (p, p, None, p), (p, p, p, None)):
        assert _lib.STATUS[L.moe_align_block_size_noalloc(nulls[0], 64, 8, 16, nulls[1], nulls[2], nulls[3],
                                                          1 << 20, None)] == "MOE_ERR_NULL_POINTER"
    assert _lib.STATUS[L.moe_align_block_size_noalloc(p, 64, 8, 16, p, p, p, 64, None)] == "MOE_ERR_CAPACITY"

