"""ctypes binding of libmoe_mi355x.so, the C ABI declared in include/moe_mi355x.h.

The library is built in-tree (``td_benchmark_amd/csrc/Makefile``) and is the
only compute path: if it is missing, every op raises -- there is no CPU or
PyTorch fallback.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libmoe_mi355x.so"
CSRC_DIR = PKG_DIR / "csrc"

STATUS = {
    0: "MOE_OK",
    -1: "MOE_ERR_NULL_POINTER",
    -2: "MOE_ERR_BAD_SHAPE",
    -3: "MOE_ERR_BAD_BLOCK_SIZE",
    -4: "MOE_ERR_CAPACITY",
    -5: "MOE_ERR_BAD_TOPK",
    -6: "MOE_ERR_BAD_EXPERTS",
    -100: "MOE_ERR_LAUNCH",
}

_P = ctypes.c_void_p
_F = ctypes.POINTER(ctypes.c_float)
_I32P = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32

# name -> (restype, argtypes); must match include/moe_mi355x.h
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "moe_quant_group128": (ctypes.c_int, [_P, _i64, _i64, _P, _P, _P]),
    "moe_quant_group128_padded": (ctypes.c_int, [_P, _i64, _i64, _P, _i64, _P, _P]),
    "moe_quant_block128": (ctypes.c_int, [_P, _i64, _i64, _i64, _P, _P, _P]),
    "moe_align_max_padded": (ctypes.c_int64, [_i64, _i32, _i32]),
    "moe_align_workspace_bytes": (ctypes.c_int64, [_i64, _i32]),
    "moe_align_block_size": (ctypes.c_int, [_P, _i64, _i32, _i32, _P, _P, _P, _i64, _P, _P]),
    "moe_align_block_size_mapped": (ctypes.c_int, [_P, _i64, _i32, _i32, _P, _P, _P, _P, _i64, _P, _P]),
    "moe_align_block_size_noalloc": (ctypes.c_int, [_P, _i64, _i32, _i32, _P, _P, _P, _i64, _P]),
    "moe_grouped_gemm": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _i64, _i32, _i32, _i64,
                                        _i64, _i32, _i32, _i64, _P, _P]),
    "moe_grouped_gemm_ordered": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _i64, _i32, _i32,
                                                _i64, _i64, _i32, _i32, _i64, _i32, _P, _P]),
    "moe_grouped_gemm_tiled": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _i64, _i32, _i32,
                                              _i64, _i64, _i32, _i32, _i64, _i32, _i32, _P, _P]),
    "moe_grouped_gemm_n_split": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _i64, _i32, _i32, _i64,
                                                _i64, _i64, _i64, _i32, _i32, _i64, _P, _P]),
    "moe_grouped_gemm_k_split": (ctypes.c_int, [_P, _P, _i64, _i64, _P, _P, _P, _P, _P, _P, _i64, _i32,
                                                _i32, _i64, _i64, _i64, _i64, _i32, _i32, _i64, _i32, _P,
                                                _P]),
    "moe_silu_mul_quant_group128": (ctypes.c_int, [_P, _i64, _i64, _P, _P, _P]),
    "moe_reduce_topk_add": (ctypes.c_int, [_P, _P, _i64, _i32, _i64, _P, _P]),
    "moe_fp8_dequant_sum": (ctypes.c_int, [_P, _P, _i64, _i64, _i64, _i64, _P, _i64, _P]),
    "moe_gather_scales_by_position": (ctypes.c_int, [_P, _i64, _i64, _P, _P, _i64, _i32, _i64, _P, _P]),
    "moe_gemm_w13_silu_quant_pos": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _i64, _i32, _i64, _i64, _i32, _i32,
                                                   _i64, _i32, _P, _P, _P]),
    "moe_grouped_gemm_pos": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _i64, _i64, _i64, _i32, _i32, _i64, _i32,
                                            _P, _P]),
    "moe_gemm_w13_silu_quant": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _i64, _i32, _i64,
                                               _i64, _i32, _i32, _i64, _P, _P, _P]),
    "moe_gemm_w13_silu_quant_tiled": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _i64, _i32, _i64,
                                                     _i64, _i32, _i32, _i64, _i32, _P, _P, _P]),
    "moe_gemm_w13_silu_quant_exact": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _i64, _i32, _i64,
                                                     _i64, _i32, _i32, _i64, _i32, _i32, _P, _P, _P]),
    "moe_silu_and_mul": (ctypes.c_int, [_P, _i64, _i64, _P, _P]),
    "moe_reduce_topk": (ctypes.c_int, [_P, _i64, _i32, _i64, _P, _P]),
}

_lib: ctypes.CDLL | None = None


class MoeKernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


def build(force: bool = True) -> Path:
    """Compile libmoe_mi355x.so for gfx950 with hipcc (no GPU needed)."""
    args = ["make", "-s", "-C", str(CSRC_DIR)]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    """Load the native library; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"td_benchmark_amd native library is missing ({LIB_PATH}); build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` -- there is no fallback path"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(status: int, op: str) -> None:
    if status != 0:
        raise MoeKernelError(f"{op} failed with {STATUS.get(status, status)}")
