"""ctypes binding of tests/libmoe_probe.so (tests/csrc/moe_probe.h): the
test-only matrix-core probes.  Built by tests/csrc/Makefile (and by
__graft_entry__.build())."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libmoe_probe.so"

_P = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32

SIGNATURES = {
    "moe_probe_mfma_dot": (ctypes.c_int, [_P, _P, _P, _i64, _i32, _P]),
    "moe_probe_block_gemm": (ctypes.c_int, [_P, _P, _P, _P, _i64, _i64, _i64, _i32, _P, _P]),
    "moe_probe_mfma_rate": (ctypes.c_int, [_i64, _i32, _i32, _P, _P]),
    "moe_probe_fp8_to_bf16": (ctypes.c_int, [_P, _i64, _P, _P]),
}

# dot forms of moe_probe.h
FORM_K128 = 0          # one 16x16x128 f8f6f4 (the grouped GEMM's form)
FORM_K32_CHAINED = 1   # four 16x16x32, accumulator chained through the instruction
FORM_K32_FP32 = 2      # four 16x16x32 from zero, fp32 adds
FORM_K128_QUARTERS = 3 # four 16x16x128 with one K quarter each, fp32 adds
FORM_BF16 = 4          # codes converted to bf16, four 16x16x32 bf16 MFMAs chained
FORM_BF16_REF_CHAIN = 5  # form 4 with the reference's scale chain (block GEMM only)
FP8_FORMS = {FORM_K128: "16x16x128", FORM_K32_CHAINED: "4x16x16x32 chained",
             FORM_K32_FP32: "4x16x16x32 + fp32 adds", FORM_K128_QUARTERS: "4x16x16x128 quarters + fp32 adds"}
FORMS = {**FP8_FORMS, FORM_BF16: "bf16 4x16x16x32"}

_lib: ctypes.CDLL | None = None


def build(force: bool = True) -> Path:
    args = ["make", "-s", "-C", str(HERE / "csrc")]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"probe library missing ({LIB_PATH}); build it with __graft_entry__.build()")
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype, fn.argtypes = res, args
        _lib = h
    return _lib


def check(status: int, op: str) -> None:
    if status != 0:
        raise RuntimeError(f"{op} failed with status {status}")
