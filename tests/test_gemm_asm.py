"""CPU: properties of the grouped GEMM's compiled gfx950 code that its source
relies on, checked on the AMD assembly of this build (hipcc -S, device side
only; no GPU needed).

* M0 belongs to the direct-to-LDS loads.  The loads are issued from inline
  asm that writes M0 (the LDS destination) and names it clobbered; the
  compiler reserves M0 and does not promise to honour that clobber.  The
  kernels are correct only if no compiler-generated instruction reads or
  writes M0: every M0 reference in the code must be one of the asm blocks'
  own `s_mov_b32 m0, <sgpr>`, followed by `s_nop 0` and the load.
"""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "td_benchmark_amd" / "csrc"
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def gemm_asm(tmp_path_factory) -> str:
    if not Path(HIPCC).exists() or shutil.which("make") is None:
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "gemm.s"
    # the device flags of csrc/Makefile
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++20", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form=1", f"-I{ROOT / 'include'}",
           "--cuda-device-only", "-S", "-o", str(out), str(CSRC / "gemm.hip")]
    subprocess.run(cmd, check=True, capture_output=True)
    return out.read_text()


def test_m0_is_written_only_by_the_direct_to_lds_loads(gemm_asm):
    lines = [ln.strip() for ln in gemm_asm.splitlines()]
    code = [ln for ln in lines if ln and not ln.startswith((";", ".", "//")) and not ln.endswith(":")]
    uses = [i for i, ln in enumerate(code) if re.search(r"\bm0\b", ln)]
    assert uses, "no M0 reference found: the direct-to-LDS loads are missing"
    kernels = len(re.findall(r"^\s*\.amdhsa_kernel\s+\S*grouped_gemm_kernel", gemm_asm, flags=re.M))
    assert kernels >= 10, f"expected the grouped GEMM instantiations, found {kernels}"
    bad = []
    for i in uses:
        ok = (re.fullmatch(r"s_mov_b32 m0, (s\d+|vcc_lo|vcc_hi)", code[i]) is not None
              and i + 2 < len(code) and code[i + 1] == "s_nop 0"
              and re.match(r"global_load_lds_dword(x4)? v\d+, s\[\d+:\d+\]( nt)?$", code[i + 2]) is not None)
        if not ok:
            bad.append(" | ".join(code[i:i + 3]))
    assert not bad, f"{len(bad)} M0 references outside the asm load blocks, e.g. {bad[:3]}"
