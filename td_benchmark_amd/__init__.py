"""MI355X-native (gfx950) rank-local FP8 MoE expert path.

Hand-written HIP kernels (``csrc/``) behind a C ABI (``include/moe_mi355x.h``,
``libmoe_mi355x.so``), torch-facing operators mirroring the vLLM calls of the
reference's ``fused_experts`` decomposition (``ops``), and a scheme plugin
(``schemes``) for the reference's benchmark harness API.
"""
from ._lib import LIB_PATH, MoeKernelError, build, lib

__all__ = ["LIB_PATH", "MoeKernelError", "build", "lib"]
