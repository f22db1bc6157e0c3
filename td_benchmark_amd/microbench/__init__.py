"""Microbench counterparts of the reference's hot-path sweeps
(microbench/mb_moe_align.py, mb_quant_kernels.py, mb_group_gemm.py,
mb_tile_order_groupgemm.py, mb_dispatch_prep.py, and the compute-stream half
of mb_chunk_overlap.py), measuring this library's kernels.  Run e.g. ``python -m td_benchmark_amd.microbench.mb_moe_align``."""

SCRIPTS = ("mb_moe_align", "mb_quant_kernels", "mb_group_gemm", "mb_tile_order_groupgemm", "mb_dispatch_prep",
           "mb_chunk_overlap")
