"""GPU: the operators reject buffers whose sizes disagree with each other.

The C ABI receives pointers and sizes only, so a scale tensor with too few
rows, an output of the wrong shape or routing tensors shorter than the sizes
say would be read or written out of bounds on the device.  The Python mirror
checks dtype and shape first and raises (TypeError / ValueError) before any
kernel is launched; each case below changes exactly one operand of a valid
call."""
from __future__ import annotations

import pytest

from moe_cases import make_case, to_gpu

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def case():
    c = make_case(40, 256, 256, 4, 2, 16, seed=5)
    return c, to_gpu(c)


def _routing(c, g):
    from td_benchmark_amd import ops
    return ops.moe_align_block_size(g["topk_ids"], c.BM, c.E)


def test_quant_outputs_must_match_input(case):
    from td_benchmark_amd import ops
    c, g = case
    x = g["x"]
    with pytest.raises(ValueError, match="out_q must have shape"):
        ops.per_token_group_quant_fp8(x, out_q=torch.empty((c.T, 128), dtype=ops.FP8, device=x.device))
    with pytest.raises(ValueError, match="out_s must have shape"):
        ops.per_token_group_quant_fp8(x, out_s=torch.empty((c.T - 1, 2), device=x.device))
    with pytest.raises(TypeError, match="x must be"):
        ops.per_token_group_quant_fp8(x.float())
    w = torch.zeros((2, 256, 256), device=x.device)
    with pytest.raises(ValueError, match="out_s must have shape"):
        ops.quantize_block128(w, out_s=torch.empty((2, 2, 1), device=x.device))


def test_grouped_gemm_checks_every_operand(case):
    from td_benchmark_amd import ops
    c, g = case
    q, s = ops.per_token_group_quant_fp8(g["x"])
    sorted_ids, eids, ntpp = _routing(c, g)
    C = torch.empty((c.T, c.k, 2 * c.I), dtype=torch.bfloat16, device=q.device)
    good = dict(A=q, B=g["w13"], C=C, A_scale=s, B_scale=g["w13_s"], B_zp=None, topk_weights=g["topk_w"],
                sorted_token_ids=sorted_ids, expert_ids=eids, num_tokens_post_padded=ntpp,
                mul_routed_weight=True, top_k=c.k, config={"BLOCK_SIZE_M": c.BM})
    ops.dispatch_fused_moe_kernel(**good)  # the valid call runs
    torch.cuda.synchronize()
    bad = [
        (TypeError, "A must be", dict(A=q.view(torch.uint8))),
        (ValueError, "A has", dict(A=q[: c.T - 1])),
        (ValueError, "A_scale must have shape", dict(A_scale=s[:, :1].contiguous())),
        (ValueError, "B_scale must have shape", dict(B_scale=g["w13_s"][:, :1].contiguous())),
        (ValueError, "whole number", dict(C=C.view(-1)[:-8])),
        (ValueError, "topk_weights has", dict(topk_weights=g["topk_w"].view(-1)[:-1])),
        (ValueError, "expert_ids has", dict(expert_ids=eids[:-1])),
        (TypeError, "sorted_token_ids must be", dict(sorted_token_ids=sorted_ids.long())),
    ]
    for exc, msg, change in bad:
        with pytest.raises(exc, match=msg):
            ops.dispatch_fused_moe_kernel(**{**good, **change})


def test_fused_w13_and_reduce_check_sizes(case):
    from td_benchmark_amd import ops
    c, g = case
    q, s = ops.per_token_group_quant_fp8(g["x"])
    sorted_ids, eids, ntpp = _routing(c, g)
    mp = sorted_ids.numel()
    with pytest.raises(ValueError, match="hq must have shape"):
        ops.gemm_w13_silu_quant(q, s, g["w13"], g["w13_s"], sorted_ids, eids, ntpp, c.S, c.k, c.BM,
                                hq=torch.empty((mp - 1, c.I), dtype=ops.FP8, device=q.device))
    with pytest.raises(ValueError, match="A has"):
        ops.gemm_w13_silu_quant(q[:, :128].contiguous(), s[:, :1].contiguous(), g["w13"], g["w13_s"],
                                sorted_ids, eids, ntpp, c.S, c.k, c.BM)
    out = torch.empty((c.T, c.H), dtype=torch.bfloat16, device=q.device)
    with pytest.raises(ValueError, match="D has"):
        ops.moe_sum(torch.empty((c.S - 1, c.H), dtype=torch.bfloat16, device=q.device), out, c.k)
    with pytest.raises(ValueError, match="out must have shape"):
        ops.silu_and_mul(torch.empty((4, c.I - 128), dtype=torch.bfloat16, device=q.device),
                         torch.empty((4, 2 * c.I), dtype=torch.bfloat16, device=q.device))


def test_runners_check_weights_and_inputs(case):
    from td_benchmark_amd import ops
    c, g = case
    with pytest.raises(ValueError, match="w13_scale must have shape"):
        ops.FusedExpertsRunner(g["w13"], g["w13_s"][:, :, :1].contiguous(), g["w2"], g["w2_s"], c.T, c.k, c.BM)
    with pytest.raises(ValueError, match="w2_scale must have shape"):
        ops.FusedExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"][:1].contiguous(), c.T, c.k, c.BM)
    r = ops.FusedExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], c.T, c.k, c.BM)
    with pytest.raises(ValueError, match="topk_weights has"):
        r.run(g["x"], g["topk_w"].view(-1)[:-1], g["topk_ids"].view(-1))
    sh = ops.SharedExpertRunner(g["w13"][:1].contiguous(), g["w13_s"][:1].contiguous(),
                                g["w2"][:1].contiguous(), g["w2_s"][:1].contiguous(), max_tokens=c.T)
    with pytest.raises(ValueError, match="x must be"):
        sh(torch.empty((c.T, 128), dtype=torch.bfloat16, device=g["x"].device))
    q, s = ops.per_token_group_quant_fp8(g["x"])
    with pytest.raises(ValueError, match="input_scale must have shape"):
        sh(q, s[:, :1].contiguous())
    torch.cuda.synchronize()


def test_launch_stream_is_torchs_current_stream():
    """Every launch goes to torch's current stream: the raw handle the ops read
    equals torch.cuda.current_stream(), also inside a stream context."""
    from td_benchmark_amd import ops

    print("case: launch stream", flush=True)
    def raw():  # the null (default) stream's handle is 0; ctypes reads it back as None
        return ops._stream().value or 0

    assert raw() == torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert raw() == side.cuda_stream == torch.cuda.current_stream().cuda_stream != 0
    assert raw() == torch.cuda.current_stream().cuda_stream
