"""Scheme plugin of the MI355X expert path, in the reference's plugin shape.

The reference registers each benchmark scheme as a ``SchemeSpec`` plus a
builder ``(cfg, ctx, data, scheme_cfg) -> SchemeInstance``
(moe_bench/schemes/base.py:18-45, registry schemes/__init__.py:18-36), and its
worker calls ``instance.run()`` in the timed loop and compares the returned
[M_local, K] bf16 tensor with the golden (worker.py:57-61, 113-146).  This
module provides the same types and the scheme "m1" (MI355X-HIP-FP8): the
whole rank-local layer -- 1x128 quant, align, W13 GEMM with fused SiLU*up and
quant, W2 GEMM with routed weights, optional shared expert, top-k reduce -- on
one GPU over that GPU's full expert set, with every buffer built by the
builder so ``run()`` only enqueues kernels.

``cfg``, ``ctx``, ``data`` and ``scheme_cfg`` are read by attribute, exactly
as the reference's builders read them (schemes/vllm_tp.py:24-36,
schemes/runtime.py:13-39): ``scheme_cfg.tunables``; ``ctx.world_size``;
``data.hidden_local``, ``data.ckpt.w1/w2.{fp8,scale}``,
``data.ckpt.shared_w1/shared_w2`` (optional) and
``data.routing.topk_ids_full/topk_weights_full``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable

import torch

from . import ops
from ._lib import LIB_PATH


class SchemeConfigError(ValueError):
    """Scheme tunables or the run context do not fit the scheme (schemes/base.py:7-8)."""


@dataclass(frozen=True)
class TunableSpec:
    typ: type
    default: Any
    description: str


@dataclass(frozen=True)
class SchemeSpec:
    code: str
    name: str
    family: str
    parallel: str
    comm: str
    weight_dtype: str
    act_quant: str
    requires_nvshmem: bool
    tunables_schema: dict[str, TunableSpec]


@dataclass
class StageResult:
    output: Any
    stage_ms: dict[str, float]


@dataclass
class SchemeInstance:
    run: Callable[[], Any]
    run_staged: Callable[[], StageResult] | None
    diagnostics: dict[str, Any]
    close: Callable[[], None]


BuilderFn = Callable[[Any, Any, Any, Any], SchemeInstance]


def validate_tunables(spec: SchemeSpec, provided: dict[str, Any] | None) -> dict[str, Any]:
    """Defaults filled in; unknown keys and wrong types raise SchemeConfigError
    (the checks of schemes/base.py:48-62; bool is not accepted as int)."""
    provided = dict(provided or {})
    extra = sorted(set(provided) - set(spec.tunables_schema))
    if extra:
        raise SchemeConfigError(
            f"{spec.code} tunables {extra} violate schema: allowed keys are {sorted(spec.tunables_schema)}")
    values = {name: t.default for name, t in spec.tunables_schema.items()}
    values.update(provided)
    for name, value in values.items():
        want = spec.tunables_schema[name].typ
        ok = isinstance(value, bool) if want is bool else (isinstance(value, want) and not isinstance(value, bool))
        if not ok:
            raise SchemeConfigError(f"{spec.code}.{name}={value!r} violates schema: expected {want.__name__}")
    return values


def base_diagnostics(spec: SchemeSpec, tunables: dict[str, Any]) -> dict[str, Any]:
    return {"scheme": spec.code, "name": spec.name, "family": spec.family, "parallel": spec.parallel,
            "weight_dtype": spec.weight_dtype, "act_quant": spec.act_quant,
            "requires_nvshmem": spec.requires_nvshmem, "tunables": tunables}


SPEC = SchemeSpec(
    code="m1",
    name="MI355X-HIP-FP8",
    family="hip_native",
    parallel="EP/local",
    comm="none (1 GPU): quant -> align -> W13+SiLU+quant -> W2(+routed w) -> [+shared] -> top-k sum",
    weight_dtype="fp8",
    act_quant="group128",
    requires_nvshmem=False,
    tunables_schema={
        "block_m": TunableSpec(int, 0, "moe_align block size (16/32/64/128/256); 0 picks from rows per expert"),
        "n_chunks": TunableSpec(int, 1, "token chunks pipelined over n_streams HIP streams"),
        "n_streams": TunableSpec(int, 1, "HIP streams for the chunk pipeline (default priority)"),
        "n_chunks_gateup": TunableSpec(int, 0, "K chunks of W13 (the b schemes' structure); 0 = one pass"),
        "n_chunks_down": TunableSpec(int, 0, "N chunks of W2 (the b schemes' structure); 0 = one pass"),
        "exact_dot": TunableSpec(bool, False, "W13 dots exact on the bf16 matrix core (no FP8 in-group "
                                              "truncation; about twice the W13 matrix-core time)"),
    },
)

_STAGES = ("quant", "align", "scales", "w13", "w2", "shared", "reduce")


def build(cfg: Any, ctx: Any, data: Any, scheme_cfg: Any) -> SchemeInstance:
    """Builder of scheme m1: every allocation and all preprocessing happen here."""
    tunables = validate_tunables(SPEC, getattr(scheme_cfg, "tunables", None))
    world = int(getattr(ctx, "world_size", 1))
    if world != 1:
        raise SchemeConfigError(f"{SPEC.code} runs the rank-local layer on one GPU; world_size={world}")
    if data is None:
        raise RuntimeError("Scheme execution requires a DataBundle; build-only tests may pass data=None.")
    bm = tunables["block_m"]
    if bm not in (0, *ops.SUPPORTED_BLOCK_M):
        raise SchemeConfigError(f"{SPEC.code}.block_m={bm} must be 0 or one of {ops.SUPPORTED_BLOCK_M}")
    if tunables["n_chunks"] < 1 or tunables["n_streams"] < 1:
        raise SchemeConfigError(f"{SPEC.code}: n_chunks and n_streams must be >= 1")
    kn = (tunables["n_chunks_gateup"], tunables["n_chunks_down"])
    if min(kn) < 0 or (min(kn) == 0) != (max(kn) == 0):
        raise SchemeConfigError(f"{SPEC.code}: n_chunks_gateup and n_chunks_down are both 0 or both >= 1")
    if kn[0] > 0 and tunables["n_chunks"] > 1:
        raise SchemeConfigError(f"{SPEC.code}: n_chunks_gateup/n_chunks_down (K/N chunks) and n_chunks "
                                "(token chunks) do not combine")
    if kn[0] > 0 and tunables["exact_dot"]:
        raise SchemeConfigError(f"{SPEC.code}: exact_dot is a mode of the fused W13; the K-split W13 "
                                "(n_chunks_gateup) does not fuse")

    ckpt = data.ckpt
    w1, w1s = ckpt.w1.fp8.contiguous(), ckpt.w1.scale.float().contiguous()
    w2, w2s = ckpt.w2.fp8.contiguous(), ckpt.w2.scale.float().contiguous()
    hidden = data.hidden_local.to(torch.bfloat16).contiguous()
    ids2d = data.routing.topk_ids_full
    T, k = ids2d.shape
    if hidden.shape[0] != T:
        raise SchemeConfigError(f"hidden has {hidden.shape[0]} rows, routing has {T}")
    ids = ids2d.to(torch.int32).contiguous().view(-1)
    wts = data.routing.topk_weights_full.to(torch.float32).contiguous().view(-1)
    shared_w = None
    if getattr(ckpt, "shared_w1", None) is not None and getattr(ckpt, "shared_w2", None) is not None:
        shared_w = (ckpt.shared_w1.fp8.contiguous(), ckpt.shared_w1.scale.float().contiguous(),
                    ckpt.shared_w2.fp8.contiguous(), ckpt.shared_w2.scale.float().contiguous())

    block_m = bm or None
    if kn[0] > 0:
        # the b schemes' compute stream: K-split W13, N-split W2 (overlap_forward.py:252-321)
        shared = ops.SharedExpertRunner(*shared_w, max_tokens=T) if shared_w is not None else None
        runner = ops.SplitExpertsRunner(w1, w1s, w2, w2s, T, k, kn[0], kn[1], block_m, shared=shared)
        first = runner
    elif tunables["n_chunks"] > 1:
        runner = ops.ChunkedExpertsRunner(w1, w1s, w2, w2s, T, k, tunables["n_chunks"], tunables["n_streams"],
                                          block_m, shared_weights=shared_w)
        for r in runner.runners:
            r.exact_dot = tunables["exact_dot"]
        first = runner.runners[0]
    else:
        shared = ops.SharedExpertRunner(*shared_w, max_tokens=T) if shared_w is not None else None
        runner = ops.FusedExpertsRunner(w1, w1s, w2, w2s, T, k, block_m, shared=shared,
                                        exact_dot=tunables["exact_dot"])
        first = runner

    state: dict[str, Any] = {"runner": runner}

    def live():
        r = state.get("runner")
        if r is None:
            raise RuntimeError(f"scheme {SPEC.code} instance was closed")
        return r

    def run() -> torch.Tensor:
        return live().run(hidden, wts, ids)

    def run_staged() -> StageResult:
        runner = live()
        if not isinstance(runner, ops.FusedExpertsRunner):
            return StageResult(output=run(), stage_ms={})
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(_STAGES) + 1)]
        ev[0].record()
        runner.stage_quant(hidden)
        ev[1].record()
        runner.stage_align(ids)
        ev[2].record()
        runner.stage_scales()
        ev[3].record()
        runner.stage_w13()
        ev[4].record()
        runner.stage_w2(wts)
        ev[5].record()
        runner.stage_shared()
        ev[6].record()
        runner.stage_reduce()
        ev[7].record()
        ev[7].synchronize()
        return StageResult(output=runner.y,
                           stage_ms={n: ev[i].elapsed_time(ev[i + 1]) for i, n in enumerate(_STAGES)})

    diag = base_diagnostics(SPEC, tunables)
    diag.update({"block_size_m": first.BM, "max_padded": first.align.max_padded,
                 "shared_expert": shared_w is not None, "library": str(LIB_PATH)})
    del runner, first

    def close() -> None:
        state["runner"] = None

    return SchemeInstance(run=run, run_staged=run_staged, diagnostics=diag, close=close)


REGISTRY: dict[str, tuple[SchemeSpec, BuilderFn]] = {SPEC.code: (SPEC, build)}


def build_scheme(cfg: Any, ctx: Any, data: Any, scheme_cfg: Any) -> SchemeInstance:
    """Look up scheme_cfg.code and build it (schemes/__init__.py:32-36)."""
    try:
        _spec, builder = REGISTRY[scheme_cfg.code]
    except KeyError as exc:
        raise SchemeConfigError(f"scheme {scheme_cfg.code!r} is not registered") from exc
    return builder(cfg, ctx, data, scheme_cfg)
