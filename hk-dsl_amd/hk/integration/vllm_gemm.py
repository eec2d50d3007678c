"""vLLM's unquantized linear layers on this build's gfx950 GEMMs, where a measured table
says they are faster.

The surface kept from the reference (python/hk/integration/vllm_gemm.py:1-693):

* the op `torch.ops.hk_vllm.linear(Tensor x, Tensor weight, Tensor? bias=None) -> Tensor`,
  y = x @ weight.T (+ bias) for x (..., K), weight (N, K); opaque to torch.compile (its
  fake gives the output's shape), launched on torch's current stream, graph-safe;
* `route_for(m, n, k, *, bf16, bias, contiguous_weight)` -> "hk" (the tile / split-K
  GEMMs), "hk_decode" (the decode kernel) or "fallback" (vLLM's own GEMM, F.linear where
  vLLM has none), read from hk/tuned/routes_vllm_linear_<arch>.json (`$HK_VLLM_ROUTES`
  overrides it); a shape the table does not hold, or an M in a gap between two measured
  runs, takes the fallback;
* `apply()` rebinds vLLM's `dispatch_unquantized_gemm` in every vllm module that bound
  it, and gives the patched engine a compile cache of its own; `revert()` puts it back;
  `decide_layers(model)` decides every linear layer once, at load.

How it is put together here. `Router` owns the table and a memo of per-call-signature
`Plan`s (path plus a launch); replacing the table starts a new generation, which drops
the memo and invalidates the decision kept on each layer. A layer is decided from its
weight alone -- whether the table routes its (N, K) at any M -- and a layer it never
routes keeps vLLM's GEMM with no wrapper in its path. Nothing here writes state while
torch.compile traces (vLLM compiles the forward whole and refuses a graph that replays
a write): the dispatch stand-in keeps no cache, and a layer decision made while
tracing is used, not stored.

One difference from the reference: a call with a bias can take the hk paths, the bias
added in the GEMM's registers (the fused epilogue); the reference sends bias calls to the
fallback (:173). `BIAS_FUSED = False` restores that.
"""

from __future__ import annotations

import functools
import sys
from collections import Counter
from typing import Callable, Dict, NamedTuple, Optional

from . import engine

#: Modules whose bindings of vLLM's dispatch function `apply` replaces.
PREFIXES = ("vllm",)
ROUTES_ENV = "HK_VLLM_ROUTES"
#: Whether a bias rides the hk paths as a fused epilogue (True) or falls back.
BIAS_FUSED = True
#: What a table's runs may name.
RUN_PATHS = ("hk", "hk_decode", "fallback")
#: Signatures memoised before deciding afresh on every call (a serving engine's prefill
#: has a new M per batch; the memo is a cache, not a record).
PLAN_CAP = 4096


def _fake(x, weight, bias=None):
    return x.new_empty((*x.shape[:-1], weight.shape[0]))


PATCH = engine.Op("hk_vllm::linear",
                  "linear(Tensor x, Tensor weight, Tensor? bias=None) -> Tensor",
                  _fake, paths=RUN_PATHS, graph="safe")
#: Calls by path (eager); `PATCH.captured` counts calls made while capturing a graph.
STATS = PATCH.stats
#: Layers left on vLLM's GEMM when decided, by reason.
UNROUTED: "Counter[str]" = Counter()


class Plan(NamedTuple):
    path: str
    run: Optional[Callable]     # (x2 (M, K), weight, bias) -> y (M, N)


_FALLBACK_PLAN = Plan("fallback", None)


class Router:
    """The table in force and what was decided from it."""

    def __init__(self):
        self._table: Optional[engine.RouteTable] = None
        self._loaded = False
        self.generation = 0
        self.plans: Dict[tuple, Plan] = {}

    def table(self) -> Optional[engine.RouteTable]:
        if not self._loaded:
            from ..target import current_arch  # noqa: PLC0415

            self._table = engine.shipped_table("vllm_linear", current_arch(), ROUTES_ENV)
            self._loaded = True
        return self._table

    def replace(self, table: Optional[engine.RouteTable], *, loaded: bool) -> None:
        self._table, self._loaded = table, loaded
        self.plans.clear()
        self.generation += 1


ROUTER = Router()


def routes() -> Optional[engine.RouteTable]:
    """The routing table for this process's arch, loaded on first use, or None."""
    return ROUTER.table()


def set_routes(table: Optional[engine.RouteTable]) -> None:
    """Route by `table` from now on; None reloads the shipped one on next use. Graphs
    captured before keep the launches they captured."""
    if any(PATCH.captured.values()):
        import warnings  # noqa: PLC0415

        warnings.warn("hk_vllm::linear: the routes changed after a CUDA graph captured calls "
                      "of the op; those graphs replay the launches of the old routes",
                      stacklevel=2)
    ROUTER.replace(table, loaded=table is not None)


# ---------------------------------------------------------------- deciding a call


def _hk_takes(path: str, m: int, n: int, k: int) -> bool:
    """Whether the kernel behind `path` takes an M x N x K call at all."""
    from ..ops import gemm_cdna  # noqa: PLC0415

    if path == "hk":
        return (n % gemm_cdna.BLOCK_N_MIN == 0 and k % gemm_cdna.K_STEP == 0
                and 2 * max(m, n) * k < gemm_cdna.OPERAND_BYTES_MAX)
    if path == "hk_decode":
        return gemm_cdna.fits("decode", m, n, k)
    return False


def route_for(m: int, n: int, k: int, *, bf16: bool = True, bias: bool = False,
              contiguous_weight: bool = True) -> str:
    """Where y = x @ W.T (+ bias), x (m, k), W (n, k), goes: "hk", "hk_decode" or
    "fallback". The table names the fastest measured path; it is taken only if its kernel
    takes the call."""
    if m < 1 or not bf16 or not contiguous_weight:
        return "fallback"
    if bias and not BIAS_FUSED:
        return "fallback"
    table = routes()
    if table is None:
        return "fallback"
    path = table.lookup(m, n, k)
    if path not in ("hk", "hk_decode") or not _hk_takes(path, m, n, k):
        return "fallback"
    return path


def route(m: int, n: int, k: int, **how) -> bool:
    """Whether the call goes to the tile GEMMs."""
    return route_for(m, n, k, **how) == "hk"


def route_decode(m: int, n: int, k: int, **how) -> bool:
    """Whether the call goes to the decode kernel."""
    return route_for(m, n, k, **how) == "hk_decode"


def _schedule(path: str, m: int, n: int, k: int) -> str:
    """The template's schedule for a routed path: the decode kernel for "hk_decode"; for
    "hk" the GEMM route's tile candidate, or -- where that route would pick the decode
    kernel, which the table measured as another path -- the tile rule's choice."""
    from ..ops import gemm_cdna  # noqa: PLC0415

    if path == "hk_decode":
        return "decode"
    name = gemm_cdna.route(m, n, k)
    if gemm_cdna.CANDIDATES[name]["kernel"] != "tile":
        name = gemm_cdna.rule(max(m, 33), n, k)      # the rule's tiles start at M = 33
    return name


def launch_for(path: str, m: int, n: int, k: int, has_bias: bool) -> Callable:
    """The launch of a routed path: (x2, weight, bias) -> y, y allocated by the template
    on the caller's stream."""
    from ..templates import gemm as T  # noqa: PLC0415

    sched = _schedule(path, m, n, k)
    if has_bias:
        return functools.partial(_with_bias, T.gemm, sched)
    return functools.partial(_plain, T.gemm, sched)


def _plain(gemm, sched, x2, weight, bias):
    return gemm(x2, weight, schedule=sched)


def _with_bias(gemm, sched, x2, weight, bias):
    return gemm(x2, weight, epilogue=gemm.bias, schedule=sched, bias=bias)


def _weight_ok(weight) -> bool:
    """A weight the kernels read in place: contiguous (N, K), 16-byte aligned."""
    return weight.dim() == 2 and weight.is_contiguous() and weight.data_ptr() % 16 == 0


def _decide(x, weight, bias, m: int, n: int, k: int) -> Plan:
    import torch  # noqa: PLC0415

    bf16 = x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
    if bias is not None and (bias.dim() != 1 or bias.shape[0] != n or bias.dtype not in (
            torch.bfloat16, torch.float16, torch.float32)):
        return _FALLBACK_PLAN
    path = route_for(m, n, k, bf16=bf16, bias=bias is not None,
                     contiguous_weight=_weight_ok(weight))
    if path == "fallback":
        return _FALLBACK_PLAN
    return Plan(path, launch_for(path, m, n, k, bias is not None))


_ENGINE_GEMM: list = []


def _fallback(x, weight, bias):
    """The engine's own GEMM: vLLM's ROCm op where vLLM registered one, else F.linear."""
    if not _ENGINE_GEMM:
        import torch  # noqa: PLC0415

        try:
            fn = torch.ops.vllm.rocm_unquantized_gemm
        except (AttributeError, RuntimeError):
            fn = torch.nn.functional.linear
        _ENGINE_GEMM.append(fn)
    return _ENGINE_GEMM[0](x, weight, bias)


def linear(x, weight, bias=None):
    """y = x @ weight.T (+ bias), on the path the table names (the op's body; reference
    python/hk/integration/vllm_gemm.py:384-416)."""
    k = x.shape[-1]
    n = weight.shape[0]
    m = x.numel() // k if k else 0
    key = (m, n, k, x.dtype, weight.dtype, None if bias is None else (bias.dtype, tuple(bias.shape)),
           _weight_ok(weight), x.get_device())
    plan = ROUTER.plans.get(key)
    if plan is None:
        plan = _decide(x, weight, bias, m, n, k)
        if len(ROUTER.plans) < PLAN_CAP:
            ROUTER.plans[key] = plan
    if plan.run is None:
        PATCH.count("fallback")
        return _fallback(x, weight, bias)
    x2 = x.reshape(m, k)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.clone(memory_format=_contiguous())
    y = plan.run(x2, weight, bias)
    PATCH.count(plan.path)
    return y.view(*x.shape[:-1], n)


def _contiguous():
    import torch  # noqa: PLC0415

    return torch.contiguous_format


def register_op() -> None:
    """Define `torch.ops.hk_vllm.linear` (idempotent)."""
    PATCH.define(linear)


# ---------------------------------------------------------------- layers and vLLM


def _unrouted_reason(weight, bias) -> str:
    """Why no call of a layer with this weight and bias can take an hk path ("" if one
    can)."""
    import torch  # noqa: PLC0415

    if weight.dtype != torch.bfloat16:
        return "weight " + str(weight.dtype).rpartition(".")[2]
    if bias is not None and not BIAS_FUSED:
        return "bias"
    if weight.dim() != 2 or not weight.is_contiguous():
        return "weight not a contiguous matrix"
    table = routes()
    if table is None or not table.routes_any(*weight.shape):
        return "no route at any M"
    return ""


def _layer_routed(layer, weight, bias) -> bool:
    """Whether a layer's calls go through the op. The decision is kept on the layer
    (`_hk_route` = (generation, reason)) and reused until the table is replaced -- except
    while torch.compile traces, where it is made and not kept."""
    kept = getattr(layer, "_hk_route", None)
    gen = ROUTER.generation
    if kept is not None and kept[0] == gen:
        return not kept[1]
    reason = _unrouted_reason(weight, bias)
    if engine.compiling():
        return not reason
    if reason and (kept is None or not kept[1]):
        UNROUTED[reason] += 1
    try:
        layer._hk_route = (gen, reason)
    except AttributeError:      # a layer that takes no attributes is decided every call
        pass
    return not reason


def _layer_gemm(engine_gemm, layer, x, weight, bias=None):
    """The GEMM a patched `dispatch_unquantized_gemm()` hands a layer: the op for a routed
    layer's GPU calls, else what vLLM's own dispatch returned (`engine_gemm`)."""
    if not _layer_routed(layer, weight, bias):
        return engine_gemm(layer, x, weight, bias)
    if not x.is_cuda:
        import torch  # noqa: PLC0415

        return torch.nn.functional.linear(x, weight, bias)
    return PATCH(x, weight, bias)


_VLLM_DISPATCH: Optional[Callable] = None


def dispatch_unquantized_gemm(*args, **kwargs):
    """Stands in for vLLM's: asks vLLM's own dispatch (its arguments pick among backends,
    which is vLLM's business) and binds what it returns as the layer's fallback. vLLM
    calls this on every forward, inside the graph it compiles, so it keeps no cache."""
    return functools.partial(_layer_gemm, _VLLM_DISPATCH(*args, **kwargs))


def rebind(prefixes, old, new) -> list:
    """Point every module-level name bound to `old` at `new`, in the loaded modules whose
    name starts with one of `prefixes`; returns "module.name" of each."""
    done = []
    for modname in sorted(sys.modules):
        if not modname.startswith(tuple(prefixes)):
            continue
        mod = sys.modules.get(modname)
        if mod is None:
            continue
        for attr, val in list(vars(mod).items()):
            if val is old:
                setattr(mod, attr, new)
                done.append(f"{modname}.{attr}")
    return done


def apply() -> str:
    """Route vLLM's unquantized linear layers. Returns what happened, in one line."""
    global _VLLM_DISPATCH
    if _VLLM_DISPATCH is not None:
        return "linear: already patched"
    try:
        from vllm.model_executor.layers import utils as vllm_utils  # noqa: PLC0415
        from vllm.platforms import current_platform  # noqa: PLC0415
    except ImportError:
        return "vllm is not importable; linear not patched"
    if not current_platform.is_rocm():
        return "linear: not patched -- not a ROCm platform"
    table = routes()
    if table is None:
        from ..target import current_arch  # noqa: PLC0415

        return (f"linear: not patched -- no routing table for {current_arch()} "
                f"(`python -m hk.integration.tune` measures one)")
    register_op()
    _VLLM_DISPATCH = vllm_utils.dispatch_unquantized_gemm
    names = rebind(PREFIXES, _VLLM_DISPATCH, dispatch_unquantized_gemm)
    cache = engine.isolate_compile_cache("linear")
    return (f"linear -> hk where {table.source or 'the table'} measured it faster "
            f"({len(names)} rebound; compile cache {cache})")


def revert() -> str:
    global _VLLM_DISPATCH
    if _VLLM_DISPATCH is None:
        return "linear: not patched"
    names = rebind(PREFIXES, dispatch_unquantized_gemm, _VLLM_DISPATCH)
    _VLLM_DISPATCH = None
    return f"linear -> vllm ({len(names)} rebound)"


def _linear_layer_bias(mod, head):
    """(is a GEMM layer, its bias) for a vLLM module: an unquantized linear (its bias
    unless vLLM adds it afterwards) or the LM head (an embedding matrix used as a GEMM)."""
    method = type(getattr(mod, "quant_method", None)).__name__
    if method == "UnquantizedLinearMethod":
        return True, (None if getattr(mod, "skip_bias_add", False) else getattr(mod, "bias", None))
    if method == "UnquantizedEmbeddingMethod":
        return (mod is head or type(mod).__name__ == "ParallelLMHead"), None
    return False, None


def decide_layers(model) -> str:
    """Decide every unquantized linear layer of a loaded vLLM model and its LM head now,
    before vLLM's profile run or any capture. Returns the report line."""
    import torch  # noqa: PLC0415

    head = getattr(model, "lm_head", None)
    routed = 0
    for mod in model.modules():
        w = getattr(mod, "weight", None)
        if not isinstance(w, torch.Tensor) or w.dim() != 2:
            continue
        is_gemm, bias = _linear_layer_bias(mod, head)
        if is_gemm:
            routed += _layer_routed(mod, w, bias)
    return f"{routed} layer{'' if routed == 1 else 's'} through hk's op; {unrouted_status()}"


def unrouted_status() -> str:
    if not UNROUTED:
        return "unrouted at load: none"
    return "unrouted at load: " + ", ".join(f"{n} ({why})" for why, n in UNROUTED.most_common())


def status() -> str:
    return "not patched" if _VLLM_DISPATCH is None else f"patched; {unrouted_status()}"


__all__ = ["PATCH", "STATS", "ROUTER", "route_for", "route", "route_decode", "linear",
           "launch_for", "register_op", "dispatch_unquantized_gemm", "apply", "revert",
           "decide_layers", "routes", "set_routes", "rebind", "status"]
