"""vLLM's unquantized linear layers on this build's gfx950 GEMMs.

Restates python/hk/integration/vllm_gemm.py's route (:1-693) over libhkx.so:

* `torch.ops.hk_vllm.linear(Tensor x, Tensor weight, Tensor? bias=None) -> Tensor`, an
  opaque op with a fake, so under torch.compile the shape-dependent choice of kernel
  is not a guard; it launches on torch's stream and declares itself graph-safe;
* `route_for(m, n, k, ...)` -- "hk" (the tile / split-K kernels), "hk_decode" (the
  decode kernel) or "fallback" (vLLM's own GEMM, or F.linear), from the measured
  route table (`engine.RouteTable`): a shape nobody measured takes the fallback;
* `dispatch_unquantized_gemm` rebound by identity in every vLLM module that imported it
  (`apply` / `revert`), and each layer decided once (`decide_layers`).

One deliberate difference: a call with a bias can take the hk path, the bias added in
the GEMM kernel's registers (the fused epilogue), where the reference sends it to the
fallback (:173) rather than pay a second pass over the output. `BIAS_FUSED = False`
restores the reference's behaviour.
"""

from __future__ import annotations

import functools
import sys
from collections import Counter
from typing import Any, Callable, Dict, Optional

from . import engine

PREFIXES = ("vllm",)
ROUTES_ENV = "HK_VLLM_ROUTES"
#: Whether a bias rides the hk path as a fused epilogue (True) or falls back.
BIAS_FUSED = True

_ORIG_DISPATCH: Optional[Callable] = None
UNROUTED: "Counter[str]" = Counter()
_GEMMS: Dict[Any, Callable] = {}
_FALLBACK: list = []
_TABLE: list = []
_GEN = [0]


def _linear_fake(x, weight, bias=None):
    return x.new_empty((*x.shape[:-1], weight.shape[0]))


RUN_PATHS = ("hk", "hk_decode", "fallback")

PATCH = engine.Op("hk_vllm::linear", "linear(Tensor x, Tensor weight, Tensor? bias=None) -> Tensor",
                  _linear_fake, paths=RUN_PATHS, graph="safe")
STATS = PATCH.stats


def routes() -> Optional[engine.RouteTable]:
    """The routing table for this process's arch (loaded once; `set_routes(None)`
    reloads it)."""
    if not _TABLE:
        from ..target import current_arch  # noqa: PLC0415

        _TABLE.append(engine.shipped_table("vllm_linear", current_arch(), ROUTES_ENV))
    return _TABLE[0]


def set_routes(table: Optional[engine.RouteTable]) -> None:
    """Route by `table` from now on; None for the shipped one."""
    if any(PATCH.captured.values()):
        import warnings  # noqa: PLC0415

        warnings.warn("hk_vllm::linear: routes changed after a CUDA graph was captured; graphs "
                      "captured before keep replaying the old routes", stacklevel=2)
    _TABLE.clear()
    _PLANS.clear()
    _GEN[0] += 1
    if table is not None:
        _TABLE.append(table)


def _gemm_takes(n: int, k: int) -> bool:
    from ..ops import gemm_cdna  # noqa: PLC0415

    return not (n % gemm_cdna.BLOCK_N_MIN or k % gemm_cdna.K_STEP)


def route_for(m: int, n: int, k: int, *, bf16: bool = True, bias: bool = False,
              contiguous_weight: bool = True) -> str:
    """"hk", "hk_decode" or "fallback" for y = x @ W.T (+ bias), x (m, k), W (n, k)."""
    if m < 1 or not bf16 or not contiguous_weight or (bias and not BIAS_FUSED):
        return "fallback"
    table = routes()
    if table is None:
        return "fallback"
    path = table.lookup(m, n, k)
    if path == "hk" and not _gemm_takes(n, k):
        return "fallback"
    if path == "hk_decode":
        from ..ops import gemm_cdna  # noqa: PLC0415

        if not gemm_cdna.fits("decode", m, n, k):
            return "fallback"
    return path if path in RUN_PATHS else "fallback"


def route(m: int, n: int, k: int, **how) -> bool:
    return route_for(m, n, k, **how) == "hk"


def route_decode(m: int, n: int, k: int, **how) -> bool:
    return route_for(m, n, k, **how) == "hk_decode"


def _fallback(x, weight, bias):
    """What vLLM would have run: its own op where it has one, else F.linear."""
    if not _FALLBACK:
        import torch  # noqa: PLC0415

        try:
            _FALLBACK.append(torch.ops.vllm.rocm_unquantized_gemm)
        except (AttributeError, RuntimeError):
            _FALLBACK.append(torch.nn.functional.linear)
    return _FALLBACK[0](x, weight, bias)


#: (M, N, K, dtypes, bias, contiguity, device) -> (path, run), decided once per shape.
_PLANS: Dict[tuple, tuple] = {}
_PLAN_CAP = 4096


def _run_for(path: str, m: int, n: int, k: int, has_bias: bool) -> Callable:
    from ..ops import gemm_cdna  # noqa: PLC0415
    from ..templates import gemm as T  # noqa: PLC0415

    schedule = None
    if path == "hk_decode":
        schedule = "decode"
    elif path == "hk":
        name = gemm_cdna.route(m, n, k)
        schedule = name if gemm_cdna.CANDIDATES[name]["kernel"] == "tile" else gemm_cdna.rule(
            max(m, 33), n, k)
    if has_bias:
        return lambda x2, w, b, out: T.gemm(x2, w, epilogue=T.bias, out=out, schedule=schedule,
                                            bias=b)
    return lambda x2, w, b, out: T.gemm(x2, w, out=out, schedule=schedule)


def _plan(x, weight, bias, m: int, n: int, k: int) -> tuple:
    import torch  # noqa: PLC0415

    path = route_for(m, n, k, bf16=x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16,
                     bias=bias is not None, contiguous_weight=weight.is_contiguous())
    if path == "fallback":
        return "fallback", None
    return path, _run_for(path, m, n, k, bias is not None)


def linear(x, weight, bias=None):
    """y = x @ weight.T (+ bias), on the kernel the table names (vllm_gemm.py:384-416)."""
    import torch  # noqa: PLC0415

    k = x.shape[-1]
    m = x.numel() // k if k else 0
    n = weight.shape[0]
    key = (m, n, k, x.dtype, weight.dtype, bias is None, weight.is_contiguous(), x.get_device())
    plan = _PLANS.get(key)
    if plan is None:
        plan = _plan(x, weight, bias, m, n, k)
        if len(_PLANS) < _PLAN_CAP:
            _PLANS[key] = plan
    path, run = plan
    if path == "fallback":
        PATCH.count("fallback")
        return _fallback(x, weight, bias)
    x2 = x.reshape(m, k)
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    out = torch.empty((m, n), device=x.device, dtype=x.dtype)
    run(x2, weight, bias, out)
    PATCH.count(path)
    return out.view(*x.shape[:-1], n)


def register_op():
    """Define `torch.ops.hk_vllm.linear`. Idempotent."""
    PATCH.define(linear)


def _unrouted(weight, bias) -> str:
    """Why the table takes no call of a layer with this weight, at any M ("" if some)."""
    import torch  # noqa: PLC0415

    if weight.dtype != torch.bfloat16:
        return f"weight {str(weight.dtype).replace('torch.', '')}"
    if bias is not None and not BIAS_FUSED:
        return "bias"
    if weight.dim() != 2 or not weight.is_contiguous():
        return "weight not a contiguous matrix"
    table = routes()
    n, k = weight.shape
    if table is None or not table.routes_any(n, k):
        return "no route at any M"
    return ""


def _compiling() -> bool:
    import torch  # noqa: PLC0415

    return torch.compiler.is_compiling()


def _takes_layer(layer, weight, bias) -> bool:
    """Whether this layer's calls go through the op at all, decided once per table
    generation and kept on the layer (read-only while torch.compile traces)."""
    memo = getattr(layer, "_hk_gemm", None)
    if memo is not None and memo[0] == _GEN[0]:
        return memo[1]
    why = _unrouted(weight, bias)
    if _compiling():
        return not why
    if why and (memo is None or memo[1]):
        UNROUTED[why] += 1
    try:
        layer._hk_gemm = (_GEN[0], not why)
    except AttributeError:
        pass
    return not why


def _gemm(layer, x, weight, bias=None):
    import torch  # noqa: PLC0415

    if not x.is_cuda:
        return torch.nn.functional.linear(x, weight, bias)
    return PATCH(x, weight, bias)


def _routed_gemm(orig, layer, x, weight, bias=None):
    if not _takes_layer(layer, weight, bias):
        return orig(layer, x, weight, bias)
    return _gemm(layer, x, weight, bias)


def dispatch_unquantized_gemm(*args, **kwargs):
    """Stands in for vLLM's: returns the routed GEMM bound to vLLM's own (kept for the
    layers the table never routes). Writes its cache only in eager code."""
    try:
        key = (args, tuple(sorted(kwargs.items())))
        hit = _GEMMS.get(key)
    except TypeError:
        key, hit = None, None
    if hit is not None:
        return hit
    g = functools.partial(_routed_gemm, _ORIG_DISPATCH(*args, **kwargs))
    if key is not None and not _compiling():
        _GEMMS[key] = g
    return g


def rebind(prefixes, old, new) -> list:
    """Replace every module-level binding of `old` by `new` in the modules whose name
    starts with one of `prefixes`, by identity. Returns the names rebound."""
    names = []
    for modname, mod in list(sys.modules.items()):
        if mod is None or not modname.startswith(tuple(prefixes)):
            continue
        for attr, val in list(vars(mod).items()):
            if val is old:
                setattr(mod, attr, new)
                names.append(f"{modname}.{attr}")
    return names


def apply() -> str:
    """Route vLLM's linear layers. Returns what happened, in one line."""
    global _ORIG_DISPATCH
    try:
        from vllm.model_executor.layers import utils as vu  # noqa: PLC0415
        from vllm.platforms import current_platform  # noqa: PLC0415
    except ImportError:
        return "vllm is not importable; linear not patched"
    if _ORIG_DISPATCH is not None:
        return "linear: already patched"
    if not current_platform.is_rocm():
        return "linear: not patched -- not a ROCm platform"
    table = routes()
    if table is None:
        from ..target import current_arch  # noqa: PLC0415

        return (f"linear: not patched -- no routing table for {current_arch()}; "
                f"`python -m hk.integration.tune` measures one")
    register_op()
    _GEMMS.clear()
    _ORIG_DISPATCH = vu.dispatch_unquantized_gemm
    names = rebind(PREFIXES, _ORIG_DISPATCH, dispatch_unquantized_gemm)
    return f"linear -> hk where {table.source or 'the table'} measured it faster ({len(names)} rebound)"


def revert() -> str:
    global _ORIG_DISPATCH
    if _ORIG_DISPATCH is None:
        return "linear: not patched"
    names = rebind(PREFIXES, dispatch_unquantized_gemm, _ORIG_DISPATCH)
    _ORIG_DISPATCH = None
    _GEMMS.clear()
    return f"linear -> vllm ({len(names)} rebound)"


def decide_layers(model) -> str:
    """Decide every unquantized linear layer of a loaded vLLM model (and its LM head) now."""
    import torch  # noqa: PLC0415

    head = getattr(model, "lm_head", None)
    routed = 0
    for _, mod in model.named_modules():
        w = getattr(mod, "weight", None)
        qm = type(getattr(mod, "quant_method", None)).__name__
        if not isinstance(w, torch.Tensor) or w.dim() != 2:
            continue
        if qm == "UnquantizedEmbeddingMethod":
            if mod is not head and type(mod).__name__ != "ParallelLMHead":
                continue
            bias = None
        elif qm == "UnquantizedLinearMethod":
            bias = None if getattr(mod, "skip_bias_add", False) else getattr(mod, "bias", None)
        else:
            continue
        routed += _takes_layer(mod, w, bias)
    return f"{routed} layer{'s' * (routed != 1)} through hk's op; {unrouted_status()}"


def unrouted_status() -> str:
    if not UNROUTED:
        return "unrouted at load: none"
    return "unrouted at load: " + ", ".join(f"{n} ({why})" for why, n in UNROUTED.most_common())


def status() -> str:
    return "not patched" if _ORIG_DISPATCH is None else f"patched; {unrouted_status()}"


__all__ = ["PATCH", "STATS", "route_for", "route", "route_decode", "linear", "register_op",
           "dispatch_unquantized_gemm", "apply", "revert", "decide_layers", "routes",
           "set_routes", "rebind"]
