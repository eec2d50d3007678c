"""The engine route on the CPU: RouteTable's semantics, the table file format, route_for's
decisions, the fallback, and the dispatch rebinding with a stand-in vLLM -- the
reference's tests/hk/ir/test_vllm_gemm.py:35-343 restated (vLLM is not installed here,
so its dispatcher and layer are stand-ins, as the reference's tests use)."""

import json
import sys
import types

import pytest
import torch

from hk.integration import engine
from hk.integration import vllm_gemm as V

TABLE = {"arch": "gfx950", "kind": "vllm_linear",
         "shapes": {"4096x4096": {"runs": [[1, 16, "hk_decode"], [64, 512, "hk"], [1024, 4096, "hk"]]},
                    "12288x4096": {"runs": [[1, 32, "hk_decode"], [33, 8192, "hk"]], "above": "fallback"},
                    "1000x64": {"runs": [[1, 8, "fallback"]]}}}


def table():
    return engine.RouteTable(engine.RouteTable.parse(TABLE), meta={"arch": "gfx950"}, source="t")


def test_lookup_inside_between_above_below():
    t = table()
    assert t.lookup(1, 4096, 4096) == "hk_decode"
    assert t.lookup(16, 4096, 4096) == "hk_decode"
    assert t.lookup(17, 4096, 4096) == "fallback"   # between two runs that disagree
    assert t.lookup(64, 4096, 4096) == "hk"
    assert t.lookup(600, 4096, 4096) == "fallback"  # between two runs (same path: still a gap)
    assert t.lookup(9999, 4096, 4096) == "hk"       # above the last run: its path
    assert t.lookup(9999, 12288, 4096) == "fallback"  # `above` says otherwise
    assert t.lookup(5, 5, 5) == "fallback" and (5, 5) in t.misses
    assert t.routes_any(4096, 4096) and not t.routes_any(1000, 64)


def test_overlapping_runs_are_refused_and_a_table_round_trips(tmp_path):
    with pytest.raises(ValueError, match="overlap"):
        engine.RouteTable({(1, 1): {"runs": [[1, 8, "hk"], [8, 9, "hk"]]}})
    t = table()
    p = tmp_path / "routes.json"
    p.write_text(json.dumps(t.to_json()))
    t2 = engine.RouteTable.from_json(p)
    for m in (1, 16, 17, 64, 600, 9999):
        assert t2.lookup(m, 4096, 4096) == t.lookup(m, 4096, 4096)
        assert t2.lookup(m, 12288, 4096) == t.lookup(m, 12288, 4096)


def test_shipped_table_env_override(tmp_path, monkeypatch):
    p = tmp_path / "r.json"
    p.write_text(json.dumps(TABLE))
    monkeypatch.setenv("HK_TEST_ROUTES", str(p))
    t = engine.shipped_table("vllm_linear", "gfx950", "HK_TEST_ROUTES")
    assert t.lookup(64, 4096, 4096) == "hk"
    monkeypatch.setenv("HK_TEST_ROUTES", str(tmp_path / "missing.json"))
    with pytest.raises(FileNotFoundError):
        engine.shipped_table("vllm_linear", "gfx950", "HK_TEST_ROUTES")
    bad = dict(TABLE, arch="gfx1100")
    p.write_text(json.dumps(bad))
    monkeypatch.setenv("HK_TEST_ROUTES", str(p))
    with pytest.raises(ValueError, match="gfx1100"):
        engine.shipped_table("vllm_linear", "gfx950", "HK_TEST_ROUTES")


@pytest.fixture
def routed():
    V.set_routes(table())
    yield
    V.set_routes(None)


def test_route_for(routed):
    assert V.route_for(64, 4096, 4096) == "hk"
    assert V.route_for(8, 4096, 4096) == "hk_decode"
    assert V.route_for(17, 4096, 4096) == "fallback"
    assert V.route_for(64, 4096, 4096, bf16=False) == "fallback"
    assert V.route_for(64, 4096, 4096, contiguous_weight=False) == "fallback"
    assert V.route_for(0, 4096, 4096) == "fallback"
    assert V.route_for(64, 4096, 4096, bias=True) == "hk"  # the bias rides the fused epilogue
    V.BIAS_FUSED = False
    try:
        assert V.route_for(64, 4096, 4096, bias=True) == "fallback"  # the reference's rule
    finally:
        V.BIAS_FUSED = True
    assert V.route_for(9999, 12288, 4096) == "fallback"


def test_no_table_routes_nothing():
    V.ROUTER.replace(None, loaded=True)     # an arch with no table
    try:
        assert V.routes() is None
        assert V.route_for(64, 4096, 4096) == "fallback"
    finally:
        V.set_routes(None)


def test_cpu_tensors_and_fallback_compute_linear(routed):
    x = torch.randn(3, 5, 64)
    w = torch.randn(1000, 64)
    b = torch.randn(1000)
    w_routed = torch.randn(4096, 4096, dtype=torch.bfloat16)
    xr = torch.ones(3, 4096, dtype=torch.bfloat16)
    layer = types.SimpleNamespace()
    y = V._layer_gemm(None, layer, xr, w_routed)                # routed, but on the CPU:
    torch.testing.assert_close(y, torch.nn.functional.linear(xr, w_routed))
    assert layer._hk_route == (V.ROUTER.generation, "")            # torch's own GEMM
    V.PATCH.reset()
    y2 = V.linear(x.bfloat16(), w.bfloat16(), None)  # the table sends (1000, 64) to the fallback
    assert V.PATCH.stats["fallback"] == 1
    ref = torch.nn.functional.linear(x.bfloat16().float(), w.bfloat16().float())
    torch.testing.assert_close(y2.float(), ref, rtol=2e-2, atol=2e-2)


def test_dispatch_rebinding_with_a_stand_in_vllm(routed, monkeypatch):
    """vLLM's `dispatch_unquantized_gemm` is replaced in every vllm module that bound it,
    by identity, and put back by revert()."""
    calls = []

    def orig_gemm(layer, x, weight, bias=None):
        calls.append("orig")
        return torch.nn.functional.linear(x, weight, bias)

    def orig_dispatch(*args, **kwargs):
        return orig_gemm

    utils = types.ModuleType("vllm.model_executor.layers.utils")
    utils.dispatch_unquantized_gemm = orig_dispatch
    other = types.ModuleType("vllm.model_executor.layers.linear")
    other.dispatch_unquantized_gemm = orig_dispatch
    platforms = types.ModuleType("vllm.platforms")
    platforms.current_platform = types.SimpleNamespace(is_rocm=lambda: True)
    mods = {"vllm": types.ModuleType("vllm"), "vllm.model_executor": types.ModuleType("vllm.model_executor"),
            "vllm.model_executor.layers": types.ModuleType("vllm.model_executor.layers"),
            "vllm.model_executor.layers.utils": utils, "vllm.model_executor.layers.linear": other,
            "vllm.platforms": platforms}
    mods["vllm.model_executor.layers"].utils = utils
    for k, v in mods.items():
        monkeypatch.setitem(sys.modules, k, v)
    monkeypatch.setenv("VLLM_CACHE_ROOT", "/tmp/vllm-cache")
    msg = V.apply()
    assert "2 rebound" in msg, msg
    assert "compile cache /tmp/vllm-cache/hk-linear" in msg
    assert __import__("os").environ["VLLM_CACHE_ROOT"] == "/tmp/vllm-cache/hk-linear"
    assert utils.dispatch_unquantized_gemm is V.dispatch_unquantized_gemm
    assert other.dispatch_unquantized_gemm is V.dispatch_unquantized_gemm
    g = utils.dispatch_unquantized_gemm()
    layer = types.SimpleNamespace()
    w = torch.randn(1000, 64, dtype=torch.bfloat16)
    g(layer, torch.randn(2, 64, dtype=torch.bfloat16), w)  # a shape the table never routes
    assert calls == ["orig"] and layer._hk_route[1] == "no route at any M"
    assert "2 rebound" in V.revert()
    assert utils.dispatch_unquantized_gemm is orig_dispatch


def test_patch_contracts():
    with pytest.raises(ValueError, match="says why"):
        engine.Patch("x::y", ["a"], graph="never")
    p = engine.Patch("x::z", ["a", "b"])
    p.count("a")
    p.count("a")
    assert p.stats == {"a": 2, "b": 0} and "a 2" in p.summary()
    assert p.guard(lambda v: v + 1)(1) == 2  # free outside capture


def test_vllm_mxfp8_route_and_patch_without_vllm():
    """The MXFP8 route: a measured table's runs where there is one (unmeasured shapes stay
    with vLLM), else M >= MIN_M; and the patch reports, rather than fails, where vLLM is
    absent (vllm_mxfp8.py:191-200's contract)."""
    from hk.integration import engine as E
    from hk.integration import vllm_mxfp8 as V

    # without a table: M >= MIN_M
    V.set_routes(None)
    V._TABLE.append(None)      # no table for this arch
    try:
        assert V.schedule(V.MIN_M, 5120, 4096)
        assert not V.schedule(V.MIN_M - 1, 5120, 4096)
        # with one: its runs, and unmeasured shapes stay with vLLM
        V.set_routes(E.RouteTable({(5120, 4096): {"runs": [[16, 256, "hk"], [384, 384, "fallback"],
                                                           [512, 8192, "hk"]]}}))
        assert V.schedule(16, 5120, 4096) and V.schedule(9000, 5120, 4096)
        assert not V.schedule(384, 5120, 4096) and not V.schedule(8, 5120, 4096)
        assert not V.schedule(4096, 2048, 4096)  # not measured
    finally:
        V.set_routes(None)
    assert not V.schedule(4096, 5124, 4096)   # N % 8
    assert not V.schedule(4096, 5120, 4000)   # K % 128
    V.ENABLED = False
    try:
        assert not V.schedule(4096, 5120, 4096)
    finally:
        V.ENABLED = True
    import importlib.util

    if importlib.util.find_spec("vllm") is None:
        assert "not importable" in V.apply_patch()
    assert V.revert() == "mxfp8: not patched"


def test_compile_cache_isolation_merges_routes(monkeypatch, tmp_path):
    """Each patched engine gets its own vLLM cache root under the current one, named for
    every route applied in any order, and a worker that inherits it adds nothing."""
    monkeypatch.setenv("VLLM_CACHE_ROOT", str(tmp_path / "vc"))
    assert engine.isolate_compile_cache("mxfp8") == str(tmp_path / "vc" / "hk-mxfp8")
    assert engine.isolate_compile_cache("linear") == str(tmp_path / "vc" / "hk-linear+mxfp8")
    assert engine.isolate_compile_cache("mxfp8") == str(tmp_path / "vc" / "hk-linear+mxfp8")
    monkeypatch.delenv("VLLM_CACHE_ROOT")
    monkeypatch.setenv("XDG_CACHE_HOME", str(tmp_path / "xdg"))
    assert engine.isolate_compile_cache("linear") == str(tmp_path / "xdg" / "vllm" / "hk-linear")


# ------------------------------------------------- the compiled forward's contract
#
# vLLM compiles its forward whole (fullgraph) and refuses to start when the code Dynamo
# produces names `update` (compilation/wrapper.py's bytecode hook): a write the graph must
# replay afterwards is lost on a CUDA-graph replay. The forward below has the shape of
# vLLM's UnquantizedLinearMethod.apply -- call dispatch_unquantized_gemm(), then the GEMM
# it returns -- and runs on the CPU with a stand-in for vLLM's own dispatch (x2, so which
# GEMM ran is visible in the output). The reference's check of the same contract is
# tests/hk/ir/test_vllm_gemm_compiled.py:85-125.

NC, KC = 256, 128


def _engine_dispatch(*args, **kwargs):
    return lambda layer, x, weight, bias=None: torch.nn.functional.linear(x, weight, bias) * 2


class _Layer(torch.nn.Module):
    def __init__(self, dtype):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.randn(NC, KC).to(dtype), requires_grad=False)

    def forward(self, x):
        return V.dispatch_unquantized_gemm()(self, x.to(self.weight.dtype), self.weight, None)


class _Net(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.layers = torch.nn.ModuleList([_Layer(torch.bfloat16), _Layer(torch.float16),
                                           _Layer(torch.bfloat16)])

    def forward(self, x):
        return sum(layer(x).float() for layer in self.layers)


@pytest.fixture
def stand_in_engine(monkeypatch):
    monkeypatch.setattr(V, "_VLLM_DISPATCH", _engine_dispatch)
    monkeypatch.setattr(V, "UNROUTED", V.Counter())
    V.set_routes(engine.RouteTable({(NC, KC): {"runs": [[1, 64, "hk_decode"]], "above": "hk"}}))
    yield
    V.set_routes(None)


def _compile_and_watch(model, x):
    """Compile `model` whole as vLLM does; return (output, names of the frames whose
    transformed code names `update`)."""
    flagged = []

    def hook(old, new):
        if "update" in new.co_names:
            flagged.append(old.co_name)

    torch._dynamo.reset()
    handle = torch._dynamo.convert_frame.register_bytecode_hook(hook)
    try:
        out = torch.compile(model, fullgraph=True, backend="eager")(x)
    finally:
        handle.remove()
        torch._dynamo.reset()
    return out, flagged


def _state(model):
    return ([getattr(layer, "_hk_route", None) for layer in model.layers], dict(V.UNROUTED),
            dict(V.ROUTER.plans))


@pytest.mark.parametrize("decided", ["at load", "never", "for a replaced table"])
def test_the_compiled_forward_writes_nothing(stand_in_engine, decided):
    model = _Net()
    if decided != "never":
        for layer in model.layers:
            V._layer_routed(layer, layer.weight, None)
    if decided == "for a replaced table":
        V.set_routes(V.routes())            # a new generation: every kept decision is stale
    before = _state(model)
    x = torch.randn(4, KC)
    out, flagged = _compile_and_watch(model, x)
    assert flagged == [], f"the traced forward writes state vLLM's guard refuses: {flagged}"
    assert _state(model) == before           # no decision, count or plan kept by the trace
    torch.testing.assert_close(out, model(x))


def test_the_compiled_forward_routes_as_eager_does(stand_in_engine):
    """Traced, the bf16 layers go through the op's CPU path (F.linear) and the fp16 one
    to the engine's GEMM (x2 in the stand-in)."""
    model = _Net()
    x = torch.randn(4, KC)
    out, _ = _compile_and_watch(model, x)
    want = sum(torch.nn.functional.linear(x.to(l.weight.dtype), l.weight).float()
               * (2 if l.weight.dtype == torch.float16 else 1) for l in model.layers)
    torch.testing.assert_close(out, want, rtol=2e-2, atol=2e-1)


def test_eager_forward_decides_each_layer_once(stand_in_engine):
    model = _Net()
    model(torch.randn(4, KC))
    model(torch.randn(4, KC))
    gen = V.ROUTER.generation
    assert [layer._hk_route for layer in model.layers] == [
        (gen, ""), (gen, "weight float16"), (gen, "")]
    assert V.UNROUTED == {"weight float16": 1}
