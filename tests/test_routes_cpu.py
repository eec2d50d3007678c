"""The measured routing tables and the tuner's decisions, on the CPU.

The decision rules restate python/hk/autotune/routes.py:92-272 (a kernel takes an M only
where it beat the engine by min_gain; a tie stays the engine's; consecutive equal answers
merge into runs; the answer at the largest M holds above it) and are checked here on
hand-made points whose answers follow from the rule alone. The shipped tables are then
checked against themselves: each route is what its own recorded points decide."""

import json
from pathlib import Path

import pytest

from hk.integration import engine, tune
from hk.ops import gemm_cdna

TUNED = Path(tune.__file__).resolve().parents[1] / "tuned"


def test_base_path_needs_the_margin():
    assert tune.base_path({"engine": 10.0, "hk": 9.0}) == "hk"          # 11% faster
    assert tune.base_path({"engine": 10.0, "hk": 9.8}) == "fallback"    # 2% < 3%
    assert tune.base_path({"engine": 10.0, "hk": 10.0}) == "fallback"   # a tie
    assert tune.base_path({"engine": 10.0, "hk": 9.0, "hk_decode": 7.0}) == "hk_decode"
    assert tune.base_path({"engine": 10.0}) == "fallback"
    assert tune.base_path({"hk": 3.0}) == "hk"  # the engine failed its check
    assert tune.base_path({"engine": 10.0, "hk": 9.8}, min_gain=0.01) == "hk"


def test_runs_merge_and_answer_above():
    pts = [[1, {"engine": 10, "hk_decode": 7}], [2, {"engine": 10, "hk_decode": 8}],
           [4, {"engine": 10, "hk": 9.9}], [8, {"engine": 10, "hk": 8}], [16, {"engine": 10, "hk": 8}]]
    rs, above = tune.runs(pts)
    assert rs == [[1, 2, "hk_decode"], [4, 4, "fallback"], [8, 16, "hk"]] and above == "hk"
    ent = tune.entry("x", pts, partial=True)
    assert ent["above"] == "fallback" and ent["partial"]
    t = engine.RouteTable({(64, 64): ent})
    assert [t.lookup(m, 64, 64) for m in (1, 2, 3, 4, 8, 16, 32)] == \
        ["hk_decode", "hk_decode", "fallback", "fallback", "hk", "hk", "fallback"]


def test_linear_shapes_of_the_two_models():
    q = {nm: (n, k) for nm, n, k, _ in tune.linear_shapes(tune.MODELS["Qwen/Qwen3-8B"])}
    assert q == {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (24576, 4096),
                 "down": (4096, 12288), "lm_head": (151936, 4096)}
    ll = {nm: (n, k) for nm, n, k, _ in tune.linear_shapes(tune.MODELS["meta-llama/Meta-Llama-3-8B"])}
    assert ll["gate_up"] == (28672, 4096) and ll["down"] == (4096, 14336)
    assert ll["lm_head"] == (128256, 4096)
    q2 = {nm: (n, k) for nm, n, k, _ in tune.linear_shapes(tune.MODELS["Qwen/Qwen3-8B"], tp=2)}
    assert q2["qkv"] == (3072, 4096) and q2["down"] == (4096, 6144)


def test_shipped_gemm_table_is_its_own_argmin():
    d = json.loads((TUNED / "routes_gemm_gfx950.json").read_text())
    assert d["arch"] == "gfx950"
    assert set(d["candidates"]) == set(gemm_cdna.CANDIDATES)
    for p in d["points"]:
        hk_us = {c[3:]: v for c, v in p["us"].items() if c.startswith("hk:")}
        assert d["routes"][f"{p['n']}x{p['k']}"][str(p["m"])] == min(hk_us, key=hk_us.get)
    # the models' shapes and the config-2 / config-4 shape are all measured
    for nk in ("6144x4096", "4096x4096", "24576x4096", "4096x12288", "151936x4096",
               "28672x4096", "4096x14336", "128256x4096", "12288x4096"):
        assert nk in d["routes"], nk


def test_gemm_route_reads_the_table(monkeypatch):
    monkeypatch.setattr(gemm_cdna, "OVERRIDE", {})
    gemm_cdna.reload_table()
    routes = gemm_cdna.table()
    assert routes["12288x4096"]["4096"] == gemm_cdna.route(4096, 12288, 4096)
    # the nearest measured M on a log scale
    assert gemm_cdna.route(3000, 12288, 4096) == routes["12288x4096"]["4096"]
    # an unmeasured shape takes the rule
    assert gemm_cdna.route(4096, 12344, 4096) == gemm_cdna.rule(4096, 12344, 4096)


def test_a_table_naming_unknown_candidates_is_refused(tmp_path, monkeypatch):
    bad = tmp_path / "r.json"
    bad.write_text(json.dumps({"arch": "gfx950", "routes": {"64x64": {"1": "nope"}}}))
    monkeypatch.setenv("HK_GEMM_ROUTES", str(bad))
    gemm_cdna.reload_table()
    with pytest.raises(ValueError, match="nope"):
        gemm_cdna.table()
    monkeypatch.delenv("HK_GEMM_ROUTES")
    gemm_cdna.reload_table()


def test_shipped_vllm_table_is_its_own_decision():
    path = TUNED / "routes_vllm_linear_gfx950.json"
    d = json.loads(path.read_text())
    assert d["arch"] == "gfx950" and d["min_gain"] == tune.MIN_GAIN
    t = engine.RouteTable.from_json(path)
    for key, ent in d["shapes"].items():
        rs, above = tune.runs(ent["points"], d["min_gain"])
        assert ent["runs"] == rs, key
        n, k = (int(v) for v in key.split("x"))
        for m, times in ent["points"]:
            assert t.lookup(m, n, k) == tune.base_path(times, d["min_gain"])
    # decode-sized M on the K = 4096 shapes goes to the decode kernel
    assert t.lookup(1, 4096, 4096) == "hk_decode" and t.lookup(16, 24576, 4096) == "hk_decode"


def test_shipped_mxfp8_table_is_its_own_decision():
    """The MXFP8 table (hk's quant + MX GEMM against the same quant + hipBLASLt's MX GEMM):
    every run is what its points decide, the route reads it, and a point where the engine
    failed its check (no engine time) goes to hk."""
    from hk.integration import vllm_mxfp8 as V

    path = TUNED / "routes_vllm_mxfp8_gfx950.json"
    d = json.loads(path.read_text())
    assert d["arch"] == "gfx950" and d["kind"] == "vllm_mxfp8"
    assert {tuple(int(v) for v in key.split("x")) for key in d["shapes"]} == set(tune.MX_SHAPES)
    t = engine.RouteTable.from_json(path)
    V.set_routes(t)
    try:
        for key, ent in d["shapes"].items():
            rs, _ = tune.runs(ent["points"], d["min_gain"])
            assert ent["runs"] == rs, key
            n, k = (int(v) for v in key.split("x"))
            for m, times in ent["points"]:
                want = tune.base_path(times, d["min_gain"])
                assert t.lookup(m, n, k) == want
                assert V.schedule(m, n, k) == (want == "hk")
                if "engine" not in times:
                    assert want == "hk"
    finally:
        V.set_routes(None)


def test_operands_of_4_gib_take_no_kernel(monkeypatch):
    # hkx_gemm refuses an A or B of 4 GiB or more (32-bit buffer offsets), so neither the
    # template's candidates nor the engine route may send one there: a bf16 weight of
    # 131072 x 16384 (exactly 4 GiB) or 131072 tokens of K = 16384 go to the engine's own
    # GEMM; one row fewer is taken
    from hk.integration import vllm_gemm

    assert gemm_cdna.OPERAND_BYTES_MAX == 1 << 32
    assert gemm_cdna.fits("decode", 8, 131068, 16384)
    assert not gemm_cdna.fits("decode", 8, 131072, 16384)
    assert gemm_cdna.fits("t256", 4096, 131068, 16384)
    assert not gemm_cdna.fits("t256", 131072, 4096, 16384)
    assert not gemm_cdna.fits("t256", 4096, 131072, 16384)
    assert gemm_cdna.fits("t256", 4096, 131072, 16384, fp8=True)

    class Everywhere:
        def __init__(self, path):
            self.path = path

        def lookup(self, m, n, k):
            return self.path

    for path in ("hk", "hk_decode"):
        monkeypatch.setattr(vllm_gemm, "routes", lambda p=path: Everywhere(p))
        assert vllm_gemm.route_for(8, 131068, 16384) == path
        assert vllm_gemm.route_for(8, 131072, 16384) == "fallback"
    monkeypatch.setattr(vllm_gemm, "routes", lambda: Everywhere("hk"))
    assert vllm_gemm.route_for(131072, 4096, 16384) == "fallback"
    assert vllm_gemm.route_for(131071, 4096, 16384) == "hk"


def test_rule_close_to_the_measured_best():
    # the route for shapes the table lacks: on the shipped table's measured points, its
    # pick is within a few percent of the fastest candidate on average and never far off
    import json as _json

    d = _json.loads((TUNED / "routes_gemm_gfx950.json").read_text())
    ratios = []
    for p in d["points"]:
        us = p["us"]
        best = min(v for c, v in us.items() if c.startswith("hk:"))
        pick = gemm_cdna.rule(p["m"], p["n"], p["k"])
        assert pick in gemm_cdna.CANDIDATES
        assert "hk:" + pick in us, (p["m"], p["n"], p["k"], pick)
        ratios.append(us["hk:" + pick] / best)
    assert sum(ratios) / len(ratios) < 1.05
    assert max(ratios) < 1.5


def test_fp8_rule_follows_its_sweep(monkeypatch):
    """The fp8 rule's picks at the sweep's points where it chose the measured best
    (scaled_mm with dequant + bias; fp8 has no measured table): 64 x 128 tiles from M = 129
    to 512, a split over K only where each split keeps 32 K units, the bf16 steps below."""
    monkeypatch.setattr(gemm_cdna, "OVERRIDE", {})
    want = {
        (256, 4096, 4096): "t64x128",        # 12.1-12.2 us; split on 128 x 128: 19.6
        (512, 4096, 4096): "t64x128",        # 13.9; the former pick 21.9
        (256, 4096, 12288): "t64x128k2",     # 23.9; unsplit 29.9
        (512, 4096, 12288): "t64x128",       # 32.4
        (1024, 4096, 4096): "t128x128",      # 22.3
        (2048, 4096, 4096): "t128",          # 37.2
        (256, 12288, 4096): "t128x128",      # 20.3-20.5
        (1024, 12288, 4096): "t256",         # 42.1
        (4096, 4096, 12288): "t256",         # 133.0
        (128, 4096, 12288): "t64x128k4",     # 18.3
    }
    for (m, n, k), name in want.items():
        assert gemm_cdna.route(m, n, k, fp8=True) == name, (m, n, k)
        assert gemm_cdna.fits(name, m, n, k, fp8=True)
