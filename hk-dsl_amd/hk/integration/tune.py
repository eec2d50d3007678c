"""Measured routing tables for gfx950: which kernel each linear shape should run on, at
every M a step can have.

Two tables, both written to hk/tuned/ (or `--out`), both measured on the machine that
runs them:

* ``routes_gemm_gfx950.json`` -- the template's own route (`hk.ops.gemm_cdna.route`): for
  each (N, K) and M of the grid, the fastest of this build's candidate kernels
  (`gemm_cdna.CANDIDATES`) that takes the shape, with every candidate's and hipBLASLt's
  TFLOP/s kept beside it. Restates tools/hk-bench/gemm_cdna_routes.py (:1-60: the grid of
  Llama-3-8B and Qwen3-8B linears, the candidates checked against fp32, then timed
  interleaved over weights rotated through more than the Infinity Cache).
* ``routes_vllm_linear_gfx950.json`` -- the vLLM route (`engine.RouteTable`, read by
  `vllm_gemm`): for each (N, K) of a model's linears, at every M of `GRID`, whether this
  build's GEMM ("hk", on the route above), its decode kernel ("hk_decode") or the engine's
  own GEMM (F.linear, i.e. hipBLASLt) is fastest; a kernel takes an M only where it beat
  the engine by `MIN_GAIN` (a tie stays the engine's), and consecutive Ms with the same
  winner merge into runs. Restates python/hk/autotune/routes.py (decisions :92-272, model
  shapes :387-478) and tools/hk-bench/route_tune.py.

How a point is timed (routes.py:618-700, "graph" timing): each path's burst -- one call on
each of `copies` weight copies that together stream at least `ROTATE_BYTES`, so every
call reads cold weights from HBM as a decode step does -- is captured once as a CUDA graph
and its replays timed with events, the paths interleaved over `rounds` rounds; a path's
time is its median round. Launch overhead is inside the graph for every path alike. Each
path's output is checked against fp32 first; a path that misses the tolerance is not timed.

A third, ``routes_vllm_mxfp8_gfx950.json`` (read by `vllm_mxfp8.schedule`), has the same
form for vLLM's block-scaled MXFP8 linears: per (N, K) of `MX_SHAPES`, hk's route (its
activation quant, then `mxfp8.gemm`) against the engine's, timed with the same
quant; the engine here is hipBLASLt's MX GEMM (`torch._scaled_mm` with E8M0 block scales),
since vLLM's own kernel (AITER's) is not importable on this machine.

    python -m hk.integration.tune gemm --out hk/tuned/routes_gemm_gfx950.json
    python -m hk.integration.tune vllm_linear --out hk/tuned/routes_vllm_linear_gfx950.json
    python -m hk.integration.tune vllm_mxfp8 --out hk/tuned/routes_vllm_mxfp8_gfx950.json
"""

from __future__ import annotations

import argparse
import datetime
import json
import statistics
import sys
import time
from pathlib import Path
from typing import Callable, Dict, List, Optional, Sequence, Tuple

#: What a kernel must beat the engine by to take an M (routes.py MIN_GAIN).
MIN_GAIN = 0.03
#: Weight bytes one timed burst streams: three times an MI355X's 256 MB Infinity Cache.
ROTATE_BYTES = 3 * 256 * 2**20
#: The Ms of the vLLM table: every decode-sized M the decode kernel takes, then a
#: geometric grid (the sawtooth between 256-row tile multiples is sampled at both ends).
GRID = (1, 2, 4, 8, 12, 16, 24, 32, 48, 64, 96, 128, 192, 256, 384, 512, 768, 1024, 1536,
        2048, 3072, 4096, 6144, 8192)
#: The Ms of the template's table (gemm_cdna_routes.py MS).
GEMM_MS = (1, 4, 16, 32, 64, 128, 256, 512, 1024, 2048, 4096, 8192)
#: vLLM computes logits for the last token of each sequence only: the LM head's M is a
#: sequence count (routes.py MAX_SEQS).
MAX_SEQS = 256
#: fp32-relative tolerance a path must meet before it is timed.
CHECK_TOL = 2e-2

#: (N, K) of the block-scaled MXFP8 linears the reference measured its route on
#: (python/hk/integration/vllm_mxfp8.py:33-36: DeepSeek-V4.1-Flash's prefill projections
#: at TP2, and the indexer's wq_b).
MX_SHAPES: Dict[Tuple[int, int], str] = {
    (1792, 5120): "dsv4_proj", (2304, 5120): "dsv4_proj", (5120, 1152): "dsv4_proj",
    (5120, 4096): "dsv4_proj", (16384, 1280): "dsv4_proj", (12800, 6144): "engram_wkv",
    (4096, 1280): "indexer_wq_b"}
#: The Ms of the MXFP8 table: from decode batches to long prefills.
MX_GRID = (16, 32, 64, 128, 256, 384, 512, 768, 1024, 1536, 2048, 3072, 4096, 6144, 8192,
           16384)

#: The config.json fields the shapes need, of the models the reference's shipped
#: tables were measured on (no network here: the values of the published configs).
MODELS: Dict[str, dict] = {
    "Qwen/Qwen3-8B": dict(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8,
                          head_dim=128, intermediate_size=12288, num_hidden_layers=36,
                          vocab_size=151936),
    "meta-llama/Meta-Llama-3-8B": dict(hidden_size=4096, num_attention_heads=32,
                                       num_key_value_heads=8, intermediate_size=14336,
                                       num_hidden_layers=32, vocab_size=128256),
}


# ------------------------------------------------------------------ shapes


def linear_shapes(cfg: dict, tp: int = 1) -> List[Tuple[str, int, int, int]]:
    """(name, N, K, calls per step) of a decoder's unquantized linears at tensor-parallel
    size `tp` (vLLM's sharding: qkv and gate_up by columns, o and down by rows), the LM
    head's rows padded to a multiple of 64 (routes.py:419-460)."""
    cfg = cfg.get("text_config", cfg)
    hid = cfg["hidden_size"]
    heads = cfg["num_attention_heads"]
    kv = cfg.get("num_key_value_heads") or heads
    hd = cfg.get("head_dim") or hid // heads
    inter = cfg["intermediate_size"]
    layers = cfg["num_hidden_layers"]
    vocab = -(-cfg["vocab_size"] // 64) * 64
    return [
        ("qkv", (heads * hd + 2 * kv * hd) // tp, hid, layers),
        ("o", hid, heads * hd // tp, layers),
        ("gate_up", 2 * inter // tp, hid, layers),
        ("down", hid, inter // tp, layers),
        ("lm_head", vocab // tp, hid, 1),
    ]


def model_shapes(models: Sequence[str], tp: int = 1) -> Dict[Tuple[int, int], str]:
    """{(N, K): names} over the models' linears, each (N, K) once."""
    out: Dict[Tuple[int, int], str] = {}
    for name in models:
        cfg = MODELS[name] if name in MODELS else json.loads(Path(name).read_text())
        for lname, n, k, _ in linear_shapes(cfg, tp):
            prev = out.get((n, k))
            out[(n, k)] = lname if prev in (None, lname) else f"{prev},{lname}"
    return out


# ------------------------------------------------------------------ decisions


def base_path(t: Dict[str, float], min_gain: float = MIN_GAIN) -> str:
    """The answer at one measured M (times in any unit, lower is better): the fastest of
    this build's paths if it beat the engine by `min_gain`, else "fallback" (the engine's
    own); no engine time -- the engine failed its check -- gives the fastest path."""
    cand = {p: v for p, v in t.items() if p != "engine"}
    if not cand:
        return "fallback"
    best = min(cand, key=cand.get)
    if "engine" not in t:
        return best
    return best if t["engine"] / t[best] - 1 >= min_gain else "fallback"


def runs(points: Sequence[list], min_gain: float = MIN_GAIN) -> Tuple[List[list], str]:
    """[[lo, hi, path], ...] over the measured Ms (sorted), consecutive equal answers
    merged, and the answer at the largest M, which the table gives above it."""
    out: List[list] = []
    for p in sorted(points, key=lambda q: q[0]):
        path = base_path(p[1], min_gain)
        if out and out[-1][2] == path:
            out[-1][1] = p[0]
        else:
            out.append([p[0], p[0], path])
    return out, (out[-1][2] if out else "fallback")


def entry(name: str, points: Sequence[list], min_gain: float = MIN_GAIN,
          partial: bool = False) -> dict:
    """A vLLM table's entry for one (N, K). A `partial` entry (its grid cut short) answers
    nothing above its largest measured M."""
    pts = sorted(points, key=lambda q: q[0])
    rs, above = runs(pts, min_gain)
    ent = dict(name=name, runs=rs, above="fallback" if partial else above, points=pts)
    if partial:
        ent["partial"] = True
    return ent


# ------------------------------------------------------------------ timing


def _where() -> dict:
    import torch  # noqa: PLC0415

    return dict(device=torch.cuda.get_device_name(0), torch=torch.__version__,
                hip=getattr(torch.version, "hip", None),
                date=datetime.date.today().isoformat())


class Bench:
    """Times paths on one (N, K): weight copies rotated through `rotate_bytes`, each
    path's burst over them captured as a CUDA graph."""

    def __init__(self, n: int, k: int, *, rotate_bytes: int = ROTATE_BYTES, seed: int = 0):
        import torch  # noqa: PLC0415

        self.torch = torch
        self.n, self.k = n, k
        self.dev = torch.device("cuda", torch.cuda.current_device())
        copies = max(2, -(-rotate_bytes // (n * k * 2)))
        free = torch.cuda.mem_get_info(self.dev)[0]
        copies = max(2, min(copies, int(0.5 * free) // (n * k * 2)))
        g = torch.Generator(device=self.dev).manual_seed(seed)
        self.ws = [(torch.randn(n, k, device=self.dev, generator=g) * k ** -0.5).to(torch.bfloat16)
                   for _ in range(copies)]
        self.g = g

    def check(self, fn: Callable, x, out) -> float:
        """fn's result on the first copy, relative to the largest fp32 reference value."""
        torch = self.torch
        got = fn(x, self.ws[0], out)
        got = out if got is None else got
        torch.cuda.synchronize()
        ref = x.float() @ self.ws[0].float().t()
        return float((got.float() - ref).abs().max() / ref.abs().max().clamp_min(1e-30))

    def graph(self, fn: Callable, x, out, calls: int):
        torch = self.torch
        s = torch.cuda.Stream(device=self.dev)
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for i in range(2):
                fn(x, self.ws[i % len(self.ws)], out)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for i in range(calls):
                fn(x, self.ws[i % len(self.ws)], out)
        return gr

    def time(self, m: int, paths: Dict[str, Callable], rounds: int = 5,
             log: Callable[[str], None] = lambda s: None) -> Dict[str, float]:
        """{path: microseconds a call} at M = m, for the paths that pass their check."""
        torch = self.torch
        x = torch.randn(m, self.k, device=self.dev, generator=self.g).to(torch.bfloat16)
        out = torch.empty(m, self.n, device=self.dev, dtype=torch.bfloat16)
        ok = {}
        for name, fn in paths.items():
            try:
                err = self.check(fn, x, out)
            except Exception as ex:  # noqa: BLE001 -- a path that cannot run is not timed
                log(f"    {name}: {type(ex).__name__}: {ex}")
                continue
            if err > CHECK_TOL:
                log(f"    {name}: error {err:.3g} over {CHECK_TOL}: not timed")
                continue
            ok[name] = fn
        # at least 8 calls a burst, and at least every copy once
        calls = max(8, len(self.ws))
        graphs = {name: self.graph(fn, x, out, calls) for name, fn in ok.items()}
        per: Dict[str, List[float]] = {name: [] for name in graphs}
        order = list(graphs)
        for gr in graphs.values():
            gr.replay()
        torch.cuda.synchronize()
        for r in range(rounds):
            for name in (order if r % 2 == 0 else order[::-1]):
                t0 = torch.cuda.Event(enable_timing=True)
                t1 = torch.cuda.Event(enable_timing=True)
                t0.record()
                graphs[name].replay()
                t1.record()
                t1.synchronize()
                per[name].append(t0.elapsed_time(t1) * 1e3 / calls)
        del graphs
        return {name: round(statistics.median(v), 3) for name, v in per.items()}


class MxBench(Bench):
    """Bench over MXFP8 weights: copies of (fp8 e4m3 W, E8M0 scales [N, K/32]) quantized
    from ~N(0, 1/K) bf16 weights, rotated through `rotate_bytes` of fp8; a path's check is
    against the fp32 product of the same quantized bytes (the activation quantized by
    `mxfp8.quant`, the rule both paths use)."""

    def __init__(self, n: int, k: int, *, rotate_bytes: int = ROTATE_BYTES, seed: int = 0):
        import torch  # noqa: PLC0415

        from ..ops import mxfp8  # noqa: PLC0415

        self.torch = torch
        self.n, self.k = n, k
        self.dev = torch.device("cuda", torch.cuda.current_device())
        copies = max(2, -(-rotate_bytes // (n * k)))
        free = torch.cuda.mem_get_info(self.dev)[0]
        copies = max(2, min(copies, int(0.5 * free) // (n * k)))
        g = torch.Generator(device=self.dev).manual_seed(seed)
        self.ws = []
        for _ in range(copies):
            w = (torch.randn(n, k, device=self.dev, generator=g) * k ** -0.5).to(torch.bfloat16)
            self.ws.append(mxfp8.quant(w))
        self.g = g

    def check(self, fn: Callable, x, out) -> float:
        torch = self.torch
        from ..ops import mxfp8  # noqa: PLC0415

        got = fn(x, self.ws[0], out)
        got = out if got is None else got
        torch.cuda.synchronize()

        def deq(q, s):
            return q.float() * torch.pow(2.0, s.float() - 127.0).repeat_interleave(32, dim=-1)

        xq, xs = mxfp8.quant(x)
        ref = deq(xq, xs) @ deq(*self.ws[0]).t()
        return float((got.float() - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


# ------------------------------------------------------------------ the tables


def _template(schedule: Optional[str]) -> Callable:
    from ..templates import gemm as T  # noqa: PLC0415

    return lambda x, w, out: T.gemm(x, w, out=out, schedule=schedule)


def tune_gemm(nks: Sequence[Tuple[int, int]], ms: Sequence[int] = GEMM_MS, *, rounds: int = 3,
              rotate_bytes: int = ROTATE_BYTES, log: Callable[[str], None] = print) -> dict:
    """The template's route table: per (N, K) and M, the fastest candidate that takes it."""
    import torch  # noqa: PLC0415

    from ..ops import gemm_cdna  # noqa: PLC0415

    routes: Dict[str, Dict[str, str]] = {}
    points: List[dict] = []
    for n, k in nks:
        bench = Bench(n, k, rotate_bytes=rotate_bytes)
        key = f"{n}x{k}"
        routes[key] = {}
        for m in ms:
            cands = [c for c in gemm_candidates(m, n, k) if gemm_cdna.fits(c, m, n, k)]
            paths = {f"hk:{c}": _template(c) for c in cands}
            paths["hipblaslt"] = lambda x, w, out: torch.matmul(x, w.t(), out=out)
            t0 = time.monotonic()
            us = bench.time(m, paths, rounds=rounds, log=log)
            fl = 2.0 * m * n * k
            tf = {p: round(fl / v / 1e6, 1) for p, v in us.items()}
            hk_us = {p[3:]: v for p, v in us.items() if p.startswith("hk:")}
            best = min(hk_us, key=hk_us.get) if hk_us else gemm_cdna.rule(m, n, k)
            routes[key][str(m)] = best
            points.append(dict(m=m, n=n, k=k, tflops=tf, us=us))
            log(f"  {key} M={m:5d}: {best:10s} {tf.get('hk:' + best, 0):7.1f} TF  "
                f"hipblaslt {tf.get('hipblaslt', 0):7.1f} TF  ({time.monotonic() - t0:.1f} s)")
        del bench
        torch.cuda.empty_cache()
    cands = {name: [c["kernel"], {k: v for k, v in c.items() if k != "kernel"}]
             for name, c in gemm_cdna.CANDIDATES.items()}
    meta = dict(_where(), rounds=rounds, stat="median", timing="graph",
                rotate_mb=rotate_bytes >> 20)
    return dict(arch="gfx950", meta=meta, candidates=cands, routes=routes, points=points)


def gemm_candidates(m: int, n: int, k: int) -> List[str]:
    """The candidates worth timing at a shape: the decode kernels at decode M, the small
    tiles and their splits below 1024 rows, the 256 x 256 kernels from 256 rows."""
    out = []
    if m <= 32:
        out += ["decode", "decode_blk"]
    if m <= 512:
        out += ["t64", "t64w8", "t64k2", "t64k4", "t64k8", "t128n128",
                "t64x128", "t64x128k2", "t64x128k4", "t64x128k8"]
    if 64 < m <= 2048:
        out += ["t128", "t128w8", "t128k2", "t128k4", "t256n128",
                "t128x128", "t128x128k2", "t128x128k4", "q128"]
    if m >= 256:
        out += ["t256", "t256w", "t256sk", "t256k2", "t256w8"]
    if 256 <= m <= 2048:
        out += ["t256k4", "t256k8"]
    return out


def tune_linear(shapes: Dict[Tuple[int, int], str], ms: Sequence[int] = GRID, *,
                rounds: int = 5, min_gain: float = MIN_GAIN, rotate_bytes: int = ROTATE_BYTES,
                log: Callable[[str], None] = print) -> Dict[str, dict]:
    """The vLLM table's entries: per (N, K), the engine against hk and hk_decode at each M."""
    import torch  # noqa: PLC0415

    from ..ops import gemm_cdna  # noqa: PLC0415
    from . import vllm_gemm  # noqa: PLC0415

    out = {}
    for (n, k), name in shapes.items():
        bench = Bench(n, k, rotate_bytes=rotate_bytes)
        pts = []
        for m in ms:
            if name == "lm_head" and m > MAX_SEQS:
                break
            # the engine's path as vLLM's unquantized linear runs it on ROCm without its
            # own op: F.linear (hipBLASLt), allocating its output
            paths = {"engine": lambda x, w, o: torch.nn.functional.linear(x, w)}
            for path in ("hk", "hk_decode"):
                if path == "hk_decode" and not gemm_cdna.fits("decode", m, n, k):
                    continue
                run = vllm_gemm.launch_for(path, m, n, k, False)
                paths[path] = (lambda run: (lambda x, w, o: run(x, w, None)))(run)
            us = bench.time(m, paths, rounds=rounds, log=log)
            pts.append([m, us])
            log(f"  {n}x{k} ({name}) M={m:5d}: {base_path(us, min_gain):9s} " +
                "  ".join(f"{p} {v:.2f}" for p, v in us.items()))
        out[f"{n}x{k}"] = entry(name, pts, min_gain)
        del bench
        torch.cuda.empty_cache()
    return out


def tune_mxfp8(shapes: Dict[Tuple[int, int], str], ms: Sequence[int] = MX_GRID, *,
               rounds: int = 5, min_gain: float = MIN_GAIN, rotate_bytes: int = ROTATE_BYTES,
               log: Callable[[str], None] = print) -> Dict[str, dict]:
    """The MXFP8 table's entries: per (N, K), hk's quant + MX GEMM against the same quant +
    hipBLASLt's MX GEMM at each M."""
    import torch  # noqa: PLC0415

    from ..ops import mxfp8  # noqa: PLC0415

    e8m0 = torch.float8_e8m0fnu

    def engine_path(x, w, o):
        q, s = mxfp8.quant(x)
        if s.shape[0] % 128:
            # hipBLASLt reads the activation's scales in whole 128-row blocks
            s = torch.nn.functional.pad(s, (0, 0, 0, 128 - s.shape[0] % 128), value=127)
        return torch._scaled_mm(q, w[0].t(), scale_a=s.view(e8m0), scale_b=w[1].view(e8m0),
                                out_dtype=torch.bfloat16)

    def hk_path(x, w, o):
        q, s = mxfp8.quant(x)
        return mxfp8.gemm(q, w[0], s, w[1], out=o)

    out = {}
    for (n, k), name in shapes.items():
        bench = MxBench(n, k, rotate_bytes=rotate_bytes)
        pts = []
        for m in ms:
            us = bench.time(m, {"engine": engine_path, "hk": hk_path}, rounds=rounds, log=log)
            pts.append([m, us])
            log(f"  {n}x{k} ({name}) M={m:5d}: {base_path(us, min_gain):9s} " +
                "  ".join(f"{p} {v:.2f}" for p, v in us.items()))
        out[f"{n}x{k}"] = entry(name, pts, min_gain)
        del bench
        torch.cuda.empty_cache()
    return out


def main(argv: Optional[Sequence[str]] = None) -> int:
    ap = argparse.ArgumentParser(prog="python -m hk.integration.tune", description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("kind", choices=("gemm", "vllm_linear", "vllm_mxfp8"))
    ap.add_argument("--models", default=",".join(MODELS),
                    help="model names (of MODELS) or config.json paths, comma-separated")
    ap.add_argument("--tp", type=int, default=1)
    ap.add_argument("--only", default="", help="NxK[,NxK...]: just these shapes")
    ap.add_argument("--ms", default="", help="M[,M...]: instead of the default grid")
    ap.add_argument("--rounds", type=int, default=0)
    ap.add_argument("--min-gain", type=float, default=MIN_GAIN)
    ap.add_argument("--out", default="", help="the table file (default: hk/tuned/)")
    args = ap.parse_args(argv)

    import torch  # noqa: PLC0415

    from ..target import current_arch  # noqa: PLC0415

    if not torch.cuda.is_available():
        print("no GPU: nothing to measure", file=sys.stderr)
        return 2
    arch = current_arch()
    shapes = (dict(MX_SHAPES) if args.kind == "vllm_mxfp8"
              else model_shapes(args.models.split(","), args.tp))
    if args.kind == "gemm":
        # the template's grid (gemm_cdna_routes.py NK): the models' (N, K), their gate and
        # up projections unmerged, and two squares
        for name in args.models.split(","):
            cfg = MODELS[name] if name in MODELS else json.loads(Path(name).read_text())
            cfg = cfg.get("text_config", cfg)
            shapes.setdefault((cfg["intermediate_size"] // args.tp, cfg["hidden_size"]), "up")
        for sq in (4096, 8192):
            shapes.setdefault((sq, sq), "square")
    if args.only:
        want = {tuple(int(v) for v in s.split("x")) for s in args.only.split(",")}
        shapes = {nk: nm for nk, nm in shapes.items() if nk in want} or {nk: "shape" for nk in want}
    ms = [int(v) for v in args.ms.split(",")] if args.ms else None
    out = Path(args.out) if args.out else (
        Path(__file__).resolve().parents[1] / "tuned" / f"routes_{args.kind}_{arch}.json")
    out.parent.mkdir(parents=True, exist_ok=True)
    t0 = time.monotonic()
    if args.kind == "gemm":
        table = tune_gemm(sorted(shapes), ms or GEMM_MS, rounds=args.rounds or 3)
        table["arch"] = arch
    elif args.kind == "vllm_mxfp8":
        ents = tune_mxfp8(shapes, ms or MX_GRID, rounds=args.rounds or 5, min_gain=args.min_gain)
        table = dict(kind="vllm_mxfp8", arch=arch, model="DeepSeek-V4.1-Flash (TP2) shapes",
                     engine="mxfp8.quant + torch._scaled_mm (hipBLASLt MX)", tp=2,
                     min_gain=args.min_gain, rounds=args.rounds or 5,
                     rotate_mb=ROTATE_BYTES >> 20, **_where(), shapes=ents)
    else:
        ents = tune_linear(shapes, ms or GRID, rounds=args.rounds or 5, min_gain=args.min_gain)
        table = dict(kind="vllm_linear", arch=arch, model=args.models, engine="F.linear",
                     tp=args.tp, min_gain=args.min_gain, rounds=args.rounds or 5,
                     rotate_mb=ROTATE_BYTES >> 20, **_where(), shapes=ents)
    out.write_text(json.dumps(table, indent=1) + "\n")
    print(f"wrote {out} ({time.monotonic() - t0:.0f} s)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
