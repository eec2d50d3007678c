"""Plumbing the engine routes share: measured route tables, an opaque custom op with
per-path counters, and a CUDA-graph contract.

The contract the reference's engine module states (python/hk/integration/engine.py:1-424)
and this one keeps:

* a table answers, for a weight shape (N, K) and a token count M, which path measured
  fastest there; it never extrapolates between two measured runs (a gap is the
  fallback), above the largest measured M it answers what the entry says (`above`,
  default the last run's path), below the smallest or for a shape not in the table the
  fallback;
* the table file is JSON `{"arch", "kind", ..., "shapes": {"NxK": {"runs": [[lo, hi,
  path], ...], "above": path, "partial": bool}}}`, overridable by an environment
  variable, refused when measured on another arch;
* the op is `torch.ops.<ns>.<name>` with a fake for torch.compile, called without the
  dispatcher from eager code, its calls counted by path (captured calls apart);
* a patch declares itself `graph="safe"` (capturable) or `graph="never"` (with the
  reason); under capture a "never" patch raises `GraphCaptureError`, and a "safe" one runs
  inside `no_host_sync`, where a host synchronisation raises a `GraphCaptureError` naming
  the patch.

The design here: a table is compiled, per shape, into a step function over M -- sorted
breakpoints and the path holding from each breakpoint to the next, gaps already turned
into fallback steps -- so a lookup is one bisect and one index. The op is registered
through `torch.library.define` / `impl` / `register_fake`.
"""

from __future__ import annotations

import bisect
import contextlib
import functools
import json
import os
import warnings
from pathlib import Path
from typing import Callable, Dict, Iterable, List, Optional, Sequence, Tuple

GRAPH_CONTRACTS = ("safe", "never")

#: Every patch made in this process, by name.
PATCHES: Dict[str, "Patch"] = {}

_CAPTURE_WORDS = ("capturing", "capture", "synchroniz")


class GraphCaptureError(RuntimeError):
    """A patch did, under CUDA-graph capture, what a graph replay cannot repeat."""


def capturing() -> bool:
    """Whether torch's current stream is capturing a graph (asks the runtime; no sync)."""
    try:
        import torch  # noqa: PLC0415
    except ImportError:
        return False
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def compiling() -> bool:
    """Whether torch.compile is tracing the caller right now."""
    try:
        import torch  # noqa: PLC0415
    except ImportError:
        return False
    return torch.compiler.is_compiling()


def _names_a_sync(err: BaseException) -> bool:
    text = str(err).lower()
    return any(w in text for w in _CAPTURE_WORDS)


@contextlib.contextmanager
def no_host_sync(what: str):
    """A block in which a host synchronisation is an error naming `what`: torch's sync
    debug mode is raised to "error" for its duration (so a synchronising call raises
    before it runs, rather than invalidating a capture or stalling a replay), and such an
    error comes out as `GraphCaptureError`. The mode in force before is restored."""
    import torch  # noqa: PLC0415

    before = torch.cuda.get_sync_debug_mode()
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")     # torch warns when the mode is turned up
        torch.cuda.set_sync_debug_mode("error")
    try:
        yield
    except GraphCaptureError:
        raise
    except RuntimeError as err:
        if not _names_a_sync(err):
            raise
        first = str(err).splitlines()[0] if str(err) else type(err).__name__
        raise GraphCaptureError(
            f"{what} synchronised with the host (or made a call a capture refuses) while a "
            f"CUDA graph was being captured; a replay runs no Python, so anything read back "
            f"would be frozen at capture time: {first}") from err
    finally:
        torch.cuda.set_sync_debug_mode(before)


# ---------------------------------------------------------------- patches


class Patch:
    """Where an engine runs this build's kernels: the paths a call can take, counters of
    which it took (eager calls in `stats`, calls made while a graph was captured in
    `captured` -- a replay runs no Python and counts nothing), and its graph contract."""

    def __init__(self, name: str, paths: Sequence[str], *, graph: str = "safe",
                 why: str = ""):
        if graph not in GRAPH_CONTRACTS:
            raise ValueError(f"{name}: graph contract {graph!r}; one of {GRAPH_CONTRACTS}")
        if graph == "never" and not why:
            raise ValueError(f"{name}: a patch that cannot be captured says why (why=...)")
        self.name = name
        self.paths = tuple(paths)
        self.graph = graph
        self.why = why
        self.stats: Dict[str, int] = dict.fromkeys(self.paths, 0)
        self.captured: Dict[str, int] = dict.fromkeys(self.paths, 0)
        PATCHES[name] = self

    def count(self, path: str) -> None:
        book = self.captured if capturing() else self.stats
        book[path] += 1

    def reset(self) -> None:
        for p in self.paths:
            self.stats[p] = self.captured[p] = 0

    def _refuse_capture(self) -> None:
        if self.graph == "never":
            raise GraphCaptureError(
                f"{self.name} cannot run inside a CUDA graph capture: {self.why}")

    def guard(self, fn: Callable) -> Callable:
        """`fn` held to this patch's graph contract. Outside a capture it is `fn`'s cost
        plus one runtime query."""

        @functools.wraps(fn)
        def held(*args, **kwargs):
            if not capturing():
                return fn(*args, **kwargs)
            self._refuse_capture()
            with no_host_sync(self.name):
                return fn(*args, **kwargs)

        return held

    def summary(self) -> str:
        eager = ", ".join(f"{p} {self.stats[p]}" for p in self.paths)
        line = f"{self.name}: {eager}"
        if any(self.captured.values()):
            line += "; captured: " + ", ".join(f"{p} {self.captured[p]}" for p in self.paths)
        return line


class Op(Patch):
    """A patch that is an opaque torch op, `torch.ops.<ns>.<name>`: torch.compile sees only
    its fake (output shape and dtype), so a shape-dependent choice of kernel inside it is
    neither a guard nor a recompile. Eager calls through `__call__` skip the dispatcher."""

    def __init__(self, qualname: str, schema: str, fake: Callable, paths: Sequence[str],
                 **contract):
        super().__init__(qualname, paths, **contract)
        self.ns, self.op_name = qualname.split("::")
        self.schema = schema
        self.fake = fake
        self.impl: Optional[Callable] = None
        self._eager_ok = False

    @property
    def defined(self) -> bool:
        return self.impl is not None

    def _packet(self):
        import torch  # noqa: PLC0415

        return getattr(getattr(torch.ops, self.ns), self.op_name)

    def define(self, impl: Callable, dispatch: str = "CUDA") -> "Op":
        """Register the op (its schema, `impl` for `dispatch` held to the graph contract,
        and the fake). Calling it again does nothing."""
        if self.impl is not None:
            return self
        import torch  # noqa: PLC0415

        held = self.guard(impl)
        try:
            self._packet()
            fresh = False
        except (AttributeError, RuntimeError):
            fresh = True
        if fresh:
            torch.library.define(self.name, self.schema[self.schema.index("("):])
            torch.library.register_fake(self.name, self.fake)
        torch.library.impl(self.name, dispatch)(held)
        self.impl = held
        self._eager_ok = dispatch == "CUDA"
        return self

    def __call__(self, *args, **kwargs):
        """Eager, with a plain GPU tensor first: the implementation itself, under the same
        contract. Otherwise (tracing, a tensor subclass, a CPU tensor) the registered op."""
        impl = self.impl
        if impl is not None and self._eager_ok and args:
            import torch  # noqa: PLC0415

            x = args[0]
            if type(x) is torch.Tensor and x.is_cuda and not torch.compiler.is_compiling():
                return impl(*args, **kwargs)
        return self._packet()(*args, **kwargs)


# ---------------------------------------------------------------- route tables


class _Steps:
    """One shape's answers as a step function over M: `starts[i]` is the first M at which
    `paths[i]` holds; before `starts[0]` the fallback holds."""

    __slots__ = ("starts", "paths", "runs", "above", "partial")

    def __init__(self, runs: List[Tuple[int, int, str]], above: str, partial: bool,
                 fallback: str):
        self.runs, self.above, self.partial = runs, above, partial
        starts: List[int] = []
        paths: List[str] = []
        for i, (lo, hi, path) in enumerate(runs):
            starts.append(lo)
            paths.append(path)
            nxt = runs[i + 1][0] if i + 1 < len(runs) else None
            if nxt is None:
                starts.append(hi + 1)
                paths.append(above)
            elif nxt > hi + 1:
                starts.append(hi + 1)
                paths.append(fallback)
        self.starts, self.paths = starts, paths


class RouteTable:
    """Measured winners per weight shape (N, K): the runs of Ms that agreed on a path.
    `shapes` maps (N, K) to an entry dict as in the file's "shapes"."""

    def __init__(self, shapes: Dict[Tuple[int, int], dict], *, fallback: str = "fallback",
                 meta: Optional[dict] = None, source: str = ""):
        self.fallback = fallback
        self.meta = dict(meta or {})
        self.source = source
        self._steps: Dict[Tuple[int, int], _Steps] = {}
        #: where each shape's entry came from (a file, or "" for a dict)
        self.origin: Dict[Tuple[int, int], str] = {}
        #: shapes asked for that the table does not hold
        self.misses: set = set()
        self.overlay(shapes, source)

    @property
    def partial(self) -> set:
        return {nk for nk, s in self._steps.items() if s.partial}

    def _entry(self, nk, ent: dict, source: str) -> _Steps:
        runs = sorted((int(lo), int(hi), str(p)) for lo, hi, p in ent["runs"])
        for lo, hi, _ in runs:
            if hi < lo:
                raise ValueError(f"{source or 'table'}: {nk}: run [{lo}, {hi}] is empty")
        for (_, hi, _), (lo2, _, _) in zip(runs, runs[1:]):
            if lo2 <= hi:
                raise ValueError(f"{source or 'table'}: {nk}: runs overlap at M={lo2}")
        partial = bool(ent.get("partial"))
        if partial:
            above = self.fallback
        elif "above" in ent:
            above = str(ent["above"])
        else:
            above = runs[-1][2] if runs else self.fallback
        return _Steps(runs, above, partial, self.fallback)

    def overlay(self, shapes: Dict[Tuple[int, int], dict], source: str = "") -> "RouteTable":
        """Add or replace entries (each shape whole)."""
        for nk, ent in shapes.items():
            nk = (int(nk[0]), int(nk[1]))
            self._steps[nk] = self._entry(nk, ent, source)
            self.origin[nk] = source
        return self

    @staticmethod
    def parse(d: dict) -> Dict[Tuple[int, int], dict]:
        """A table file's "shapes", keyed by (N, K)."""
        out = {}
        for key, ent in d.get("shapes", {}).items():
            n, _, k = key.partition("x")
            out[(int(n), int(k))] = ent
        return out

    @classmethod
    def from_json(cls, path) -> "RouteTable":
        path = Path(path)
        d = json.loads(path.read_text())
        return cls(cls.parse(d), meta={k: v for k, v in d.items() if k != "shapes"},
                   source=str(path))

    def to_json(self) -> dict:
        shapes = {}
        for (n, k), s in self._steps.items():
            ent = {"runs": [list(r) for r in s.runs]}
            if s.partial:
                ent["partial"] = True
            elif s.above != (s.runs[-1][2] if s.runs else self.fallback):
                ent["above"] = s.above
            shapes[f"{n}x{k}"] = ent
        return {**self.meta, "shapes": shapes}

    def shapes(self) -> Iterable[Tuple[int, int]]:
        return self._steps.keys()

    def paths(self) -> set:
        """Every path some M of some shape takes."""
        return {p for s in self._steps.values() for p in s.paths}

    def routes_any(self, n: int, k: int) -> bool:
        """Whether some M of (N, K) takes a path other than the fallback."""
        s = self._steps.get((n, k))
        return s is not None and any(p != self.fallback for p in s.paths)

    def lookup(self, m: int, n: int, k: int) -> str:
        s = self._steps.get((n, k))
        if s is None:
            self.misses.add((n, k))
            return self.fallback
        i = bisect.bisect_right(s.starts, m)
        return s.paths[i - 1] if i else self.fallback


def shipped_table(kind: str, arch: str, env: str) -> Optional[RouteTable]:
    """The table for `kind` on `arch`: the file `$env` names if set (it must exist), else
    hk/tuned/routes_<kind>_<arch>.json if present, else None. A table whose "arch" is
    another one is refused."""
    named = os.environ.get(env)
    if named:
        path = Path(named)
        if not path.is_file():
            raise FileNotFoundError(f"${env} names {path}, which does not exist")
    else:
        path = Path(__file__).resolve().parents[1] / "tuned" / f"routes_{kind}_{arch}.json"
        if not path.is_file():
            return None
    table = RouteTable.from_json(path)
    measured_on = table.meta.get("arch")
    if measured_on is not None and measured_on != arch:
        raise ValueError(f"{path} holds routes measured on {measured_on}; this is {arch}")
    return table


# ---------------------------------------------------------------- vLLM compile cache


def isolate_compile_cache(route: str) -> str:
    """Point vLLM's cache root (`VLLM_CACHE_ROOT`) at a directory of its own for the
    patched engine, and return it.

    vLLM keys its compiled graphs by its config and source, not by what is patched into
    it; sharing a root with an unpatched run, a patched engine would load a graph whose
    linear layers call vLLM's GEMM and never reach the route (the reference does the
    same, python/hk/integration/vllm_gemm.py:573-598). The directory is
    `<root>/hk-<routes>`, `<routes>` the sorted '+'-joined names of every route
    applied, so the order routes are applied in does not matter, and a worker process
    that inherits the variable adds nothing."""
    env = os.environ
    root = env.get("VLLM_CACHE_ROOT")
    if not root:
        home = env.get("XDG_CACHE_HOME") or os.path.join(os.path.expanduser("~"), ".cache")
        root = os.path.join(home, "vllm")
    root = os.path.normpath(root)
    routes = {route}
    parent, leaf = os.path.split(root)
    if leaf.startswith("hk-"):
        routes.update(r for r in leaf[3:].split("+") if r)
        root = parent
    own = os.path.join(root, "hk-" + "+".join(sorted(routes)))
    env["VLLM_CACHE_ROOT"] = own
    return own


__all__ = ["Op", "Patch", "RouteTable", "GraphCaptureError", "capturing", "compiling",
           "no_host_sync",
           "shipped_table", "isolate_compile_cache", "PATCHES"]
