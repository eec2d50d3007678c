"""What an engine patch needs: an opaque torch custom op with a fake, counters of which
way calls went, a CUDA-graph contract that is checked, and a route table that is a
measurement rather than a rule.

Restates python/hk/integration/engine.py's contract (:1-424):

* `Op` -- `torch.ops.<ns>.<name>` defined with a schema and a fake (what torch.compile
  traces), its implementation called directly in eager code (no dispatcher on the hot
  path), guarded under capture;
* `Patch.guard` -- under CUDA-graph capture a `graph="never"` patch raises
  `GraphCaptureError`, and a `graph="safe"` one runs with torch's sync debug mode set
  to error, so a host sync inside it raises there, naming the patch (`no_host_sync`);
* `RouteTable` -- for each (N, K), runs `[lo, hi, path]` of measured Ms that agreed; an
  M inside a run takes its path, an M between two runs takes the fallback (the table
  does not guess which side of a tooth it is on), above the largest run the path
  measured there (`above`), below the smallest or for an unmeasured shape the fallback;
* `shipped_table` -- the table file for a kind and arch, `$env` overriding it.
"""

from __future__ import annotations

import bisect
import contextlib
import functools
import json
import os
from pathlib import Path
from typing import Callable, Dict, Iterable, List, Optional, Sequence, Tuple

GRAPH_CONTRACTS = ("safe", "never")

#: Every patch constructed, by name.
PATCHES: Dict[str, "Patch"] = {}


class GraphCaptureError(RuntimeError):
    """A patch did, under CUDA-graph capture, something a replay cannot repeat."""


def capturing() -> bool:
    """Whether the current stream is capturing a CUDA graph (no sync)."""
    try:
        import torch  # noqa: PLC0415
    except ImportError:
        return False
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


@contextlib.contextmanager
def no_host_sync(what: str):
    """Raise `GraphCaptureError` naming `what` at any host sync inside."""
    import warnings  # noqa: PLC0415

    import torch  # noqa: PLC0415

    prev = torch.cuda.get_sync_debug_mode()
    with warnings.catch_warnings():
        warnings.filterwarnings("ignore", message="Synchronization debug mode")
        torch.cuda.set_sync_debug_mode("error")
    try:
        yield
    except RuntimeError as ex:
        msg = str(ex)
        if isinstance(ex, GraphCaptureError) or not ("synchroniz" in msg
                                                     or "stream is capturing" in msg):
            raise
        raise GraphCaptureError(
            f"{what} synchronized with the host while a CUDA graph was being captured; a "
            f"replay runs no Python, so whatever it read back is frozen at the capture's "
            f"value. ({msg.splitlines()[0]})") from ex
    finally:
        torch.cuda.set_sync_debug_mode(prev)


class Patch:
    """One place an engine runs this build's kernels: its paths, counted (captured calls
    apart), and its CUDA-graph contract."""

    def __init__(self, name: str, paths: Sequence[str], *, graph: str = "safe", why: str = ""):
        if graph not in GRAPH_CONTRACTS:
            raise ValueError(f"graph contract {graph!r} is not one of {GRAPH_CONTRACTS}")
        if graph != "safe" and not why:
            raise ValueError(f"{name}: a patch that cannot be captured says why")
        self.name, self.paths, self.graph, self.why = name, tuple(paths), graph, why
        self.stats: Dict[str, int] = {p: 0 for p in self.paths}
        self.captured: Dict[str, int] = {p: 0 for p in self.paths}
        PATCHES[name] = self

    def count(self, path: str) -> None:
        (self.captured if capturing() else self.stats)[path] += 1

    def reset(self) -> None:
        for d in (self.stats, self.captured):
            for p in d:
                d[p] = 0

    def check_capture(self) -> None:
        if self.graph == "never" and capturing():
            raise GraphCaptureError(f"{self.name} is declared graph='never' and is being "
                                    f"captured: {self.why}")

    def guard(self, fn: Callable) -> Callable:
        """`fn` under this patch's contract; free outside capture."""

        @functools.wraps(fn)
        def guarded(*args, **kwargs):
            if not capturing():
                return fn(*args, **kwargs)
            self.check_capture()
            with no_host_sync(self.name):
                return fn(*args, **kwargs)

        return guarded

    def summary(self) -> str:
        def fmt(d):
            return ", ".join(f"{p} {n}" for p, n in d.items())

        cap = sum(self.captured.values())
        return f"{self.name}: {fmt(self.stats)}" + (f"; captured: {fmt(self.captured)}" if cap else "")


class Op(Patch):
    """A patch that is an opaque torch custom op `torch.ops.<ns>.<name>`."""

    def __init__(self, qualname: str, schema: str, fake: Callable, paths: Sequence[str], **kw):
        super().__init__(qualname, paths, **kw)
        self.ns, self.op_name = qualname.split("::")
        self.schema, self.fake = schema, fake
        self._lib = None
        self._op = None
        self._direct = None

    @property
    def defined(self) -> bool:
        return self._lib is not None

    def define(self, impl: Callable, dispatch: str = "CUDA") -> "Op":
        """Register `impl`, guarded, and the fake. Idempotent."""
        if self._lib is not None:
            return self
        import torch  # noqa: PLC0415

        lib = torch.library.Library(self.ns, "FRAGMENT")
        lib.define(self.schema)
        guarded = self.guard(impl)
        lib.impl(self.op_name, guarded, dispatch)
        torch.library.register_fake(self.name, self.fake, lib=lib)
        self._lib = lib
        self._op = getattr(getattr(torch.ops, self.ns), self.op_name)
        if dispatch == "CUDA":
            self._direct = (guarded, torch.Tensor, torch.compiler.is_compiling)
        return self

    def __call__(self, *args, **kwargs):
        """The op -- or, in eager code on a GPU tensor, what it would run, called without
        the dispatcher under the same capture contract."""
        if self._direct is not None and args:
            guarded, tensor, compiling = self._direct
            x = args[0]
            if type(x) is tensor and x.is_cuda and not compiling():
                return guarded(*args, **kwargs)
        op = self._op
        if op is None:
            import torch  # noqa: PLC0415

            op = getattr(getattr(torch.ops, self.ns), self.op_name)
        return op(*args, **kwargs)


class RouteTable:
    """Measured winners: for each (N, K), which path each measured M took, as runs
    `[lo, hi, path]` (see the module docstring)."""

    def __init__(self, shapes: Dict[Tuple[int, int], dict], *, fallback: str = "fallback",
                 meta: Optional[dict] = None, source: str = ""):
        self.fallback = fallback
        self.meta = meta or {}
        self.source = source
        self._runs: Dict[Tuple[int, int], List[Tuple[int, int, str]]] = {}
        self._lows: Dict[Tuple[int, int], List[int]] = {}
        self._above: Dict[Tuple[int, int], str] = {}
        self.origin: Dict[Tuple[int, int], str] = {}
        self.partial: set = set()
        self.misses: set = set()
        for nk, ent in shapes.items():
            self._add(nk, ent, source)

    def _add(self, nk, ent: dict, source: str) -> None:
        rs = sorted((int(lo), int(hi), str(p)) for lo, hi, p in ent["runs"])
        for (lo1, hi1, _), (lo2, _, _) in zip(rs, rs[1:]):
            if lo2 <= hi1:
                raise ValueError(f"{source}: runs for {nk} overlap at M={lo2}")
        for lo, hi, _ in rs:
            if hi < lo:
                raise ValueError(f"{source}: run [{lo}, {hi}] for {nk} is empty")
        self._runs[nk] = rs
        self._lows[nk] = [r[0] for r in rs]
        self._above[nk] = str(ent.get("above", rs[-1][2] if rs else self.fallback))
        if ent.get("partial"):
            self.partial.add(nk)
            self._above[nk] = self.fallback
        else:
            self.partial.discard(nk)
        self.origin[nk] = source

    def overlay(self, shapes: Dict[Tuple[int, int], dict], source: str) -> "RouteTable":
        """Replace or add entries, each shape whole."""
        for nk, ent in shapes.items():
            self._add(nk, ent, source)
        return self

    @staticmethod
    def parse(d: dict) -> Dict[Tuple[int, int], dict]:
        out = {}
        for key, ent in d.get("shapes", {}).items():
            n, k = (int(v) for v in key.split("x"))
            out[(n, k)] = ent
        return out

    @classmethod
    def from_json(cls, path) -> "RouteTable":
        path = Path(path)
        d = json.loads(path.read_text())
        meta = {k: v for k, v in d.items() if k != "shapes"}
        return cls(cls.parse(d), meta=meta, source=str(path))

    def to_json(self) -> dict:
        shapes = {}
        for (n, k), rs in self._runs.items():
            ent = {"runs": [list(r) for r in rs]}
            if self._above[(n, k)] != (rs[-1][2] if rs else self.fallback):
                ent["above"] = self._above[(n, k)]
            if (n, k) in self.partial:
                ent["partial"] = True
            shapes[f"{n}x{k}"] = ent
        return {**self.meta, "shapes": shapes}

    def shapes(self) -> Iterable[Tuple[int, int]]:
        return self._runs.keys()

    def paths(self) -> set:
        return {p for rs in self._runs.values() for _, _, p in rs} | set(self._above.values())

    def routes_any(self, n: int, k: int) -> bool:
        """Whether some M of (N, K) takes a path other than the fallback."""
        rs = self._runs.get((n, k))
        if not rs:
            return False
        return any(p != self.fallback for _, _, p in rs) or self._above[(n, k)] != self.fallback

    def lookup(self, m: int, n: int, k: int) -> str:
        rs = self._runs.get((n, k))
        if not rs:
            self.misses.add((n, k))
            return self.fallback
        i = bisect.bisect_right(self._lows[(n, k)], m) - 1
        if i < 0:
            return self.fallback
        lo, hi, path = rs[i]
        if m <= hi:
            return path
        return self._above[(n, k)] if i == len(rs) - 1 else self.fallback


def shipped_table(kind: str, arch: str, env: str) -> Optional[RouteTable]:
    """The routing table for `kind` on `arch`: `$env` if set, else hk/tuned/'s file,
    else None. A table measured on another arch is refused."""
    override = os.environ.get(env)
    path = Path(override) if override else (
        Path(__file__).resolve().parents[1] / "tuned" / f"routes_{kind}_{arch}.json")
    if override and not path.is_file():
        raise FileNotFoundError(f"${env} names {path}, which does not exist")
    t = RouteTable.from_json(path) if path.is_file() else None
    if t is not None and t.meta.get("arch") not in (None, arch):
        raise ValueError(f"{path} was measured on {t.meta['arch']}, not {arch}")
    return t


__all__ = ["Op", "Patch", "RouteTable", "GraphCaptureError", "no_host_sync", "capturing",
           "shipped_table", "PATCHES"]
