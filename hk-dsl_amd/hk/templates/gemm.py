"""hk.templates.gemm: a GEMM whose store is yours, on hand-written gfx950 kernels.

    import hk

    def bias_gelu(acc, ctx):            # acc: the fp32 accumulator tile
        return (acc + ctx.bias).gelu()  # ctx.bias: one value per column of C

    y = hk.templates.gemm(x, w, epilogue=bias_gelu, bias=b)   # gelu(x @ w.T + b)

C = epilogue(A @ B^T accumulated in fp32, ctx), A (M, K) and B (N, K) bf16 (F.linear's
layout), C (M, N) in `out_dtype` (bf16 by default; fp16, fp32, int8, float8_e4m3fn).
The surface is the reference's (python/hk/templates/gemm.py:1-51, 956-1004): the same
call, the bound form, the operand kinds, `ctx`, the ready-made epilogues, `chain`,
`init_from`, `plan`, `kernels`, `kernel_for`. Behind it every launch is libhkx.so's
(include/hkx.h): the route (hk.ops.gemm_cdna.route) picks the tile kernel, its split-K
form or the decode kernel, and the epilogue runs where C is stored:

* an epilogue of the fused form -- act(acc * per-row * per-column * number + bias +
  tile + number), act gelu(tanh) / silu / relu -- in the GEMM kernel's registers
  before its one store;
* any other one in the pass that sums a split-K plan's shares (for a one-share plan,
  the GEMM stores its fp32 sum and the pass runs the epilogue) -- never on a share,
  so an epilogue that is not linear is right whatever the route.

The epilogue is a traced function: `acc` is a tile of C, `ctx` what it can read:

    ctx.<name>   an operand passed to gemm() by that name, loaded for the tile and
                 converted to fp32. Its kind follows torch's broadcasting against C:
                   (N,) or (1, N)   a row vector, one value per column (bias, scale)
                   (M, 1)           a column vector, one value per row (per-token)
                   (M, N)           a tile of C's shape (residual)
                   a Python number  baked in (a value that changes per call is a tensor)
    ctx.row, ctx.col   C's element coordinates
    ctx.m              C's rows

It returns the tile to store (or None, having changed `acc` in place): `+ - * /` with
tiles, vectors and numbers, `.gelu()` (tanh), `.silu()`, `.relu()`, `.exp()`,
`.exp2()`, `.rsqrt()`, `.maximum()`, ..., and the fills (`right_fill_` ...).

Ready-made epilogues are attributes: `gemm.bias`, `gemm.gelu`, `gemm.bias_gelu`,
`gemm.silu`, `gemm.bias_silu`, `gemm.relu`, `gemm.bias_relu`, `gemm.residual`,
`gemm.bias_residual`, `gemm.scale`, `gemm.chain(f, g, ...)`; and, new here,
`gemm.silu_and_mul`: B is (2I, K), its gate rows then its up rows (vLLM's merged
gate_up layout), and C (M, I) = silu(x @ gate^T) * (x @ up^T), both halves accumulated
in one kernel and combined in its registers.
"""

from __future__ import annotations

import ctypes
import hashlib
import inspect
import re
import sys
import types
import weakref
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Optional, Tuple

from .. import _native as nat
from . import _trace

# ---------------------------------------------------------------- operands

#: What an operand is, by its shape against C (templates/gemm.py:71).
ROW, COL, TILE, CONST = "row", "col", "tile", "const"

_RESERVED = {"a", "b", "c", "ws", "cnt", "x", "w", "epilogue", "out", "out_dtype",
             "schedule"}

_KIND_CODE = {ROW: nat.ROW, COL: nat.COL, TILE: nat.TILE}


def _torch():
    import torch  # noqa: PLC0415

    return torch


def _dtype_ok(t) -> None:
    torch = _torch()
    ok = (torch.bfloat16, torch.float16, torch.float32, torch.int8, torch.float8_e4m3fn,
          torch.float8_e5m2)
    if t not in ok:
        raise TypeError(f"hk.templates.gemm: {t} is not a dtype hk stores or loads here "
                        f"(bf16, fp16, fp32, int8, float8_e4m3fn, float8_e5m2)")


def _kind(name: str, v, m: int, n: int) -> str:
    """An operand's kind by its shape against C (M, N), as torch broadcasts it
    (templates/gemm.py:116-135)."""
    torch = _torch()
    if isinstance(v, bool) or not isinstance(v, (int, float, torch.Tensor)):
        raise TypeError(f"hk.templates.gemm: operand {name}={v!r}: a tensor or a Python number")
    if not isinstance(v, torch.Tensor):
        return CONST
    s = tuple(v.shape)
    if s == (m, n):
        return TILE  # (1, N) at M = 1 is C's shape: a tile
    if s in ((n,), (1, n)):
        return ROW
    if s == (m, 1):
        return COL
    raise ValueError(
        f"hk.templates.gemm: operand {name} is {s}; against C ({m}, {n}) it must broadcast "
        f"as torch would and be one of ({n},) or (1, {n}) -- one value a column --, "
        f"({m}, 1) -- one a row --, or ({m}, {n}). A scalar is a Python number (baked in), "
        f"or a ({n},)-shaped tensor of it.")


# ---------------------------------------------------------------- the hook

class _Tile:
    """What `ctx.tile` describes: the accumulator tile's element type (fp32)."""

    dtype = "fp32"

    def __repr__(self):
        return "RegTile(fp32, elementwise)"


class Context:
    """What an epilogue reads: operands by name, coordinates, C's rows
    (templates/gemm.py:141-227). Reading an operand gemm() was not given raises
    AttributeError naming it."""

    def __init__(self, ep: "Epilogue", g: _trace.Graph):
        self._ep, self._g = ep, g

    @property
    def row(self):
        """C's row of the element (the tile's first element's, on the reference's tiles)."""
        self._ep.uses_coords = True
        return _trace.Sym(self._g, self._g.make("ROW", kind=_trace.COLV))

    @property
    def col(self):
        """C's column of the element, in the whole C (a launch on a column slice adds its
        offset, EP_COL0 in the reference)."""
        self._ep.uses_coords = True
        return _trace.Sym(self._g, self._g.make("COL", kind=_trace.ROWV))

    @property
    def m(self):
        """C's rows."""
        return _trace.Sym(self._g, self._g.make("M", kind=_trace.SCALAR))

    @property
    def tile(self):
        return _Tile()

    def __getattr__(self, name: str):
        if name.startswith("_"):
            raise AttributeError(name)
        ep = self._ep
        kind = ep.kinds.get(name)
        if kind is None:
            raise AttributeError(
                f"the epilogue reads ctx.{name}, and gemm() was given no operand {name!r} "
                f"(it has {sorted(ep.kinds) or 'none'}). Pass it as "
                f"gemm(a, b, epilogue=..., {name}=tensor_or_number).")
        if kind == CONST:
            return ep.consts_by_name[name]
        k = {ROW: _trace.ROWV, COL: _trace.COLV, TILE: _trace.TILEV}[kind]
        return _trace.Sym(self._g, self._g.make("LOAD", name=name, kind=k))


class _Signature:
    """How an epilogue takes its arguments after the accumulator: each positional name is
    `ctx` (the context) or an operand read by that name; each keyword-only one is a number
    with a default that an operand of that name overrides. The contract of
    templates/gemm.py:341-366: fn(acc), fn(acc, ctx), fn(acc, bias, residual, *, alpha=1.0)."""

    __slots__ = ("positional", "numbers")

    def __init__(self, fn):
        label = getattr(fn, "__name__", repr(fn))
        sig = inspect.signature(fn)
        P = inspect.Parameter
        positional, numbers = [], {}
        for p in sig.parameters.values():
            if p.kind in (P.VAR_POSITIONAL, P.VAR_KEYWORD):
                positional = None
                break
            if p.kind is P.KEYWORD_ONLY:
                if p.default is P.empty:
                    raise TypeError(f"{label}: a keyword-only parameter of an epilogue is a "
                                    f"number with a default")
                numbers[p.name] = p.default
            else:
                positional.append(p.name)
        if not positional:
            raise TypeError(f"an epilogue is fn(acc, ...): the accumulator, then `ctx` or "
                            f"operands by name; {label} is {sig}")
        self.positional = tuple(positional[1:])
        self.numbers = numbers

    def invoke(self, fn, acc, ctx):
        given = ctx._ep.kinds
        args = [ctx if name == "ctx" else getattr(ctx, name) for name in self.positional]
        kwargs = {name: getattr(ctx, name) if name in given else default
                  for name, default in self.numbers.items()}
        return fn(acc, *args, **kwargs)


_SIGNATURES: "weakref.WeakKeyDictionary[Any, _Signature]" = weakref.WeakKeyDictionary()


def _signature(fn) -> _Signature:
    """`fn`'s checked signature (TypeError if it cannot be an epilogue)."""
    try:
        return _SIGNATURES[fn]
    except (KeyError, TypeError):
        pass
    sig = _Signature(fn)
    try:
        _SIGNATURES[fn] = sig
    except TypeError:
        pass
    return sig


def _params(fn):
    """(positional names after acc, keyword-only numbers with defaults) of an epilogue."""
    sig = _signature(fn)
    return list(sig.positional), dict(sig.numbers)


def _call(fn, acc, ctx):
    """`fn` applied to the tile `acc`, its parameters bound from `ctx`; None means `acc`."""
    got = _signature(fn).invoke(fn, acc, ctx)
    return acc if got is None else got


def _value_key(v) -> str:
    if isinstance(v, (bool, int, float, str, type(None))):
        return repr(v)
    if isinstance(v, tuple):
        return "(" + ",".join(_value_key(x) for x in v) + ")"
    if callable(v):
        return _fn_key(v)
    return type(v).__qualname__


def _fn_key(fn) -> str:
    """An epilogue's identity that holds across processes, for the binding's tag: a
    composed epilogue by its parts; a function by where it is defined, its byte code and
    constants, and the values its closure holds; anything else by repr."""
    if isinstance(fn, _Composed):
        return fn.key()
    code = getattr(fn, "__code__", None)
    if code is None:
        return repr(fn)
    digest = hashlib.sha1(code.co_code)
    digest.update(repr(code.co_names).encode())
    digest.update(",".join(_value_key(c) for c in code.co_consts
                           if not inspect.iscode(c)).encode())
    for sub in code.co_consts:        # nested functions and lambdas
        if inspect.iscode(sub):
            digest.update(sub.co_code)
    cells = []
    for cell in fn.__closure__ or ():
        try:
            cells.append(_value_key(cell.cell_contents))
        except ValueError:            # an empty cell
            cells.append("<empty>")
    return f"{fn.__module__}.{fn.__qualname__}#{digest.hexdigest()[:16]}[{';'.join(cells)}]"


class Epilogue:
    """A user's epilogue bound to its operands' kinds and dtypes and C's dtype, traced
    and compiled (templates/gemm.py:229-273). `compiled` is the form libhkx.so runs;
    `tag` a deterministic name."""

    def __init__(self, fn: Callable, kinds: Dict[str, str], dtypes: Dict[str, Any],
                 consts: Dict[str, float], out_dtype):
        self.fn = fn
        self.kinds = dict(kinds)
        self.dtypes = dict(dtypes)
        self.consts_by_name = dict(consts)
        self.out_dtype = out_dtype
        self.uses_coords = False
        self.paired = fn is silu_and_mul
        if not self.paired:
            _signature(fn)
        self.init = fn.init if isinstance(fn, _Composed) else None
        if self.init is not None and kinds.get(self.init) != TILE:
            raise ValueError(
                f"the epilogue starts the accumulator as ctx.{self.init} (init_from), so "
                f"gemm() needs {self.init}= an (M, N) tensor; it has {self.init} as "
                f"{kinds.get(self.init, 'nothing')}")
        #: Tensor operands, sorted by name: their order in the launch (the reference's
        #: ep_* parameters, templates/gemm.py:253).
        self.tensors = [n for n in sorted(kinds) if kinds[n] != CONST]
        h = hashlib.sha1(repr((_fn_key(fn), sorted(kinds.items()),
                               sorted((k, str(v)) for k, v in dtypes.items()),
                               sorted(consts.items()), str(out_dtype))).encode())
        base = re.sub(r"\W", "_", getattr(fn, "__name__", "fn"))[:24]
        self.tag = f"ep_{base}_{h.hexdigest()[:8]}"
        self.compiled = self._compile()

    def _trace(self):
        g = _trace.Graph()
        ctx = Context(self, g)
        acc = _trace.Sym(g, g.make("ACC", kind=_trace.TILEV))
        if self.init is not None:
            acc = acc + getattr(ctx, self.init)
        body = self.fn.stages_call if isinstance(self.fn, _Composed) else self.fn
        got = _call(body, acc, ctx)
        if not isinstance(got, _trace.Sym) or got.node.kind != _trace.TILEV:
            what = getattr(got, "node", None)
            raise TypeError(
                f"the epilogue {getattr(self.fn, '__name__', self.fn)} returned "
                f"{'a vector' if what is not None else type(got).__name__}; it returns the "
                f"tile it was given or one of the same shape -- C's elements, computed "
                f"elementwise")
        return got.node

    def _compile(self) -> _trace.Compiled:
        if self.paired:
            c = _trace.Compiled()
            c.form = "silu_mul"
            return c
        out = self._trace()
        fused = match_fused(out, self.kinds)
        if fused is not None:
            fused.uses_coords = self.uses_coords
            return fused
        index = {name: i for i, name in enumerate(self.tensors)}
        c = _trace.compile_program(out, index, nat.MAX_REGS, nat.MAX_INSTR)
        return c

    @property
    def runs_in_kernel(self) -> bool:
        """Whether the GEMM kernel's own store runs it (the fused form, or nothing)."""
        return self.compiled.form in ("none", "fused", "silu_mul")

    def struct(self) -> nat.HkxEpilogue:
        """The HkxEpilogue for this binding, operand pointers left for the call."""
        ep = nat.HkxEpilogue()
        ep.col_scale = ep.row_scale = ep.row_add = ep.tile_add = -1
        ep.cmul = 1.0
        c = self.compiled
        index = {name: i for i, name in enumerate(self.tensors)}
        ep.nops = len(self.tensors)
        if len(self.tensors) > nat.MAX_OPERANDS:
            raise ValueError(f"hk.templates.gemm: at most {nat.MAX_OPERANDS} tensor operands")
        for i, name in enumerate(self.tensors):
            ep.ops[i].kind = _KIND_CODE[self.kinds[name]]
        if c.form == "none":
            ep.form = nat.EP_NONE
        elif c.form == "silu_mul":
            ep.form = nat.EP_SILU_MUL
        elif c.form == "fused":
            ep.form = nat.EP_FUSED
            ep.act = {"none": nat.ACT_NONE, "gelu_tanh": nat.ACT_GELU_TANH,
                      "silu": nat.ACT_SILU, "relu": nat.ACT_RELU}[c.act]
            ep.cmul, ep.cadd = c.cmul, c.cadd
            for slot in ("col_scale", "row_scale", "row_add", "tile_add"):
                name = getattr(c, slot)
                setattr(ep, slot, index[name] if name else -1)
        else:
            ep.form = nat.EP_PROGRAM
            ep.nins, ep.out_reg = len(c.ins), c.out_reg
            for i, (op, d, a, b, cc, imm) in enumerate(c.ins):
                ep.ins[i] = nat.HkxInstr(nat.OP[op], d, a, b, cc, 0, 0, 0, imm)
        return ep


def match_fused(out, kinds):
    return _trace.match_fused(out, kinds)


_EPILOGUES: Dict[Any, Epilogue] = {}


def bind(fn: Callable, operands: Dict[str, Any], m: int, n: int, out_dtype) -> Epilogue:
    """The Epilogue for `fn` with these operands (tensors by kind and dtype, numbers by
    value) and C's dtype -- made once per distinct binding (templates/gemm.py:403-422)."""
    kinds, dtypes, consts = {}, {}, {}
    for name, v in operands.items():
        if name in _RESERVED or not name.isidentifier() or name.startswith("_"):
            raise ValueError(f"hk.templates.gemm: {name!r} cannot name an operand")
        k = kinds[name] = _kind(name, v, m, n)
        if k == CONST:
            consts[name] = float(v)
        else:
            _dtype_ok(v.dtype)
            dtypes[name] = v.dtype
    key = (fn, tuple(sorted(kinds.items())), tuple(sorted((k, str(d)) for k, d in dtypes.items())),
           tuple(sorted(consts.items())), str(out_dtype))
    ep = _EPILOGUES.get(key)
    if ep is None:
        ep = _EPILOGUES[key] = Epilogue(fn, kinds, dtypes, consts, out_dtype)
    return ep


# ---------------------------------------------------------------- plans

@dataclass
class Step:
    """One launch of a plan (schedules/gemm.py:36-67's fields): the kernel family, its
    schedule, the columns of C it covers, whether it carries the epilogue, where it
    stores ("out" or "scratch"), and the route candidate it came from."""

    kernel: str
    sched: Dict[str, Any]
    cols: Tuple[int, int]
    epilogue: bool = True
    into: str = "out"
    route: Optional[str] = None
    schedule: Any = field(default=None, repr=False)


def _check(m: int, n: int, k: int, ab_bytes: int = 2) -> None:
    if m < 1 or k < 1:
        raise ValueError(f"hk.templates.gemm: M={m}, K={k}; nothing to multiply")
    kstep = 128 // ab_bytes
    if k % kstep or n % 4:
        raise ValueError(f"hk.templates.gemm: K={k} must be a multiple of {kstep} and N={n} "
                         f"of 4 on gfx950; M may be anything")


def _sched_record(schedule) -> Dict[str, Any]:
    """A schedule passed to gemm(): a dict {"kernel": "tile" | "decode", ...} or a
    candidate name of hk.ops.gemm_cdna.CANDIDATES."""
    from ..ops import gemm_cdna  # noqa: PLC0415

    if isinstance(schedule, str):
        if schedule not in gemm_cdna.CANDIDATES:
            raise ValueError(f"hk.templates.gemm: schedule {schedule!r} is not one of "
                             f"{sorted(gemm_cdna.CANDIDATES)}")
        return dict(gemm_cdna.CANDIDATES[schedule], name=schedule)
    if isinstance(schedule, dict):
        rec = dict(schedule)
        if rec.get("kernel") not in ("tile", "decode"):
            raise ValueError(f"hk.templates.gemm: a schedule record names kernel 'tile' or "
                             f"'decode', got {rec.get('kernel')!r}")
        return rec
    raise TypeError(f"hk.templates.gemm: schedule is a candidate name or a record dict, "
                    f"not {type(schedule).__name__}")


def plan(m: int, n: int, k: int, arch: Optional[str] = None, *, schedule=None,
         fp8: bool = False, epilogue_in_kernel: bool = True) -> List[Step]:
    """The launches gemm() makes for an M x N x K problem, in order, and the one that
    carries the epilogue (templates/gemm.py:506-547). Needs no GPU.

    Exactly one launch writes each column of C, and it runs the epilogue; a split-K
    plan's shares go to a scratch and a reduction runs the epilogue once on their sum
    -- as does the one-share plan of an epilogue outside the fused form
    (`epilogue_in_kernel=False`)."""
    from ..ops import gemm_cdna  # noqa: PLC0415
    from ..target import current_arch  # noqa: PLC0415

    arch = arch or current_arch()
    if arch != "gfx950":
        raise ValueError(f"hk.templates.gemm: this build's kernels are gfx950's, not {arch}")
    _check(m, n, k, 1 if fp8 else 2)
    if schedule is not None:
        rec = _sched_record(schedule)
        name = rec.pop("name", "schedule")
    else:
        name = gemm_cdna.route(m, n, k, fp8=fp8)
        rec = dict(gemm_cdna.CANDIDATES[name])
    rec = gemm_cdna.resolve(rec, m, n, k, fp8=fp8)
    kernel = rec["kernel"]
    splits = rec.get("splits", 1)
    cols = (0, n)
    if splits > 1 or not epilogue_in_kernel:
        return [Step(kernel, rec, cols, False, "scratch", route=name),
                Step("reduce", {"splits": splits}, cols, True, route=name)]
    return [Step(kernel, rec, cols, True, route=name)]


# ---------------------------------------------------------------- kernels

@dataclass
class KernelDesc:
    """What a step launches in libhkx.so: the kernel template instance, by name."""

    name: str
    sched: Dict[str, Any]

    def source(self) -> str:
        return {"tile": "hk-dsl_amd/csrc/hkx_ring.hpp (ring) / hkx_pp.hpp (ping-pong) / "
                        "hkx_tile4.hpp (4 waves) / hkx_tile.hpp (8 waves)",
                "decode": "hk-dsl_amd/csrc/hkx_decode.hpp",
                "reduce": "hk-dsl_amd/csrc/hkx_reduce.hpp"}[self.name.split("<")[0]]


def kernel_for(step: Step, ep: Optional[Epilogue] = None, arch: Optional[str] = None) -> KernelDesc:
    """The kernel a step launches (with the epilogue if the step carries it)."""
    s = step.sched
    if step.kernel == "tile":
        name = (f"tile<{s['tile_m']}x{s['tile_n']}, {s['schedule']}, "
                f"splits {s.get('splits', 1)}>")
    elif step.kernel == "decode":
        name = (f"decode<waves {s.get('waves', 8)}, rows {s.get('rows', 16)}, "
                f"splits {s.get('splits', 1)}>")
    else:
        name = f"reduce<splits {s['splits']}>"
    if step.epilogue and ep is not None:
        name += f" + {ep.tag}: {ep.compiled.describe()}"
    return KernelDesc(name, dict(s))


def kernels(m: int, n: int, k: int, *, epilogue=None, out_dtype=None, arch=None,
            schedule=None, **operands):
    """The kernels gemm() would launch for an M x N x K call with these operands, as
    [(step, kernel, constexprs)]. Operands may be tensors on the "meta" device: only
    their shapes and dtypes are read. Needs no GPU."""
    tdt = _out_dtype(out_dtype)
    nn = n // 2 if epilogue is silu_and_mul else n
    ep = bind(epilogue or _identity, operands, m, nn, tdt)
    steps = plan(m, n, k, arch=arch, schedule=schedule,
                 epilogue_in_kernel=ep.runs_in_kernel)
    return [(st, kernel_for(st, ep), {}) for st in steps]


# ---------------------------------------------------------------- launch

def _operand_tensor(name: str, kind: str, v, m: int, n: int):
    """An operand as the kernels take it: fp32 / bf16 / fp16, the alignment the 4-wide
    loads need, and its stride (`ld`) -- a row vector 1 (0 where it is one broadcast
    value), a column vector its row stride, a tile its row stride."""
    torch = _torch()
    if v.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        v = v.float()  # converted to fp32 where it is loaded either way
    eb = v.element_size()
    if kind == ROW:
        v = v.reshape(n) if v.dim() == 2 else v
        if v.stride(0) == 0:
            return v, 0
        if v.stride(0) != 1 or v.data_ptr() % (4 * eb):
            v = v.contiguous().clone()
        return v, 1
    if kind == COL:
        return v, v.stride(0)
    if v.stride(1) != 1 or v.data_ptr() % (4 * eb) or (v.stride(0) * eb) % (4 * eb):
        v = v.contiguous()
    return v, v.stride(0)


class _Launch:
    """A call signature made ready: the HkxGemmArgs with everything but the pointers, and
    how each operand is prepared. `__call__` fills in the pointers and launches."""

    def __init__(self, ep: Epilogue, steps: List[Step], m: int, n: int, k: int, out_shape,
                 out_dtype, fp8: bool):
        self.ep, self.steps, self.m, self.n, self.k = ep, steps, m, n, k
        self.out_shape, self.out_dtype = out_shape, out_dtype
        st = steps[0]
        s = st.sched
        args = nat.HkxGemmArgs()
        args.m, args.n, args.k = m, out_shape[1], k
        args.ab_dtype = nat.FP8E4M3 if fp8 else nat.BF16
        args.c_dtype = nat.dtype_code(out_dtype)
        if st.kernel == "tile":
            args.kernel = nat.KERNEL_TILE
            args.tile_m, args.tile_n = s["tile_m"], s["tile_n"]
            args.tile_schedule = nat.SCHEDULES[s["schedule"]]
            args.variant = s.get("variant", 0)
        else:
            args.kernel = nat.KERNEL_DECODE
            args.decode_waves = s.get("waves", 8)
            # the paired form needs each workgroup's gate and up fragments together
            args.decode_rows = 32 if ep.paired else s.get("rows", 16)
            args.variant = s.get("variant", 0)
        args.splits = s.get("splits", 1)
        args.ep = ep.struct()
        self.args = args
        self.size = ctypes.sizeof(nat.HkxGemmArgs)
        self.lib = nat.lib()
        self.ncnt = None  # arrival counters the plan takes (asked once, at the first call)

    def __call__(self, a, b, out, operands: Dict[str, Any]):
        if a.stride(1) != 1 or (a.stride(0) * a.element_size()) % 16 or a.data_ptr() % 16:
            a = a.contiguous()
        if b.stride(1) != 1 or (b.stride(0) * b.element_size()) % 16 or b.data_ptr() % 16:
            b = b.contiguous()
        args = nat.HkxGemmArgs()
        ctypes.memmove(ctypes.addressof(args), ctypes.addressof(self.args), self.size)
        args.a, args.b, args.c = a.data_ptr(), b.data_ptr(), out.data_ptr()
        args.lda, args.ldb, args.ldc = a.stride(0), b.stride(0), out.stride(0)
        keep = []
        for i, name in enumerate(self.ep.tensors):
            t, ld = _operand_tensor(name, self.ep.kinds[name], operands[name], self.m,
                                    self.out_shape[1])
            keep.append(t)
            o = args.ep.ops[i]
            o.ptr, o.dtype, o.ld = t.data_ptr(), nat.dtype_code(t.dtype), ld
        dev = a.device
        L = self.lib
        need = L.hkx_gemm_workspace(ctypes.byref(args))
        if need:
            ws = nat.workspace(dev, need)
            args.ws, args.ws_bytes = ws.data_ptr(), ws.numel() * 4
        if self.ncnt is None:
            # a decode split finishes in the kernel (one launch; measured level with the
            # two-launch form); a tile split keeps its reduction launch (the in-kernel finish
            # of the 4-wave kernel measured 4-10 us slower at M = 16-128)
            self.ncnt = (L.hkx_gemm_counters(ctypes.byref(args))
                         if args.kernel == nat.KERNEL_DECODE else 0)
        if self.ncnt:
            cnt = nat.counters(dev, self.ncnt)
            if cnt is not None:
                args.counters, args.counters_len = cnt.data_ptr(), cnt.numel()
        nat.check(L.hkx_gemm(ctypes.byref(args), ctypes.c_void_p(nat.stream_of(dev))))
        return out


#: (epilogue, shapes, dtypes, device, operand signatures) -> a prepared launch: a call
#: that hits it only fills pointers and launches (templates/gemm.py:728-760).
_LAUNCH: Dict[Tuple, Any] = {}


def _sig(item):
    name, v = item
    try:
        return (name, tuple(v.shape), v.dtype, v.stride())
    except AttributeError:
        return (name, type(v), v)


def _out_dtype(out_dtype):
    torch = _torch()
    if out_dtype is None:
        return torch.bfloat16
    if out_dtype not in (torch.bfloat16, torch.float16, torch.float32, torch.int8,
                         torch.float8_e4m3fn):
        raise TypeError(f"hk.templates.gemm: out_dtype {out_dtype}; bf16, fp16, fp32, int8 "
                        f"or float8_e4m3fn")
    return out_dtype


def _identity(acc):
    return acc


def _gemm(a, b, epilogue=None, out=None, out_dtype=None, schedule=None, **operands):
    key = (epilogue, tuple(a.shape), tuple(b.shape), a.dtype, b.dtype,
           out_dtype if out is None else (tuple(out.shape), out.dtype, out.stride()),
           a.device, tuple(map(_sig, operands.items())),
           None if schedule is None else repr(sorted(_sched_record(schedule).items())))
    try:
        got = _LAUNCH[key]
    except KeyError:
        got = _LAUNCH[key] = _slow(a, b, epilogue, out, out_dtype, operands, schedule)
    except TypeError:  # an unhashable operand
        got = _slow(a, b, epilogue, out, out_dtype, operands, schedule)
    go, shape, dtype = got
    if out is None:
        out = _torch().empty(shape, device=a.device, dtype=dtype)
    return go(a, b, out, operands)


def _slow(a, b, epilogue, out, out_dtype, operands, schedule=None):
    """Check a call and make its launch: (go, C's shape, C's dtype)
    (templates/gemm.py:770-803)."""
    torch = _torch()
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError(f"hk.templates.gemm: want A (M, K) and B (N, K), got "
                         f"{tuple(a.shape)} and {tuple(b.shape)}")
    m, k = a.shape
    n, kb = b.shape
    if kb != k:
        raise ValueError(f"hk.templates.gemm: A is (M={m}, K={k}) and B is (N={n}, K={kb}); "
                         f"B is passed (N, K), as to F.linear")
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise TypeError(f"hk.templates.gemm: A and B are bf16, got {a.dtype} and {b.dtype}")
    if not a.is_cuda or b.device != a.device:
        raise ValueError("hk.templates.gemm: A and B are on one GPU")
    paired = epilogue is silu_and_mul
    if paired and n % 2:
        raise ValueError(f"hk.templates.gemm: silu_and_mul takes B (2I, K), gate rows then "
                         f"up rows; N={n} is odd")
    cn = n // 2 if paired else n
    tdt = out.dtype if out is not None else _out_dtype(out_dtype)
    _out_dtype(tdt)
    if out is not None and (tuple(out.shape) != (m, cn) or out.stride(1) != 1):
        raise ValueError(f"hk.templates.gemm: out is {tuple(out.shape)}, expected ({m}, {cn}) "
                         f"with unit column stride")
    ep = bind(epilogue or _identity, operands, m, cn, tdt)
    for name in ep.tensors:
        if operands[name].device != a.device:
            raise ValueError(f"hk.templates.gemm: operand {name} is on {operands[name].device}, "
                             f"A on {a.device}")
    steps = plan(m, cn if not paired else n, k, schedule=schedule,
                 epilogue_in_kernel=ep.runs_in_kernel)
    if paired:
        for st in steps:
            st.cols = (0, cn)
    go = _Launch(ep, steps, m, cn, k, (m, cn), tdt, fp8=False)
    return go, (m, cn), tdt


# ---------------------------------------------------------------- ready-made

def bias(acc, ctx):
    """acc + bias, bias one value per column of C: F.linear's."""
    return acc + ctx.bias


#: GELU(tanh) is x * sigmoid(2u), u = sqrt(2/pi)(x + 0.044715 x^3). The kernels evaluate
#: it as x * rsqrt(1 + 2^(x (A x^2 + B)))^2 -- one exp2 and one rsqrt (the reference's
#: instruction form, templates/gemm.py:814-837); here it is one traced `gelu` op.
def gelu_tanh(x):
    """GELU, tanh approximation, of a tile, in place; returns it."""
    return x.gelu_()


def gelu(acc):
    """GELU, tanh approximation (F.gelu(..., approximate="tanh"))."""
    return gelu_tanh(acc)


def silu(acc):
    """SiLU, x * sigmoid(x)."""
    return acc.silu()


def relu(acc):
    return acc.relu()


def bias_gelu(acc, ctx):
    """gelu(acc + bias), tanh approximation."""
    acc += ctx.bias
    return gelu_tanh(acc)


def bias_silu(acc, ctx):
    return (acc + ctx.bias).silu()


def bias_relu(acc, ctx):
    return (acc + ctx.bias).relu()


def _residual(acc):
    """acc + residual, residual (M, N): the accumulator starts as the residual."""
    return acc


def _bias_residual(acc, ctx):
    """acc + bias + residual, the accumulator starting as the residual."""
    return acc + ctx.bias


_residual.__name__ = "residual"
_bias_residual.__name__ = "bias_residual"


def scale(acc, ctx):
    """acc * scale: a number, a per-channel (N,) or a per-row (M, 1) vector. With
    out_dtype int8 or float8_e4m3fn this is a quantizer: the store rounds to nearest
    even and saturates (fp8 at +-448, where torch's cast gives NaN)."""
    return acc * ctx.scale


def silu_and_mul(acc, ctx=None):
    """The paired epilogue: with B (2I, K) -- gate rows then up rows -- C (M, I) =
    silu(A gate^T) * (A up^T), fp32 math, one rounding (vLLM's SiluAndMul fused into the
    gate_up GEMM; the reference runs it as a separate kernel, ops/fused.py:80-114)."""
    raise TypeError("silu_and_mul is a paired epilogue: pass it as "
                    "gemm(x, w_gate_up, epilogue=gemm.silu_and_mul)")


class _Composed:
    """An epilogue built from others: optionally an (M, N) operand the accumulator starts
    from (`init`), then `stages` applied in order, each to what the previous returned, all
    reading the same ctx. What `chain` and `init_from` return."""

    def __init__(self, stages: Tuple[Callable, ...], init: Optional[str], name: str,
                 qualname: str, doc: Optional[str] = None):
        for f in stages:
            _signature(f)
        self.stages = tuple(stages)
        self.init = init
        self.__name__ = name
        self.__qualname__ = qualname
        self.__doc__ = doc

    def stages_call(self, acc, ctx):
        """The stages alone, the accumulator already started from `init`."""
        for f in self.stages:
            acc = _call(f, acc, ctx)
        return acc

    def __call__(self, acc, ctx):
        return self.stages_call(acc, ctx)

    def key(self) -> str:
        inner = ",".join(_fn_key(f) for f in self.stages)
        return f"init_from({self.init})[{inner}]" if self.init else f"chain[{inner}]"

    def __repr__(self) -> str:
        return f"<epilogue {self.__qualname__}>"


def _label(f, attr="__name__") -> str:
    return getattr(f, attr, None) or type(f).__name__


def chain(*fns: Callable) -> Callable:
    """One epilogue that applies `fns` in order, each to what the previous returned, all
    reading the same ctx (templates/gemm.py:891-915). An `init_from` epilogue may only
    come first: it decides where the accumulator starts."""
    for f in fns[1:]:
        if isinstance(f, _Composed) and f.init:
            raise ValueError("chain: an init_from epilogue starts the accumulator, so it can "
                             "only come first")
    init = None
    stages: List[Callable] = []
    for i, f in enumerate(fns):
        if i == 0 and isinstance(f, _Composed) and f.init:
            init = f.init
            stages.extend(f.stages)
        else:
            stages.append(f)
    name = "_".join(_label(f) for f in fns)
    qual = "chain(" + ", ".join(_label(f, "__qualname__") for f in fns) + ")"
    if init:
        qual = f"init_from({init!r})({qual})"
    return _Composed(tuple(stages), init, name, qual)


def init_from(name: str) -> Callable:
    """Decorator: the accumulator starts as the (M, N) operand `name` instead of zero, so
    C = fn(name + A @ B^T, ctx) -- BLAS's beta * C with beta 1 (templates/gemm.py:924-945).
    The kernels add it where they store, in fp32, before the epilogue."""
    if not isinstance(name, str) or not name.isidentifier():
        raise TypeError(f"init_from takes an operand's name, not {name!r}")

    def start_from(fn):
        if isinstance(fn, _Composed):
            if fn.init:
                raise ValueError(f"init_from({name!r}): {fn.__qualname__} already starts "
                                 f"from {fn.init!r}")
            stages = fn.stages
        else:
            stages = (fn,)
        return _Composed(stages, name, _label(fn),
                         f"init_from({name!r})({_label(fn, '__qualname__')})",
                         getattr(fn, "__doc__", None))

    return start_from


residual = init_from("residual")(_residual)
bias_residual = init_from("residual")(_bias_residual)

READY = {f.__name__: f for f in (bias, gelu, silu, relu, bias_gelu, bias_silu, bias_relu,
                                 residual, bias_residual, scale, gelu_tanh, silu_and_mul)}


class _Bound:
    """gemm(epilogue=..., **operands) with no A and B: the same call waiting for them.
    Calling it with (a, b) and optionally out= and more operands launches."""

    def __init__(self, epilogue, out, out_dtype, schedule, operands):
        self._epilogue, self._out, self._out_dtype = epilogue, out, out_dtype
        self._schedule, self._operands = schedule, operands
        self.__name__ = f"gemm[{getattr(epilogue, '__name__', 'plain')}]"

    def __call__(self, a, b, *, out=None, **more):
        ops = dict(self._operands)
        ops.update(more)
        return _gemm(a, b, epilogue=self._epilogue,
                     out=self._out if out is None else out,
                     out_dtype=self._out_dtype, schedule=self._schedule, **ops)

    def __repr__(self) -> str:
        return f"<{self.__name__}>"


class _GemmModule(types.ModuleType):
    """This module is itself the template: `hk.templates.gemm(a, b, ...)` -- and, after
    `import hk.templates.gemm`, the module that name now binds -- launches, and its
    attributes (the ready-made epilogues, `plan`, `kernels`, `kernel_for`, `chain`,
    `init_from`, `Context`, `Step`) are the module's own (templates/gemm.py:956-1004)."""

    def __call__(self, a=None, b=None, *, epilogue=None, out=None, out_dtype=None,
                 schedule=None, **operands):
        if a is None and b is None:
            return _Bound(epilogue, out, out_dtype, schedule, operands)
        if a is None or b is None:
            raise TypeError("hk.templates.gemm(a, b, ...) takes both A and B, or neither (to "
                            "bind the epilogue for later)")
        return _gemm(a, b, epilogue=epilogue, out=out, out_dtype=out_dtype,
                     schedule=schedule, **operands)

    def __repr__(self) -> str:
        return "<hk.templates.gemm>"


sys.modules[__name__].__class__ = _GemmModule
#: The template (this module): `from hk.templates.gemm import gemm` works too.
gemm = sys.modules[__name__]

__all__ = ["gemm", "plan", "kernels", "kernel_for", "bind", "init_from", "Step", "Context",
           "Epilogue", "chain", "READY", *READY]
