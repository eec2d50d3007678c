"""The boundary: libhkx.so's C ABI (include/hkx.h) through ctypes.

The reference launches a code object per Step with hipModuleLaunchKernel on torch's
current stream (python/hk/runtime/codeobj.py:265-276, mlir/python/HKLaunch.c:1-25).
Here one C call, `hkx_gemm(&args, stream)`, makes every launch of a plan on the stream
passed in -- torch's current stream -- and returns a status code; a non-zero code
raises with the library's message.

There is no fallback: if the library is not built, `lib()` raises and nothing runs.
"""

from __future__ import annotations

import ctypes
import os
import threading
from ctypes import (POINTER, Structure, c_char_p, c_float, c_int, c_int32, c_int64,
                    c_size_t, c_uint8, c_void_p)
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libhkx.so"

# ---- constants of include/hkx.h
OK, ERR_SHAPE, ERR_DTYPE, ERR_WORKSPACE, ERR_LAUNCH, ERR_ARG = range(6)
BF16, FP16, FP32, FP8E4M3, INT8 = range(5)
#: ab_dtype codes of fp8 operand pairs with e5m2: both, A e4m3 x B e5m2, A e5m2 x B e4m3
FP8E5M2, FP8_E4M3_E5M2, FP8_E5M2_E4M3 = 5, 6, 7
ROW, COL, TILE = 1, 2, 3
EP_NONE, EP_FUSED, EP_PROGRAM, EP_SILU_MUL = range(4)
ACT_NONE, ACT_GELU_TANH, ACT_SILU, ACT_RELU = range(4)
KERNEL_AUTO, KERNEL_TILE, KERNEL_DECODE = range(3)
TILE_AUTO, TILE_PINGPONG, TILE_W4, TILE_W8, TILE_RING = range(5)
PP_MFMA32, PP_ONE_TILE = 1, 2
RING_WAVESPLIT, RING_STREAMK, RING_HALFSTAGE = 4, 8, 16
#: The tile schedules by name (the route candidates' "schedule").
#: HKX_KERNEL_DECODE variant bit: the streaming kernel where it takes the call.
DEC_STREAM = 1

SCHEDULES = {"pp": TILE_PINGPONG, "w4": TILE_W4, "w8": TILE_W8, "ring": TILE_RING}

OPS = ["MOV", "LOAD", "CONST", "ROW", "COL", "ADD", "SUB", "MUL", "DIV", "MAX", "MIN",
       "EXP", "EXP2", "LOG", "LOG2", "ABS", "RELU", "GELU", "SILU", "SQRT", "RSQRT",
       "NEG", "STEP", "SELLE", "M", "TANH", "SIGMOID", "SQUARE"]
OP = {name: i for i, name in enumerate(OPS)}
MAX_OPERANDS, MAX_INSTR, MAX_REGS = 8, 64, 16


class HkxOperand(Structure):
    _fields_ = [("ptr", c_void_p), ("kind", c_int32), ("dtype", c_int32), ("ld", c_int64)]


class HkxInstr(Structure):
    _fields_ = [("op", c_uint8), ("dst", c_uint8), ("a", c_uint8), ("b", c_uint8),
                ("c", c_uint8), ("pad0", c_uint8), ("pad1", c_uint8), ("pad2", c_uint8),
                ("imm", c_float)]


class HkxEpilogue(Structure):
    _fields_ = [("form", c_int32), ("act", c_int32), ("col_scale", c_int32),
                ("row_scale", c_int32), ("row_add", c_int32), ("tile_add", c_int32),
                ("cmul", c_float), ("cadd", c_float), ("nins", c_int32), ("out_reg", c_int32),
                ("col0", c_int32), ("nops", c_int32), ("ops", HkxOperand * MAX_OPERANDS),
                ("ins", HkxInstr * MAX_INSTR)]


class HkxGemmArgs(Structure):
    _fields_ = [("a", c_void_p), ("b", c_void_p), ("c", c_void_p), ("lda", c_int64),
                ("ldb", c_int64), ("ldc", c_int64), ("m", c_int32), ("n", c_int32),
                ("k", c_int32), ("ab_dtype", c_int32), ("c_dtype", c_int32),
                ("kernel", c_int32), ("tile_m", c_int32), ("tile_n", c_int32),
                ("splits", c_int32), ("tile_schedule", c_int32), ("variant", c_int32),
                ("decode_waves", c_int32), ("decode_rows", c_int32),
                ("ws", c_void_p), ("ws_bytes", c_size_t), ("ep", HkxEpilogue),
                ("counters", c_void_p), ("counters_len", c_int64)]


#: Every function include/hkx.h declares.
SYMBOLS = ("hkx_abi_version", "hkx_abi_sizes", "hkx_last_error", "hkx_gemm_workspace",
           "hkx_gemm_counters",
           "hkx_gemm_check", "hkx_gemm", "hkx_scaled_mm", "hkx_mx_gemm", "hkx_mx_gemm_workspace",
           "hkx_mx_quant", "hkx_gemm_noalloc")

_LIB = None
_LOCK = threading.Lock()


class HkxError(RuntimeError):
    """libhkx.so refused or failed a call; `code` is its status."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


def lib() -> ctypes.CDLL:
    """libhkx.so, loaded once (after torch, so the HIP runtime torch loaded is the one
    the library binds to). Raises if it is not built: there is no other path."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        try:
            import torch  # noqa: F401,PLC0415 -- loads libamdhip64 first
        except ImportError:
            pass
        path = Path(os.environ.get("HKX_LIB", LIB_PATH))
        if not path.is_file():
            raise RuntimeError(f"hk: the gfx950 kernel library {path} is not built; run "
                               f"`python hk-dsl_amd/build.py` (or __graft_entry__.build())")
        L = ctypes.CDLL(str(path))
        L.hkx_abi_version.restype = c_int
        L.hkx_abi_sizes.argtypes = [POINTER(c_size_t)]
        L.hkx_last_error.restype = c_char_p
        L.hkx_gemm_workspace.argtypes = [POINTER(HkxGemmArgs)]
        L.hkx_gemm_workspace.restype = c_size_t
        L.hkx_gemm_counters.argtypes = [POINTER(HkxGemmArgs)]
        L.hkx_gemm_counters.restype = c_size_t
        L.hkx_gemm_check.argtypes = [POINTER(HkxGemmArgs)]
        L.hkx_gemm.argtypes = [POINTER(HkxGemmArgs), c_void_p]
        L.hkx_gemm_noalloc.argtypes = [POINTER(HkxGemmArgs), c_void_p]
        L.hkx_mx_gemm.argtypes = [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                  c_void_p, c_int64, c_void_p, c_int64, c_int32, c_int32,
                                  c_int32, c_void_p, c_size_t, c_void_p]
        L.hkx_mx_gemm_workspace.argtypes = [c_int32, c_int32, c_int32]
        L.hkx_mx_gemm_workspace.restype = c_size_t
        L.hkx_mx_quant.argtypes = [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                   c_int32, c_int32, c_void_p]
        L.hkx_scaled_mm.argtypes = [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                    c_void_p, c_int32, c_void_p, c_void_p, c_int64, c_int32,
                                    c_int32, c_int32, c_void_p, c_size_t, c_void_p]
        sizes = (c_size_t * 4)()
        L.hkx_abi_sizes(sizes)
        want = [ctypes.sizeof(t) for t in (HkxOperand, HkxInstr, HkxEpilogue, HkxGemmArgs)]
        if list(sizes) != want:
            raise RuntimeError(f"hk: libhkx.so's struct sizes {list(sizes)} differ from the "
                               f"binding's {want}; rebuild the library")
        _LIB = L
    return _LIB


def last_error() -> str:
    return lib().hkx_last_error().decode(errors="replace")


def check(code: int) -> None:
    if code != OK:
        raise HkxError(code, last_error())


# ---- torch glue

def dtype_code(dt) -> int:
    import torch  # noqa: PLC0415

    m = {torch.bfloat16: BF16, torch.float16: FP16, torch.float32: FP32,
         torch.float8_e4m3fn: FP8E4M3, torch.int8: INT8, torch.float8_e5m2: FP8E5M2}
    if dt not in m:
        raise TypeError(f"hk: {dt} is not an element type the kernels take")
    return m[dt]


def stream_of(device) -> int:
    import torch  # noqa: PLC0415

    return torch.cuda.current_stream(device).cuda_stream


_WS: dict = {}


def capturing(device) -> bool:
    """Whether `device`'s current stream is capturing a CUDA graph."""
    import torch  # noqa: PLC0415

    return torch.cuda.is_current_stream_capturing()


def workspace(device, nbytes: int):
    """A cached fp32 workspace of at least `nbytes` for (device, current stream): the
    reference's module-owned scratch (python/hk/ops/gemm_cdna_dp.py:330-338). Calls on
    one stream run in order, so they can share it.

    Under CUDA-graph capture a graph bakes the buffer's address in, so a captured call gets
    a buffer of its own, allocated in the capture -- i.e. from the graph's private memory
    pool, which lives exactly as long as the graph -- and not kept here: the caller holds it
    until its launches are enqueued, after which the capture may hand the same memory to a
    later allocation of the same graph (that runs after those launches on the stream, as
    any temporary of a captured region). The eager cache is never used in a capture: its
    buffer could be replaced (and freed) under a graph still replaying it, and two graphs
    replayed at once on different streams would share it. (Keeping every captured call's
    buffer for the life of the process, as an earlier form did, grows without bound in a
    process that captures many graphs.)"""
    import torch  # noqa: PLC0415

    if nbytes == 0:
        return None
    if capturing(device):
        return torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=device)
    key = (device, stream_of(device))
    buf = _WS.get(key)
    if buf is None or buf.numel() * 4 < nbytes:
        buf = torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=device)
        _WS[key] = buf
    return buf


_CNT: dict = {}
_CNT_GRAPH: dict = {}


def counters(device, n: int):
    """int32 arrival counters (at least `n`, all zero) for a decode call split over K, or
    None: the reference's per-shape `cnt` (python/hk/ops/decode_gemm.py:283-298), zeroed
    once when made and kept at zero by the kernel (its last arriver resets its counter).

    Eager calls get a buffer per (device, stream), since calls on one stream run in order.
    A call under CUDA-graph capture gets the device's graph buffer -- made, zeroed, by an
    eager call before the capture (e.g. a warm-up), as the reference's is -- and None if no
    eager call made one: the capture then records the split's two-launch form, with no
    memset or fill in the graph. Graphs replayed at the same time on several streams of one
    device share the graph buffer, so such replays must not overlap."""
    import torch  # noqa: PLC0415

    if n <= 0:
        return None
    if capturing(device):
        buf = _CNT_GRAPH.get(device)
        return buf if buf is not None and buf.numel() >= n else None
    key = (device, stream_of(device))
    buf = _CNT.get(key)
    if buf is None or buf.numel() < n:
        size = max(n, 4096)
        buf = torch.zeros(size, dtype=torch.int32, device=device)
        _CNT[key] = buf
        g = _CNT_GRAPH.get(device)
        if g is None or g.numel() < size:
            _CNT_GRAPH[device] = torch.zeros(size, dtype=torch.int32, device=device)
    return buf


def gemm_args(a, b, c, *, kernel=KERNEL_AUTO, tile_m=0, tile_n=0, splits=1, schedule=TILE_AUTO,
              variant=0, decode_waves=0, decode_rows=0, ep: HkxEpilogue = None) -> HkxGemmArgs:
    """HkxGemmArgs for A (M, K), B (N, K) -- (2N, K) paired -- and C (M, N) tensors."""
    args = HkxGemmArgs()
    args.a, args.b, args.c = a.data_ptr(), b.data_ptr(), c.data_ptr()
    args.lda, args.ldb, args.ldc = a.stride(0), b.stride(0), c.stride(0)
    args.m, args.k = a.shape
    args.n = c.shape[1]
    args.ab_dtype = dtype_code(a.dtype)
    args.c_dtype = dtype_code(c.dtype)
    args.kernel, args.tile_m, args.tile_n, args.splits = kernel, tile_m, tile_n, splits
    args.tile_schedule, args.variant = schedule, variant
    args.decode_waves, args.decode_rows = decode_waves, decode_rows
    if ep is not None:
        args.ep = ep
    else:
        args.ep.form = EP_NONE
        args.ep.cmul = 1.0
        args.ep.col_scale = args.ep.row_scale = args.ep.row_add = args.ep.tile_add = -1
    return args


def run(args: HkxGemmArgs, device) -> None:
    """Launch `args` on `device`'s current stream, with the workspace its plan needs."""
    L = lib()
    need = L.hkx_gemm_workspace(ctypes.byref(args))
    if need:
        ws = workspace(device, need)
        args.ws, args.ws_bytes = ws.data_ptr(), ws.numel() * 4
    # arrival counters for a decode split (one launch instead of two, measured level with
    # them); a tile kernel's split keeps its reduction launch, which measured faster
    ncnt = L.hkx_gemm_counters(ctypes.byref(args)) if args.kernel == KERNEL_DECODE else 0
    cnt = counters(device, ncnt) if ncnt and not args.counters else None
    if cnt is not None:
        args.counters, args.counters_len = cnt.data_ptr(), cnt.numel()
    check(L.hkx_gemm(ctypes.byref(args), c_void_p(stream_of(device))))


#: The no-allocation entry point's scratch per GPU (HKX_NOALLOC_SCRATCH_BYTES in hkx.h).
NOALLOC_SCRATCH_BYTES = 64 << 20


def run_noalloc(args: HkxGemmArgs, device) -> None:
    """Launch `args` through hkx_gemm_noalloc on `device`'s current stream: the workspace
    is the library's static per-GPU scratch, so nothing is allocated (calls overlapping on
    one GPU race on that scratch)."""
    check(lib().hkx_gemm_noalloc(ctypes.byref(args), c_void_p(stream_of(device))))


__all__ = ["lib", "check", "run_noalloc", "NOALLOC_SCRATCH_BYTES", "HkxError", "HkxGemmArgs", "HkxEpilogue", "HkxOperand", "HkxInstr",
           "gemm_args", "run", "workspace", "counters", "dtype_code", "SYMBOLS", "OP", "OPS"]
