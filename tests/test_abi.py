"""The C-ABI library on the CPU: it loads, exports every function include/hkx.h declares,
agrees with the ctypes binding on struct layouts, checks arguments the way the
reference's Python raises (templates/gemm.py:770-803), sizes workspaces, and every kernel
it launches was actually compiled into it. No kernel is launched here."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from hk import _native as nat

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "hkx.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|void|const char\*)\s+(hkx_\w+)\(", text, re.M)))


def test_the_library_exports_every_declared_symbol():
    L = nat.lib()
    names = _declared()
    assert set(names) == set(nat.SYMBOLS)
    for name in names:
        assert hasattr(L, name), name
    assert L.hkx_abi_version() == 4


def test_no_kernel_launch_stub_is_missing():
    """Every kernel a launcher names is defined in the library: a launch stub the host
    pass dropped would be an undefined symbol (and the library would not load)."""
    out = subprocess.run(["nm", "-D", "--undefined-only", str(nat.LIB_PATH)], capture_output=True,
                         text=True).stdout
    assert "__device_stub__" not in out


def _args(m=64, n=128, k=128, **kw):
    a = nat.HkxGemmArgs()
    a.a, a.b, a.c = 0x10000, 0x20000, 0x30000  # never dereferenced: no launch happens
    a.lda = a.ldb = k
    a.ldc = n
    a.m, a.n, a.k = m, n, k
    a.ab_dtype, a.c_dtype = nat.BF16, nat.BF16
    a.kernel = nat.KERNEL_TILE
    a.tile_m, a.tile_n, a.splits = 128, 256, 1
    a.ep.form = nat.EP_NONE
    a.ep.cmul = 1.0
    a.ep.col_scale = a.ep.row_scale = a.ep.row_add = a.ep.tile_add = -1
    for key, v in kw.items():
        setattr(a, key, v)
    return a


def _check(args):
    L = nat.lib()
    rc = L.hkx_gemm_check(ctypes.byref(args))
    return rc, nat.last_error()


def test_argument_checks():
    assert _check(_args()) == (nat.OK, "")
    rc, msg = _check(_args(k=100))
    assert rc == nat.ERR_SHAPE and "multiple of 64" in msg
    rc, msg = _check(_args(n=130))
    assert rc == nat.ERR_SHAPE
    rc, msg = _check(_args(ab_dtype=nat.FP32))
    assert rc == nat.ERR_DTYPE
    rc, msg = _check(_args(m=0))
    assert rc == nat.ERR_SHAPE and "nothing to multiply" in msg
    rc, msg = _check(_args(tile_m=96))
    assert rc == nat.ERR_ARG
    rc, msg = _check(_args(kernel=nat.KERNEL_DECODE, m=40))
    assert rc == nat.ERR_SHAPE and "M <= 32" in msg
    rc, msg = _check(_args(lda=100))
    assert rc == nat.ERR_SHAPE
    # fp8 takes K in 128s
    rc, msg = _check(_args(ab_dtype=nat.FP8E4M3, k=192, lda=192, ldb=192))
    assert rc == nat.ERR_SHAPE and "multiple of 128" in msg
    # the paired silu-and-mul form is bf16 / e4m3 only: an e5m2 pair is refused for that
    e5 = _args(ab_dtype=nat.FP8E5M2, k=256, lda=256, ldb=256, m=256, n=256, tile_m=256,
               tile_n=256, kernel=nat.KERNEL_TILE)
    e5.ep.form = nat.EP_SILU_MUL
    rc, msg = _check(e5)
    assert rc == nat.ERR_ARG and "silu-and-mul" in msg and "e5m2" in msg


def test_epilogue_checks():
    a = _args()
    a.ep.form = nat.EP_FUSED
    a.ep.row_add = 0
    a.ep.nops = 1
    a.ep.ops[0] = nat.HkxOperand(0x40000, nat.COL, nat.BF16, 1)  # a COL where a ROW belongs
    rc, msg = _check(a)
    assert rc == nat.ERR_ARG and "row_add" in msg
    a.ep.ops[0] = nat.HkxOperand(0x40000, nat.ROW, nat.INT8, 1)
    rc, msg = _check(a)
    assert rc == nat.ERR_DTYPE
    a.ep.ops[0] = nat.HkxOperand(0x40002, nat.ROW, nat.BF16, 1)  # misaligned for 8-byte loads
    rc, msg = _check(a)
    assert rc == nat.ERR_SHAPE
    a.ep.ops[0] = nat.HkxOperand(0x40000, nat.ROW, nat.BF16, 1)
    assert _check(a)[0] == nat.OK
    p = _args()
    p.ep.form = nat.EP_PROGRAM
    p.ep.nins = 1
    p.ep.ins[0] = nat.HkxInstr(nat.OP["LOAD"], 1, 3, 0, 0, 0, 0, 0, 0.0)  # operand 3 of 0
    p.ws, p.ws_bytes = 0x50000, 1 << 30
    rc, msg = _check(p)
    assert rc == nat.ERR_ARG and "loads operand" in msg


def test_workspace_sizes():
    L = nat.lib()
    assert L.hkx_gemm_workspace(ctypes.byref(_args())) == 0
    assert L.hkx_gemm_workspace(ctypes.byref(_args(splits=2))) == 2 * 64 * 128 * 4
    # 2 k-steps cannot take 3 splits: capped at 2
    assert L.hkx_gemm_workspace(ctypes.byref(_args(splits=3))) == 2 * 64 * 128 * 4
    prog = _args()
    prog.ep.form = nat.EP_PROGRAM
    assert L.hkx_gemm_workspace(ctypes.byref(prog)) == 64 * 128 * 4
    pair = _args()
    pair.ep.form = nat.EP_SILU_MUL
    pair.splits = 2
    assert L.hkx_gemm_workspace(ctypes.byref(pair)) == 2 * 64 * 256 * 4
    # a plan that needs a workspace refuses to run without one
    rc, msg = _check(_args(splits=2))
    assert rc == nat.ERR_WORKSPACE
    # stream-K on the ring route: 2048 rows (8 tile rows, 32 tile columns a wave of the 256
    # CUs this host-only call assumes), N = 9216: the last 1024 columns (32 tiles) split
    # min(256 / 32, 8 K units / 4, 8) = 2 ways -> 2 shares of 2048 x 1024 fp32
    sk = _args(m=2048, n=9216, k=512, tile_m=256, tile_n=256, tile_schedule=nat.TILE_RING,
               variant=nat.RING_STREAMK)
    assert L.hkx_gemm_workspace(ctypes.byref(sk)) == 2 * 2048 * 1024 * 4
    sk.n = 8192  # whole waves: nothing is split
    assert L.hkx_gemm_workspace(ctypes.byref(sk)) == 0
    sk.variant = nat.RING_STREAMK | nat.RING_WAVESPLIT
    assert _check(sk)[0] == nat.ERR_ARG
    # HKX_RING_HALFSTAGE combines with either; it is a ring-schedule bit only
    for v in (nat.RING_HALFSTAGE, nat.RING_HALFSTAGE | nat.RING_WAVESPLIT,
              nat.RING_HALFSTAGE | nat.RING_STREAMK):
        sk.variant = v
        assert _check(sk)[0] == nat.OK, v
    pp = _args(m=2048, n=8192, k=512, tile_m=256, tile_n=256, tile_schedule=nat.TILE_PINGPONG,
               variant=nat.RING_HALFSTAGE)
    assert _check(pp)[0] == nat.ERR_ARG


def test_arrival_counter_counts():
    """hkx_gemm_counters: one int32 a block of decode rows for an unpaired decode call split
    over K, one a tile for the 4-wave tile kernel split over K, none otherwise; a call given
    too few counters is refused before any launch."""
    L = nat.lib()
    d = _args(m=16, n=4100, k=4096, kernel=nat.KERNEL_DECODE, splits=4)
    assert L.hkx_gemm_counters(ctypes.byref(d)) == 257
    d.decode_rows = 32
    assert L.hkx_gemm_counters(ctypes.byref(d)) == 129
    d.splits = 1
    assert L.hkx_gemm_counters(ctypes.byref(d)) == 0
    # the 4-wave tile kernel split over K: one a tile; the 256 x 256 ring tiles: none
    assert L.hkx_gemm_counters(ctypes.byref(_args(m=300, n=1000, splits=2))) == 3 * 4
    ring = _args(m=512, n=512, k=512, tile_m=256, tile_n=256, tile_schedule=nat.TILE_RING, splits=2)
    assert L.hkx_gemm_counters(ctypes.byref(ring)) == 0
    pair = _args(m=16, n=4096, k=4096, kernel=nat.KERNEL_DECODE, splits=4, decode_rows=32)
    pair.ep.form = nat.EP_SILU_MUL
    assert L.hkx_gemm_counters(ctypes.byref(pair)) == 0
    short = _args(m=16, n=4100, k=4096, kernel=nat.KERNEL_DECODE, splits=4)
    short.ws, short.ws_bytes = 0x50000, 1 << 30
    short.counters, short.counters_len = 0x60000, 100
    rc, msg = _check(short)
    assert rc == nat.ERR_WORKSPACE and "counters" in msg
    short.counters_len = 257
    assert _check(short)[0] == nat.OK


def test_mx_workspace_sizes():
    """The MX GEMM splits K where its 256 x 256 tiles fill less than half of (this host's
    assumed) 256 CUs: min(CUs / tiles, k-tiles / 8, 8) splits, trimmed so none is empty."""
    L = nat.lib()
    ws = L.hkx_mx_gemm_workspace
    assert ws(4096, 4096, 4096) == 0                       # 256 tiles: one pass
    assert ws(2048, 1792, 5120) == 4 * 2048 * 1792 * 4     # 56 tiles, 40 k-tiles: 4 splits
    assert ws(300, 512, 2048) == 2 * 300 * 512 * 4         # 16 k-tiles: 2 splits of 8
    assert ws(64, 512, 4224) == 4 * 64 * 512 * 4           # 33 k-tiles: 9, 9, 9 and 6
    assert ws(300, 512, 1152) == 0                         # 9 k-tiles: too few to split
    # a split call refuses to run without its workspace (checked before any launch)
    p = 1 << 20
    rc = L.hkx_mx_gemm(p, 5120, p, 5120, p, 160, p, 160, p, 1792, 2048, 1792, 5120, None, 0, None)
    assert rc == nat.ERR_WORKSPACE and b"workspace" in L.hkx_last_error()


def test_the_build_refuses_spills():
    from importlib import import_module

    import sys
    sys.path.insert(0, str(ROOT / "hk-dsl_amd"))
    build = import_module("build")
    remarks = ("x: remark: Function Name: k1\nx: remark:     ScratchSize [bytes/lane]: 0\n"
               "x: remark: Function Name: k2\nx: remark:     ScratchSize [bytes/lane]: 16\n")
    assert build._spills(remarks) == [("k2", 16)]
