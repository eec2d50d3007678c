"""The gfx950 kernels through the C ABI (hk._native), against the CPU oracle:
every tile shape and store mode, bf16 and fp8, split-K, the decode kernel, the paired
silu-and-mul form and the epilogue-program pass. Inputs are made on the CPU from a
seeded generator, so the oracle sees exactly the operands the GPU does."""

import ctypes

import pytest
import torch

from hk import _native as nat
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _data(m, n, k, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed * 1000003 + m * 7919 + n * 31 + k)
    a = torch.randn(m, k, generator=g).to(dtype)
    b = (torch.randn(n, k, generator=g) * k ** -0.5).to(dtype)
    return a, b


def _fused(ops, *, act=nat.ACT_NONE, cs=-1, rs=-1, ra=-1, ta=-1, cmul=1.0, cadd=0.0):
    ep = nat.HkxEpilogue()
    ep.form = nat.EP_FUSED
    ep.act, ep.col_scale, ep.row_scale, ep.row_add, ep.tile_add = act, cs, rs, ra, ta
    ep.cmul, ep.cadd = cmul, cadd
    ep.nops = len(ops)
    for i, (t, kind) in enumerate(ops):
        ep.ops[i] = nat.HkxOperand(t.data_ptr(), kind, nat.dtype_code(t.dtype),
                                   1 if kind == nat.ROW else t.stride(0))
    return ep


def _run(a, b, c, **kw):
    print(f"case: A{tuple(a.shape)} B{tuple(b.shape)} C{tuple(c.shape)} {c.dtype} {kw}", flush=True)
    args = nat.gemm_args(a, b, c, **{k: v for k, v in kw.items() if k != "ep"}, ep=kw.get("ep"))
    nat.run(args, a.device)
    torch.cuda.synchronize()


PP, W4, W8, RING = nat.TILE_PINGPONG, nat.TILE_W4, nat.TILE_W8, nat.TILE_RING
SNAME = {PP: "pp", W4: "w4", W8: "w8", RING: "ring"}
#: (tile_m, tile_n, schedule, variant): the ring kernel, the ping-pong kernel (16 x 16 and
#: 32 x 32 MFMAs, one workgroup a CU or one a tile), the 4-wave (32 x 32 MFMA) and 8-wave
#: (16 x 16) kernels
TILES = [(256, 256, RING, 0), (256, 256, PP, 0), (256, 256, PP, nat.PP_MFMA32),
         (256, 256, PP, nat.PP_ONE_TILE),
         (256, 256, W4, 0), (128, 256, W4, 0), (64, 256, W4, 0), (256, 256, W8, 0),
         (128, 256, W8, 0), (64, 256, W8, 0), (128, 128, W8, 0), (256, 128, W8, 0),
         (128, 128, W4, 0), (64, 128, W4, 0), (128, 256, RING, 0)]


def tile_id(t):
    return f"{t[0]}x{t[1]}{SNAME[t[2]]}" + (f"v{t[3]}" if len(t) > 3 and t[3] else "")


TILE_IDS = [tile_id(t) for t in TILES]


@pytest.mark.parametrize("tile", TILES, ids=TILE_IDS)
@pytest.mark.parametrize("shape", [(300, 512, 256), (1, 256, 128), (257, 1000, 640),
                                   (513, 768, 4096)])
def test_tile_plain_bf16(tile, shape):
    m, n, k = shape
    a, b = _data(m, n, k)
    ref = O.gemm_fp32(a, b)
    c = torch.full((m, n), 7.0, dtype=torch.bfloat16, device=DEV)
    _run(a.to(DEV), b.to(DEV), c, kernel=nat.KERNEL_TILE, tile_m=tile[0], tile_n=tile[1],
         schedule=tile[2], variant=tile[3])
    O.assert_close(c, ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("tile", [(128, W4), (128, W8), (256, PP), (256, RING)],
                         ids=lambda t: f"{t[0]}{SNAME[t[1]]}")
@pytest.mark.parametrize("splits", [1, 2, 3, 4])
def test_tile_bias_gelu_and_split(splits, tile):
    m, n, k = 200, 1408, 640
    a, b = _data(m, n, k, seed=1)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    ref = O.apply_epilogue("bias_gelu", O.gemm_fp32(a, b), bias=bias)
    c = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    bd = bias.to(DEV)
    ep = _fused([(bd, nat.ROW)], act=nat.ACT_GELU_TANH, ra=0)
    _run(a.to(DEV), b.to(DEV), c, kernel=nat.KERNEL_TILE, tile_m=tile[0], tile_n=256,
         splits=splits, schedule=tile[1], ep=ep)
    O.assert_close(c, ref, rtol=1e-2, atol=1e-2)


def test_tile_nothing_past_m():
    m, n, k = 100, 512, 256
    a, b = _data(m, n, k, seed=2)
    room = torch.full((108, n), 7.0, dtype=torch.bfloat16, device=DEV)
    _run(a.to(DEV), b.to(DEV), room[:m], kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256)
    O.assert_close(room[:m], O.gemm_fp32(a, b), rtol=1e-2, atol=1e-2)
    assert torch.equal(room[m:].cpu(), torch.full((8, n), 7.0, dtype=torch.bfloat16))


@pytest.mark.parametrize("sched", [(W4, 0), (W8, 0), (PP, 0), (PP, nat.PP_MFMA32), (RING, 0)],
                         ids=lambda t: SNAME[t[0]] + str(t[1]))
@pytest.mark.parametrize("out", [torch.float32, torch.float16])
def test_tile_out_dtypes_residual_colscale(out, sched):
    m, n, k = 300, 768, 512
    a, b = _data(m, n, k, seed=3)
    g = torch.Generator().manual_seed(9)
    res = torch.randn(m, n, generator=g).to(torch.bfloat16)
    rs = torch.rand(m, 1, generator=g) + 0.5
    ref = (O.gemm_fp32(a, b) * rs + res.float())
    c = torch.empty((m, n), dtype=out, device=DEV)
    resd, rsd = res.to(DEV), rs.to(DEV)
    ep = _fused([(rsd, nat.COL), (resd, nat.TILE)], cs=0, ta=1)
    _run(a.to(DEV), b.to(DEV), c, kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256, ep=ep,
         schedule=sched[0], variant=sched[1])
    O.assert_close(c, ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("tile", [(256, 256, RING), (256, 256, PP), (256, 256, W4), (64, 256, W4),
                                  (256, 256, W8), (128, 128, W8), (128, 128, W4), (64, 128, W4)],
                         ids=tile_id)
def test_tile_fp8_scaled(tile):
    m, n, k = 300, 512, 1024
    g = torch.Generator().manual_seed(11)
    a8 = (torch.randn(m, k, generator=g) * 2).to(torch.float8_e4m3fn)
    b8 = (torch.randn(n, k, generator=g) * 2).to(torch.float8_e4m3fn)
    sa = (torch.rand(m, 1, generator=g) * 1.5 + 0.5) / 448
    sb = (torch.rand(n, generator=g) * 1.5 + 0.5) / 448
    bias = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16)
    ref = O.scaled_mm(a8, b8, sa, sb)
    c = torch.empty((m, n), dtype=torch.float32, device=DEV)
    sad, sbd, bd = sa.to(DEV), sb.to(DEV), bias.to(DEV)
    ep = _fused([(sad, nat.COL), (sbd, nat.ROW)], cs=0, rs=1)
    _run(a8.to(DEV), b8.to(DEV), c, kernel=nat.KERNEL_TILE, tile_m=tile[0], tile_n=tile[1],
         schedule=tile[2], ep=ep)
    assert O.rel_to_max(c.cpu(), ref) < 1e-4
    # with the bias, into bf16
    c2 = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    ep = _fused([(sad, nat.COL), (sbd, nat.ROW), (bd, nat.ROW)], cs=0, rs=1, ra=2)
    _run(a8.to(DEV), b8.to(DEV), c2, kernel=nat.KERNEL_TILE, tile_m=tile[0], tile_n=tile[1],
         schedule=tile[2], ep=ep)
    O.assert_close(c2, O.scaled_mm(a8, b8, sa, sb, bias), rtol=3e-2, atol=1e-2)


@pytest.mark.parametrize("bm", [128, 64])
@pytest.mark.parametrize("form", ["plain", "bias_gelu", "residual", "silu_mul", "int8", "fp32"])
@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("k", [64, 192, 640])
def test_w4_128_columns(bm, form, splits, k):
    """The 4-wave kernel's 128-column tiles (four LDS stages): K-tile counts below, at and
    past the stage count (1, 3, 10), split over K, ragged M and N, every store mode."""
    m, n = 300, 520
    kw = dict(kernel=nat.KERNEL_TILE, tile_m=bm, tile_n=128, schedule=W4, splits=splits)
    if form == "silu_mul":
        a, b = _data(m, 2 * n, k, seed=81)
        acc = O.gemm_fp32(a, b)
        c = torch.full((m, n), 7.0, dtype=torch.bfloat16, device=DEV)
        ep = nat.HkxEpilogue()
        ep.form = nat.EP_SILU_MUL
        _run(a.to(DEV), b.to(DEV), c, ep=ep, **kw)
        O.assert_close(c, O.silu_and_mul(acc[:, :n], acc[:, n:]), rtol=1e-2, atol=1e-2)
        return
    a, b = _data(m, n, k, seed=80)
    acc = O.gemm_fp32(a, b)
    g = torch.Generator().manual_seed(82)
    if form == "int8":
        sd = torch.full((n,), 40.0).to(DEV)
        c = torch.empty((m, n), dtype=torch.int8, device=DEV)
        _run(a.to(DEV), b.to(DEV), c, ep=_fused([(sd, nat.ROW)], rs=0), **kw)
        assert (c.cpu().float() - O.quantize_int8(acc * 40)).abs().max().item() <= 1.0
        return
    c = torch.full((m, n), 7.0, dtype=torch.float32 if form == "fp32" else torch.bfloat16,
                   device=DEV)
    if form in ("plain", "fp32"):
        _run(a.to(DEV), b.to(DEV), c, **kw)
        ref = acc
    elif form == "bias_gelu":
        bias = torch.randn(n, generator=g).to(torch.bfloat16)
        ref = O.apply_epilogue("bias_gelu", acc, bias=bias)
        bd = bias.to(DEV)
        _run(a.to(DEV), b.to(DEV), c, ep=_fused([(bd, nat.ROW)], ra=0, act=nat.ACT_GELU_TANH), **kw)
    else:
        res = torch.randn(m, n, generator=g).to(torch.bfloat16)
        rs = torch.rand(m, 1, generator=g) + 0.5
        ref = acc * rs + res.float()
        resd, rsd = res.to(DEV), rs.to(DEV)
        _run(a.to(DEV), b.to(DEV), c, ep=_fused([(rsd, nat.COL), (resd, nat.TILE)], cs=0, ta=1), **kw)
    O.assert_close(c, ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("m", [1, 5, 16, 17, 32])
@pytest.mark.parametrize("cfg", [(8, 16, 1), (4, 32, 1), (16, 16, 4), (8, 32, 2)])
def test_decode(m, cfg):
    waves, rows, splits = cfg
    n, k = 1536, 2048
    a, b = _data(m, n, k, seed=4)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    ref = O.apply_epilogue("bias", O.gemm_fp32(a, b), bias=bias)
    c = torch.full((m, n), 7.0, dtype=torch.bfloat16, device=DEV)
    bd = bias.to(DEV)
    _run(a.to(DEV), b.to(DEV), c, kernel=nat.KERNEL_DECODE, decode_waves=waves,
         decode_rows=rows, splits=splits, ep=_fused([(bd, nat.ROW)], ra=0))
    O.assert_close(c, ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("kernel", ["tile", "tile_split", "decode", "decode_split", "tile_fp32",
                                    "tile8", "tile8_split", "tilepp", "tilepp_split",
                                    "tilepp_fp32", "tilering", "tilering_split", "tilering_fp32"])
def test_silu_and_mul(kernel):
    m = 5 if kernel.startswith("decode") else 300
    n, k = 768, 512
    a, b = _data(m, 2 * n, k, seed=7)
    acc = O.gemm_fp32(a, b)
    ref = O.silu_and_mul(acc[:, :n], acc[:, n:])
    dt = torch.float32 if kernel.endswith("fp32") else torch.bfloat16
    c = torch.empty((m, n), dtype=dt, device=DEV)
    ep = nat.HkxEpilogue()
    ep.form = nat.EP_SILU_MUL
    kw = dict(ep=ep, splits=2 if kernel.endswith("split") else 1)
    if kernel.startswith("decode"):
        kw.update(kernel=nat.KERNEL_DECODE, decode_rows=32)
    else:
        kw.update(kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256,
                  schedule=W8 if kernel.startswith("tile8") else (
                      PP if kernel.startswith("tilepp") else (
                          RING if kernel.startswith("tilering") else W4)))
    _run(a.to(DEV), b.to(DEV), c, **kw)
    O.assert_close(c, ref, rtol=1e-2, atol=1e-2)


def test_program_pass():
    """An epilogue outside the fused form: (acc + bias) * 0.5 + gelu(acc * t), cols >= 300
    set to 0 -- through the register program."""
    m, n, k = 130, 512, 256
    a, b = _data(m, n, k, seed=8)
    g = torch.Generator().manual_seed(10)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    t = torch.randn(m, n, generator=g).to(torch.bfloat16)
    acc = O.gemm_fp32(a, b)
    ref = (acc + bias.float()) * 0.5 + O.gelu_tanh(acc * t.float())
    ref[:, 300:] = 0
    bd, td = bias.to(DEV), t.to(DEV)
    ep = nat.HkxEpilogue()
    ep.form = nat.EP_PROGRAM
    ep.nops = 2
    ep.ops[0] = nat.HkxOperand(bd.data_ptr(), nat.ROW, nat.BF16, 1)
    ep.ops[1] = nat.HkxOperand(td.data_ptr(), nat.TILE, nat.BF16, n)
    P = nat.OP
    prog = [("LOAD", 1, 0, 0, 0, 0.0), ("ADD", 1, 0, 1, 0, 0.0), ("CONST", 2, 0, 0, 0, 0.5),
            ("MUL", 1, 1, 2, 0, 0.0), ("LOAD", 2, 1, 0, 0, 0.0), ("MUL", 2, 0, 2, 0, 0.0),
            ("GELU", 2, 2, 0, 0, 0.0), ("ADD", 1, 1, 2, 0, 0.0),
            ("CONST", 3, 0, 0, 0, 300.0), ("COL", 4, 0, 0, 0, 0.0), ("SUB", 3, 3, 4, 0, 0.0),
            ("CONST", 5, 0, 0, 0, 0.0), ("SELLE", 1, 3, 5, 1, 0.0)]
    for i, (op, d, x, y, z, imm) in enumerate(prog):
        ep.ins[i] = nat.HkxInstr(P[op], d, x, y, z, 0, 0, 0, imm)
    ep.nins, ep.out_reg = len(prog), 1
    for kw in (dict(kernel=nat.KERNEL_TILE, tile_m=128, tile_n=256),
               dict(kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256, schedule=PP),
               dict(kernel=nat.KERNEL_TILE, tile_m=64, tile_n=256, splits=2),
               dict(kernel=nat.KERNEL_TILE, tile_m=128, tile_n=128, schedule=nat.TILE_W8)):
        c = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
        _run(a.to(DEV), b.to(DEV), c, ep=ep, **kw)
        O.assert_close(c, ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("tile", [(128, W4), (128, W8), (256, PP), (256, RING)],
                         ids=lambda t: f"{t[0]}{SNAME[t[1]]}")
def test_quantizing_stores(tile):
    m, n, k = 128, 512, 512
    a, b = _data(m, n, k, seed=12)
    acc = O.gemm_fp32(a, b)
    s = torch.full((n,), 40.0)
    sd = s.to(DEV)
    c = torch.empty((m, n), dtype=torch.int8, device=DEV)
    _run(a.to(DEV), b.to(DEV), c, kernel=nat.KERNEL_TILE, tile_m=tile[0], tile_n=256,
         schedule=tile[1], ep=_fused([(sd, nat.ROW)], rs=0))
    assert (c.cpu().float() - O.quantize_int8(acc * 40)).abs().max().item() <= 1.0
    c8 = torch.empty((m, n), dtype=torch.float8_e4m3fn, device=DEV)
    s2 = torch.rand(n, generator=torch.Generator().manual_seed(3)) * 900
    s2d = s2.to(DEV)
    _run(a.to(DEV), b.to(DEV), c8, kernel=nat.KERNEL_TILE, tile_m=tile[0], tile_n=256,
         schedule=tile[1], ep=_fused([(s2d, nat.ROW)], rs=0))
    want = (acc * s2).clamp(-448, 448)
    got = c8.cpu().float()
    big = want.abs() > 16
    assert ((got - want).abs() / want.abs())[big].max().item() < 0.07
    assert got.abs().max().item() == 448.0


# ---------------------------------------------------------------- the ring kernel's forms

@pytest.mark.parametrize("act", [nat.ACT_NONE, nat.ACT_GELU_TANH, nat.ACT_SILU, nat.ACT_RELU])
@pytest.mark.parametrize("shape", [(300, 1000, 512), (512, 768, 1024), (17, 264, 256)])
def test_ring_bias_act(act, shape):
    """The compiled bias + activation forms (bf16 bias vector, bf16 C), ragged M and N
    (N % 256 != 0; N % 8 == 0), rows past M untouched."""
    m, n, k = shape
    a, b = _data(m, n, k, seed=21)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(22)) * 0.1).to(torch.bfloat16)
    name = {nat.ACT_NONE: "bias", nat.ACT_GELU_TANH: "bias_gelu", nat.ACT_SILU: "bias_silu",
            nat.ACT_RELU: "bias_relu"}[act]
    acc = O.gemm_fp32(a, b) + bias.float()
    ref = {"bias": acc, "bias_gelu": O.gelu_tanh(acc), "bias_silu": O.silu(acc),
           "bias_relu": acc.clamp_min(0)}[name]
    c = torch.full((m + 3, n), 7.0, dtype=torch.bfloat16, device=DEV)
    bd = bias.to(DEV)
    _run(a.to(DEV), b.to(DEV), c[:m], kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256,
         schedule=RING, ep=_fused([(bd, nat.ROW)], ra=0, act=act))
    O.assert_close(c[:m], ref, rtol=1e-2, atol=1e-2)
    assert (c[m:].float() == 7.0).all()


def test_ring_unaligned_col_scale_falls_back():
    """A 16-bit per-token scale that starts 2 bytes into a word (a slice at an odd
    element) is not the ring kernel's (its slots are aligned words): the 256 x 256 call
    runs on the ping-pong kernel, with the same result."""
    m, n, k = 300, 512, 256
    a, b = _data(m, n, k, seed=29)
    full = (torch.rand(m + 1, 1, generator=torch.Generator().manual_seed(30)) + 0.5).to(torch.float16)
    ref = O.gemm_fp32(a, b) * full[1:].float()
    fd = full.to(DEV)
    c = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    _run(a.to(DEV), b.to(DEV), c, kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256,
         schedule=RING, ep=_fused([(fd[1:], nat.COL)], cs=0))
    O.assert_close(c, ref, rtol=1e-2, atol=1e-2)


def test_ring_fp8_dequant_forms():
    """fp8: the compiled dequant forms (fp32 column and row scales, with and without a
    bf16 bias) and the generic one (a broadcast row scale), 2 x 3 tiles a workgroup."""
    m, n, k = 600, 1280, 2048
    g = torch.Generator().manual_seed(23)
    a8 = (torch.randn(m, k, generator=g) * 2).to(torch.float8_e4m3fn)
    b8 = (torch.randn(n, k, generator=g) * 2).to(torch.float8_e4m3fn)
    sa = (torch.rand(m, 1, generator=g) * 1.5 + 0.5) / 448
    sb = (torch.rand(n, generator=g) * 1.5 + 0.5) / 448
    bias = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16)
    sad, sbd, bd = sa.to(DEV), sb.to(DEV), bias.to(DEV)
    c = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    _run(a8.to(DEV), b8.to(DEV), c, kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256,
         schedule=RING, ep=_fused([(sad, nat.COL), (sbd, nat.ROW)], cs=0, rs=1))
    assert O.rel_to_max(c.cpu(), O.scaled_mm(a8, b8, sa, sb)) < 8e-3
    _run(a8.to(DEV), b8.to(DEV), c, kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256,
         schedule=RING, ep=_fused([(sad, nat.COL), (sbd, nat.ROW), (bd, nat.ROW)], cs=0, rs=1, ra=2))
    O.assert_close(c, O.scaled_mm(a8, b8, sa, sb, bias), rtol=3e-2, atol=1e-2)
    one = torch.tensor([2.0 / 448], device=DEV)
    ep = _fused([(sad, nat.COL), (one, nat.ROW)], cs=0, rs=1)
    ep.ops[1].ld = 0  # one value for every column
    _run(a8.to(DEV), b8.to(DEV), c, kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256,
         schedule=RING, ep=ep)
    ref = O.gemm_fp32(a8.float(), b8.float()) * sa * (2.0 / 448)
    assert O.rel_to_max(c.cpu(), ref) < 8e-3


def test_ring_c_past_4gib_falls_back():
    """C spanning 4 GiB or more (here a 512-column view of rows 2 MiB apart) is past the
    ring kernel's 32-bit store offsets: the call runs on the ping-pong kernel, right to
    the last row."""
    m, n, k = 2100, 512, 256
    a, b = _data(m, n, k, seed=31)
    big = torch.empty((m, 1 << 20), dtype=torch.bfloat16, device=DEV)
    c = big[:, :n]
    _run(a.to(DEV), b.to(DEV), c, kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256, schedule=RING)
    O.assert_close(c, O.gemm_fp32(a, b), rtol=1e-2, atol=1e-2)
    del big


def test_ring_falls_back_for_ragged_n():
    """N % 8 != 0 (a C the ring kernel cannot store in 16-byte pieces) runs on the
    ping-pong kernel and is still right."""
    m, n, k = 300, 1004, 512
    a, b = _data(m, n, k, seed=24)
    c = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    _run(a.to(DEV), b.to(DEV), c, kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256, schedule=RING)
    O.assert_close(c, O.gemm_fp32(a, b), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("m", [1, 4, 16, 17, 24, 32])
@pytest.mark.parametrize("nk", [(1536, 4096), (1000, 2048), (12288, 1024), (256, 1024), (4100, 3072),
                                (4096, 12288), (1000, 14336), (300, 5120), (16, 6144)])
def test_decode_stream(m, nk):
    """The streaming decode kernel (M <= 16, or M <= 32 as two 16-token fragments from K =
    2048; K a multiple of 1024; past 4096 X is streamed with the chunks): bias epilogue,
    ragged N (rows of W past N read as zeros, columns past N never written), ragged M
    (rows past M never written), chunk counts per workgroup from 1 up (3 ahead of the
    ring). At K = 1024 and M > 16 the call goes to decode_kernel."""
    n, k = nk
    a, b = _data(m, n, k, seed=25)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(26)).to(torch.bfloat16)
    ref = O.apply_epilogue("bias", O.gemm_fp32(a, b), bias=bias)
    c = torch.full((m, n + 8), 7.0, dtype=torch.bfloat16, device=DEV)
    bd = bias.to(DEV)
    _run(a.to(DEV), b.to(DEV), c[:, :n], kernel=nat.KERNEL_DECODE, variant=nat.DEC_STREAM,
         ep=_fused([(bd, nat.ROW)], ra=0))
    O.assert_close(c[:, :n], ref, rtol=1e-2, atol=1e-2)
    assert (c[:, n:].float() == 7.0).all()


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9, 13, 16])
@pytest.mark.parametrize("n", [12288, 1004, 4100, 8])
def test_decode_rows(m, n):
    """The whole-row decode kernels at M <= 4 (K = 4096, chunks of 4 rows: short workgroups
    of one chunk at M <= 2, of two at M = 3 and at M = 4 up to N = 8192 -- 1004 and 4100
    rows end on a workgroup whose second chunk is past N --, the persistent kernel with
    chunks strided over the workgroups at M = 4 and N = 12288), the stream kernel above:
    bias, chunk counts a workgroup from 1 up (1025 chunks: one workgroup with a group of
    one), a W of row stride K + 64, an output of row stride N + 8 with sentinels (columns
    past N never written)."""
    k = 4096
    a, b = _data(m, n, k, seed=31)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(32)).to(torch.bfloat16)
    ref = O.apply_epilogue("bias", O.gemm_fp32(a, b), bias=bias)
    wide = torch.zeros(n, k + 64, dtype=b.dtype)
    wide[:, :k] = b
    c = torch.full((m, n + 8), 7.0, dtype=torch.bfloat16, device=DEV)
    bd = bias.to(DEV)
    _run(a.to(DEV), wide.to(DEV)[:, :k], c[:, :n], kernel=nat.KERNEL_DECODE,
         variant=nat.DEC_STREAM, ep=_fused([(bd, nat.ROW)], ra=0))
    O.assert_close(c[:, :n], ref, rtol=1e-2, atol=1e-2)
    assert (c[:, n:].float() == 7.0).all()


@pytest.mark.parametrize("m,n", [(m, n) for m in (1, 3, 4) for n in (16384, 20004, 32768)]
                         + [(1, 40004), (2, 40004), (1, 65540)])
def test_decode_rows_bias_many_groups(m, n):
    """The whole-row decode kernel with a bias where a workgroup walks 4 or more groups of
    chunks (N > 12288 on 256 CUs), so the three bias slots of its LDS are each reused: a
    DMA of one group's bias words must leave the other slots' words alone (N = 20004 also
    ends on a ragged chunk); past N = 32768 at M <= 2, the short-workgroup form that the LM
    heads' N takes (N = 40004 and 65540 here)."""
    k = 4096
    a, b = _data(m, n, k, seed=36)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(37)).to(torch.bfloat16)
    ref = O.apply_epilogue("bias", O.gemm_fp32(a, b), bias=bias)
    c = torch.full((m, n + 8), 7.0, dtype=torch.bfloat16, device=DEV)
    _run(a.to(DEV), b.to(DEV), c[:, :n], kernel=nat.KERNEL_DECODE, variant=nat.DEC_STREAM,
         ep=_fused([(bias.to(DEV), nat.ROW)], ra=0))
    O.assert_close(c[:, :n], ref, rtol=1e-2, atol=1e-2)
    assert (c[:, n:].float() == 7.0).all()


@pytest.mark.parametrize("m", [1, 2, 3])
@pytest.mark.parametrize("nk", [(12288, 1024), (49152, 1024), (4100, 2048), (24576, 2048), (1000, 1024),
                                (8, 2048), (2056, 1024)])
def test_decode_per_wave_rows(m, nk):
    """The per-wave whole-row decode kernel (K = 1024 with M <= 3, K = 2048 with M <= 2; the
    stream kernel above): bias, rows a wave from 1 to 24 (49152 rows), ragged N (rows past N
    read zero and are never written), a W of row stride K + 64, an output of row stride
    N + 8 with sentinels."""
    n, k = nk
    a, b = _data(m, n, k, seed=38)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(39)).to(torch.bfloat16)
    ref = O.apply_epilogue("bias", O.gemm_fp32(a, b), bias=bias)
    wide = torch.zeros(n, k + 64, dtype=b.dtype)
    wide[:, :k] = b
    c = torch.full((m, n + 8), 7.0, dtype=torch.bfloat16, device=DEV)
    _run(a.to(DEV), wide.to(DEV)[:, :k], c[:, :n], kernel=nat.KERNEL_DECODE,
         variant=nat.DEC_STREAM, ep=_fused([(bias.to(DEV), nat.ROW)], ra=0))
    O.assert_close(c[:, :n], ref, rtol=1e-2, atol=1e-2)
    assert (c[:, n:].float() == 7.0).all()


@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float16, torch.float32, torch.int8,
                                 torch.float8_e4m3fn], ids=["bf16", "fp16", "fp32", "int8", "fp8"])
def test_decode_per_wave_rows_forms(odt):
    """The per-wave kernel's epilogue and stores: none; a broadcast per-token scale with cmul,
    a bias, cadd and GELU; and the 8-bit stores (int8 within one quantizer step of the
    oracle's, fp8 e4m3 saturating at 448)."""
    m, n, k = 2, 3000, 2048
    a, b = _data(m, n, k, seed=40)
    acc = O.gemm_fp32(a, b)
    ad, bdev = a.to(DEV), b.to(DEV)
    if odt in (torch.int8, torch.float8_e4m3fn):
        mul = 40.0 if odt == torch.int8 else 300.0
        c = torch.empty((m, n), dtype=odt, device=DEV)
        _run(ad, bdev, c, kernel=nat.KERNEL_DECODE, variant=nat.DEC_STREAM, ep=_fused([], cmul=mul))
        if odt == torch.int8:
            assert (c.cpu().float() - O.quantize_int8(acc * mul)).abs().max().item() <= 1.0
        else:
            want = (acc * mul).clamp(-448, 448)
            got = c.cpu().float()
            big = want.abs() > 16
            assert ((got - want).abs() / want.abs())[big].max().item() < 0.07
            assert got.abs().max().item() == 448.0
        return
    c = torch.empty((m, n), dtype=odt, device=DEV)
    _run(ad, bdev, c, kernel=nat.KERNEL_DECODE, variant=nat.DEC_STREAM)
    O.assert_close(c, acc, rtol=1e-2, atol=1e-2)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(41)).to(torch.bfloat16)
    sd = torch.full((1, 1), 0.75, device=DEV).expand(m, 1)
    ep = _fused([(sd, nat.COL), (bias.to(DEV), nat.ROW)], cs=0, ra=1, act=nat.ACT_GELU_TANH,
                cmul=0.5, cadd=0.25)
    c2 = torch.empty((m, n), dtype=odt, device=DEV)
    _run(ad, bdev, c2, kernel=nat.KERNEL_DECODE, variant=nat.DEC_STREAM, ep=ep)
    O.assert_close(c2, O.gelu_tanh(acc * 0.375 + bias.float() + 0.25), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("m", [1, 3, 7, 16])
@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float16, torch.float32],
                         ids=["bf16", "fp16", "fp32"])
def test_decode_rows_forms(m, odt):
    """The decode kernels' epilogue forms and output types (the whole-row kernel at M = 1 and
    3, the stream kernel at 7 and 16): none, and a broadcast per-token scale with cmul, a bias,
    cadd and GELU."""
    n, k = 1000, 4096
    a, b = _data(m, n, k, seed=33)
    acc = O.gemm_fp32(a, b)
    ad, bdev = a.to(DEV), b.to(DEV)
    c = torch.empty((m, n), dtype=odt, device=DEV)
    _run(ad, bdev, c, kernel=nat.KERNEL_DECODE, variant=nat.DEC_STREAM)
    O.assert_close(c, acc, rtol=1e-2, atol=1e-2)
    g = torch.Generator().manual_seed(34)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    sd = torch.full((1, 1), 0.75, device=DEV).expand(m, 1)
    bd = bias.to(DEV)
    ep = _fused([(sd, nat.COL), (bd, nat.ROW)], cs=0, ra=1, act=nat.ACT_GELU_TANH,
                cmul=0.5, cadd=0.25)
    c2 = torch.empty((m, n), dtype=odt, device=DEV)
    _run(ad, bdev, c2, kernel=nat.KERNEL_DECODE, variant=nat.DEC_STREAM, ep=ep)
    O.assert_close(c2, O.gelu_tanh(acc * 0.375 + bias.float() + 0.25), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("m", [1, 4])
def test_decode_rows_quantizing_stores(m):
    """The whole-row decode kernel's 8-bit stores, one byte a lane: int8 and fp8 e4m3
    (saturating at 448) of acc times a broadcast per-token scale."""
    n, k = 4096, 4096
    a, b = _data(m, n, k, seed=35)
    acc = O.gemm_fp32(a, b)
    ad, bdev = a.to(DEV), b.to(DEV)
    s40 = torch.full((1, 1), 40.0, device=DEV).expand(m, 1)
    c = torch.empty((m, n), dtype=torch.int8, device=DEV)
    _run(ad, bdev, c, kernel=nat.KERNEL_DECODE, variant=nat.DEC_STREAM,
         ep=_fused([(s40, nat.COL)], cs=0))
    assert (c.cpu().float() - O.quantize_int8(acc * 40)).abs().max().item() <= 1.0
    s300 = torch.full((1, 1), 300.0, device=DEV).expand(m, 1)
    c8 = torch.empty((m, n), dtype=torch.float8_e4m3fn, device=DEV)
    _run(ad, bdev, c8, kernel=nat.KERNEL_DECODE, variant=nat.DEC_STREAM,
         ep=_fused([(s300, nat.COL)], cs=0))
    want = (acc * 300).clamp(-448, 448)
    got = c8.cpu().float()
    big = want.abs() > 16
    assert ((got - want).abs() / want.abs())[big].max().item() < 0.07
    assert got.abs().max().item() == 448.0


@pytest.mark.parametrize("m", [1, 7, 16, 20, 32])
@pytest.mark.parametrize("nk", [(1000, 2048), (12288, 1024), (1000, 6144)])
def test_decode_stream_fused_forms(m, nk):
    """The streaming decode kernel's whole fused form: a per-token scale with a stride (a
    16-bit column of a wider tensor, odd elements in the high half of their word), a
    per-channel fp32 scale, a bf16 column add, a residual tile, GELU -- the vectors staged
    through LDS one block ahead."""
    n, k = nk
    a, b = _data(m, n, k, seed=27)
    g = torch.Generator().manual_seed(28)
    sa3 = (torch.rand(m, 3, generator=g) + 0.5).to(torch.float16)
    sb = torch.rand(n, generator=g) + 0.5
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    res = torch.randn(m, n, generator=g).to(torch.bfloat16)
    acc = O.gemm_fp32(a, b)
    ref = O.gelu_tanh(acc * sa3[:, 1:2].float() * sb * 0.5 + bias.float() + res.float() + 0.25)
    c = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    sa3d, sbd, bd, resd = sa3.to(DEV), sb.to(DEV), bias.to(DEV), res.to(DEV)
    ep = _fused([(sa3d[:, 1:2], nat.COL), (sbd, nat.ROW), (bd, nat.ROW), (resd, nat.TILE)],
                cs=0, rs=1, ra=2, ta=3, act=nat.ACT_GELU_TANH, cmul=0.5, cadd=0.25)
    _run(a.to(DEV), b.to(DEV), c, kernel=nat.KERNEL_DECODE, variant=nat.DEC_STREAM, ep=ep)
    O.assert_close(c, ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("m", [1, 9, 16, 24, 32])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32],
                         ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("nk", [(1000, 2048), (4096, 12288)])
def test_decode_stream_residual(m, dt, nk):
    """A residual tile on the streaming decode kernel (staged through LDS by DMA a block
    ahead, like the vector operands): 16- and 32-bit operands, a strided view (row stride
    N + 4), X held or streamed (K = 12288)."""
    n, k = nk
    a, b = _data(m, n, k, seed=29)
    g = torch.Generator().manual_seed(30)
    acc = O.gemm_fp32(a, b)
    # row stride N + 4: 8-byte aligned 16-bit rows (the generic epilogue form, 4-byte DMA);
    # bf16 also with N + 8 (16-byte aligned rows: the fast form), alone and with a bias
    for extra, with_bias in ((4, False),) + (((8, False), (8, True)) if dt == torch.bfloat16 else ()):
        room = torch.randn(m, n + extra, generator=g).to(dt)
        res = room[:, :n]
        c = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
        resd = room.to(DEV)[:, :n]
        if with_bias:
            bias = torch.randn(n, generator=g).to(torch.bfloat16)
            bd = bias.to(DEV)
            _run(a.to(DEV), b.to(DEV), c, kernel=nat.KERNEL_DECODE, variant=nat.DEC_STREAM,
                 ep=_fused([(bd, nat.ROW), (resd, nat.TILE)], ra=0, ta=1))
            O.assert_close(c, acc + bias.float() + res.float(), rtol=1e-2, atol=1e-2)
        else:
            _run(a.to(DEV), b.to(DEV), c, kernel=nat.KERNEL_DECODE, variant=nat.DEC_STREAM,
                 ep=_fused([(resd, nat.TILE)], ta=0))
            O.assert_close(c, acc + res.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("variant", [nat.RING_WAVESPLIT, nat.RING_STREAMK], ids=["ppw", "sk"])
@pytest.mark.parametrize("form", ["bias_gelu", "residual_colscale", "silu_mul", "fp8_deq_bias"])
def test_ring_wave_split(form, variant):
    """HKX_RING_WAVESPLIT at 2048 rows (8 tile rows: 32 tile columns a wave of 256 CUs) and
    N = 9216 (36 tile columns): columns 0-8191 on the ring kernel, 8192-9215 on 128 x 256
    tiles, the per-column operands (bias, row scale) and the residual taken from column
    8192 for the second launch; the paired form with its gate and up rows a full N apart.
    HKX_RING_STREAMK: the rest on 256 x 256 ring tiles split 2 ways over K into fp32
    shares, summed with the epilogue by the reduction (one pass for fp8, whose 4 K units
    make no split)."""
    m, n, k = 2048, 9216, 512
    g = torch.Generator().manual_seed(50)
    kw = dict(kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256, schedule=RING, variant=variant)
    if form == "fp8_deq_bias":
        a8 = (torch.randn(m, k, generator=g) * 2).to(torch.float8_e4m3fn)
        b8 = (torch.randn(n, k, generator=g) * 2).to(torch.float8_e4m3fn)
        sa = (torch.rand(m, 1, generator=g) + 0.5) / 448
        sb = (torch.rand(n, generator=g) + 0.5) / 448
        bias = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16)
        c = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
        sad, sbd, bd = sa.to(DEV), sb.to(DEV), bias.to(DEV)
        _run(a8.to(DEV), b8.to(DEV), c, ep=_fused([(sad, nat.COL), (sbd, nat.ROW), (bd, nat.ROW)],
                                                  cs=0, rs=1, ra=2), **kw)
        O.assert_close(c, O.scaled_mm(a8, b8, sa, sb, bias), rtol=3e-2, atol=1e-2)
        return
    if form == "silu_mul":
        a, b = _data(m, 2 * n, k, seed=51)
        acc = O.gemm_fp32(a, b)
        ref = O.silu_and_mul(acc[:, :n], acc[:, n:])
        c = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
        ep = nat.HkxEpilogue()
        ep.form = nat.EP_SILU_MUL
        _run(a.to(DEV), b.to(DEV), c, ep=ep, **kw)
        O.assert_close(c, ref, rtol=1e-2, atol=1e-2)
        return
    a, b = _data(m, n, k, seed=52)
    acc = O.gemm_fp32(a, b)
    c = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    if form == "bias_gelu":
        bias = torch.randn(n, generator=g).to(torch.bfloat16)
        ref = O.apply_epilogue("bias_gelu", acc, bias=bias)
        bd = bias.to(DEV)
        _run(a.to(DEV), b.to(DEV), c, ep=_fused([(bd, nat.ROW)], ra=0, act=nat.ACT_GELU_TANH), **kw)
    else:
        res = torch.randn(m, n, generator=g).to(torch.bfloat16)
        rs = torch.rand(m, 1, generator=g) + 0.5
        ref = acc * rs + res.float()
        resd, rsd = res.to(DEV), rs.to(DEV)
        _run(a.to(DEV), b.to(DEV), c, ep=_fused([(rsd, nat.COL), (resd, nat.TILE)], cs=0, ta=1), **kw)
    O.assert_close(c, ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("half", [False, True, "q128"], ids=["quad", "halfstage", "quad128"])
@pytest.mark.parametrize("form", ["plain", "bias", "bias_gelu", "silu", "silu_mul", "residual",
                                  "bias_residual_gelu"])
@pytest.mark.parametrize("mnk", [(256, 256, 64), (300, 520, 128), (4096, 4352, 192),
                                 (1000, 2048, 1088), (2048, 9216, 512)])
def test_ring_quad(form, mnk, half):
    """The quadrant kernel (the ring schedule's default for these forms) and, with
    HKX_RING_HALFSTAGE, the half-stage ring kernel on the same calls: one K-tile a tile
    (its fills run on into the next tile), ragged M and N, 272 tiles on 256 workgroups
    (some walk two), K-tiles past what two LDS slots hold; with wave split (the rest of N
    on 128 x 256 tiles) at 2048 x 9216; the paired silu * up form (128 C columns a tile,
    gate and up rows N apart). Its wait counts and fill order run on K-tile counts 1-17.
    "quad128": the same calls on 128 x 256 tiles (one phase a K-tile, three slots)."""
    m, n, k = mnk
    if half == "q128":  # 128 x 256 tiles: the quadrant kernel's one-phase form
        kw = dict(kernel=nat.KERNEL_TILE, tile_m=128, tile_n=256, schedule=RING)
    else:
        variant = (nat.RING_HALFSTAGE if half else 0) | (nat.RING_WAVESPLIT if n == 9216 else 0)
        kw = dict(kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256, schedule=RING, variant=variant)
    if form == "silu_mul":  # B holds the gate rows, then the up rows
        a, b = _data(m, 2 * n, k, seed=62)
        acc = O.gemm_fp32(a, b)
        c = torch.full((m, n), 7.0, dtype=torch.bfloat16, device=DEV)
        ep = nat.HkxEpilogue()
        ep.form = nat.EP_SILU_MUL
        _run(a.to(DEV), b.to(DEV), c, ep=ep, **kw)
        O.assert_close(c, O.silu_and_mul(acc[:, :n], acc[:, n:]), rtol=1e-2, atol=1e-2)
        return
    a, b = _data(m, n, k, seed=60)
    acc = O.gemm_fp32(a, b)
    g = torch.Generator().manual_seed(61)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    c = torch.full((m, n), 7.0, dtype=torch.bfloat16, device=DEV)
    bd = bias.to(DEV)
    if form == "plain":
        ref = acc
        _run(a.to(DEV), b.to(DEV), c, **kw)
    elif form == "bias":
        ref = acc + bias.float()
        _run(a.to(DEV), b.to(DEV), c, ep=_fused([(bd, nat.ROW)], ra=0), **kw)
    elif form == "bias_gelu":
        ref = O.apply_epilogue("bias_gelu", acc, bias=bias)
        _run(a.to(DEV), b.to(DEV), c, ep=_fused([(bd, nat.ROW)], ra=0, act=nat.ACT_GELU_TANH), **kw)
    elif form in ("residual", "bias_residual_gelu"):
        # the tile operand a strided view: row stride N + 8 (16-byte aligned rows: the
        # quadrant kernel's form), or N + 4 with a bias and GELU (8-byte aligned rows: the
        # quadrant kernel declines, the ring kernel's generic form runs)
        room = torch.randn(m, n + (8 if form == "residual" else 4), generator=g).to(torch.bfloat16)
        res = room[:, :n]
        resd = room.to(DEV)[:, :n]
        if form == "residual":
            ref = acc + res.float()
            _run(a.to(DEV), b.to(DEV), c, ep=_fused([(resd, nat.TILE)], ta=0), **kw)
        else:
            ref = O.gelu_tanh(acc + bias.float() + res.float())
            _run(a.to(DEV), b.to(DEV), c,
                 ep=_fused([(bd, nat.ROW), (resd, nat.TILE)], ra=0, ta=1, act=nat.ACT_GELU_TANH), **kw)
    else:
        ref = O.silu(acc)
        _run(a.to(DEV), b.to(DEV), c, ep=_fused([], act=nat.ACT_SILU), **kw)
    O.assert_close(c, ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("splits", [2, 3, 4])
@pytest.mark.parametrize("form", ["plain", "bias_gelu", "residual", "fp8_deq_bias"])
def test_quad_split_k(form, splits):
    """The quadrant kernel split over K (blockIdx.y the split, fp32 shares summed in split
    order by the reduction, which applies the epilogue): 17 bf16 or 9 fp8 K-tiles, so the
    last split is short; ragged M and N."""
    m, n = 300, 520
    kw = dict(kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256, schedule=RING, splits=splits)
    g = torch.Generator().manual_seed(90)
    c = torch.full((m, n), 7.0, dtype=torch.bfloat16, device=DEV)
    if form == "fp8_deq_bias":
        k = 9 * 128
        a8 = (torch.randn(m, k, generator=g) * 2).to(torch.float8_e4m3fn)
        b8 = (torch.randn(n, k, generator=g) * 2).to(torch.float8_e4m3fn)
        sa = (torch.rand(m, 1, generator=g) + 0.5) / 448
        sb = (torch.rand(n, generator=g) + 0.5) / 448
        bias = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16)
        sad, sbd, bd = sa.to(DEV), sb.to(DEV), bias.to(DEV)
        _run(a8.to(DEV), b8.to(DEV), c,
             ep=_fused([(sad, nat.COL), (sbd, nat.ROW), (bd, nat.ROW)], cs=0, rs=1, ra=2), **kw)
        O.assert_close(c, O.scaled_mm(a8, b8, sa, sb, bias), rtol=3e-2, atol=1e-2)
        return
    k = 17 * 64
    a, b = _data(m, n, k, seed=91)
    acc = O.gemm_fp32(a, b)
    if form == "plain":
        _run(a.to(DEV), b.to(DEV), c, **kw)
        ref = acc
    elif form == "bias_gelu":
        bias = torch.randn(n, generator=g).to(torch.bfloat16)
        bd = bias.to(DEV)
        _run(a.to(DEV), b.to(DEV), c, ep=_fused([(bd, nat.ROW)], ra=0, act=nat.ACT_GELU_TANH), **kw)
        ref = O.apply_epilogue("bias_gelu", acc, bias=bias)
    else:
        res = torch.randn(m, n, generator=g).to(torch.bfloat16)
        resd = res.to(DEV)
        _run(a.to(DEV), b.to(DEV), c, ep=_fused([(resd, nat.TILE)], ta=0), **kw)
        ref = acc + res.float()
    O.assert_close(c, ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("half", [False, True], ids=["quad", "halfstage"])
@pytest.mark.parametrize("form", ["plain", "deq", "deq_bias"])
@pytest.mark.parametrize("mnk", [(256, 256, 128), (300, 520, 256), (4096, 4352, 384),
                                 (1000, 2048, 1152), (2048, 9216, 512)])
def test_ring_quad_fp8(form, mnk, half):
    """fp8 e4m3 on the quadrant kernel (K-tiles of 128: a whole line) and, with
    HKX_RING_HALFSTAGE, on the half-stage ring kernel: unscaled, per-token x per-channel
    dequant, and dequant + bias; K-tile counts 1-9, ragged M and N, two tiles a workgroup,
    wave split at 2048 x 9216."""
    m, n, k = mnk
    g = torch.Generator().manual_seed(70)
    a8 = (torch.randn(m, k, generator=g) * 2).to(torch.float8_e4m3fn)
    b8 = (torch.randn(n, k, generator=g) * 2).to(torch.float8_e4m3fn)
    sa = (torch.rand(m, 1, generator=g) + 0.5) / 448
    sb = (torch.rand(n, generator=g) + 0.5) / 448
    bias = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16)
    variant = (nat.RING_HALFSTAGE if half else 0) | (nat.RING_WAVESPLIT if n == 9216 else 0)
    kw = dict(kernel=nat.KERNEL_TILE, tile_m=256, tile_n=256, schedule=RING, variant=variant)
    c = torch.full((m, n), 7.0, dtype=torch.bfloat16, device=DEV)
    sad, sbd, bd = sa.to(DEV), sb.to(DEV), bias.to(DEV)
    if form == "plain":
        _run(a8.to(DEV), b8.to(DEV), c, **kw)
        ref = O.gemm_fp32(a8.float(), b8.float())
        O.assert_close(c, ref, rtol=1e-2, atol=1e-2 * ref.abs().max().item())
        return
    if form == "deq":
        _run(a8.to(DEV), b8.to(DEV), c, ep=_fused([(sad, nat.COL), (sbd, nat.ROW)], cs=0, rs=1), **kw)
        O.assert_close(c, O.scaled_mm(a8, b8, sa, sb), rtol=3e-2, atol=1e-2)
        return
    _run(a8.to(DEV), b8.to(DEV), c, ep=_fused([(sad, nat.COL), (sbd, nat.ROW), (bd, nat.ROW)],
                                              cs=0, rs=1, ra=2), **kw)
    O.assert_close(c, O.scaled_mm(a8, b8, sa, sb, bias), rtol=3e-2, atol=1e-2)
