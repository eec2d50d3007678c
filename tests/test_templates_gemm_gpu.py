"""hk.templates.gemm on the GPU against the CPU oracle: every ready-made epilogue and the
operand kinds through the routed plan, every route candidate forced, the out dtypes and
quantizing stores, in-place and bound forms -- the cases of the reference's
tests/hk/gpu/test_templates_gemm.py:43-215, with this build's kernels.

Inputs are made on the CPU from a seeded generator and copied to the GPU, so the oracle
(torch fp32 on the CPU) sees the same operands. Check: max|got - ref| / max|ref| < 1e-2
(the reference's measure, :33-35), and for the BASELINE configs elementwise rtol = atol =
1e-2."""

import importlib

import pytest
import torch

import hk
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
T = hk.templates.gemm
TG = importlib.import_module("hk.templates.gemm")


def _data(m, n, k, seed=0):
    g = torch.Generator().manual_seed(seed + m + n + k)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    b = (torch.randn(n, k, generator=g) * k ** -0.5).to(torch.bfloat16)
    return a, b, O.gemm_fp32(a, b)


def _close(got, ref, rel=1e-2):
    err = O.rel_to_max(got.cpu(), ref)
    assert err < rel, f"rel err {err:.3g}"


def mask_cols(acc, ctx):
    """C[:, 1000:] = 0, through the coordinates."""
    return acc.right_fill_(1000 - ctx.col, 0.0)


def _cases(m, n, k):
    g = torch.Generator().manual_seed(7)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    res = torch.randn(m, n, generator=g).to(torch.bfloat16)
    rs = torch.rand(m, 1, generator=g) + 0.5
    gl = O.gelu_tanh
    return {
        "bias": (T.bias, dict(bias=bias), lambda c: c + bias.float()),
        "bias_gelu": (T.bias_gelu, dict(bias=bias), lambda c: gl(c + bias.float())),
        "bias_silu": (T.bias_silu, dict(bias=bias), lambda c: O.silu(c + bias.float())),
        "residual": (T.residual, dict(residual=res), lambda c: c + res.float()),
        "bias_residual": (T.bias_residual, dict(bias=bias, residual=res),
                          lambda c: c + bias.float() + res.float()),
        "row_scale": (T.scale, dict(scale=rs), lambda c: c * rs),
        "number": (T.scale, dict(scale=0.25), lambda c: c * 0.25),
        "own_gelu": (lambda acc, ctx: (acc + ctx.bias).gelu(), dict(bias=bias),
                     lambda c: gl(c + bias.float())),
        "coords": (mask_cols, {}, lambda c: torch.cat([c[:, :1000], c[:, 1000:] * 0], 1)),
        "chain": (T.chain(T.residual, T.relu), dict(residual=res),
                  lambda c: O.relu(c + res.float())),
        "named": (lambda acc, bias, residual, *, alpha=0.5: (acc + bias) * alpha + residual,
                  dict(bias=bias, residual=res), lambda c: (c + bias.float()) * 0.5 + res.float()),
        "tile_mul": (lambda acc, ctx: acc * ctx.gate, dict(gate=res), lambda c: c * res.float()),
    }


NAMES = ["bias", "bias_gelu", "bias_silu", "residual", "bias_residual", "row_scale", "number",
         "own_gelu", "coords", "chain", "tile_mul", "named"]
SHAPES = [(1, 4096, 4096), (33, 6144, 4096), (128, 4096, 4096), (200, 1408, 640),
          (1024, 4096, 4096), (2048, 12288, 4096), (4096, 4224, 1024)]
CASES = ([(s, nm) for s in SHAPES[2:4] for nm in NAMES]
         + [(s, nm) for s in SHAPES[:2] + SHAPES[4:] for nm in ("bias_gelu", "residual", "coords")])


def _to(ops):
    return {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in ops.items()}


@pytest.mark.parametrize("shape,name", CASES, ids=[f"{nm}-{'x'.join(map(str, s))}" for s, nm in CASES])
def test_the_routed_plan_is_right(shape, name):
    m, n, k = shape
    a, b, acc = _data(m, n, k)
    fn, ops, ref = _cases(m, n, k)[name]
    print(f"case {name} {shape} plan {T.plan(m, n, k)}", flush=True)
    _close(T(a.to(DEV), b.to(DEV), epilogue=fn, **_to(ops)), ref(acc))


@pytest.mark.parametrize("cand", sorted(hk.ops.gemm_cdna.CANDIDATES))
@pytest.mark.parametrize("name", ["bias_gelu", "residual", "coords"])
def test_every_candidate_carries_the_epilogue(cand, name):
    """Each candidate a route can name, forced: the epilogue in its store or in the
    reduction of its split, right against the oracle."""
    m, n, k = (257, 1536, 2048) if not cand.startswith("decode") else (17, 1536, 2048)
    a, b, acc = _data(m, n, k)
    fn, ops, ref = _cases(m, n, k)[name]
    print(f"case {cand} {name}", flush=True)
    _close(T(a.to(DEV), b.to(DEV), epilogue=fn, schedule=cand, **_to(ops)), ref(acc))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_out_dtypes(dtype):
    a, b, acc = _data(300, 4096, 1024)
    bias = torch.randn(4096, generator=torch.Generator().manual_seed(1))
    got = T(a.to(DEV), b.to(DEV), epilogue=T.bias, out_dtype=dtype, bias=bias.to(DEV))
    assert got.dtype == dtype
    _close(got, acc + bias, rel=1e-2 if dtype != torch.float32 else 1e-5)


def test_an_int8_quantizer_rounds_and_saturates():
    a, b, acc = _data(128, 4096, 4096)
    s = torch.full((4096,), 40.0)
    got = T(a.to(DEV), b.to(DEV), epilogue=T.scale, out_dtype=torch.int8, scale=s.to(DEV))
    ref = O.quantize_int8(acc * 40.0)
    assert got.dtype == torch.int8
    assert (got.cpu().float() - ref).abs().max().item() <= 1.0  # bf16 vs fp32 GEMM


def test_an_fp8_quantizer_rounds_and_saturates():
    a, b, acc = _data(300, 4096, 1024)
    s = torch.rand(4096, generator=torch.Generator().manual_seed(2)) * 900  # some past 448
    got = T(a.to(DEV), b.to(DEV), epilogue=T.scale, out_dtype=torch.float8_e4m3fn, scale=s.to(DEV))
    assert got.dtype == torch.float8_e4m3fn
    want = (acc * s).clamp(-448, 448)
    big = want.abs() > 16
    rel = ((got.cpu().float() - want).abs() / want.abs())[big]
    assert rel.max().item() < 0.07  # e4m3: 3 mantissa bits
    assert got.cpu().float().abs().max().item() == 448.0


def test_out_is_written_in_place_and_nothing_past_m():
    a, b, acc = _data(100, 4096, 1024)
    room = torch.full((108, 4096), 7.0, device=DEV, dtype=torch.bfloat16)
    res = torch.randn(100, 4096, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    got = T(a.to(DEV), b.to(DEV), epilogue=T.residual, out=room[:100], residual=res.to(DEV))
    assert got.data_ptr() == room.data_ptr()
    _close(room[:100], acc + res.float())
    assert torch.equal(room[100:].cpu(), torch.full((8, 4096), 7.0, dtype=torch.bfloat16))


def test_the_bound_form_and_an_in_place_residual():
    """gemm(epilogue=...) without tensors binds for later; out may be the residual
    itself (each element is read before it is written)."""
    a, b, acc = _data(512, 4096, 1024)
    lin = T(epilogue=T.residual)
    res = torch.randn(512, 4096, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    want = acc + res.float()
    rd = res.to(DEV)
    got = lin(a.to(DEV), b.to(DEV), out=rd, residual=rd)
    _close(got, want)


def test_a_column_operand_at_a_ragged_m():
    for m in (1, 17, 255, 257):
        a, b, acc = _data(m, 4096, 1024)
        s = torch.rand(m, 1, generator=torch.Generator().manual_seed(m)) + 0.5
        _close(T(a.to(DEV), b.to(DEV), epilogue=T.scale, scale=s.to(DEV)), acc * s)


def heavy(acc, ctx):
    """Four tile operands and a GELU each: the register program."""
    for t in (ctx.r0, ctx.r1, ctx.r2, ctx.r3):
        acc += T.gelu_tanh(acc * t)
    return acc


def test_an_epilogue_outside_the_fused_form_runs_in_the_pass():
    for (m, n, k) in [(4, 4096, 4096), (4096, 4096, 1024)]:
        a, b, acc = _data(m, n, k)
        g = torch.Generator().manual_seed(5)
        rs = [torch.randn(m, n, generator=g).to(torch.bfloat16) for _ in range(4)]
        got = T(a.to(DEV), b.to(DEV), epilogue=heavy, **{f"r{i}": r.to(DEV) for i, r in enumerate(rs)})
        want = acc
        for t in rs:
            want = want + O.gelu_tanh(want * t.float())
        _close(got, want, rel=2e-2)


def test_silu_and_mul_epilogue():
    for m in (5, 300):
        a, b, acc = _data(m, 2 * 768, 1024)
        got = T(a.to(DEV), b.to(DEV), epilogue=T.silu_and_mul)
        assert tuple(got.shape) == (m, 768)
        O.assert_close(got, O.silu_and_mul(acc[:, :768], acc[:, 768:]), rtol=1e-2, atol=1e-2)


def test_misuse_is_named():
    a, b, _ = _data(64, 4096, 1024)
    a, b = a.to(DEV), b.to(DEV)
    with pytest.raises(ValueError, match="broadcast"):
        T(a, b, epilogue=T.bias, bias=torch.zeros(64, device=DEV))
    with pytest.raises(AttributeError, match="ctx.bias"):
        T(a, b, epilogue=T.bias, scale=1.0)
    with pytest.raises(TypeError, match="bf16"):
        T(a.float(), b, epilogue=T.bias, bias=torch.zeros(4096, device=DEV))


# ---------------------------------------------------------------- the BASELINE configs

def _cfg_inputs(m, k, n, seed):
    """x ~N(0,1), w (K, N) ~N(0, 0.02), b ~N(0, 0.1), all bf16, from a CPU generator;
    w is handed to the GEMM as w.t().contiguous() (N, K) -- F.linear's layout."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(k, n, generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16)
    return x, w, b


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_config1_linear_bias_gelu(seed):
    x, w, b = _cfg_inputs(256, 1024, 1024, seed)
    ref = O.linear_bias_gelu(x, w, b)
    got = T(x.to(DEV), w.t().contiguous().to(DEV), epilogue=T.bias_gelu, bias=b.to(DEV))
    O.assert_close(got, ref, rtol=1e-2, atol=1e-2)


def test_config2_bias_gelu_full_size():
    """Config 2 at its full size, 4096 x 4096 x 12288 (K x N), elementwise rtol=atol=1e-2."""
    x, w, b = _cfg_inputs(4096, 4096, 12288, 0)
    xd, wd, bd = x.to(DEV), w.t().contiguous().to(DEV), b.to(DEV)
    got = T(xd, wd, epilogue=T.bias_gelu, bias=bd)
    ref = O.gelu_tanh(xd.float() @ wd.float().t() + bd.float())  # fp32 reference on the GPU
    torch.testing.assert_close(got.float(), ref, rtol=1e-2, atol=1e-2)
    # and the CPU oracle on the whole output (fp32 on the host's cores, about a second)
    O.assert_close(got, O.linear_bias_gelu(x, w, b), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("m", [2048, 8192])
def test_config3_gate_up_silu_and_mul(m):
    x, w, _ = _cfg_inputs(m, 4096, 24576, 3)
    xd, wd = x.to(DEV), w.t().contiguous().to(DEV)
    got = T(xd, wd, epilogue=T.silu_and_mul)
    acc = xd.float() @ wd.float().t()
    ref = O.silu_and_mul(acc[:, :12288], acc[:, 12288:])
    torch.testing.assert_close(got.float(), ref, rtol=1e-2, atol=1e-2)
    # and the CPU oracle on the whole output
    a = O.gemm_fp32(x, w.t().contiguous())
    O.assert_close(got, O.silu_and_mul(a[:, :12288], a[:, 12288:]), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("m", [1, 4, 16])
@pytest.mark.parametrize("with_bias", [False, True])
def test_config4_decode(m, with_bias):
    x, w, b = _cfg_inputs(m, 4096, 12288, 4)
    wd = w.t().contiguous().to(DEV)
    acc = O.gemm_fp32(x, w.t().contiguous())
    if with_bias:
        got = T(x.to(DEV), wd, epilogue=T.bias, bias=b.to(DEV))
        ref = acc + b.float()
    else:
        got = T(x.to(DEV), wd)
        ref = acc
    assert T.plan(m, 12288, 4096)[0].kernel == "decode"
    O.assert_close(got, ref, rtol=1e-2, atol=1e-2)


def test_config5_fp8_scaled_dequant():
    g = torch.Generator().manual_seed(5)
    m, k, n = 8192, 4096, 4096
    x8 = torch.randn(m, k, generator=g).to(torch.float8_e4m3fn)
    w8 = torch.randn(k, n, generator=g).to(torch.float8_e4m3fn)  # (K, N) as configured
    sa = (torch.rand(m, 1, generator=g) * 1.5 + 0.5) / 448
    sb = (torch.rand(n, generator=g) * 1.5 + 0.5) / 448
    bias = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16)
    b8 = w8.t().contiguous()
    xd, bd8 = x8.to(DEV), b8.to(DEV)
    got = hk.ops.scaled_mm(xd, bd8, sa.to(DEV), sb.to(DEV), bias=bias.to(DEV))
    ref = (xd.float() @ bd8.float().t()) * sa.to(DEV) * sb.to(DEV) + bias.to(DEV).float()
    torch.testing.assert_close(got.float(), ref, rtol=3e-2, atol=1e-2)
    # no bias: the reference tests' rel-to-max measure (|acc sa sb| ~ 1e-4 << atol)
    got0 = hk.ops.scaled_mm(xd, bd8, sa.to(DEV), sb.to(DEV))
    ref0 = (xd.float() @ bd8.float().t()) * sa.to(DEV) * sb.to(DEV)
    assert O.rel_to_max(got0, ref0) < 8e-3
    # and the CPU oracle on the whole output, with and without the bias
    O.assert_close(got, O.scaled_mm(x8, b8, sa, sb, bias), rtol=3e-2, atol=1e-2)
    assert O.rel_to_max(got0.cpu(), O.scaled_mm(x8, b8, sa, sb)) < 8e-3


def test_scaled_mm_per_tensor_and_ragged_m():
    g = torch.Generator().manual_seed(6)
    for m in (1, 33, 300):
        a8 = torch.randn(m, 1024, generator=g).to(torch.float8_e4m3fn)
        b8 = torch.randn(768, 1024, generator=g).to(torch.float8_e4m3fn)
        got = hk.ops.scaled_mm(a8.to(DEV), b8.to(DEV), 0.5, 0.25)
        ref = O.scaled_mm(a8, b8, 0.5, 0.25)
        assert O.rel_to_max(got.cpu(), ref) < 8e-3
