"""hk.templates.gemm's host side, on the CPU with meta tensors: epilogue binding and
capture, the compiled forms, plans and routes, misuse -- the reference's ir-tier checks
(tests/hk/ir/test_templates_gemm.py:54-274) restated for this build. A Python
interpreter of the HKX register program checks the program compiler against the
epilogue evaluated directly."""

import math

import numpy as np
import pytest
import torch

import hk
from hk import _native as nat
from hk.ops import gemm_cdna
from oracle import gemm_oracle as O

T = hk.templates.gemm


def meta(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, device="meta", dtype=dtype)


def compiled(fn, m=64, n=256, **ops):
    return T.bind(fn, ops, m, n, torch.bfloat16).compiled


# ------------------------------------------------------------------ forms

def test_ready_made_epilogues_compile_to_the_fused_form():
    b, r = meta(256), meta(64, 256)
    s_col, s_row = meta(64, 1, dtype=torch.float32), meta(256, dtype=torch.float32)
    assert compiled(T.bias, bias=b).describe() == "acc + bias"
    assert compiled(T.bias_gelu, bias=b).describe() == "gelu_tanh(acc + bias)"
    assert compiled(T.bias_silu, bias=b).describe() == "silu(acc + bias)"
    assert compiled(T.bias_relu, bias=b).describe() == "relu(acc + bias)"
    assert compiled(T.gelu).describe() == "gelu_tanh(acc)"
    assert compiled(T.residual, residual=r).describe() == "acc + residual"
    assert compiled(T.bias_residual, bias=b, residual=r).form == "fused"
    assert compiled(T.scale, scale=s_col).describe() == "acc * scale"
    assert compiled(T.scale, scale=s_row).describe() == "acc * scale"
    assert compiled(T.scale, scale=0.25).describe() == "acc * 0.25"
    assert compiled(T.chain(T.residual, T.relu), residual=r).describe() == "relu(acc + residual)"
    own = lambda acc, ctx: (acc + ctx.bias).gelu()  # noqa: E731
    assert compiled(own, bias=b).describe() == "gelu_tanh(acc + bias)"
    deq = lambda acc, ctx: acc * ctx.sa * ctx.sb + ctx.bias  # noqa: E731
    c = compiled(deq, sa=s_col, sb=s_row, bias=b)
    assert (c.form, c.col_scale, c.row_scale, c.row_add) == ("fused", "sa", "sb", "bias")
    assert compiled(lambda acc: acc).form == "none"


def test_other_epilogues_compile_to_a_program():
    b, r = meta(256), meta(64, 256)
    named = lambda acc, bias, residual, *, alpha=0.5: (acc + bias) * alpha + residual  # noqa: E731
    assert compiled(named, bias=b, residual=r).form == "program"
    coords = lambda acc, ctx: acc.right_fill_(1000 - ctx.col, 0.0)  # noqa: E731
    c = compiled(coords)
    assert c.form == "program" and c.uses_coords
    assert compiled(lambda acc, ctx: acc * ctx.gate, gate=r).form == "program"


# ------------------------------------------------------------------ the program, interpreted

def _interp(c, acc, ops, m_rows):
    """Run a compiled program on the CPU over a whole C (float64), the kernels' semantics
    (hk-dsl_amd/csrc/hkx_reduce.hpp run_program)."""
    M, N = acc.shape
    R = [np.zeros((M, N)) for _ in range(nat.MAX_REGS)]
    R[0] = acc.copy()
    rows = np.arange(M)[:, None] * np.ones((1, N))
    cols = np.ones((M, 1)) * np.arange(N)[None, :]
    names = sorted(ops)
    for op, d, a, b, cc, imm in c.ins:
        A, B = R[a], R[b]
        if op == "LOAD":
            v = ops[names[a]]
            r = np.broadcast_to(v, (M, N)).astype(np.float64)
        elif op == "CONST":
            r = np.full((M, N), imm)
        elif op == "ROW":
            r = rows
        elif op == "COL":
            r = cols
        elif op == "M":
            r = np.full((M, N), float(m_rows))
        else:
            f = {"MOV": lambda: A, "ADD": lambda: A + B, "SUB": lambda: A - B, "MUL": lambda: A * B,
                 "DIV": lambda: A / B, "MAX": lambda: np.maximum(A, B), "MIN": lambda: np.minimum(A, B),
                 "EXP": lambda: np.exp(A), "EXP2": lambda: np.exp2(A), "LOG": lambda: np.log(A),
                 "LOG2": lambda: np.log2(A), "ABS": lambda: np.abs(A), "RELU": lambda: np.maximum(A, 0),
                 "GELU": lambda: O.gelu_tanh(torch.from_numpy(A)).double().numpy(),
                 "SILU": lambda: A / (1 + np.exp(-A)), "SQRT": lambda: np.sqrt(A),
                 "RSQRT": lambda: 1 / np.sqrt(A), "NEG": lambda: -A, "STEP": lambda: (A > 0) * 1.0,
                 "SELLE": lambda: np.where(A <= 0, B, R[cc]), "TANH": lambda: np.tanh(A),
                 "SIGMOID": lambda: 1 / (1 + np.exp(-A)), "SQUARE": lambda: A * A}[op]
            r = f()
        R[d] = np.array(r, dtype=np.float64)
    return R[c.out_reg]


def test_programs_compute_what_the_epilogue_says():
    g = np.random.default_rng(0)
    M, N = 6, 1200
    acc = g.standard_normal((M, N))
    bias = g.standard_normal(N)
    res = g.standard_normal((M, N))
    r0, r1 = g.standard_normal((M, N)), g.standard_normal((M, N))
    cases = [
        (lambda acc, bias, residual, *, alpha=0.5: (acc + bias) * alpha + residual,
         dict(bias=bias, residual=res), (acc + bias) * 0.5 + res),
        (lambda acc, ctx: acc.right_fill_(1000 - ctx.col, 0.0), {},
         np.where(np.arange(N)[None, :] >= 1000, 0.0, acc)),
        (lambda acc, ctx: acc.left_fill_(3 - ctx.row, -1.0), {},
         np.where(np.arange(M)[:, None] < 3, -1.0, acc)),
        (lambda acc, ctx: acc * ctx.gate, dict(gate=res), acc * res),
    ]

    def heavy(acc, ctx):
        for t in (ctx.r0, ctx.r1):
            acc += T.gelu_tanh(acc * t)
        return acc

    h = acc.copy()
    for t in (r0, r1):
        h = h + O.gelu_tanh(torch.from_numpy(h * t)).double().numpy()
    cases.append((heavy, dict(r0=r0, r1=r1), h))

    def quadratic(acc, ctx):
        q = acc * acc
        q *= 0.5
        q += ctx.bias
        q.exp2_()
        q += 1.0
        q.rsqrt_()
        return acc * q * q - ctx.m + acc.maximum(0.0).minimum(2.0)

    qq = np.exp2(acc * acc * 0.5 + bias) + 1
    cases.append((quadratic, dict(bias=bias), acc / qq - M + np.clip(acc, 0, 2)))
    for fn, ops, want in cases:
        kinds = {k: torch.empty(v.shape if v.ndim == 2 else (v.shape[0],), device="meta")
                 for k, v in ops.items()}
        c = T.bind(fn, kinds, M, N, torch.bfloat16).compiled
        assert c.form == "program"
        got = _interp(c, acc, {k: (v if v.ndim == 2 else v[None, :]) for k, v in ops.items()}, M)
        np.testing.assert_allclose(got, want, rtol=1e-9, atol=1e-9)


def test_registers_are_reused():
    """A long chain of operations fits the 16 registers: values die and their registers
    are taken again."""
    def long(acc, ctx):
        for i in range(25):
            acc = acc * 1.001 + ctx.bias
        return acc

    c = compiled(long, bias=meta(256))
    assert c.form == "program"
    assert max(max(i[1], i[2], i[3]) for i in c.ins) < 4


# ------------------------------------------------------------------ binding and misuse

def test_operand_kinds_follow_broadcasting():
    m, n = 64, 256
    assert T._kind("x", meta(n), m, n) == "row"
    assert T._kind("x", meta(1, n), m, n) == "row"
    assert T._kind("x", meta(m, 1), m, n) == "col"
    assert T._kind("x", meta(m, n), m, n) == "tile"
    assert T._kind("x", meta(1, n), 1, n) == "tile"  # (1, N) at M = 1 is C's shape
    assert T._kind("x", 2.0, m, n) == "const"
    with pytest.raises(ValueError, match="broadcast"):
        T._kind("x", meta(m), m, n)
    with pytest.raises(TypeError):
        T._kind("x", True, m, n)


def test_misuse_is_named():
    with pytest.raises(AttributeError, match="ctx.bias"):
        T.bind(T.bias, {"scale": 1.0}, 64, 256, torch.bfloat16)
    with pytest.raises(TypeError, match="returned"):
        T.bind(lambda acc, ctx: ctx.bias, {"bias": meta(256)}, 64, 256, torch.bfloat16)
    with pytest.raises(TypeError, match="returned"):
        T.bind(lambda acc: 3.0, {}, 64, 256, torch.bfloat16)
    with pytest.raises(ValueError, match="cannot name"):
        T.bind(T.bias, {"out": meta(256)}, 64, 256, torch.bfloat16)
    with pytest.raises(TypeError, match="keyword-only"):
        T.bind(lambda acc, *, alpha: acc, {}, 64, 256, torch.bfloat16)
    with pytest.raises(ValueError, match="init_from"):
        T.bind(T.residual, {"residual": meta(256)}, 64, 256, torch.bfloat16)
    with pytest.raises(TypeError, match="truth value"):
        T.bind(lambda acc: acc if acc else acc, {}, 64, 256, torch.bfloat16)
    with pytest.raises(ValueError, match="only come first"):
        T.chain(T.relu, T.residual)


def test_tags_are_deterministic_and_bindings_cached():
    e1 = T.bind(T.bias_gelu, {"bias": meta(256)}, 64, 256, torch.bfloat16)
    e2 = T.bind(T.bias_gelu, {"bias": meta(256)}, 64, 256, torch.bfloat16)
    assert e1 is e2 and e1.tag.startswith("ep_bias_gelu_")
    e3 = T.bind(T.bias_gelu, {"bias": meta(256, dtype=torch.float32)}, 64, 256, torch.bfloat16)
    assert e3.tag != e1.tag


def test_binding_by_parameter_name_and_keyword_defaults():
    fn = lambda acc, bias, *, alpha=2.0: acc * alpha + bias  # noqa: E731
    c = compiled(fn, bias=meta(256))
    assert (c.form, c.cmul, c.row_add) == ("fused", 2.0, "bias")
    c = compiled(fn, bias=meta(256), alpha=3.0)
    assert c.cmul == 3.0


# ------------------------------------------------------------------ plans and routes

LAYERS = [(4096, 4096), (12288, 4096), (4096, 12288), (6144, 4096), (1408, 640), (24576, 4096)]
MS = [1, 4, 16, 17, 32, 33, 100, 128, 200, 1024, 2048, 4096, 8192]


@pytest.mark.parametrize("n,k", LAYERS)
def test_every_column_is_written_once_and_carries_the_epilogue_once(n, k):
    for m in MS:
        steps = T.plan(m, n, k)
        writers = [s for s in steps if s.into == "out"]
        assert len(writers) == 1 and writers[0].epilogue and writers[0].cols == (0, n)
        for s in steps:
            if s.into == "scratch":
                assert not s.epilogue  # split shares never run the epilogue
        if any(s.sched.get("splits", 1) > 1 for s in steps):
            assert [s.kernel for s in steps][-1] == "reduce"


def test_an_epilogue_outside_the_fused_form_gets_the_reduction():
    steps = T.plan(4096, 4096, 4096, epilogue_in_kernel=False)
    assert [(s.kernel, s.into, s.epilogue) for s in steps] == [
        ("tile", "scratch", False), ("reduce", "out", True)]


def test_routes():
    assert gemm_cdna.route(1, 12288, 4096) == "decode"
    assert gemm_cdna.route(16, 12288, 4096) == "decode"
    assert gemm_cdna.route(4096, 12288, 4096).startswith("t256")
    assert gemm_cdna.route(8192, 24576, 4096).startswith("t256")
    # a grid too small for the GPU splits over K
    assert "k" in gemm_cdna.rule(64, 4096, 4096)
    # fp8 has no decode kernel
    assert gemm_cdna.route(16, 4096, 4096, fp8=True).startswith("t64")
    for name in gemm_cdna.CANDIDATES:
        rec = gemm_cdna.resolve(gemm_cdna.CANDIDATES[name], 17, 1536, 2048)
        assert rec["splits"] >= 1


def test_a_user_override_wins():
    gemm_cdna.OVERRIDE[(4096, 12288, 4096)] = "t128"
    try:
        assert T.plan(4096, 12288, 4096)[0].route == "t128"
    finally:
        gemm_cdna.OVERRIDE.clear()


def test_schedule_records():
    steps = T.plan(300, 4096, 1024, schedule={"kernel": "tile", "tile_m": 64, "tile_n": 256,
                                              "splits": 2})
    assert steps[0].sched["splits"] == 2 and steps[-1].kernel == "reduce"
    with pytest.raises(ValueError):
        T.plan(300, 4096, 1024, schedule="nonsense")


def test_kernels_describe_the_launches_with_meta_tensors():
    ks = T.kernels(4096, 12288, 4096, epilogue=T.bias_gelu, bias=meta(12288))
    (step, kern, _), = ks
    assert step.kernel == "tile" and "gelu_tanh(acc + bias)" in kern.name
    ks = T.kernels(4096, 24576, 4096, epilogue=T.silu_and_mul)
    assert ks[-1][0].epilogue


def test_shape_checks():
    with pytest.raises(ValueError, match="multiple of 64"):
        T.plan(16, 4096, 100)
    with pytest.raises(ValueError, match="nothing to multiply"):
        T.plan(0, 4096, 4096)


def test_workspace_under_capture_is_the_graphs_own(monkeypatch):
    """Each call captured into a graph gets a fresh workspace, allocated in the capture (the
    graph's private pool owns it for the graph's life) and not kept in the eager cache; so a
    process that captures many graphs keeps nothing per captured call. Outside capture one
    buffer per stream is reused and grown."""
    from hk import _native as nat

    monkeypatch.setattr(nat, "stream_of", lambda dev: 12345)
    monkeypatch.setattr(nat, "_WS", {})
    monkeypatch.setattr(nat, "capturing", lambda dev: True)
    first = nat.workspace("cpu", 64)
    again = nat.workspace("cpu", 32)
    assert again is not first
    second = nat.workspace("cpu", 4096)
    assert second.numel() * 4 >= 4096
    assert nat._WS == {}                       # captured buffers are not the eager cache
    assert not hasattr(nat, "_PINNED")
    assert nat.workspace("cpu", 0) is None
    # outside capture, one buffer per stream, replaced when a call needs more
    monkeypatch.setattr(nat, "capturing", lambda dev: False)
    small = nat.workspace("cpu", 64)
    assert nat.workspace("cpu", 32) is small
    big = nat.workspace("cpu", 4096)
    assert big is not small and nat._WS[("cpu", 12345)] is big


def test_scaled_mm_argument_errors_on_the_cpu():
    """scaled_mm refuses what the reference refuses before any launch
    (python/hk/ops/gemm.py:911-966): a non-fp8 operand, a bias with an fp32 out, and
    accumulate=True without an fp32 out."""
    import torch

    import hk

    a8 = torch.zeros(4, 128, dtype=torch.float8_e5m2)
    b8 = torch.zeros(8, 128, dtype=torch.float8_e4m3fn)
    with pytest.raises(TypeError, match="float8_e4m3fn or float8_e5m2"):
        hk.ops.scaled_mm(a8.half(), b8, 1.0, 1.0)
    with pytest.raises(ValueError, match="fp32 out takes no bias"):
        hk.ops.scaled_mm(a8, b8, 1.0, 1.0, bias=torch.zeros(8), out=torch.zeros(4, 8))
    with pytest.raises(ValueError, match="accumulate=True"):
        hk.ops.scaled_mm(a8, b8, 1.0, 1.0, accumulate=True)
    from hk import _native as nat
    from hk.ops import gemm as G

    assert G._pair_code(a8, b8) == nat.FP8_E5M2_E4M3
    assert G._pair_code(b8, a8) == nat.FP8_E4M3_E5M2
    assert G._pair_code(a8, a8) == nat.FP8E5M2 and G._pair_code(b8, b8) == nat.FP8E4M3
