"""Pins the CPU oracle (oracle/gemm_oracle.py) before anything is checked against it.

Each oracle function is checked against something that does not share its code: torch's
own implementations (F.gelu(approximate="tanh"), F.silu, the float8_e4m3fn cast), a
float64 brute force on tiny shapes, the formulas' closed forms and special values, and
the fixtures in tests/golden/golden.npz, which make_golden.py computes in numpy float64
from the definitions. The checks are chosen so a plausible slip -- a wrong GELU
constant or sign, a transposed operand, a scale on the wrong axis, a dropped bias, an
fp8 exponent bias off by one -- fails one of them."""

import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gemm_oracle as O

G = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz", allow_pickle=False)


def _bf16(arr16: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(arr16.astype(np.int16)).view(torch.bfloat16)


# ------------------------------------------------------------------ GELU / SiLU

def test_gelu_tanh_matches_torch_and_closed_form():
    x = torch.linspace(-12, 12, 20001, dtype=torch.float64)
    want = F.gelu(x, approximate="tanh")
    assert (O.gelu_tanh(x).double() - want).abs().max().item() < 2e-6
    # special values of 0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3)))
    assert O.gelu_tanh(torch.tensor([0.0])).item() == 0.0
    v = 0.5 * (1 + math.tanh(math.sqrt(2 / math.pi) * (1 + 0.044715)))
    assert abs(O.gelu_tanh(torch.tensor([1.0])).item() - v) < 1e-6
    assert abs(O.gelu_tanh(torch.tensor([10.0])).item() - 10.0) < 1e-5
    assert abs(O.gelu_tanh(torch.tensor([-10.0])).item()) < 1e-5


def test_the_exp2_rsqrt_form_is_the_same_function():
    """The reference's instruction form (templates/gemm.py:814-837) -- and the kernels' --
    equals the textbook tanh-GELU: its constants pinned to a few fp32 ulps everywhere."""
    x = torch.linspace(-20, 20, 40001)
    a, b = O.gelu_tanh_exp2(x), O.gelu_tanh(x)
    assert ((a - b).abs() <= 2e-6 + 1e-5 * b.abs()).all()
    # a sign slip in B would make gelu(1) ~ 1.0 + ...; a dropped A would miss at |x| ~ 2
    assert abs(O.gelu_tanh_exp2(torch.tensor([2.0])).item() - F.gelu(torch.tensor(2.0), approximate="tanh").item()) < 1e-6
    assert O.GELU_B < 0 and O.GELU_A < 0 and abs(O.GELU_A / O.GELU_B - 0.044715) < 1e-15


def test_silu_and_silu_and_mul():
    x = torch.linspace(-30, 30, 6001, dtype=torch.float64)
    assert (O.silu(x).double() - F.silu(x)).abs().max().item() < 1e-5
    g = torch.randn(64, 32, generator=torch.Generator().manual_seed(0))
    u = torch.randn(64, 32, generator=torch.Generator().manual_seed(1))
    assert torch.allclose(O.silu_and_mul(g, u), F.silu(g) * u, atol=1e-6)
    assert O.silu(torch.tensor([-1e4])).item() == 0.0  # saturates, no NaN
    assert O.relu(torch.tensor([-1.0, 2.0])).tolist() == [0.0, 2.0]


# ------------------------------------------------------------------ the GEMM

def test_gemm_fp32_against_a_float64_brute_force():
    g = torch.Generator().manual_seed(3)
    a = torch.randn(8, 128, generator=g).to(torch.bfloat16)
    b = torch.randn(64, 128, generator=g).to(torch.bfloat16)
    brute = np.zeros((8, 64))
    av, bv = a.double().numpy(), b.double().numpy()
    for i in range(8):
        for j in range(64):
            brute[i, j] = sum(av[i, t] * bv[j, t] for t in range(128))
    got = O.gemm_fp32(a, b).double().numpy()
    assert np.abs(got - brute).max() < 1e-4
    # B is (N, K): a transposed operand would not even have this shape
    assert tuple(O.gemm_fp32(a, b).shape) == (8, 64)
    assert np.abs(O.gemm_f64(a, b).numpy() - brute).max() < 1e-10


def test_split_k_sums_whole_k_steps_in_order():
    g = torch.Generator().manual_seed(4)
    a = torch.randn(16, 640, generator=g).to(torch.bfloat16)
    b = torch.randn(32, 640, generator=g).to(torch.bfloat16)
    whole = O.gemm_f64(a, b)
    for splits in (1, 2, 3, 4, 7, 10):
        got = O.split_k(a, b, splits, 64)
        assert (got.double() - whole).abs().max().item() < 1e-3
    # 10 k-steps in 3 splits: shares of 4, 4, 2 steps -- ceil division
    share0 = O.gemm_fp32(a[:, :256], b[:, :256])
    share1 = O.gemm_fp32(a[:, 256:512], b[:, 256:512])
    share2 = O.gemm_fp32(a[:, 512:], b[:, 512:])
    assert torch.equal(O.split_k(a, b, 3, 64), (share0 + share1) + share2)


@pytest.mark.parametrize("m,n,k", [(m, n, k) for m in (1, 5, 17) for n in (128, 256) for k in (64, 128)])
def test_epilogues_against_the_golden_vectors(m, n, k):
    key = f"t_{m}_{n}_{k}"
    a, b = _bf16(G[key + "_a"]), _bf16(G[key + "_b"])
    bias, res = _bf16(G[key + "_bias"]), _bf16(G[key + "_res"])
    sc = torch.from_numpy(G[key + "_scale"])
    acc = O.gemm_fp32(a, b)
    assert np.abs(acc.double().numpy() - G[key + "_acc"]).max() < 1e-4
    tol = dict(rtol=1e-5, atol=1e-5)
    for name, ops in (("bias_gelu", dict(bias=bias)), ("bias_silu", dict(bias=bias)),
                      ("bias_relu", dict(bias=bias)), ("bias_residual", dict(bias=bias, residual=res))):
        np.testing.assert_allclose(O.apply_epilogue(name, acc, **ops).double().numpy(),
                                   G[key + "_" + name], **tol)
    np.testing.assert_allclose(O.apply_epilogue("scale", acc, scale=sc).double().numpy(),
                               G[key + "_scale_out"], **tol)
    if n == 256:
        np.testing.assert_allclose(O.silu_and_mul(acc[:, :128], acc[:, 128:]).double().numpy(),
                                   G[key + "_silu_and_mul"], **tol)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_config1_against_its_golden_slice(seed):
    """Config 1's inputs are the seeded generator's (their sha256 pins it), and the oracle's
    y = gelu_tanh(x @ w + b) matches the float64 fixture."""
    import hashlib

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(256, 1024, generator=g).to(torch.bfloat16)
    w = (torch.randn(1024, 1024, generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(1024, generator=g) * 0.1).to(torch.bfloat16)
    shas = [hashlib.sha256(t.view(torch.int16).numpy().tobytes()).hexdigest() for t in (x, w, b)]
    assert shas == list(G[f"cfg1_s{seed}_sha"])
    y = O.linear_bias_gelu(x[:16], w, b)
    np.testing.assert_allclose(y.numpy(), G[f"cfg1_s{seed}_y16"], rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------------ fp8 e4m3

def test_e4m3_decode_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ours = O.e4m3_decode(codes).astype(np.float64)
    fixture = G["e4m3_values"]
    torch_vals = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().double().numpy()
    nan = np.isnan(fixture)
    assert list(np.nonzero(nan)[0]) == [0x7F, 0xFF]
    assert np.array_equal(np.isnan(ours), nan) and np.array_equal(np.isnan(torch_vals), nan)
    assert np.array_equal(ours[~nan], fixture[~nan])
    assert np.array_equal(torch_vals[~nan], fixture[~nan])
    assert fixture[0x7E] == 448.0 and fixture[0x01] == 2.0 ** -9 and fixture[0x08] == 2.0 ** -6


def test_e4m3_encode_rounds_to_nearest_even_and_saturates():
    g = torch.Generator().manual_seed(5)
    x = torch.cat([torch.randn(20000, generator=g) * s for s in (0.01, 1.0, 30.0, 200.0)])
    x = x[x.abs() <= 448]
    ours = O.e4m3_encode(x.numpy())
    theirs = x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()  # torch rounds to nearest even
    assert np.array_equal(ours, theirs)
    # ties go to the even code: 1.0625 lies halfway between 1.0 (0x38) and 1.125 (0x39)
    assert O.e4m3_encode(np.array([1.0625], np.float32))[0] == 0x38
    assert O.e4m3_encode(np.array([1.1875], np.float32))[0] == 0x3A
    # past 448 the quantizing store saturates (torch's cast would not)
    assert list(O.e4m3_encode(np.array([500.0, -1e6, 448.0], np.float32))) == [0x7E, 0xFE, 0x7E]


def test_int8_quantizer():
    x = torch.tensor([2.5, -2.5, 3.5, 0.49, 126.6, 300.0, -300.0])
    assert O.quantize_int8(x).tolist() == [2.0, -2.0, 4.0, 0.0, 127.0, 127.0, -128.0]


def test_scaled_mm_against_the_golden_vector_and_special_cases():
    a8 = torch.from_numpy(G["fp8_a"]).view(torch.float8_e4m3fn)
    b8 = torch.from_numpy(G["fp8_b"]).view(torch.float8_e4m3fn)
    sa, sb = torch.from_numpy(G["fp8_sa"]), torch.from_numpy(G["fp8_sb"])
    bias = _bf16(G["fp8_bias"])
    np.testing.assert_allclose(O.scaled_mm(a8, b8, sa, sb, bias).double().numpy(), G["fp8_out"],
                               rtol=1e-5, atol=1e-7)
    # identity operands: the product is the scales' outer product -- each on its own axis
    eye = torch.eye(16).to(torch.float8_e4m3fn)
    sa2 = torch.arange(1, 17, dtype=torch.float32).reshape(16, 1)
    sb2 = torch.arange(1, 17, dtype=torch.float32) * 10
    out = O.scaled_mm(eye, eye, sa2, sb2)
    assert torch.equal(out, torch.diag(sa2.reshape(16) * sb2))
    # per-tensor scales broadcast
    assert torch.equal(O.scaled_mm(eye, eye, 2.0, 3.0), torch.eye(16) * 6.0)


def test_rel_to_max_and_assert_close():
    ref = torch.tensor([1.0, -4.0, 2.0])
    assert O.rel_to_max(ref + torch.tensor([0.0, 0.04, 0.0]), ref) == pytest.approx(0.01)
    with pytest.raises(AssertionError):
        O.assert_close(ref * 1.1, ref, rtol=1e-2, atol=1e-2)


# ------------------------------------------------------------------ MX fp8 (the oracle pinned)


def test_e8m0_is_a_power_of_two():
    s = torch.tensor([0, 100, 127, 130, 254], dtype=torch.uint8)
    assert O.e8m0(s).tolist() == [2.0 ** -127, 2.0 ** -27, 1.0, 8.0, 2.0 ** 127]


def test_mx_quant_hand_blocks():
    """Blocks whose answer follows from the rule by hand: a max of exactly 448 keeps e = 0;
    480 needs e = 1 (values halved); a max of 1 gives e = -8 (1 -> 256); a block of zeros
    and a tiny block clamp their byte at 0 while q is scaled by the unclamped e."""
    rows = [[448.0] + [1.0] * 31,
            [480.0] + [0.5] * 31,
            [1.0] + [0.25] * 31,
            [0.0] * 32,
            [2.0 ** -130] + [0.0] * 31]
    x = torch.tensor(rows).to(torch.bfloat16)
    q, s = O.mx_quant(x)
    assert s.flatten().tolist() == [127, 128, 119, 0, 0]
    qf = q.float()
    assert qf[0, :2].tolist() == [448.0, 1.0]
    assert qf[1, :2].tolist() == [240.0, 0.25]
    assert qf[2, :2].tolist() == [256.0, 64.0]
    assert (qf[3] == 0).all()
    assert qf[4, 0].item() == 16.0  # 2^-130 / 2^-134


def test_mx_quant_scale_is_the_smallest_that_fits():
    """Every block of random rows (magnitudes 2^-20..2^20): the block max lands in (224, 448]
    after scaling (one power of two less would overflow 448); dequant is within e4m3's half
    ulp of x (relative 2^-4 at the block scale)."""
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(64, 256, generator=g) *
         torch.exp2(torch.randint(-20, 20, (64, 1), generator=g).float())).to(torch.bfloat16)
    q, s = O.mx_quant(x)
    v = x.float().reshape(64, 8, 32)
    scaled_max = v.abs().amax(-1) / O.e8m0(s)
    assert (scaled_max <= 448.0).all() and (scaled_max > 224.0).all()
    err = (O.mx_dequant(q, s) - x.float()).abs().reshape(64, 8, 32)
    assert (err <= O.e8m0(s)[..., None] * 448.0 * 2.0 ** -4).all()


def test_mx_quant_round_trips_representable_values():
    """Values that are e4m3 numbers times the block's scale come back exactly."""
    g = torch.Generator().manual_seed(8)
    base = torch.randn(16, 128, generator=g).clamp(-440, 440).to(torch.float8_e4m3fn).float()
    base[:, ::32] = 448.0  # pin every block's max, so e = 0 before the row factor
    x = (base * torch.exp2(torch.randint(-6, 6, (16, 1), generator=g).float())).to(torch.bfloat16)
    q, s = O.mx_quant(x)
    assert torch.equal(O.mx_dequant(q, s), x.float())


def test_mx_gemm_is_the_scaled_product():
    """Against a float64 brute force over (m, n, k) with the scales applied term by term."""
    g = torch.Generator().manual_seed(9)
    m, n, k = 3, 5, 64
    a = torch.randn(m, k, generator=g).to(torch.float8_e4m3fn)
    b = torch.randn(n, k, generator=g).to(torch.float8_e4m3fn)
    sa = torch.randint(120, 135, (m, k // 32), generator=g, dtype=torch.uint8)
    sb = torch.randint(120, 135, (n, k // 32), generator=g, dtype=torch.uint8)
    ref = [[sum(float(a[i, t]) * 2.0 ** (int(sa[i, t // 32]) - 127) *
                float(b[j, t]) * 2.0 ** (int(sb[j, t // 32]) - 127) for t in range(k))
            for j in range(n)] for i in range(m)]
    got = O.mx_gemm(a, b, sa, sb).double()
    assert torch.allclose(got, torch.tensor(ref, dtype=torch.float64), rtol=1e-5, atol=1e-6)
