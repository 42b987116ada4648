"""GPU parity: the Hadamard rotation (tolerance vs the float64 closed form
and vs the oracle's rounding points -- the reference FWHT's bits are not
pinnable) and the fused rotation + sign + quant (bit-exact given the same
rotated fp16 input)."""
import math

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import hadamard as oh
from oracle import quant as oq
from tests.gpu_util import assert_bitexact, outlier_input, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def C():
    from signrot_amd import _CUDA
    return _CUDA


def _hadk(k, dtype=torch.float16):
    return to_dev(oh.had_table(k).astype(np.float32)).to(dtype)


@pytest.mark.parametrize("n", [8, 32, 128, 512, 4096, 16384, 32768])
@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_hadamard_transform_closed_form(C, n, dtype):
    rng = np.random.default_rng(n)
    rows = 3 if n >= 16384 else 17
    x = rng.standard_normal((rows, n)).astype(dtype)
    scale = 1.0 / math.sqrt(n)
    out = to_np(C.hadamard_transform(to_dev(x), scale))
    want = oh.fwht(x.astype(np.float64)) * np.float64(np.float32(scale))
    # fp32 accumulation: log2(n) rounded adds of partial sums bounded by the
    # row's L1 norm (times scale)
    acc = np.log2(n) * 2.0 ** -23 * scale * np.abs(x.astype(np.float64)).sum(-1, keepdims=True)
    if dtype == np.float16:
        ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
        # one fp16 rounding of the fp32-accumulated value
        assert np.all(np.abs(out.astype(np.float64) - want) <= ulp + acc), "fp16 FWHT error"
        # and almost always the correctly rounded value
        exact = want.astype(np.float16)
        assert np.mean(out != exact) < 1e-3
    else:
        assert np.all(np.abs(out.astype(np.float64) - want) <= acc + 1e-30)


@pytest.mark.parametrize("n", [4096, 14336, 28672, 12 * 64, 11008, 128, 32, 6144, 10240,
                               12288, 20480])
def test_online_hadamard_vs_oracle(C, n):
    rng = np.random.default_rng(n + 1)
    x = outlier_input(rng, 9, n, n_out=min(8, n // 4), mag=50.0)
    had, k = oh.get_hadK(n)
    sign = rng.choice([-1, 1], n).astype(np.int8)
    hk = _hadk(k) if k > 1 else None
    out = to_np(C.online_hadamard(to_dev(x), hk, k, to_dev(sign)))
    want = oh.online_hadamard(x, sign)
    exact = oh.matmul_hadU_f64(x.astype(np.float64)) * sign
    # rtol 1e-2 / atol 1e-2 against the oracle ...
    np.testing.assert_allclose(out.astype(np.float32), want.astype(np.float32),
                               rtol=1e-2, atol=1e-2)
    # ... and agreement in (nearly) every bit: differences only where fp32
    # accumulation order moves a value across an fp16 rounding boundary
    assert np.mean(out.view(np.uint16) != want.view(np.uint16)) < 5e-3
    np.testing.assert_allclose(out.astype(np.float64), exact, rtol=1e-2, atol=1e-2)


def test_online_hadamard_fp32_mode(C):
    rng = np.random.default_rng(2)
    n = 14336
    x = outlier_input(rng, 4, n, n_out=8, mag=50.0)
    out = to_np(C.online_hadamard(to_dev(x), _hadk(28, torch.float32), 28, None, True))
    exact = oh.matmul_hadU_f64(x.astype(np.float64))
    # a single rounding at the end (plus the fp32 accumulation error of the
    # FWHT and the 28-term mix)
    ulp = np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64)
    acc = 16 * 2.0 ** -23 * np.abs(x.astype(np.float64)).sum(-1, keepdims=True) / np.sqrt(n)
    assert np.all(np.abs(out.astype(np.float64) - exact) <= ulp + acc)
    assert np.mean(out != exact.astype(np.float16)) < 1e-3


@pytest.mark.parametrize("n,rows", [(4096, 16), (14336, 64), (28672, 5), (128, 33),
                                    (11008, 3), (32, 10), (14336, 7), (14336, 3001),
                                    (14336, 1), (14336, 513), (14336, 1024),
                                    (6144, 9), (10240, 13), (28672, 700), (12288, 3),
                                    (20480, 2),
                                    # the register/shuffle kernel of the plain
                                    # 2^k rotations (one block per row, grid
                                    # stride past 4096 rows)
                                    (4096, 1), (2048, 5), (8192, 7), (8192, 1), (4096, 4200),
                                    # config 2 at M = 8192, config 4 at M = 4096
                                    (14336, 8192), (28672, 4096)])
@pytest.mark.parametrize("use_sign", [False, True])
def test_had_sign_quant_bitexact(C, n, rows, use_sign):
    rng = np.random.default_rng(n + rows)
    x = outlier_input(rng, rows, n, n_out=min(8, n // 4), mag=100.0)
    _, k = oh.get_hadK(n)
    hk = _hadk(k) if k > 1 else None
    sign_np = rng.choice([-1, 1], n).astype(np.int8) if use_sign else np.ones(n, np.int8)
    sign = to_dev(sign_np) if use_sign else None
    xd = to_dev(x)
    rot = C.online_hadamard(xd, hk, k, sign)
    q, s = C.had_sign_quant(xd, hk, k, sign)
    qw, sw = oq.sym_quant_dynamic(to_np(rot))
    assert_bitexact(to_np(s), sw, "scale")
    assert_bitexact(to_np(q), qw, "codes")
    # same as the unfused GPU composition
    q2, s2 = C.sym_quant_dynamic(rot.view(rows, n))
    assert torch.equal(q, q2) and torch.equal(s, s2)
    # the rotation itself on the first and last rows and on rows next to the
    # persistent kernels' grid strides (256 and 512 blocks)
    idx = sorted({i for i in (0, 255, 256, 511, 512, rows - 1) if i < rows})
    want = oh.online_hadamard(x[idx], sign_np)
    got = to_np(rot)[idx]
    np.testing.assert_allclose(got.astype(np.float32), want.astype(np.float32),
                               rtol=1e-2, atol=1e-2)
    assert np.mean(got.view(np.uint16) != want.view(np.uint16)) < 5e-3


@pytest.mark.parametrize("n", [2048, 4096, 8192])
def test_had_sign_quant_pow2_unaligned_sign(C, n):
    # a sign vector that is not 16-byte aligned takes the generic kernel:
    # the same codes and scales as the aligned one
    rng = np.random.default_rng(n)
    x = to_dev(outlier_input(rng, 9, n, n_out=8, mag=100.0))
    sign_np = rng.choice([-1, 1], n).astype(np.int8)
    buf = torch.empty(n + 16, dtype=torch.int8, device="cuda")
    buf[3:n + 3] = to_dev(sign_np)
    unaligned = buf[3:n + 3]
    assert unaligned.data_ptr() % 16 != 0
    q1, s1 = C.had_sign_quant(x, None, 1, to_dev(sign_np))
    q2, s2 = C.had_sign_quant(x, None, 1, unaligned)
    assert torch.equal(q1, q2) and torch.equal(s1, s2)


def test_zero_sign_raises_in_module():
    from signrot_amd.nn import OnlineHadamard
    m = OnlineHadamard(4096, had_adj=True).cuda()
    m.had_adj_sign[5] = 0
    with pytest.raises(RuntimeError):
        m(torch.zeros(2, 4096, dtype=torch.float16, device="cuda"))


@pytest.mark.parametrize("n", [14336, 28672])
@pytest.mark.parametrize("case", ["zeros", "tiny", "subnormal_scale", "clip", "huge"])
def test_had_sign_quant_edge_cases(C, case, n):
    """Rows the MFMA fast paths (n = 28 x 512, 28 x 1024) must treat like the
    reference: an all-zero row (scale 0, codes 0), tiny values (subnormal
    fp16 scale), a row whose scale underflows to 0, clip < 1 (codes clamp
    at -8), and large magnitudes."""
    rows = 8
    rng = np.random.default_rng(42)
    x = rng.standard_normal((rows, n)).astype(np.float16)
    clip = 1.0
    if case == "zeros":
        x[2] = 0
        x[5] = 0
    elif case == "tiny":
        x = (x.astype(np.float32) * 1e-5).astype(np.float16)
    elif case == "subnormal_scale":
        x[:] = 0
        x[1, 100] = np.float16(2 ** -24)
        x[3, 7] = -np.float16(2 ** -23)
    elif case == "clip":
        clip = 0.8
    else:
        x = (x.astype(np.float32) * 300).astype(np.float16)
    hk = _hadk(28)
    sign = to_dev(rng.choice([-1, 1], n).astype(np.int8))
    xd = to_dev(x)
    rot = C.online_hadamard(xd, hk, 28, sign)
    q, s = C.had_sign_quant(xd, hk, 28, sign, clip)
    qw, sw = oq.sym_quant_dynamic(to_np(rot), clip)
    assert_bitexact(to_np(s), sw, "scale")
    assert_bitexact(to_np(q), qw, "codes")


@pytest.mark.parametrize("n", [14336, 28672])
@pytest.mark.parametrize("clip", [1.0, 0.8])
def test_had_sign_quant_mixed_rows(C, clip, n):
    """One launch whose persistent blocks meet rows of every kind in turn:
    ordinary rows, all-zero rows, rows whose fp16 scale is subnormal or
    underflows (the clamped path) and large rows -- each row's codes and
    scale must not depend on its neighbours."""
    rows = 1100
    rng = np.random.default_rng(7)
    x = outlier_input(rng, rows, n, n_out=8, mag=50.0).astype(np.float32)
    kind = rng.integers(0, 5, rows)
    x[kind == 1] = 0
    x[kind == 2] *= 1e-6
    x[kind == 3] = 0
    x[np.nonzero(kind == 3)[0], 11] = 2.0 ** -24
    x[kind == 4] *= 200
    x = x.astype(np.float16)
    hk = _hadk(28)
    sign = to_dev(rng.choice([-1, 1], n).astype(np.int8))
    xd = to_dev(x)
    rot = C.online_hadamard(xd, hk, 28, sign)
    q, s = C.had_sign_quant(xd, hk, 28, sign, clip)
    qw, sw = oq.sym_quant_dynamic(to_np(rot), clip)
    assert_bitexact(to_np(s), sw, "scale")
    assert_bitexact(to_np(q), qw, "codes")
