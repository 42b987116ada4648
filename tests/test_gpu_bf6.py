"""GPU parity of the bf6 GEMM path: the int4 -> bf6 conversion against the
NumPy layout statement (bit-exact), and matmul_bf6 / w4a4_linear_bf6
against the oracle's int4 products and fused dequant (bit-exact), at small,
ragged and config shapes."""
import numpy as np
import pytest
import torch

from oracle import quant as oq
from tests.bf6_layout import encode
from tests.gpu_util import assert_bitexact, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def C():
    from signrot_amd import _CUDA
    return _CUDA


def _rand_packed(rng, r, k):
    return rng.integers(0, 256, (r, k // 2)).astype(np.uint8)


@pytest.mark.parametrize("R,K", [(1, 128), (32, 128), (45, 256), (300, 1024), (4096, 640)])
def test_i4_to_bf6_matches_layout(C, R, K):
    rng = np.random.default_rng(R + K)
    w = _rand_packed(rng, R, K)
    got = to_np(C.i4_to_bf6(to_dev(w)))
    assert_bitexact(got, encode(oq.unpack_i4(w)), "bf6 bytes")


BF6_SHAPES = [
    (1, 32, 128), (7, 5, 128), (256, 128, 128), (300, 200, 256), (33, 1000, 384),
    (512, 512, 4096), (1024, 4096, 1024), (2048, 4096, 1536), (600, 4160, 2048),
]


@pytest.mark.parametrize("M,N,K", BF6_SHAPES)
def test_matmul_bf6_bitexact(C, M, N, K):
    rng = np.random.default_rng(M * 3 + N * 5 + K)
    a, b = _rand_packed(rng, M, K), _rand_packed(rng, N, K)
    a6, b6 = C.i4_to_bf6(to_dev(a)), C.i4_to_bf6(to_dev(b))
    c = to_np(C.matmul_bf6(a6, b6, M, N, K))
    assert_bitexact(c, oq.matmul_s4s4(a, b), "int32 C")
    # and equal to the int8-MFMA GEMM on the packed operands
    assert np.array_equal(c, to_np(C.matmul(to_dev(a), to_dev(b))))


@pytest.mark.parametrize("M,N,K", [(256, 128, 128), (300, 200, 256), (2048, 4096, 1536),
                                   (65, 4100, 4096)])
@pytest.mark.parametrize("bias", [False, True])
def test_w4a4_linear_bf6_bitexact(C, M, N, K, bias):
    rng = np.random.default_rng(M + N + K + bias)
    a, b = _rand_packed(rng, M, K), _rand_packed(rng, N, K)
    sa = (np.abs(rng.standard_normal(M)) * 0.05 + 1e-3).astype(np.float16)
    sb = (np.abs(rng.standard_normal(N)) * 0.01 + 1e-4).astype(np.float16)
    bs = (rng.standard_normal(N) * 0.5).astype(np.float16) if bias else None
    a6, b6 = C.i4_to_bf6(to_dev(a)), C.i4_to_bf6(to_dev(b))
    out = C.w4a4_linear_bf6(a6, to_dev(sa), b6, to_dev(sb), M, N, K,
                            to_dev(bs) if bias else None)
    assert_bitexact(to_np(out), oq.w4a4_linear(a, sa, b, sb, bs), "fp16 out")


def test_bf6_extreme_values(C):
    # every code -8 at K = 28672 (the cfg4 down_proj depth): 64 K per output
    K = 28672
    a = np.full((40, K // 2), 0x88, np.uint8)
    b = np.full((33, K // 2), 0x88, np.uint8)
    c = to_np(C.matmul_bf6(C.i4_to_bf6(to_dev(a)), C.i4_to_bf6(to_dev(b)), 40, 33, K))
    assert np.all(c == 64 * K)
    b2 = np.full((33, K // 2), 0x77, np.uint8)
    c2 = to_np(C.matmul_bf6(C.i4_to_bf6(to_dev(a)), C.i4_to_bf6(to_dev(b2)), 40, 33, K))
    assert np.all(c2 == -56 * K)


def test_bf6_empty(C):
    a6 = torch.zeros(3072, dtype=torch.uint8, device="cuda")  # one block
    assert C.matmul_bf6(a6, a6, 0, 5, 128).shape == (0, 5)
    out = C.w4a4_linear_bf6(a6, torch.ones(3, dtype=torch.float16, device="cuda"), a6,
                            torch.ones(4, dtype=torch.float16, device="cuda"), 3, 4, 0)
    assert torch.equal(out, torch.zeros(3, 4, dtype=torch.float16, device="cuda"))


def _sample_rows(rng, M, n=48):
    fixed = {0, 1, 127, 128, 255, 256, M // 2, M - 257, M - 256, M - 2, M - 1}
    rand = set(rng.choice(M, n, replace=False).tolist())
    return np.array(sorted(r for r in fixed | rand if 0 <= r < M))


@pytest.mark.parametrize("M,N,K", [(2048, 4096, 14336), (8192, 4096, 14336),
                                   (512, 57344, 8192), (4096, 8192, 28672)])
def test_bf6_config_shapes_sampled_rows(C, M, N, K):
    rng = np.random.default_rng(M + N + K)
    a, b = _rand_packed(rng, M, K), _rand_packed(rng, N, K)
    sa = (np.abs(rng.standard_normal(M)) * 0.05 + 1e-3).astype(np.float16)
    sb = (np.abs(rng.standard_normal(N)) * 0.01 + 1e-4).astype(np.float16)
    a6, b6 = C.i4_to_bf6(to_dev(a)), C.i4_to_bf6(to_dev(b))
    c = C.matmul_bf6(a6, b6, M, N, K)
    out = C.w4a4_linear_bf6(a6, to_dev(sa), b6, to_dev(sb), M, N, K)
    rows = _sample_rows(rng, M)
    ridx = torch.from_numpy(rows).cuda()
    assert_bitexact(to_np(c[ridx]), oq.matmul_s4s4(a[rows], b), "int32 C")
    assert_bitexact(to_np(out[ridx]), oq.w4a4_linear(a[rows], sa[rows], b, sb), "fp16 out")


# ------------------------------------------------- quantizer with bf6 output

def _had_inputs(rng, M, K, chunk, outliers=True):
    from oracle import hadamard as oh
    n = K * chunk
    x = rng.standard_normal((M, n)).astype(np.float16)
    if outliers:
        cols = rng.choice(n, 8, replace=False)
        x[:, cols] *= 50
    sign = (rng.integers(0, 2, n) * 2 - 1).astype(np.int8)
    return x, oh.had_table(K).astype(np.float16), sign


@pytest.mark.parametrize("M,K,chunk,clip", [(1, 28, 512, 1.0), (33, 28, 512, 1.0),
                                            (300, 12, 512, 0.9), (64, 28, 1024, 1.0),
                                            (2048, 28, 512, 1.0), (70, 20, 1024, 0.8)])
def test_had_sign_quant_bf6_matches_int4_path(C, M, K, chunk, clip):
    """Same codes (decoded from the bf6 layout) and scales as had_sign_quant."""
    from tests.bf6_layout import decode
    rng = np.random.default_rng(M + K + chunk)
    x, hk, sign = _had_inputs(rng, M, K, chunk)
    dx, dh, ds = to_dev(x), to_dev(hk), to_dev(sign)
    q6, s6 = C.had_sign_quant_bf6(dx, dh, K, ds, clip)
    q4, s4 = C.had_sign_quant(dx, dh, K, ds, clip)
    assert torch.equal(s6, s4)
    n = K * chunk
    assert np.array_equal(decode(to_np(q6), M, n), oq.unpack_i4(to_np(q4))), "codes"


def test_had_sign_quant_bf6_nonfinite_rows(C):
    """Rows holding inf / NaN take the exact per-element path: same codes."""
    from tests.bf6_layout import decode
    rng = np.random.default_rng(5)
    M, K = 40, 28
    x, hk, sign = _had_inputs(rng, M, K, 512, outliers=False)
    x[3, 100] = np.inf
    x[7, 5] = np.nan
    x[11, :] = 0
    dx, dh, ds = to_dev(x), to_dev(hk), to_dev(sign)
    q6, s6 = C.had_sign_quant_bf6(dx, dh, K, ds)
    q4, s4 = C.had_sign_quant(dx, dh, K, ds)
    assert torch.equal(s6.view(torch.int16), s4.view(torch.int16))
    assert np.array_equal(decode(to_np(q6), M, K * 512), oq.unpack_i4(to_np(q4)))


def test_bf6_qlinear_chain(C):
    """had_sign_quant_bf6 -> w4a4_linear_bf6 == had_sign_quant -> w4a4_linear
    (bit-identical fp16 output), the cfg2 QLinear chain at a reduced M."""
    rng = np.random.default_rng(9)
    M, K, N = 96, 28, 256
    x, hk, sign = _had_inputs(rng, M, K, 512)
    n = K * 512
    w = _rand_packed(rng, N, n)
    sb = (np.abs(rng.standard_normal(N)) * 0.01 + 1e-4).astype(np.float16)
    dx, dh, ds, dw, dsb = to_dev(x), to_dev(hk), to_dev(sign), to_dev(w), to_dev(sb)
    q6, s6 = C.had_sign_quant_bf6(dx, dh, K, ds)
    out6 = C.w4a4_linear_bf6(q6, s6, C.i4_to_bf6(dw), dsb, M, N, n)
    q4, s4 = C.had_sign_quant(dx, dh, K, ds)
    out4 = C.w4a4_linear(q4, s4, dw, dsb)
    assert torch.equal(out6, out4)
