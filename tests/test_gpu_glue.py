"""GPU parity of the decode-layer glue against the CPU oracle (cases from
benchmarks/test_fused_equivalence.py:92-122): RoPE bit-exact; RMSNorm and
SwiGLU within one fp16 ulp (the device rsqrt/exp are AMD's own, so the
reference's bit-exactness against torch-CUDA does not carry over)."""
import numpy as np
import pytest
import torch

from oracle import glue
from tests.gpu_util import assert_bitexact, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def C():
    from signrot_amd import _CUDA
    return _CUDA


def _within_ulp(got, want, what, ulps=1):
    g = np.asarray(got, np.float16).astype(np.float64)
    w = np.asarray(want, np.float16).astype(np.float64)
    spacing = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    d = np.abs(g - w)
    bad = d > ulps * spacing
    assert not bad.any(), f"{what}: {bad.sum()} / {bad.size} beyond {ulps} ulp, max {d.max()}"


@pytest.mark.parametrize("rows,cols", [(1, 4096), (16, 4096), (2048, 4096), (1, 11008),
                                       (32, 14336), (3, 128), (5, 100), (2, 8200)])
def test_rmsnorm(C, rows, cols):
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float16)
    got = to_np(C.rmsnorm(to_dev(x), 1e-5, cols))
    _within_ulp(got, glue.rmsnorm(x, 1e-5, cols), "rmsnorm")


def test_rmsnorm_mean_dim_and_module(C):
    from signrot_amd.nn import RMSNorm
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((4, 4096)) * 30).astype(np.float16)
    got = to_np(RMSNorm(1024, eps=1e-6)(to_dev(x)))
    _within_ulp(got, glue.rmsnorm(x, 1e-6, 1024), "rmsnorm mean_dim")
    z = np.zeros((2, 4096), np.float16)
    assert np.all(to_np(C.rmsnorm(to_dev(z), 1e-5, 4096)) == 0)


@pytest.mark.parametrize("b,t,hq,hk,d", [(1, 1, 32, 32, 128), (16, 1, 32, 32, 128),
                                         (1, 2048, 32, 32, 128), (4, 3, 32, 8, 128),
                                         (32, 1, 32, 8, 128), (2, 5, 4, 2, 64)])
def test_rope_bitexact(C, b, t, hq, hk, d):
    rng = np.random.default_rng(b * 31 + t)
    q = rng.standard_normal((b, t, hq, d)).astype(np.float16)
    k = rng.standard_normal((b, t, hk, d)).astype(np.float16)
    for cb in sorted({1, b}):
        c = rng.standard_normal((cb, t, d)).astype(np.float16)
        s = rng.standard_normal((cb, t, d)).astype(np.float16)
        qw, kw = glue.rope_qk(q, k, c, s)
        dq, dk = to_dev(q), to_dev(k)
        C.rope_qk(dq, dk, to_dev(c), to_dev(s))
        assert_bitexact(to_np(dq), qw, f"q cos_b={cb}")
        assert_bitexact(to_np(dk), kw, f"k cos_b={cb}")


def test_rope_signed_zeros(C):
    """Zeros of both signs, fp16 underflow and their sums in every (x0, x1,
    cos, sin) combination: the kernel's output bits, the sign of zero
    included, are the oracle's (a multiply rounded through fma(x, y, +0)
    once turned -0 products into +0 here)."""
    vals = np.array([0.0, -0.0, 1e-7, -1e-7, 6e-8, -6e-8, 0.5, -0.5, 3.0, -3.0], np.float16)
    n = len(vals)
    x0, x1, c, s = np.meshgrid(vals, vals, vals, vals, indexing="ij")
    q = np.stack([x0.reshape(-1), x1.reshape(-1)], -1).reshape(1, n ** 4, 1, 2)
    cos = np.stack([c.reshape(-1)] * 2, -1).reshape(1, n ** 4, 2)
    sin = np.stack([s.reshape(-1)] * 2, -1).reshape(1, n ** 4, 2)
    qw, _ = glue.rope_qk(q, q, cos, sin)
    dq, dk = to_dev(q), to_dev(q.copy())
    C.rope_qk(dq, dk, to_dev(cos), to_dev(sin))
    assert_bitexact(to_np(dq), qw, "rope q signed zeros")
    assert_bitexact(to_np(dk), qw, "rope k signed zeros")


@pytest.mark.parametrize("shape", [(1, 11008), (16, 11008), (2048, 11008), (32, 14336), (7,)])
def test_swiglu(C, shape):
    rng = np.random.default_rng(sum(shape))
    g = (rng.standard_normal(shape) * 4).astype(np.float16)
    u = (rng.standard_normal(shape) * 4).astype(np.float16)
    got = to_np(C.swiglu(to_dev(g), to_dev(u))).astype(np.float64)
    want = glue.swiglu(g, u)
    # a one-ulp flip of the rounded silu (device expf vs float64 exp) moves
    # the product by |up| * ulp(silu), plus the final rounding's ulp
    silu = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))).astype(np.float16)
    tol = (np.spacing(np.abs(want)).astype(np.float64) +
           np.abs(u.astype(np.float64)) * np.spacing(np.abs(silu)).astype(np.float64))
    d = np.abs(got - want.astype(np.float64))
    assert (d <= tol).all(), f"swiglu: {(d > tol).sum()} beyond tolerance, max {d.max()}"
    # nearly all elements agree exactly
    assert (d == 0).mean() > 0.999
