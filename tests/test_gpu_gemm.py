"""GPU parity: int4 GEMM (int32, bit-exact) and the fused W4A4 linear
(fp16, bit-exact) vs the CPU oracle; fused == unfused on the GPU."""
import numpy as np
import pytest
import torch

from oracle import quant as oq
from tests.gpu_util import assert_bitexact, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def C():
    from signrot_amd import _CUDA
    return _CUDA


GEMM_SHAPES = [
    (1, 4096, 4096), (16, 4096, 4096), (1, 4096, 14336), (16, 4096, 14336),
    (17, 100, 768), (32, 768, 2048), (33, 64, 32), (64, 2048, 768), (65, 130, 4096),
    (128, 4096, 14336), (300, 513, 800), (513, 2048, 768), (2048, 4096, 14336),
    (2, 16, 32), (5, 3, 64), (1100, 300, 4128), (1024, 128, 256), (4096, 256, 1024),
    # M <= 32 weight-streaming kernel: decode shapes, several column blocks per
    # workgroup, ragged N and K, every A-register depth, and the fallback
    # past its limits (K > 16384, > 16 column blocks per workgroup)
    (32, 6144, 4096), (32, 28672, 4096), (32, 4096, 14336), (24, 4112, 16384),
    (16, 1000, 8192), (1, 57344, 8192), (3, 17, 4128), (20, 50, 96), (32, 16, 32),
    (9, 4096, 2048), (32, 300, 8320), (2, 70000, 256), (32, 64, 28672),
    # K > 16384: A through registers in batches of units (exact batches,
    # a ragged last batch, the cfg4 down-proj shapes)
    (1, 8192, 28672), (32, 8192, 28672), (16, 520, 20000), (7, 333, 40064),
    (25, 1000, 30016),
    # 256 x 128 tile kernel: the tile grid split over the 8 XCDs into 1, 2, 4
    # or 8 row parts (the split with the fewest panel rows per XCD), and
    # row-major where no split divides the grid
    (1024, 4096, 256), (2048, 512, 256),
    # 256 x 256 tile kernel (>= 256 such tiles): XCD-aware tile order, ragged
    # M and N with a K tail (row-major order), a grid of two waves of tiles
    (4096, 4096, 1024), (4352, 4160, 4128), (8192, 4096, 640),
]


def _rand_packed(rng, r, k):
    return rng.integers(0, 256, (r, k // 2)).astype(np.uint8)


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_matmul_bitexact(C, M, N, K):
    rng = np.random.default_rng(M * 7 + N * 13 + K)
    a, b = _rand_packed(rng, M, K), _rand_packed(rng, N, K)
    c = C.matmul(to_dev(a), to_dev(b))
    assert_bitexact(to_np(c), oq.matmul_s4s4(a, b), "int32 C")


def test_matmul_extreme_values(C):
    K = 28672
    a = np.full((3, K // 2), 0x88, np.uint8)
    b = np.full((17, K // 2), 0x88, np.uint8)
    c = to_np(C.matmul(to_dev(a), to_dev(b)))
    assert np.all(c == 64 * K)
    b2 = np.full((17, K // 2), 0x77, np.uint8)
    c2 = to_np(C.matmul(to_dev(a), to_dev(b2)))
    assert np.all(c2 == -56 * K)
    # the 256 x 256 tile kernel at the cfg4 down-proj depth
    a = np.full((4096, K // 2), 0x88, np.uint8)
    b = np.full((4096, K // 2), 0x77, np.uint8)
    c3 = to_np(C.matmul(to_dev(a), to_dev(b)))
    assert np.all(c3 == -56 * K)
    # the streaming kernel's deepest register configuration (M = 32, K =
    # 16384) and its batched form (K = 28672, four batches of A)
    for K in (16384, 28672):
        a = np.full((32, K // 2), 0x88, np.uint8)
        b = np.full((40, K // 2), 0x88, np.uint8)
        assert np.all(to_np(C.matmul(to_dev(a), to_dev(b))) == 64 * K)


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (16, 4096, 4096), (33, 300, 768),
                                   (128, 4096, 14336), (2048, 4096, 14336), (7, 5, 64),
                                   (32, 6144, 4096), (32, 28672, 4096), (32, 4096, 14336),
                                   (13, 4100, 8192), (4096, 4096, 2048),
                                   # the batched weight-streaming form (K > 16384)
                                   (32, 8192, 28672), (5, 1030, 20000),
                                   # mid-size M with >= 192 tiles of 128 x 128: the
                                   # grouped kernel's dense form (ragged M and N,
                                   # N not a multiple of 8)
                                   (300, 8192, 1024), (700, 4100, 2048), (129, 28672, 512)])
@pytest.mark.parametrize("bias", [False, True])
def test_w4a4_linear_bitexact(C, M, N, K, bias):
    rng = np.random.default_rng(M + N + K + bias)
    a, b = _rand_packed(rng, M, K), _rand_packed(rng, N, K)
    sa = (np.abs(rng.standard_normal(M)) * 0.05 + 1e-3).astype(np.float16)
    sb = (np.abs(rng.standard_normal(N)) * 0.01 + 1e-4).astype(np.float16)
    bs = (rng.standard_normal(N) * 0.5).astype(np.float16) if bias else None
    out = C.w4a4_linear(to_dev(a), to_dev(sa), to_dev(b), to_dev(sb),
                        to_dev(bs) if bias else None)
    want = oq.w4a4_linear(a, sa, b, sb, bs)
    assert_bitexact(to_np(out), want, "fp16 out")
    # the fused kernel equals the unfused GPU pair
    unf = C.sym_dequant(C.matmul(to_dev(a), to_dev(b)), to_dev(sa), to_dev(sb))
    if bias:
        unf = unf + to_dev(bs)
    assert torch.equal(out, unf)


@pytest.mark.parametrize("M,N,K", [(300, 8192, 1024), (700, 4104, 512)])
def test_w4a4_linear_residual_dense_grouped(C, M, N, K):
    """The residual (and bias) epilogue of the grouped kernel's dense form:
    linear + residual equals the oracle-checked linear plus the residual in
    fp16, in place too."""
    rng = np.random.default_rng(M + N)
    a, b = _rand_packed(rng, M, K), _rand_packed(rng, N, K)
    sa = to_dev((np.abs(rng.standard_normal(M)) * 0.05 + 1e-3).astype(np.float16))
    sb = to_dev((np.abs(rng.standard_normal(N)) * 0.01 + 1e-4).astype(np.float16))
    bs = to_dev((rng.standard_normal(N) * 0.5).astype(np.float16))
    res = to_dev((rng.standard_normal((M, N)) * 3.0).astype(np.float16))
    da, db = to_dev(a), to_dev(b)
    for bias in (None, bs):
        out = C.w4a4_linear_residual(da, sa, db, sb, res, bias=bias)
        want = C.w4a4_linear(da, sa, db, sb, bias) + res
        assert torch.equal(out, want)
    inplace = res.clone()
    C.w4a4_linear_residual(da, sa, db, sb, inplace, out=inplace)
    assert torch.equal(inplace, C.w4a4_linear(da, sa, db, sb) + res)


@pytest.mark.parametrize("M,N,K", [(128, 4096, 14336), (128, 14336, 4096), (200, 4100, 8192),
                                   (100, 14336, 4640), (512, 4096, 14336), (65, 1032, 28672),
                                   (99, 1001, 28672),
                                   # the big kernel's split: the cfg4 70B down_proj at M = 512;
                                   # ragged M with K chunks of 4352 and 3968 codes
                                   (512, 8192, 28672), (300, 8192, 8320)])
def test_w4a4_linear_split_k(C, M, N, K):
    """Mid-size M with few output tiles: the workspace entry points split K
    into int32 partials; the result is bit for bit the plain entry point's
    (itself pinned against the oracle above), with bias and residual, in
    place too; a K tail chunk (K = 4640: chunks of 2560 and 2080), M N not
    a multiple of 4 (99 x 1001: the one-output reduce)."""
    from signrot_amd import _native
    rng = np.random.default_rng(M * 7 + N + K)
    a, b = to_dev(_rand_packed(rng, M, K)), to_dev(_rand_packed(rng, N, K))
    sa = to_dev((np.abs(rng.standard_normal(M)) * 0.05 + 1e-3).astype(np.float16))
    sb = to_dev((np.abs(rng.standard_normal(N)) * 0.01 + 1e-4).astype(np.float16))
    bs = to_dev((rng.standard_normal(N) * 0.5).astype(np.float16))
    res = to_dev((rng.standard_normal((M, N)) * 3.0).astype(np.float16))
    nbytes = int(_native.lib().srq_w4a4_linear_ws_bytes(M, N, K))
    assert nbytes > 0, "shape expected to split"
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    p = lambda t: 0 if t is None else t.data_ptr()
    for bias in (None, bs):
        plain = torch.empty(M, N, dtype=torch.float16, device="cuda")
        split = torch.empty_like(plain)
        _native.call("srq_w4a4_linear", p(a), p(sa), p(b), p(sb), p(bias), M, N, K, p(plain), st)
        _native.call("srq_w4a4_linear_ws", p(a), p(sa), p(b), p(sb), p(bias), M, N, K, p(split),
                     p(ws), nbytes, st)
        assert torch.equal(plain, split)
        plain_r = torch.empty_like(plain)
        _native.call("srq_w4a4_linear_residual", p(a), p(sa), p(b), p(sb), p(bias), p(res), M, N,
                     K, p(plain_r), st)
        inplace = res.clone()
        _native.call("srq_w4a4_linear_residual_ws", p(a), p(sa), p(b), p(sb), p(bias),
                     p(inplace), M, N, K, p(inplace), p(ws), nbytes, st)
        assert torch.equal(plain_r, inplace)
    # the torch wrapper takes the split path and equals the oracle-checked one
    assert torch.equal(C.w4a4_linear(a, sa, b, sb, bs), split)


def test_matmul_rejects_bad_k(C):
    a = torch.zeros(4, 8, dtype=torch.uint8, device="cuda")  # K = 16
    with pytest.raises(RuntimeError):
        C.matmul(a, a)
    with pytest.raises(RuntimeError):
        C.matmul(torch.zeros(4, 16, dtype=torch.uint8, device="cuda"),
                 torch.zeros(4, 32, dtype=torch.uint8, device="cuda"))


def test_matmul_empty(C):
    a = torch.zeros(0, 16, dtype=torch.uint8, device="cuda")
    b = torch.zeros(5, 16, dtype=torch.uint8, device="cuda")
    assert C.matmul(a, b).shape == (0, 5)


def _sample_rows(rng, M, n=48):
    """Edge rows, rows at 128/256-row tile boundaries and random rows."""
    fixed = {0, 1, 127, 128, 255, 256, M // 2, M - 257, M - 256, M - 2, M - 1}
    rand = set(rng.choice(M, n, replace=False).tolist())
    return np.array(sorted(r for r in fixed | rand if 0 <= r < M))


@pytest.mark.parametrize("M,N,K,what", [
    (8192, 4096, 14336, "cfg2 down_proj M=8192"),
    (4096, 57344, 8192, "cfg4 gate/up (fused) M=4096"),
    (4096, 8192, 28672, "cfg4 down_proj M=4096"),
    (2048, 4096, 14336, "cfg2 down_proj M=2048"),
    (512, 57344, 8192, "cfg4 gate/up M=512"),
])
def test_config_shapes_sampled_rows(C, M, N, K, what):
    """The configs' full GEMM shapes (each kernel at its real tile grid), the
    int32 product and the fused W4A4 linear checked bit-exactly on sampled
    rows against the brute-force oracle."""
    rng = np.random.default_rng(M + N + K)
    a, b = _rand_packed(rng, M, K), _rand_packed(rng, N, K)
    sa = (np.abs(rng.standard_normal(M)) * 0.05 + 1e-3).astype(np.float16)
    sb = (np.abs(rng.standard_normal(N)) * 0.01 + 1e-4).astype(np.float16)
    da, db = to_dev(a), to_dev(b)
    c = C.matmul(da, db)
    out = C.w4a4_linear(da, to_dev(sa), db, to_dev(sb))
    rows = _sample_rows(rng, M)
    want_c = oq.matmul_s4s4(a[rows], b)
    assert_bitexact(to_np(c[torch.from_numpy(rows).cuda()]), want_c, f"{what}: int32 C")
    want = oq.w4a4_linear(a[rows], sa[rows], b, sb)
    assert_bitexact(to_np(out[torch.from_numpy(rows).cuda()]), want, f"{what}: fp16 out")
