"""GPU parity of the asymmetric-activation path: the uint4 quantizers
(dynamic, MoE sign rows, given scale/zero), sum_i4, the zero-point outer
product, the unsigned-A GEMM on every kernel path, the fused asymmetric
linear (dense and grouped), and the modules built on them -- bit-exact
against the oracle and against the reference's unfused op chains."""
import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle import quant as oq
from tests.gpu_util import DEV, assert_bitexact, outlier_input, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def C():
    from signrot_amd import _CUDA
    return _CUDA


def _zero_bits(z):
    """fp16 zero points as bits with every NaN folded to one pattern."""
    z = np.asarray(z, np.float16)
    b = z.view(np.uint16).copy()
    b[np.isnan(z)] = 0x7E00
    return b


def _degenerate(x):
    x = x.copy()
    x[0] = 0                                  # all-zero: scale 0, zero NaN
    if x.shape[0] > 1:
        x[1] = 3                              # constant: scale 0, zero -inf
    if x.shape[0] > 2:
        x[2] = np.float16(2 ** -24)           # scale underflows, ratio -inf
        x[2, 0] = np.float16(2 ** -23)
    if x.shape[0] > 3:
        x[3] = x[3] * 300                     # large magnitudes
    if x.shape[0] > 4:
        x[4] = np.abs(x[4]) + 100             # all positive, zero far below 0
    return x


@pytest.mark.parametrize("rows,cols,clip", [(64, 4096, 1.0), (7, 14336, 1.0), (33, 33, 1.0),
                                            (16, 4096, 0.8), (9, 7, 1.0), (300, 512, 0.9)])
def test_asym_quant_dynamic(C, rows, cols, clip):
    rng = np.random.default_rng(rows * 31 + cols)
    x = _degenerate(outlier_input(rng, rows, cols, n_out=min(4, cols // 2), mag=40.0))
    q, s, z = C.asym_quant_dynamic(to_dev(x), clip)
    qw, sw, zw = oq.asym_quant_dynamic(x, clip)
    assert_bitexact(to_np(s), sw, "scale")
    assert np.array_equal(_zero_bits(to_np(z)), _zero_bits(zw)), "zero"
    assert_bitexact(to_np(q), qw, "codes")


@pytest.mark.parametrize("signed", [False, True])
def test_asym_quant_given(C, signed):
    rng = np.random.default_rng(11)
    x = outlier_input(rng, 40, 1000, mag=20.0)
    s = (np.abs(rng.standard_normal(40)) * 0.3 + 0.01).astype(np.float16)
    z = rng.integers(-10, 25, 40).astype(np.float16)
    f = C.asym_quant_f16_si4 if signed else C.asym_quant_f16_ui4
    q = f(to_dev(x), to_dev(s), to_dev(z))
    want = (oq.asym_quant_f16_si4 if signed else oq.asym_quant_f16_ui4)(x, s, z)
    assert_bitexact(to_np(q), want, "codes")


def test_asym_quantizer_module_matches_reference_form():
    from signrot_amd.nn import AsymQuantizer
    rng = np.random.default_rng(12)
    for clip in (1.0, 0.85):
        x = to_dev(outlier_input(rng, 24, 4096, mag=30.0))
        m = AsymQuantizer(clip_ratio=clip)
        a, b = m(x), m.forward_reference(x)
        assert torch.equal(a.quantized_x, b.quantized_x)
        assert torch.equal(a.scales_x, b.scales_x.to(torch.float16))
        assert torch.equal(a.zeros_x, b.zeros_x)


@pytest.mark.parametrize("rows,cols,experts", [(200, 4096, 8), (37, 14336, 4)])
def test_asym_quant_dynamic_moe(C, rows, cols, experts):
    rng = np.random.default_rng(rows + cols)
    x = outlier_input(rng, rows, cols, mag=25.0)
    eid = rng.integers(0, experts, rows).astype(np.int32)
    sign = rng.choice([-1, 1], (experts, cols)).astype(np.int8)
    q, s, z = C.asym_quant_dynamic_moe(to_dev(x), to_dev(sign), to_dev(eid), 1.0)
    qw, sw, zw = om.asym_quant_dynamic_moe(x, sign, eid)
    assert_bitexact(to_np(s), sw, "scale")
    assert np.array_equal(_zero_bits(to_np(z)), _zero_bits(zw)), "zero"
    assert_bitexact(to_np(q), qw, "codes")
    q2, s2, z2 = C.asym_quant_dynamic_moe(to_dev(x), None, to_dev(eid), 1.0)
    qw2, sw2, _ = oq.asym_quant_dynamic(x)
    assert_bitexact(to_np(q2), qw2, "codes (no sign)")


@pytest.mark.parametrize("signed", [True, False])
def test_sum_i4(C, signed):
    rng = np.random.default_rng(13)
    p = rng.integers(0, 256, (300, 7169)).astype(np.uint8)
    assert_bitexact(to_np(C.sum_i4(to_dev(p), signed)), oq.sum_i4(p, signed), "sum")


def test_matmul_colrow(C):
    rng = np.random.default_rng(14)
    a = rng.integers(-128, 128, (77, 1)).astype(np.int8)
    b = rng.integers(-2 ** 31, 2 ** 31, (1, 300), dtype=np.int64).astype(np.int32)
    got = C.matmul_colrow_i8_i32(to_dev(a), to_dev(b))
    assert_bitexact(to_np(got), oq.matmul_colrow_i8_i32(a, b), "colrow")


U4_SHAPES = [  # every kernel of the dispatcher: stream (M <= 32), skinny,
    # tile (64 < M < 1024), 256x128 (M >= 1024), 256x256 (>= 256 tiles)
    (1, 4096, 4096), (16, 4096, 14336), (32, 6144, 4096), (40, 1000, 8192), (64, 2048, 768),
    (200, 513, 800), (700, 4096, 1024), (2048, 4096, 1024), (4096, 4096, 512), (5, 3, 64),
    (32, 1000, 28672), (3, 700, 20000)]  # the batched stream form (K > 16384)


@pytest.mark.parametrize("M,N,K", U4_SHAPES)
def test_matmul_ui4_si4(C, M, N, K):
    rng = np.random.default_rng(M * 3 + N + K)
    a = rng.integers(0, 256, (M, K // 2)).astype(np.uint8)
    b = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
    got = C.matmul_ui4_si4(to_dev(a), to_dev(b))
    assert_bitexact(to_np(got), oq.matmul_u4s4(a, b), "int32 C")


def test_matmul_ui4_si4_extremes(C):
    K = 28672
    a = np.full((3, K // 2), 0xFF, np.uint8)      # all 15
    b = np.full((40, K // 2), 0x88, np.uint8)     # all -8
    assert np.all(to_np(C.matmul_ui4_si4(to_dev(a), to_dev(b))) == -120 * K)


@pytest.mark.parametrize("M,N,K,bias", [(1, 4096, 4096, False), (32, 4096, 14336, True),
                                        (130, 512, 2048, False), (2048, 4096, 2048, True),
                                        (4096, 4096, 512, False), (300, 8192, 1024, True)])
def test_w4a4_linear_asym(C, M, N, K, bias):
    rng = np.random.default_rng(M + N + K)
    x = outlier_input(rng, M, K, mag=30.0) + np.float16(0.5)
    q, s, z = oq.asym_quant_dynamic(x)
    zi = z[:, 0].astype(np.int8)
    w = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
    sw = (np.abs(rng.standard_normal(N)) * 0.01 + 1e-4).astype(np.float16)
    bs = (rng.standard_normal(N) * 0.5).astype(np.float16) if bias else None
    ws = oq.sum_i4(w)
    dq, ds, dz, dw, dsw, dws = map(to_dev, (q, s, zi, w, sw, ws))
    dbs = to_dev(bs) if bias else None
    out = C.w4a4_linear_asym(dq, ds.view(-1), dz, dw, dsw, dws.view(-1), dbs)
    assert_bitexact(to_np(out), oq.w4a4_linear_asym(q, s, zi, w, sw, bs), "fp16 out")
    # the reference's unfused chain on the GPU
    c = C.matmul_ui4_si4(dq, dw) - C.matmul_colrow_i8_i32(dz.view(-1, 1), dws.view(1, -1))
    unf = C.sym_dequant(c, ds.view(-1), dsw)
    if bias:
        unf = unf + dbs
    assert torch.equal(out, unf)


def test_linear4bit_asym_module():
    from signrot_amd.nn import AsymQuantizer, Linear4bit
    from signrot_amd.functional import kernel
    rng = np.random.default_rng(15)
    lin = Linear4bit(4096, 1024, bias=True).to(DEV)
    lin.weight.copy_(to_dev(rng.integers(0, 256, (1024, 2048)).astype(np.uint8)))
    lin.weight_scales.copy_(to_dev((np.abs(rng.standard_normal((1024, 1))) * 0.01)
                                   .astype(np.float32)))
    lin.bias.copy_(to_dev(rng.standard_normal(1024).astype(np.float16)))
    x = to_dev(outlier_input(rng, 2, 4096, mag=25.0)).view(2, 1, 4096)
    p = AsymQuantizer()(x)
    out = lin(p)
    c = kernel.matmul_ui4_si4(p.quantized_x, lin.weight)
    c = c - kernel.matmul_colrow_i8_i32(p.zeros_x, kernel.sum_i4(lin.weight).mT)
    ref = kernel.sym_dequant(c, p.scales_x, lin.weight_scales.half()) + lin.bias
    assert out.shape == (2, 1, 1024)
    assert torch.equal(out, ref)


def test_asym_symm_linear_module():
    from signrot_amd.nn import AsymSymmLinear4bit
    from signrot_amd.functional import kernel
    rng = np.random.default_rng(16)
    fp = torch.nn.Linear(512, 256, bias=True).half().to(DEV)
    sc = torch.full((256, 1), 0.01, dtype=torch.float16, device=DEV)
    with torch.no_grad():
        fp.weight.copy_((torch.randint(-8, 8, (256, 512), device=DEV).half() * sc))
    m = AsymSymmLinear4bit.from_float(fp, sc).to(DEV)
    x = to_dev(outlier_input(rng, 8, 512, mag=10.0))
    s = (x.float().abs().amax(-1, keepdim=True) / 7).half()
    z = torch.randint(-3, 4, (8, 1), dtype=torch.int8, device=DEV)
    q = kernel.asym_quant_f16_si4(x, s, z.half())
    out = m(kernel.PackedQuantizedTensor(q, s, z))
    c = oq.matmul_s4s4(to_np(q), to_np(m.weight)).astype(np.int64)
    c = oq.wrap_i32(c - oq.matmul_colrow_i8_i32(to_np(z), oq.sum_i4(to_np(m.weight))[:, 0]))
    want = oq.add_bias(oq.sym_dequant(c, to_np(s), to_np(m.weight_scales).reshape(-1)),
                       to_np(fp.bias))
    assert_bitexact(to_np(out), want, "AsymSymmLinear4bit")


def test_grouped_unsigned_and_moe_asym_linear(C):
    rng = np.random.default_rng(17)
    counts = [5, 0, 130, 64]
    E, N, K = len(counts), 384, 1024
    R = sum(counts)
    a = rng.integers(0, 256, (R, K // 2)).astype(np.uint8)
    w = rng.integers(0, 256, (E, N, K // 2)).astype(np.uint8)
    sa = (np.abs(rng.standard_normal(R)) * 0.05 + 1e-3).astype(np.float16)
    sw = (np.abs(rng.standard_normal((E, N))) * 0.01 + 1e-4).astype(np.float16)
    za = rng.integers(-5, 20, R).astype(np.int8)
    ws = np.stack([oq.sum_i4(w[e])[:, 0] for e in range(E)])
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    eid = np.repeat(np.arange(E), counts).astype(np.int32)
    da, dw = to_dev(a), to_dev(w)
    out = C.w4a4_linear_moe_asym(da, to_dev(sa), to_dev(za), dw, to_dev(sw), to_dev(ws),
                                 to_dev(off))
    want = np.empty((R, N), np.float16)
    for e in range(E):
        r = slice(off[e], off[e + 1])
        if counts[e]:
            want[r] = oq.w4a4_linear_asym(a[r], sa[r], za[r], w[e], sw[e])
    assert_bitexact(to_np(out), want, "grouped asym linear")
    # pointer-array grouped GEMM with unsigned A == dense u4s4 per expert
    c = torch.zeros((R, N), dtype=torch.int32, device=DEV)
    ps = to_dev(np.array([[m, N, K] for m in counts], np.int32))
    row0 = np.concatenate([[0], np.cumsum(counts)[:-1]])
    pa = to_dev((da.data_ptr() + row0 * (K // 2)).astype(np.int64))
    pb = to_dev((dw.data_ptr() + np.arange(E) * N * (K // 2)).astype(np.int64))
    pc = to_dev((c.data_ptr() + row0 * N * 4).astype(np.int64))
    ld = to_dev(np.full(E, K, np.int64))
    ldc = to_dev(np.full(E, N, np.int64))
    C.matmul_grouped(ps, pa, pb, pc, ld, ld, ldc, signed_a=False)
    torch.cuda.synchronize()
    for e in range(E):
        r = slice(off[e], off[e + 1])
        if counts[e]:
            assert_bitexact(to_np(c)[r], oq.matmul_u4s4(a[r], w[e]), f"grouped u4 expert {e}")
    # the reference's composition: grouped int32 + sym_dequant_moe(zero, wsum)
    unf = C.sym_dequant_moe(c, to_dev(sa).view(-1, 1), to_dev(sw), to_dev(eid), to_dev(za),
                            to_dev(ws))
    assert torch.equal(out, unf)


def _asym_block(seed, hidden=512, inter=1536, experts=8, top_k=2):
    from signrot_amd.nn import SignRotMoEBlock
    g = torch.Generator(device=DEV).manual_seed(seed)
    gate = torch.nn.Linear(hidden, experts, bias=False, dtype=torch.float16, device=DEV)
    with torch.no_grad():
        gate.weight.normal_(0, 0.1, generator=g)

    def w(n, k):
        return torch.randint(0, 256, (experts, n, k // 2), dtype=torch.uint8, device=DEV,
                             generator=g)

    def s(n, k):
        return torch.full((experts, n), 1.0 / k, dtype=torch.float16, device=DEV)

    sign = torch.randint(0, 2, (experts, inter), dtype=torch.int8, device=DEV,
                         generator=g) * 2 - 1
    return SignRotMoEBlock(gate, top_k=top_k, norm_topk_prob=True,
                           w_gate=w(inter, hidden), s_gate=s(inter, hidden),
                           w_up=w(inter, hidden), s_up=s(inter, hidden),
                           w_down=w(hidden, inter), s_down=s(hidden, inter),
                           sign_down=sign, asym=True).eval()


@pytest.mark.parametrize("hidden,inter,tokens", [(512, 1536, 19), (4096, 14336, 64)])
@torch.no_grad()
def test_moe_block_asym_grouped_equals_loop(hidden, inter, tokens):
    blk = _asym_block(seed=hidden + tokens, hidden=hidden, inter=inter)
    x = torch.randn(1, tokens, hidden, device=DEV, dtype=torch.float16)
    blk.use_grouped = True
    out, logits = blk(x)
    blk.use_grouped = False
    out2, logits2 = blk(x)
    assert torch.equal(logits, logits2)
    assert torch.equal(out, out2)
    assert torch.isfinite(out).all()


def _hadk(k):
    from oracle import hadamard as oh
    return to_dev(oh.had_table(k).astype(np.float16))


@pytest.mark.parametrize("n,K,rows,clip,use_sign", [
    (14336, 28, 2048, 1.0, True), (14336, 28, 7, 0.8, True), (28672, 28, 300, 1.0, True),
    (12288, 12, 5, 1.0, False), (6144, 12, 513, 1.0, True), (4096, 1, 9, 1.0, True)])
def test_had_sign_asym_quant(C, n, K, rows, clip, use_sign):
    """Fused rotation + sign + asymmetric quantizer == online_hadamard then
    asym_quant_dynamic (GPU chain) == the oracle's quantizer on the GPU's
    rotated values, bit for bit (the K = 1 shape takes the two-launch form)."""
    rng = np.random.default_rng(n + rows)
    x = outlier_input(rng, rows, n, n_out=8, mag=40.0)
    if rows >= 7:
        x[1] = 0                          # all-zero row
        x[2] = np.float16(1.5)            # constant row (rotates to one spike)
        x[3] *= 300                       # large
        x[4, 5] = np.float16(np.inf)      # non-finite rows take the exact route
        x[5, 9] = np.float16(np.nan)
        x[6] = np.abs(x[6]) + np.float16(20)
    hk = _hadk(K) if K > 1 else None
    sign = to_dev(rng.choice([-1, 1], n).astype(np.int8)) if use_sign else None
    xd = to_dev(x)
    q, s, z = C.had_sign_asym_quant(xd, hk, K, sign, clip)
    rot = C.online_hadamard(xd, hk, K, sign)
    q2, s2, z2 = C.asym_quant_dynamic(rot, clip)
    assert torch.equal(s, s2), "scale vs chain"
    assert np.array_equal(_zero_bits(to_np(z)), _zero_bits(to_np(z2))), "zero vs chain"
    assert torch.equal(q, q2), "codes vs chain"
    qw, sw, zw = oq.asym_quant_dynamic(to_np(rot), clip)
    assert_bitexact(to_np(s), sw, "scale")
    assert np.array_equal(_zero_bits(to_np(z)), _zero_bits(zw)), "zero"
    assert_bitexact(to_np(q), qw, "codes")


@torch.no_grad()
def test_hadamard_asym_quantizer_module_and_linear():
    """Sequential(OnlineHadamard, AsymQuantizer, Linear4bit) fused by
    fuse_online_hadamard gives the unfused sequence's output bit for bit."""
    from signrot_amd.nn import (AsymQuantizer, HadamardQuantizer, Linear4bit, OnlineHadamard,
                                fuse_online_hadamard)
    rng = np.random.default_rng(21)
    n, out_f = 14336, 512
    lin = Linear4bit(n, out_f).to(DEV)
    lin.weight.copy_(to_dev(rng.integers(0, 256, (out_f, n // 2)).astype(np.uint8)))
    lin.weight_scales.copy_(to_dev(np.full((out_f, 1), 1e-3, np.float32)))
    had = OnlineHadamard(n, lin, had_adj=True).to(DEV)
    had.had_adj_sign.copy_(to_dev(rng.choice([-1, 1], n).astype(np.int8)))
    seq = torch.nn.Sequential(had, AsymQuantizer(), lin)
    x = to_dev(outlier_input(rng, 33, n, mag=50.0))
    want = seq(x)
    holder = torch.nn.Module()
    holder.mlp = seq
    fuse_online_hadamard(holder)
    assert isinstance(holder.mlp[0], HadamardQuantizer)
    got = holder.mlp(x)
    assert torch.equal(got, want)
