"""GPU parity on rows holding NaN or ±inf, for every quantizer entry point.

The reference reduces each row with fmaxf / fminf, which skip NaN, and maps
NaN quotients to code 0 (signrot/kernels/fused.cu:17-28, 83-111, 236-266;
moe.cu:60-101).  The vectorised kernels here send rows holding a non-finite
value through an exact per-element branch; these cases exercise that branch
and the fused quantizers (rotation, SwiGLU, RMSNorm in front) against the
oracle, whose handling of such rows is pinned by hand-worked known answers
in tests/test_oracle_nonfinite.py.  Each case mixes ordinary rows with the
special ones so a row's result cannot depend on its neighbours."""
import numpy as np
import pytest
import torch

from oracle import hadamard as oh
from oracle import moe as om
from oracle import quant as oq
from tests.gpu_util import assert_bitexact, outlier_input, to_dev, to_np

pytestmark = pytest.mark.gpu
NAN, INF = np.float16(np.nan), np.float16(np.inf)


@pytest.fixture(scope="module")
def C():
    from signrot_amd import _CUDA
    return _CUDA


def _special_rows(rng, rows, cols, scale=3.0):
    """rows x cols fp16: every third row ordinary; the others hold one or two
    NaN, +inf, -inf, both infinities, all NaN, or NaN next to an outlier."""
    x = (rng.standard_normal((rows, cols)) * scale).astype(np.float16)
    kinds = []
    for r in range(rows):
        k = r % 9
        c = rng.integers(0, cols, 2)
        if k == 1:
            x[r, c[0]] = NAN
        elif k == 2:
            x[r, c[0]] = INF
        elif k == 3:
            x[r, c[0]] = -INF
        elif k == 4:
            x[r, c[0]] = INF
            x[r, c[1]] = -INF
        elif k == 5:
            x[r] = NAN
        elif k == 7:
            x[r, c[0]] = NAN
            x[r, c[1]] = np.float16(-300.0)
        elif k == 8:
            x[r, c] = NAN
        kinds.append(k)
    return x


@pytest.mark.parametrize("rows,cols", [(45, 4096), (18, 14336), (27, 28672), (9, 4095),
                                       (18, 8), (9, 128), (2048, 4096)])
@pytest.mark.parametrize("clip", [1.0, 0.9])
def test_sym_quant_dynamic_nonfinite(C, rows, cols, clip):
    rng = np.random.default_rng(rows * 31 + cols)
    x = _special_rows(rng, rows, cols)
    q, s = C.sym_quant_dynamic(to_dev(x), clip)
    qw, sw = oq.sym_quant_dynamic(x, clip)
    assert_bitexact(to_np(s), sw, "scale")
    assert_bitexact(to_np(q), qw, "codes")


@pytest.mark.parametrize("rows,cols,experts", [(27, 14336, 8), (45, 4096, 8), (18, 768, 128)])
@pytest.mark.parametrize("with_sign", [True, False])
def test_sym_quant_dynamic_moe_nonfinite(C, rows, cols, experts, with_sign):
    rng = np.random.default_rng(rows + cols)
    x = _special_rows(rng, rows, cols)
    eid = rng.integers(0, experts, rows).astype(np.int32)
    sign = (rng.integers(0, 2, (experts, cols)) * 2 - 1).astype(np.int8)
    q, s = C.sym_quant_dynamic_moe(to_dev(x), to_dev(sign) if with_sign else None,
                                   to_dev(eid), 1.0)
    qw, sw = om.sym_quant_dynamic_moe(x, sign if with_sign else None, eid, 1.0)
    assert_bitexact(to_np(s), sw, "scale")
    assert_bitexact(to_np(q), qw, "codes")


def _hadk(k):
    return to_dev(oh.had_table(k).astype(np.float16)) if k > 1 else None


@pytest.mark.parametrize("n", [4096, 14336, 28672])
@pytest.mark.parametrize("clip", [1.0, 0.8])
def test_had_sign_quant_nonfinite(C, n, clip):
    """NaN anywhere in a row makes the whole rotated row NaN (scale 0, codes
    0); a single ±inf makes it all ±inf (scale inf, codes 0); a finite row
    whose rotation overflows fp16 turns inf inside the kernel."""
    rows = 27
    rng = np.random.default_rng(n)
    x = _special_rows(rng, rows, n)
    x[6] = np.float16(1000.0)        # rotation of a constant row overflows
    x[15] = np.float16(-1000.0)
    _, k = oh.get_hadK(n)
    hk = _hadk(k)
    sign_np = rng.choice([-1, 1], n).astype(np.int8)
    sign = to_dev(sign_np)
    xd = to_dev(x)
    rot = C.online_hadamard(xd, hk, k, sign)
    q, s = C.had_sign_quant(xd, hk, k, sign, clip)
    rot_np = to_np(rot)
    # the non-finite pattern of the rotation is fixed by the Hadamard signs
    want = oh.online_hadamard(x, sign_np)
    assert np.array_equal(np.isnan(rot_np), np.isnan(want)), "NaN positions of the rotation"
    assert np.array_equal(np.isinf(rot_np), np.isinf(want)), "inf positions of the rotation"
    fin = np.isfinite(want)
    np.testing.assert_array_equal(np.sign(rot_np[~fin & ~np.isnan(want)]),
                                  np.sign(want[~fin & ~np.isnan(want)]))
    qw, sw = oq.sym_quant_dynamic(rot_np, clip)
    assert_bitexact(to_np(s), sw, "scale")
    assert_bitexact(to_np(q), qw, "codes")


@pytest.mark.parametrize("rows,K,chunk", [(18, 28, 512), (18, 28, 1024)])
def test_swiglu_had_sign_quant_nonfinite(C, rows, K, chunk):
    """SwiGLU(NaN) and SwiGLU(-inf, u) are NaN, SwiGLU(+inf, u) is ±inf: the
    fused op equals swiglu -> had_sign_quant on such rows."""
    rng = np.random.default_rng(rows + chunk)
    n = K * chunk
    gu = (rng.standard_normal((rows, 2 * n)) * 2.0).astype(np.float16)
    gu[:, :n] = _special_rows(rng, rows, n, 2.0)
    gu[3, n + 5] = NAN              # NaN in the up half
    gu[12, n + 9] = INF
    gu = to_dev(gu)
    hk = _hadk(K)
    sign = to_dev(rng.choice([-1, 1], n).astype(np.int8))
    q, s = C.swiglu_had_sign_quant(gu, hk, K, sign)
    a = C.swiglu(gu[:, :n].contiguous(), gu[:, n:].contiguous())
    q_ref, s_ref = C.had_sign_quant(a, hk, K, sign)
    torch.cuda.synchronize()
    assert_bitexact(to_np(s), to_np(s_ref), "scales")
    assert_bitexact(to_np(q), to_np(q_ref), "codes")
    qw, sw = oq.sym_quant_dynamic(to_np(C.online_hadamard(a, hk, K, sign)))
    assert_bitexact(to_np(s), sw, "scales vs oracle")
    assert_bitexact(to_np(q), qw, "codes vs oracle")


def test_swiglu_had_sign_quant_moe_nonfinite(C):
    rows, n, K, experts = 27, 14336, 28, 8
    rng = np.random.default_rng(5)
    gate = to_dev(_special_rows(rng, rows, n, 2.0))
    up = to_dev((rng.standard_normal((rows, n)) * 2).astype(np.float16))
    eid = to_dev(rng.integers(0, experts, rows).astype(np.int32))
    sign = to_dev(rng.choice([-1, 1], (experts, n)).astype(np.int8))
    hk = _hadk(K)
    q, s = C.swiglu_had_sign_quant_moe(gate, up, hk, K, sign, eid, 1.0)
    rot = C.online_hadamard(C.swiglu(gate, up), hk, K, None)
    q2, s2 = C.sym_quant_dynamic_moe(rot, sign, eid, 1.0)
    torch.cuda.synchronize()
    assert_bitexact(to_np(s), to_np(s2), "scales")
    assert_bitexact(to_np(q), to_np(q2), "codes")


@pytest.mark.parametrize("n,K", [(14336, 28), (28672, 28)])
def test_had_sign_quant_moe_nonfinite(C, n, K):
    """The plain MoE down-proj input op (rotation + per-expert sign rows +
    quantizer) on rows holding NaN / inf: equal to the rotation then
    sym_quant_dynamic_moe."""
    rows, experts = 27, 8
    rng = np.random.default_rng(n + 1)
    x = to_dev(_special_rows(rng, rows, n, 2.0))
    eid = to_dev(rng.integers(0, experts, rows).astype(np.int32))
    sign = to_dev(rng.choice([-1, 1], (experts, n)).astype(np.int8))
    hk = _hadk(K)
    q, s = C.had_sign_quant_moe(x, hk, K, sign, eid, 1.0)
    rot = C.online_hadamard(x, hk, K, None)
    q2, s2 = C.sym_quant_dynamic_moe(rot, sign, eid, 1.0)
    torch.cuda.synchronize()
    assert_bitexact(to_np(s), to_np(s2), "scales")
    assert_bitexact(to_np(q), to_np(q2), "codes")


def test_sym_quant_dynamic_rows_nonfinite(C):
    """Rows holding NaN / inf quantized straight from gathered token rows:
    equal to sym_quant_dynamic of the gathered rows."""
    rows, cols = 27, 4096
    rng = np.random.default_rng(11)
    x = to_dev(_special_rows(rng, rows, cols, 3.0))
    idx = to_dev(rng.integers(0, rows, 54).astype(np.int32))
    q, s = C.sym_quant_dynamic_rows(x, idx)
    q2, s2 = C.sym_quant_dynamic(x[idx.long()].contiguous())
    torch.cuda.synchronize()
    assert_bitexact(to_np(s), to_np(s2), "scales")
    assert_bitexact(to_np(q), to_np(q2), "codes")


@pytest.mark.parametrize("rows,cols", [(27, 4096), (18, 8192), (9, 1024)])
def test_rmsnorm_quant_nonfinite(C, rows, cols):
    """A NaN makes the sum of squares NaN (the whole row NaN: scale 0); an
    inf makes rsqrt 0 (finite -> 0, inf -> NaN)."""
    rng = np.random.default_rng(rows * cols)
    x = to_dev(_special_rows(rng, rows, cols, 1.0))
    q, s, h = C.rmsnorm_quant(x, 1e-5, cols, 1.0, return_norm=True)
    h_ref = C.rmsnorm(x, 1e-5, cols)
    torch.cuda.synchronize()
    assert_bitexact(to_np(h), to_np(h_ref), "normalized x")
    qw, sw = oq.sym_quant_dynamic(to_np(h_ref))
    assert_bitexact(to_np(s), sw, "scales vs oracle")
    assert_bitexact(to_np(q), qw, "codes vs oracle")


@pytest.mark.parametrize("shape", [(3, 3, 8, 128), (1, 18, 1, 128), (2, 9, 6), (9, 64)])
def test_kv_quant_pack_nonfinite(C, shape):
    rng = np.random.default_rng(sum(shape))
    rows = int(np.prod(shape[:-1]))
    x = _special_rows(rng, rows, shape[-1], 2.0).reshape(shape)
    q, p = C.kv_quant_pack(to_dev(x))
    qw, pw = oq.kv_quant_pack(x)
    assert_bitexact(to_np(p), pw, "param")
    assert_bitexact(to_np(q), qw, "codes")


def test_head_had_quant_nonfinite(C):
    """The o_proj head-axis rotation + quantizer (one row per request): NaN
    or inf in one head spreads over that head-axis column only, so rows mix
    NaN, inf and finite values."""
    from signrot_amd.functional.hadamard import _inv_sqrt_f32, matmul_hadU_cuda
    B, H, D = 27, 32, 128
    rng = np.random.default_rng(77)
    x_np = _special_rows(rng, B, H * D, 2.0).reshape(B, H, D)
    x = to_dev(x_np)
    q, s, rot = C.head_had_quant(x, _inv_sqrt_f32(H), return_rot=True)
    t = matmul_hadU_cuda(x.transpose(-1, -2).contiguous(), None, 1)
    ref = t.transpose(-1, -2).reshape(B, H * D).contiguous()
    torch.cuda.synchronize()
    assert_bitexact(to_np(rot), to_np(ref), "rotated rows")
    qw, sw = oq.sym_quant_dynamic(to_np(ref))
    assert_bitexact(to_np(s).reshape(-1), sw.reshape(-1), "scales vs oracle")
    assert_bitexact(to_np(q), qw, "codes vs oracle")


def test_qkv_rope_had_append_nonfinite_kv():
    """A NaN or inf in one new K or V row: the fused q/k/v step writes the
    same cache bytes and [scale, zero] as rope -> update (kv_quant_pack ->
    append), and they match the oracle's quantizer of the cached rows."""
    from signrot_amd.functional import kernel
    from signrot_amd.transformers import MultiLayerPagedKVCache4Bit
    from signrot_amd.transformers.decode_layer import rope_cos_sin
    from tests.test_gpu_fused_decode import _clone_cache
    B, T, Hq, Hkv, page, D = 4, 20, 8, 2, 16, 128
    rng = np.random.default_rng(19)
    cache_a = MultiLayerPagedKVCache4Bit(B, page, T + 2, "cuda", 1, Hkv, D,
                                         group_size=Hq // Hkv)
    kv = rng.standard_normal((2, B, T, Hkv, D)).astype(np.float16)
    cache_a.update(to_dev(kv[0]), to_dev(kv[1]), 0, {})
    cache_b = _clone_cache(cache_a)
    cache_c = _clone_cache(cache_a)
    qkv_np = (rng.standard_normal((B, (Hq + 2 * Hkv) * D)) * 2.0).astype(np.float16)
    k0, v0 = Hq * D, (Hq + Hkv) * D
    qkv_np[0, k0 + 5] = NAN                  # K head 0 of request 0
    qkv_np[1, k0 + D + 7] = INF              # K head 1 of request 1
    qkv_np[2, v0 + 3] = NAN                  # V head 0 of request 2
    qkv_np[3, v0 + D + 1] = -INF             # V head 1 of request 3
    qkv = to_dev(qkv_np)
    cos, sin = rope_cos_sin([T], D, 500000.0, "cuda")
    q = qkv[:, : Hq * D].contiguous().view(B, 1, Hq, D)
    k = qkv[:, k0:v0].contiguous().view(B, 1, Hkv, D)
    v = qkv[:, v0:].contiguous().view(B, 1, Hkv, D)
    kernel.rope_qk(q, k, cos, sin)
    cache_a.update(k, v, 0, {"attention_mask": None})
    cache_b.update_qkv_fused(qkv, cos, sin, 0, Hq)
    cache_c.update_qkv_decode(qkv, cos, sin, 0, Hq)  # the form fused with the attention
    torch.cuda.synchronize()
    assert_bitexact(to_np(cache_b.pages), to_np(cache_a.pages), "cache codes")
    assert_bitexact(to_np(cache_b.scales), to_np(cache_a.scales), "cache params")
    assert_bitexact(to_np(cache_c.pages), to_np(cache_a.pages), "cache codes (qkv_decode_i4)")
    assert_bitexact(to_np(cache_c.scales), to_np(cache_a.scales), "cache params (qkv_decode_i4)")
    # the new token's V rows (no rotation) against the oracle quantizer,
    # located by the page rule of the cache's own index buffers
    from oracle import attention as oa
    spec = cache_a.specs()
    indptr, indices = to_np(spec["kv_indptr"]), to_np(spec["kv_indices"])
    pw, prw = oq.kv_quant_pack(to_np(v).reshape(B * Hkv, D))
    pages, params = to_np(cache_a.pages), to_np(cache_a.scales)
    got_v, got_p = [], []
    for b in range(B):
        pg, e = oa.slot(indptr, indices, page, b, T)      # the appended token
        got_v.append(pages[pg, 0, 1, :, e])
        got_p.append(params[pg, 0, 1, :, e])
    assert_bitexact(np.stack(got_v).reshape(B * Hkv, D // 2), pw, "V codes vs oracle")
    assert_bitexact(np.stack(got_p).reshape(B * Hkv, 2), prw, "V params vs oracle")
