"""GPU parity of the fused decode-step kernels.

Each fused entry point is checked bit for bit against the chain of
separate ops it replaces (each of those is pinned against the oracle in the
other GPU tests), and the fused decoder layer against the op-by-op layer,
including the cache contents it leaves behind.  The chains are the
reference's: RMSNorm -> Quantizer (modeling_llama.py), rope_qk -> K/q
Hadamard -> kv_quant_pack -> append_kv_i4 (kv_cache.py:144-170, 295-415),
transpose -> head-axis Hadamard -> Quantizer (modeling_llama.py:94, 117),
swiglu -> OnlineHadamard -> Quantizer (modeling_llama.py:125-137), and the
residual add after o_proj / down_proj.
"""
import math

import numpy as np
import scipy.linalg
import pytest
import torch

from oracle import hadamard as oh
from oracle import quant as oq
from tests.gpu_util import assert_bitexact, outlier_input, to_dev, to_np

pytestmark = pytest.mark.gpu


def _ops():
    from signrot_amd import _CUDA
    return _CUDA


@pytest.mark.parametrize("rows,cols,clip", [(1, 4096, 1.0), (32, 4096, 1.0), (33, 1024, 0.9),
                                            (5, 8192, 1.0), (7, 8, 1.0), (64, 4104, 1.0)])
def test_rmsnorm_quant_equals_rmsnorm_then_quant(rows, cols, clip):
    C = _ops()
    rng = np.random.default_rng(rows * 7 + cols)
    x = to_dev(outlier_input(rng, rows, cols, n_out=3, mag=30.0))
    q, s, h = C.rmsnorm_quant(x, 1e-5, cols, clip, return_norm=True)
    h_ref = C.rmsnorm(x, 1e-5, cols)
    q_ref, s_ref = C.sym_quant_dynamic(h_ref, clip)
    torch.cuda.synchronize()
    assert_bitexact(to_np(h), to_np(h_ref), "normalized x")
    assert_bitexact(to_np(q), to_np(q_ref), "codes")
    assert_bitexact(to_np(s), to_np(s_ref), "scales")
    q2, s2 = C.rmsnorm_quant(x, 1e-5, cols, clip)  # no normalized output
    assert_bitexact(to_np(q2), to_np(q_ref), "codes (out=NULL)")
    assert_bitexact(to_np(s2), to_np(s_ref), "scales (out=NULL)")


def test_rmsnorm_quant_rejects_unsupported_width():
    C = _ops()
    x = torch.zeros(2, 8200, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="8192"):
        C.rmsnorm_quant(x, 1e-5, 8200)


@pytest.mark.parametrize("B,H,D", [(32, 32, 128), (1, 32, 128), (3, 8, 64), (4, 64, 128),
                                   (2, 16, 256)])
def test_head_had_quant_equals_unfused_chain(B, H, D):
    from signrot_amd.functional.hadamard import _inv_sqrt_f32, matmul_hadU_cuda
    C = _ops()
    rng = np.random.default_rng(B * 100 + H + D)
    x = to_dev((rng.standard_normal((B, H, D)) * 2.0).astype(np.float16))
    q, s, rot = C.head_had_quant(x, _inv_sqrt_f32(H), return_rot=True)
    # the decoder's op-by-op chain (modeling_llama.py:94, 117)
    t = matmul_hadU_cuda(x.transpose(-1, -2).contiguous(), None, 1)
    ref = t.transpose(-1, -2).reshape(B, H * D).contiguous()
    q_ref, s_ref = C.sym_quant_dynamic(ref)
    torch.cuda.synchronize()
    assert_bitexact(to_np(rot), to_np(ref), "rotated rows")
    assert_bitexact(to_np(q), to_np(q_ref), "codes vs sym_quant_dynamic")
    assert_bitexact(to_np(s), to_np(s_ref), "scales vs sym_quant_dynamic")
    qw, sw = oq.sym_quant_dynamic(to_np(rot))
    assert_bitexact(to_np(q), qw, "codes vs the oracle quantizer of the rotated rows")
    assert_bitexact(to_np(s).reshape(-1), sw.reshape(-1), "scales vs the oracle")
    # rotation itself within the fp16 tolerance of the float64 closed form
    want = oh.rotate(to_np(x).transpose(0, 2, 1).reshape(-1, H)).reshape(B, D, H)
    np.testing.assert_allclose(to_np(rot).reshape(B, H, D).astype(np.float32),
                               want.transpose(0, 2, 1).astype(np.float32), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("M", [1, 16, 32, 48, 200, 1024])
def test_w4a4_linear_residual(M):
    C = _ops()
    rng = np.random.default_rng(M)
    K, N = 512, 384
    A = to_dev(oq.pack_i4(rng.integers(-8, 8, (M, K)).astype(np.int8)))
    B = to_dev(oq.pack_i4(rng.integers(-8, 8, (N, K)).astype(np.int8)))
    sa = to_dev((rng.random(M) * 0.02 + 1e-3).astype(np.float16))
    sb = to_dev((rng.random(N) * 0.02 + 1e-3).astype(np.float16))
    bias = to_dev((rng.standard_normal(N) * 0.1).astype(np.float16))
    res = to_dev((rng.standard_normal((M, N)) * 3.0).astype(np.float16))
    for b in (None, bias):
        out = C.w4a4_linear_residual(A, sa, B, sb, res, bias=b)
        ref = C.w4a4_linear(A, sa, B, sb, b) + res
        torch.cuda.synchronize()
        assert_bitexact(to_np(out), to_np(ref), f"linear + residual (bias={b is not None})")
    inplace = res.clone()
    C.w4a4_linear_residual(A, sa, B, sb, inplace, out=inplace)
    ref = C.w4a4_linear(A, sa, B, sb) + res
    torch.cuda.synchronize()
    assert_bitexact(to_np(inplace), to_np(ref), "in-place residual")


@pytest.mark.parametrize("rows,K,chunk", [(1, 28, 512), (32, 28, 512), (77, 28, 512),
                                         (4, 12, 512), (1, 28, 1024), (32, 28, 1024),
                                         (300, 28, 1024), (4, 12, 1024), (6, 20, 1024)])
def test_swiglu_had_sign_quant_equals_chain(rows, K, chunk):
    C = _ops()
    rng = np.random.default_rng(rows + K + chunk)
    n = K * chunk
    gu = to_dev((rng.standard_normal((rows, 2 * n)) * 2.0).astype(np.float16))
    # the K table named by the case (get_hadK(20480) would pick 40 x 512)
    k = K
    hk = to_dev(oh.had_table(K).astype(np.float16))
    sign = to_dev(rng.choice([-1, 1], n).astype(np.int8))
    q, s = C.swiglu_had_sign_quant(gu, hk, k, sign)
    a = C.swiglu(gu[:, :n].contiguous(), gu[:, n:].contiguous())
    q_ref, s_ref = C.had_sign_quant(a, hk, k, sign)
    torch.cuda.synchronize()
    assert_bitexact(to_np(q), to_np(q_ref), "codes")
    assert_bitexact(to_np(s), to_np(s_ref), "scales")


def test_swiglu_had_sign_quant_rejects_generic_sizes():
    C = _ops()
    n = 28 * 64  # had_28 x H_64: no fused SwiGLU form
    had, k = oh.get_hadK(n)
    gu = torch.zeros(2, 2 * n, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="512"):
        C.swiglu_had_sign_quant(gu, to_dev(had.astype(np.float16)), k)
    # K = 32 with H_1024 chunks: the SwiGLU form stops at K = 28
    assert not C.swiglu_had_fusable(32 * 1024, 32) and C.swiglu_had_fusable(28 * 1024, 28)
    h32 = to_dev(scipy.linalg.hadamard(32).astype(np.float16))
    gu = torch.zeros(2, 2 * 32 * 1024, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="1024"):
        C.swiglu_had_sign_quant(gu, h32, 32)


def _prefilled_cache(B, T, Hkv, Hq, page, layers, rng):
    from signrot_amd.transformers import MultiLayerPagedKVCache4Bit
    cache = MultiLayerPagedKVCache4Bit(B, page, T + 2, "cuda", layers, Hkv, 128,
                                       group_size=Hq // Hkv)
    gen = torch.Generator(device="cuda").manual_seed(int(rng.integers(1 << 30)))
    for li in range(layers):
        kv = torch.randn((2, B, T, Hkv, 128), device="cuda", generator=gen).half()
        cache.update(kv[0], kv[1], li, {})
    return cache


def _clone_cache(cache):
    return cache.clone()


@pytest.mark.parametrize("B,T,Hq,Hkv,page,cos_batch", [(3, 37, 8, 2, 16, 1), (32, 255, 32, 8, 256, 1),
                                                       (2, 16, 4, 4, 16, 2)])
def test_qkv_rope_had_append_equals_update_chain(B, T, Hq, Hkv, page, cos_batch):
    from signrot_amd.functional import kernel
    from signrot_amd.transformers.decode_layer import rope_cos_sin
    rng = np.random.default_rng(B * 1000 + T)
    cache_a = _prefilled_cache(B, T, Hkv, Hq, page, 2, rng)
    cache_b = _clone_cache(cache_a)
    D = 128
    qkv = to_dev((rng.standard_normal((B, (Hq + 2 * Hkv) * D)) * 2.0).astype(np.float16))
    if cos_batch == 1:
        cos, sin = rope_cos_sin([T], D, 500000.0, "cuda")
    else:
        cos, sin = rope_cos_sin(list(range(T, T + B)), D, 10000.0, "cuda")
        cos, sin = cos.view(B, 1, D), sin.view(B, 1, D)
    for li in (0, 1):
        # op-by-op: rope_qk, cache.update (K Hadamard, kv_quant_pack, append),
        # the stub's q Hadamard
        q = qkv[:, : Hq * D].contiguous().view(B, 1, Hq, D)
        k = qkv[:, Hq * D: (Hq + Hkv) * D].contiguous().view(B, 1, Hkv, D)
        v = qkv[:, (Hq + Hkv) * D:].contiguous().view(B, 1, Hkv, D)
        kernel.rope_qk(q, k, cos, sin)
        attend = cache_a.update(k, v, li, {"attention_mask": None})
        out_a = attend(q).view(B, Hq, D)
        q_rot = cache_b.update_qkv_fused(qkv, cos, sin, li, Hq)
        out_b = cache_b.decode_rotated(q_rot, li)
        from signrot_amd.transformers.kv_cache import matmul_had_cuda
        q_ref = matmul_had_cuda(q.view(B, Hq, D), torch.float16)
        torch.cuda.synchronize()
        assert cache_a.length == cache_b.length
        assert_bitexact(to_np(q_rot), to_np(q_ref), f"rotated q (layer {li})")
        assert_bitexact(to_np(cache_b.pages), to_np(cache_a.pages), f"cache codes (layer {li})")
        assert_bitexact(to_np(cache_b.scales), to_np(cache_a.scales), f"cache params (layer {li})")
        assert_bitexact(to_np(out_b), to_np(out_a), f"attention output (layer {li})")


@pytest.mark.parametrize("B,T,Hq,Hkv,page,cos_batch,chunks,rotate", [
    (3, 37, 8, 2, 16, 1, 1, True), (32, 255, 32, 8, 256, 1, 1, True), (2, 16, 4, 4, 16, 2, 1, True),
    (3, 300, 8, 2, 64, 1, 3, True), (4, 100, 8, 1, 32, 1, 1, True), (1, 40, 16, 16, 16, 1, 2, True),
    (5, 70, 8, 4, 8, 5, 1, True), (3, 37, 8, 2, 16, 1, 1, False),
    # config 3: unsplit (one eight-wave block per CU) and split in two
    (32, 4095, 32, 8, 256, 1, 1, True), (32, 4095, 32, 8, 256, 1, 2, True)])
def test_qkv_decode_i4_equals_append_then_decode(B, T, Hq, Hkv, page, cos_batch, chunks, rotate):
    """qkv_decode_i4 (the q/k/v step fused into the decode attention) against
    qkv_rope_had_append followed by batch_decode_i4: the cache bytes, the
    attention output and the o_proj input codes are bit-identical, split or
    not, with the new token in the last tile of its chunk (its codes written
    by the block and attended from LDS) and in the page-table (stage_tile)
    form for page sizes below 32."""
    from signrot_amd.functional.hadamard import _inv_sqrt_f32
    from signrot_amd.transformers.decode_layer import rope_cos_sin
    from signrot_amd.transformers.kv_cache import _SplitDecoder
    rng = np.random.default_rng(B * 1000 + T + chunks)
    cache_a = _prefilled_cache(B, T, Hkv, Hq, page, 2, rng)
    caches = [cache_a, _clone_cache(cache_a), _clone_cache(cache_a)]
    for c in caches:
        if not rotate:
            c.hadamard_dtype = None
        c._decoder = _SplitDecoder(B, Hq, 128, chunks, "cuda", c.hadamard_dtype)
    cache_a, cache_b, cache_c = caches
    D = 128
    if cos_batch == 1:
        cos, sin = rope_cos_sin([T], D, 500000.0, "cuda")
    else:
        cos, sin = rope_cos_sin(list(range(T, T + B)), D, 10000.0, "cuda")
        cos, sin = cos.view(B, 1, D), sin.view(B, 1, D)
    scale = _inv_sqrt_f32(Hq)
    for li in (0, 1):
        qkv = to_dev((rng.standard_normal((B, (Hq + 2 * Hkv) * D)) * 2.0).astype(np.float16))
        q_rot = cache_a.update_qkv_fused(qkv, cos, sin, li, Hq)
        o_a = cache_a.decode_rotated(q_rot, li)
        qa_a, sa_a = cache_a.decode_rotated_quant(q_rot, li, scale)
        o_b = cache_b.update_qkv_decode(qkv, cos, sin, li, Hq)
        qa_c, sa_c = cache_c.update_qkv_decode_quant(qkv, cos, sin, li, Hq, scale)
        torch.cuda.synchronize()
        assert cache_a.length == cache_b.length == cache_c.length
        for name, c in (("qkv_decode_i4", cache_b), ("qkv_decode_i4 + quant", cache_c)):
            assert_bitexact(to_np(c.pages), to_np(cache_a.pages), f"cache codes, {name} (layer {li})")
            assert_bitexact(to_np(c.scales), to_np(cache_a.scales), f"cache params, {name} (layer {li})")
        assert_bitexact(to_np(o_b), to_np(o_a), f"attention output (layer {li})")
        assert_bitexact(to_np(qa_c), to_np(qa_a), f"o_proj input codes (layer {li})")
        assert_bitexact(to_np(sa_c), to_np(sa_a), f"o_proj input scales (layer {li})")


def test_qkv_decode_i4_argument_errors():
    C = _ops()
    rng = np.random.default_rng(3)
    cache = _prefilled_cache(2, 20, 2, 8, 16, 1, rng)
    spec = cache.specs()
    qkv = torch.zeros(2, 12 * 128, dtype=torch.float16, device="cuda")
    cos = torch.zeros(1, 128, dtype=torch.float16, device="cuda")
    o = torch.empty(2, 8, 128, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="qkv must be"):
        C.qkv_decode_i4(o, qkv[:, :-128].contiguous(), cos, cos, **spec, layer_idx=0, n_q_heads=8,
                        had_scale=1.0)
    with pytest.raises(RuntimeError, match="split"):
        C.qkv_decode_i4(None, qkv, cos, cos, **spec, layer_idx=0, n_q_heads=8, had_scale=1.0)
    with pytest.raises(RuntimeError, match="cos/sin"):
        C.qkv_decode_i4(o, qkv, torch.zeros(3, 128, dtype=torch.float16, device="cuda"),
                        torch.zeros(3, 128, dtype=torch.float16, device="cuda"), **spec, layer_idx=0,
                        n_q_heads=8, had_scale=1.0)


@pytest.mark.parametrize("M,ffn,K", [
    (32, 14336, 4096), (1, 14336, 4096), (16, 896, 1024), (7, 8, 256), (32, 28672, 8192),
    (20, 1000, 4128),
    # every other kernel of the dispatch: ring (the skinny kernel is skipped),
    # dense grouped, big, 256 x 256 square tiles
    (48, 896, 1024), (70, 256, 256), (600, 512, 2048), (128, 14336, 4096), (300, 4096, 1024),
    (1100, 1504, 1024), (4096, 4096, 512), (2048, 14336, 512),
    # big-kernel grids with a last round over at most half the CUs: those
    # columns on the dense grouped form (the cfg4 70B gate/up at M = 512; a
    # ragged M)
    (512, 28672, 8192), (300, 20480, 512)])
def test_w4a4_linear_swiglu_equals_linear_then_swiglu(M, ffn, K):
    """The SwiGLU epilogue of the gate/up projection, on every kernel the
    shape dispatches to: bit-identical to the fp16 gate/up GEMM outputs fed
    to srq_swiglu (fused.cu:367-390)."""
    C = _ops()
    rng = np.random.default_rng(M * 7 + ffn + K)
    A = to_dev(rng.integers(0, 256, (M, K // 2)).astype(np.uint8))
    sa = to_dev((rng.random(M) * 0.05 + 1e-3).astype(np.float16))
    w = to_dev(rng.integers(0, 256, (2 * ffn, K // 2)).astype(np.uint8))
    sw = to_dev((rng.random(2 * ffn) * 0.01 + 1e-4).astype(np.float16))
    gu = C.w4a4_linear(A, sa, w, sw)
    want = C.swiglu(gu[:, :ffn].contiguous(), gu[:, ffn:].contiguous())
    w_il, s_il = C.interleave_gate_up(w, sw, ffn)
    got = C.w4a4_linear_swiglu(A, sa, w_il, s_il)
    torch.cuda.synchronize()
    assert_bitexact(to_np(got), to_np(want), "swiglu(gate, up)")


def test_w4a4_linear_swiglu_rejects_unpaired_columns():
    C = _ops()
    A = torch.zeros(33, 128, dtype=torch.uint8, device="cuda")
    w = torch.zeros(40, 128, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match="16"):
        C.w4a4_linear_swiglu(A, torch.ones(33, dtype=torch.float16, device="cuda"), w,
                             torch.ones(40, dtype=torch.float16, device="cuda"))


@pytest.mark.parametrize("B,T,Hq,Hkv,chunks", [(32, 4096, 32, 8, 2), (3, 300, 8, 2, 5),
                                                (1, 40, 16, 16, 3), (4, 1000, 32, 8, 1),
                                                (2, 700, 4, 4, 31)])
def test_merge_head_had_quant_equals_merge_then_head_had_quant(B, T, Hq, Hkv, chunks):
    """The split-KV merge folded into the head-axis Hadamard + quantizer:
    bit-identical to batch_decode_i4's merged output fed to head_had_quant
    (chunks = 1 takes the unsplit path of the cache's decoder)."""
    from signrot_amd.functional.hadamard import _inv_sqrt_f32
    C = _ops()
    rng = np.random.default_rng(B * 10 + T + chunks)
    cache = _prefilled_cache(B, T, Hkv, Hq, 256, 1, rng)
    spec = cache.specs()
    q = to_dev((rng.standard_normal((B, Hq, 128)) * 2.0).astype(np.float16))
    scale = _inv_sqrt_f32(Hq)
    o = torch.empty_like(q)
    tmp = torch.empty((B, Hq, chunks, 132), dtype=torch.float32, device="cuda")
    C.batch_decode_i4(o, q, **spec, layer_idx=0, tmp=tmp, num_chunks=chunks)
    q_ref, s_ref = C.head_had_quant(o, scale)
    if chunks > 1:
        tmp2 = torch.full_like(tmp, float("nan"))
        C.batch_decode_i4(None, q, **spec, layer_idx=0, tmp=tmp2, num_chunks=chunks)
        qg, sg, rot = C.merge_head_had_quant(tmp2, scale, return_rot=True)
        _, _, rot_ref = C.head_had_quant(o, scale, return_rot=True)
        torch.cuda.synchronize()
        assert_bitexact(to_np(rot), to_np(rot_ref), "rotated rows")
    else:
        with pytest.raises(RuntimeError, match="split"):
            C.batch_decode_i4(None, q, **spec, layer_idx=0, tmp=tmp, num_chunks=1)
        from signrot_amd.transformers.kv_cache import _SplitDecoder
        dec = _SplitDecoder(B, Hq, 128, 1, "cuda", None)
        qg, sg = dec.attend_head_had_quant(q, spec, 0, scale)
    torch.cuda.synchronize()
    assert_bitexact(to_np(qg), to_np(q_ref), "codes")
    assert_bitexact(to_np(sg), to_np(s_ref), "scales")


def test_merge_head_had_quant_rejects_too_many_records():
    C = _ops()
    tmp = torch.zeros((1, 32, 4, 132), dtype=torch.float32, device="cuda")  # 128 > 124
    with pytest.raises(RuntimeError, match="LDS"):
        C.merge_head_had_quant(tmp, 1.0)


@pytest.mark.parametrize("hidden,Hq,Hkv,ffn,T,B,page", [
    (1024, 8, 2, 14336, 40, 4, 64), (4096, 32, 8, 896, 300, 4, 64),
    # config 3 at its full shape (what bench.py times)
    (4096, 32, 8, 14336, 4096, 32, 256)])
def test_fused_decode_layer_equals_op_by_op(hidden, Hq, Hkv, ffn, T, B, page):
    from signrot_amd.transformers.decode_layer import W4A4LlamaDecodeLayer, rope_cos_sin
    rng = np.random.default_rng(hidden + ffn)
    layers = [W4A4LlamaDecodeLayer.random(hidden, Hq, Hkv, 128, ffn, layer_idx=i, seed=5 + i)
              for i in range(2)]
    cache_a = _prefilled_cache(B, T, Hkv, Hq, page, 2, rng)
    cache_b = _clone_cache(cache_a)
    h0_np = (rng.standard_normal((B, 1, hidden)) * 0.5).astype(np.float16)
    h0 = to_dev(h0_np)
    cos, sin = rope_cos_sin([T], 128, 500000.0, "cuda")
    ha, hb = h0.clone(), h0
    for layer in layers:
        ha = layer(ha, cache_a, cos, sin, fused=False)
        hb = layer(hb, cache_b, cos, sin, fused=True)
    torch.cuda.synchronize()
    assert_bitexact(to_np(hb), to_np(ha), "layer output")
    assert_bitexact(to_np(cache_b.pages), to_np(cache_a.pages), "cache codes")
    assert_bitexact(to_np(cache_b.scales), to_np(cache_a.scales), "cache params")
    assert_bitexact(to_np(h0), h0_np, "input hidden state (must not be modified)")
