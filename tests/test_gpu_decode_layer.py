"""GPU parity of one W4A4 Llama decoder layer decode step (the config-3
path), stage by stage: each stage's HIP output is compared with the oracle
applied to the HIP output of the previous stage, so integer stages are
checked bit-exactly on identical fp16 inputs (int4 codes flip on one-ulp
input changes, which end-to-end comparisons would amplify).  Shapes: a
reduced layer (hidden 1024, 8 query / 2 or 4 KV heads of 128, FFN 896 =
28 x 32, so the down-proj rotation is had_28 x H_32), the config-3 head
layout (32 / 8 heads) with a reduced FFN, and config 3 itself (hidden 4096,
32 / 8 heads, FFN 14336, batch 32, 4096 cached tokens).
"""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import glue
from oracle import hadamard as oh
from oracle import quant as oq
from tests.gpu_util import assert_bitexact, to_dev, to_np

pytestmark = pytest.mark.gpu


def _ulps(got, want, what, n=1):
    g = np.asarray(got, np.float16).astype(np.float64)
    w = np.asarray(want, np.float16).astype(np.float64)
    tol = n * np.spacing(np.abs(np.asarray(want, np.float16))).astype(np.float64)
    bad = np.abs(g - w) > tol
    assert not bad.any(), f"{what}: {bad.sum()} / {bad.size} beyond {n} ulp"


def _linear(x, w):
    q, s = oq.sym_quant_dynamic(x)
    return oq.w4a4_linear(q, s.reshape(-1), *w)


def _run(B, T, hidden, Hq, Hkv, ffn, page, seed):
    from signrot_amd.transformers import MultiLayerPagedKVCache4Bit
    from signrot_amd.transformers.decode_layer import W4A4LlamaDecodeLayer, rope_cos_sin
    D = 128
    rng = np.random.default_rng(seed)
    layer = W4A4LlamaDecodeLayer.random(hidden, Hq, Hkv, D, ffn, layer_idx=1, seed=seed)
    cache = MultiLayerPagedKVCache4Bit(B, page, T + 1, "cuda", 2, Hkv, D, group_size=Hq // Hkv)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    for li in range(2):  # prefill both layers (init_kv_i4)
        kv = torch.randn((2, B, T, Hkv, D), device="cuda", generator=gen).half()
        cache.update(kv[0], kv[1], li, {})
    k0 = torch.zeros(B, 1, Hkv, D, dtype=torch.float16, device="cuda")
    cache.update(k0, k0, 0, {})  # layer 0's step: the cache now counts T + 1 tokens
    data, param = to_np(cache.pages).copy(), to_np(cache.scales).copy()
    h = (rng.standard_normal((B, hidden)) * 0.5).astype(np.float16)
    cos, sin = rope_cos_sin([T], D, 500000.0, "cuda")
    tr = {}
    out = to_np(layer(to_dev(h).view(B, 1, hidden), cache, cos, sin, trace=tr)).reshape(B, hidden)
    tr = {k: to_np(v) for k, v in tr.items()}
    w = layer.unpacked()

    # attention block
    _ulps(tr["norm1"], glue.rmsnorm(h, 1e-5, hidden), "input rmsnorm")
    assert_bitexact(tr["qkv"], _linear(tr["norm1"], w["qkv"]), "q/k/v projection")
    q = tr["qkv"][:, : Hq * D].reshape(B, 1, Hq, D)
    k = tr["qkv"][:, Hq * D: (Hq + Hkv) * D].reshape(B, 1, Hkv, D)
    v = tr["qkv"][:, (Hq + Hkv) * D:].reshape(B, 1, Hkv, D)
    qw, kw = glue.rope_qk(q, k, to_np(cos), to_np(sin))
    assert_bitexact(tr["q_rope"], qw, "rope q")
    assert_bitexact(tr["k_rope"], kw, "rope k")
    # the appended token: K rotated (within the FWHT tolerance), quantized
    # bit-exactly from the rotated fp16 values the cache stored
    indptr, indices, last = oa.page_table(B, T + 1, page)
    got_data, got_param = to_np(cache.pages), to_np(cache.scales)
    kr = oh.rotate(tr["k_rope"].reshape(-1, D)).reshape(B, Hkv, D)
    vq, vp = oq.kv_quant_pack(tr["qkv"][:, (Hq + Hkv) * D:].reshape(B, Hkv, D))
    for b in range(B):
        pg, e = oa.slot(indptr, indices, page, b, T)
        assert_bitexact(got_data[pg, 1, 1, :, e], vq[b], f"appended V codes b={b}")
        assert_bitexact(got_param[pg, 1, 1, :, e], vp[b], f"appended V params b={b}")
        kd = oq.kv_dequant(got_data[pg, 1, 0, :, e], got_param[pg, 1, 0, :, e])
        err = np.abs(kd - kr[b].astype(np.float32))
        assert (err <= got_param[pg, 1, 0, :, e, 0:1].astype(np.float32) * 0.51 + 2e-3).all()
    # attention over the cache as stored (incl. the appended token)
    qr = oh.rotate(tr["q_rope"].reshape(-1, D)).reshape(B, Hq, D)
    att = oa.decode(qr, got_data, got_param, indptr, indices, last, 1)
    d = np.abs(tr["attn"].reshape(B, Hq, D).astype(np.float64) - att)
    assert (d <= 1e-2 + 1e-2 * np.abs(att)).all(), d.max()
    a_rot = oh.rotate(np.ascontiguousarray(tr["attn"].reshape(B, Hq, D).transpose(0, 2, 1))
                      .reshape(-1, Hq)).reshape(B, D, Hq).transpose(0, 2, 1).reshape(B, hidden)
    _ulps(tr["attn_rot"], a_rot, "head-axis Hadamard")
    o = _linear(tr["attn_rot"], w["o"])
    assert_bitexact(tr["resid1"], (h.astype(np.float32) + o.astype(np.float32)).astype(np.float16),
                    "o_proj + residual")
    # MLP block
    _ulps(tr["norm2"], glue.rmsnorm(tr["resid1"], 1e-5, hidden), "post-attention rmsnorm")
    assert_bitexact(tr["gu"], _linear(tr["norm2"], w["gu"]), "gate/up projection")
    sw = glue.swiglu(tr["gu"][:, :ffn], tr["gu"][:, ffn:])
    mism = (tr["act"].view(np.uint16) != sw.view(np.uint16)).mean()
    assert mism < 1e-3, mism
    qd, sd = oq.sym_quant_dynamic(oh.online_hadamard(tr["act"], w["down_sign"]))
    assert (tr["down_q"] != qd).mean() < 0.01  # codes may flip on one-ulp rotation differences
    assert_bitexact(tr["down"], oq.w4a4_linear(tr["down_q"], tr["down_s"].reshape(-1),
                                               *w["down"]), "down_proj")
    assert_bitexact(out, (tr["resid1"].astype(np.float32) + tr["down"].astype(np.float32))
                    .astype(np.float16), "final residual")


@pytest.mark.parametrize("B,T,hidden,Hq,Hkv,ffn,page,seed", [
    (3, 70, 1024, 8, 2, 896, 32, 1),
    (4, 300, 1024, 8, 4, 896, 64, 2),
    (2, 200, 4096, 32, 8, 896, 64, 3),
    # config 3 at its full shape: Llama-3-8B layer, batch 32, 4096 cached
    # tokens in 256-token pages, FFN 14336 (had_28 x H_512)
    (32, 4096, 4096, 32, 8, 14336, 256, 4),
])
def test_decode_layer_stagewise(B, T, hidden, Hq, Hkv, ffn, page, seed):
    _run(B, T, hidden, Hq, Hkv, ffn, page, seed)
