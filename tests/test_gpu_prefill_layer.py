"""GPU parity of the decoder layer's prefill (its first update: T tokens per
request, optionally left-padded) followed by decode steps, stage by stage
against the oracle chain (tests/layer_check.py), the prefill attention
against oracle.attention.prefill (the flash-attn 2 varlen call of
modeling_llama.py:81-90), the cached K/V entries against the quantizer
applied to the rotated fp16 K and to V (kv_cache.py:295-395), and each
decode step's fused path bit for bit against its op-by-op path."""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import glue
from oracle import hadamard as oh
from oracle import quant as oq
from tests import layer_check as lc
from tests.gpu_util import assert_bitexact, to_dev, to_np

pytestmark = pytest.mark.gpu

D = 128


def _rope(positions, theta=500000.0):
    """cos/sin fp16 [B, T, D] for per-request positions [B, T]."""
    from signrot_amd.transformers.decode_layer import rope_cos_sin
    cs = [rope_cos_sin(list(map(int, p)), D, theta, "cuda") for p in positions]
    return (torch.cat([c for c, _ in cs]).contiguous(), torch.cat([s for _, s in cs]).contiguous())


@pytest.mark.parametrize("masked", [False, True])
def test_prefill_then_decode(masked):
    from signrot_amd.transformers import MultiLayerPagedKVCache4Bit
    from signrot_amd.transformers.decode_layer import W4A4LlamaDecodeLayer
    B, T, hidden, Hq, Hkv, ffn, page, steps = 3, 40, 1024, 8, 2, 896, 32, 2
    seed = 11 + masked
    lengths = np.array([40, 33, 36] if masked else [T] * B)   # same page count (2)
    mask = (np.arange(T)[None, :] >= (T - lengths)[:, None]).astype(np.int32)
    positions = np.maximum(np.cumsum(mask, axis=1) - 1, 0)     # HF position_ids
    layer = W4A4LlamaDecodeLayer.random(hidden, Hq, Hkv, D, ffn, layer_idx=0, seed=seed)
    w = layer.unpacked()
    cache = MultiLayerPagedKVCache4Bit(B, page, T + steps, "cuda", 1, Hkv, D,
                                       group_size=Hq // Hkv)
    rng = np.random.default_rng(seed)
    h = (rng.standard_normal((B, T, hidden)) * 0.5).astype(np.float16)
    cos, sin = _rope(positions)
    mask_d = torch.from_numpy(mask).cuda() if masked else None
    tr = {}
    out = to_np(layer.prefill(to_dev(h), cache, cos, sin, attention_mask=mask_d, trace=tr))
    tr = {k: to_np(v) for k, v in tr.items()}
    live = mask.reshape(-1).nonzero()[0]                       # real-token rows

    # ---- prefill: projections, RoPE, attention, the cache, then o_proj + MLP
    hf = h.reshape(B * T, hidden)
    lc.ulps(tr["norm1"], glue.rmsnorm(hf, 1e-5, hidden), "input rmsnorm")
    assert_bitexact(tr["qkv"], lc.linear(tr["norm1"], w["qkv"]), "q/k/v projection")
    q = tr["qkv"][:, : Hq * D].reshape(B, T, Hq, D)
    k = tr["qkv"][:, Hq * D: (Hq + Hkv) * D].reshape(B, T, Hkv, D)
    v = tr["qkv"][:, (Hq + Hkv) * D:].reshape(B, T, Hkv, D)
    qw, kw = glue.rope_qk(q, k, to_np(cos), to_np(sin))
    assert_bitexact(tr["q_rope"], qw, "rope q")
    assert_bitexact(tr["k_rope"], kw, "rope k")
    att = oa.prefill(tr["q_rope"], tr["k_rope"], v, mask if masked else None, causal=True)
    d = np.abs(tr["attn"].astype(np.float64) - att).reshape(B * T, -1)[live]
    assert (d <= 1e-2 + 1e-2 * np.abs(att.reshape(B * T, -1)[live])).all(), d.max()
    data, param = to_np(cache.pages), to_np(cache.scales)
    indptr, indices, last = lc.page_table(lengths, page)
    kr = oh.rotate(tr["k_rope"].reshape(-1, D)).reshape(B, T, Hkv, D)
    for b in range(B):
        vq, vp = oq.kv_quant_pack(v[b, T - lengths[b]:])
        for j in range(lengths[b]):  # real token j of request b sits at position j
            pg, e = oa.slot(indptr, indices, page, b, j)
            assert_bitexact(data[pg, 0, 1, :, e], vq[j], f"prefill V codes b={b} t={j}")
            assert_bitexact(param[pg, 0, 1, :, e], vp[j], f"prefill V params b={b} t={j}")
            lc.check_k_entry(data, param, pg, e, 0, kr[b, T - lengths[b] + j],
                             f"prefill K b={b} t={j}")
    lc.check_attn_out_and_mlp(tr, hf, w, hidden, Hq, ffn, out, rows=live)

    # ---- decode steps: op path checked against the oracle, fused path
    # bit-identical to it on a clone of the cache
    for s in range(steps):
        hs = (rng.standard_normal((B, hidden)) * 0.5).astype(np.float16)
        pos = lengths + s
        c1, s1 = _rope(pos[:, None])
        ext = None
        if masked:
            ext = torch.from_numpy(np.concatenate([mask, np.ones((B, s + 1), np.int32)], 1)).cuda()
        fused_cache = cache.clone()
        fused = to_np(layer(to_dev(hs).view(B, 1, hidden), fused_cache, c1, s1,
                            attention_mask=ext))
        tr = {}
        got = to_np(layer(to_dev(hs).view(B, 1, hidden), cache, c1, s1, trace=tr,
                          attention_mask=ext))
        assert_bitexact(fused, got, f"fused vs op-by-op decode step {s}")
        tr = {k: to_np(x) for k, x in tr.items()}
        lc.check_decode_step(tr, hs, w, got.reshape(B, hidden), to_np(c1), to_np(s1),
                             to_np(cache.pages), to_np(cache.scales),
                             lc.page_table(pos + 1, page), pos, 0, hidden, Hq, Hkv, ffn, page)
