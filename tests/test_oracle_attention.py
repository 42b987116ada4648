"""Pins of oracle.attention: the page table against the reference's layout
rule (physical page j * B + b, kv_cache.py:417-433), the append restatement
against hand-placed tokens, and the decode attention against torch's
scaled_dot_product_attention (a library routine, float64, on the CPU) over
the dense dequantized K/V, plus closed forms (one token, identical keys) and
invariance under a permutation of the physical pages."""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import quant as oq


def _random_cache(rng, B, T, H, page, L=2, layer=1, spare=3):
    pages_per = (T + page - 1) // page
    P = pages_per * B + spare
    data = rng.integers(0, 256, (P, L, 2, H, page, 64), dtype=np.uint8)
    param = np.empty((P, L, 2, H, page, 2), np.float16)
    param[..., 0] = rng.uniform(0.05, 0.5, param.shape[:-1]).astype(np.float16)
    param[..., 1] = rng.uniform(-2, 2, param.shape[:-1]).astype(np.float16)
    indptr, indices, last = oa.page_table(B, T, page)
    return data, param, indptr, indices, last


def test_page_table_layout():
    indptr, indices, last = oa.page_table(3, 10, 4)
    assert indptr.tolist() == [0, 3, 6, 9]
    # request b page j -> j * B + b
    assert indices.tolist() == [0, 3, 6, 1, 4, 7, 2, 5, 8]
    assert last.tolist() == [2, 2, 2]
    _, _, last = oa.page_table(2, 8, 4)
    assert last.tolist() == [4, 4]
    assert oa.request_len(*oa.page_table(2, 8, 4)[0:1], last, 4, 1) == 8


def test_append_places_tokens():
    B, H, page, T = 2, 3, 4, 6
    data = np.zeros((8, 1, 2, H, page, 64), np.uint8)
    param = np.zeros((8, 1, 2, H, page, 2), np.float16)
    indptr, indices, last = oa.page_table(B, T, page)
    k = np.arange(B * T * H * 64, dtype=np.int64).reshape(B * T, H, 64).astype(np.uint8)
    v = (255 - k).astype(np.uint8)
    kp = np.arange(B * T * H * 2).reshape(B * T, H, 2).astype(np.float16)
    seq = np.array([0, T, 2 * T], np.int32)
    oa.append(data, param, indptr, indices, last, 0, k, v, kp, kp, seq)
    for b in range(B):
        for t in range(T):
            pg = (t // page) * B + b
            assert np.array_equal(data[pg, 0, 0, :, t % page], k[b * T + t])
            assert np.array_equal(data[pg, 0, 1, :, t % page], v[b * T + t])
            assert np.array_equal(param[pg, 0, 1, :, t % page], kp[b * T + t])
    # decode append: one more token lands at position T
    indptr, indices, last = oa.page_table(B, T + 1, page)
    k1 = np.full((B, H, 64), 7, np.uint8)
    oa.append(data, param, indptr, indices, last, 0, k1, k1, kp[:B], kp[:B])
    for b in range(B):
        assert np.array_equal(data[(T // page) * B + b, 0, 0, :, T % page], k1[b])


@pytest.mark.parametrize("B,T,H,G,page", [(2, 37, 2, 1, 16), (1, 300, 2, 4, 128),
                                          (3, 64, 1, 8, 32)])
def test_decode_matches_torch_sdpa(B, T, H, G, page):
    rng = np.random.default_rng(T)
    data, param, indptr, indices, last = _random_cache(rng, B, T, H, page)
    q = rng.standard_normal((B, H * G, 128)).astype(np.float16)
    got = oa.decode(q, data, param, indptr, indices, last, 1)
    for b in range(B):
        # dense K̂/V̂ straight from the layout rule, not through oracle.gather
        ks, vs = [], []
        for t in range(T):
            pg = (t // page) * B + b
            ks.append(oq.kv_dequant(data[pg, 1, 0, :, t % page], param[pg, 1, 0, :, t % page]))
            vs.append(oq.kv_dequant(data[pg, 1, 1, :, t % page], param[pg, 1, 1, :, t % page]))
        k = torch.from_numpy(np.stack(ks).astype(np.float64)).permute(1, 0, 2)  # [H, T, D]
        v = torch.from_numpy(np.stack(vs).astype(np.float64)).permute(1, 0, 2)
        k = k.repeat_interleave(G, dim=0)
        v = v.repeat_interleave(G, dim=0)
        qq = torch.from_numpy(q[b].astype(np.float64)).unsqueeze(1)  # [Hq, 1, D]
        ref = torch.nn.functional.scaled_dot_product_attention(qq, k, v).squeeze(1).numpy()
        np.testing.assert_allclose(got[b], ref, rtol=1e-10, atol=1e-10)


def test_decode_closed_forms():
    rng = np.random.default_rng(5)
    data, param, indptr, indices, last = _random_cache(rng, 1, 1, 2, 16)
    q = rng.standard_normal((1, 2, 128)).astype(np.float16)
    got = oa.decode(q, data, param, indptr, indices, last, 1)
    v = oq.kv_dequant(data[0, 1, 1, :, 0], param[0, 1, 1, :, 0])
    np.testing.assert_array_equal(got[0], v.astype(np.float64))
    # identical keys -> uniform weights -> mean of the values
    data, param, indptr, indices, last = _random_cache(rng, 1, 20, 1, 8)
    data[:, :, 0] = data[0, 1, 0, 0, 0]
    param[:, :, 0] = param[0, 1, 0, 0, 0]
    got = oa.decode(q[:, :1], data, param, indptr, indices, last, 1)
    vs = [oq.kv_dequant(data[(t // 8), 1, 1, 0, t % 8], param[(t // 8), 1, 1, 0, t % 8])
          for t in range(20)]
    np.testing.assert_allclose(got[0, 0], np.mean(np.stack(vs).astype(np.float64), 0),
                               rtol=1e-12, atol=1e-12)


def test_decode_page_permutation_invariance():
    rng = np.random.default_rng(9)
    B, T, H, page = 3, 50, 2, 8
    data, param, indptr, indices, last = _random_cache(rng, B, T, H, page, spare=0)
    q = rng.standard_normal((B, H, 128)).astype(np.float16)
    ref = oa.decode(q, data, param, indptr, indices, last, 1)
    perm = rng.permutation(data.shape[0])          # new slot of each physical page
    data2 = np.empty_like(data)
    param2 = np.empty_like(param)
    data2[perm] = data
    param2[perm] = param
    got = oa.decode(q, data2, param2, indptr, perm[indices].astype(np.int32), last, 1)
    np.testing.assert_array_equal(got, ref)


# ---------------------------------------------------------------- prefill

@pytest.mark.parametrize("B,T,Hq,Hkv,causal", [(2, 33, 4, 2, True), (1, 70, 2, 2, False),
                                               (2, 17, 8, 1, True)])
def test_prefill_matches_torch_sdpa(B, T, Hq, Hkv, causal):
    rng = np.random.default_rng(B * 100 + T)
    q = rng.standard_normal((B, T, Hq, 128))
    k = rng.standard_normal((B, T, Hkv, 128))
    v = rng.standard_normal((B, T, Hkv, 128))
    mask = (rng.random((B, T)) > 0.25).astype(np.int32)
    mask[:, 0] = 1
    got = oa.prefill(q, k, v, mask, causal)
    G = Hq // Hkv
    for b in range(B):
        qq = torch.from_numpy(q[b]).permute(1, 0, 2)
        kk = torch.from_numpy(k[b]).permute(1, 0, 2).repeat_interleave(G, dim=0)
        vv = torch.from_numpy(v[b]).permute(1, 0, 2).repeat_interleave(G, dim=0)
        allow = torch.from_numpy(mask[b] != 0)[None, :].expand(T, T)
        if causal:
            allow = allow & torch.ones(T, T, dtype=torch.bool).tril()
        ref = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, attn_mask=allow)
        ref = ref.permute(1, 0, 2).numpy()
        live = mask[b] != 0
        np.testing.assert_allclose(got[b][live], ref[live], rtol=1e-10, atol=1e-10)
        assert np.all(got[b][~live] == 0)


def test_prefill_closed_forms():
    T, D = 9, 128
    rng = np.random.default_rng(3)
    v = rng.standard_normal((1, T, 1, D))
    q = rng.standard_normal((1, T, 1, D))
    k = np.zeros((1, T, 1, D))           # equal logits: causal cumulative mean
    got = oa.prefill(q, k, v)
    want = np.cumsum(v[0, :, 0], axis=0) / np.arange(1, T + 1)[:, None]
    np.testing.assert_allclose(got[0, :, 0], want, rtol=1e-12)
    # a key far above the rest takes all the weight once it is visible
    k2 = np.zeros((1, T, 1, D))
    k2[0, 4, 0] = 50.0
    q2 = np.ones((1, T, 1, D))
    got2 = oa.prefill(q2, k2, v)
    np.testing.assert_allclose(got2[0, 4:, 0], np.broadcast_to(v[0, 4, 0], (T - 4, D)),
                               rtol=1e-12, atol=1e-12)


def test_prefill_left_padding_is_unpadding():
    """A left-padded sequence gives, on its valid rows, the attention of the
    unpadded sequence alone (the unpad / varlen / pad round trip)."""
    rng = np.random.default_rng(11)
    T, pad = 20, 6
    q = rng.standard_normal((1, T, 2, 128))
    k = rng.standard_normal((1, T, 1, 128))
    v = rng.standard_normal((1, T, 1, 128))
    mask = np.ones((1, T), np.int32)
    mask[0, :pad] = 0
    got = oa.prefill(q, k, v, mask)
    alone = oa.prefill(q[:, pad:], k[:, pad:], v[:, pad:])
    np.testing.assert_allclose(got[0, pad:], alone[0], rtol=1e-12, atol=1e-12)
    assert np.all(got[0, :pad] == 0)
