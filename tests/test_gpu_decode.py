"""GPU parity of the paged int4 KV cache: the append kernels must place
bytes exactly where the oracle's layout rule puts them (bit-exact), and the
decode attention must match the oracle within the fp16 tolerance
(|d| <= 1e-2 + 1e-2 |ref|; the reference checks 3e-2 against an fp32
reference and 2e-3 split vs unsplit, benchmarks/test_split_decode.py:58-85).
Cases restate test_split_decode.py:88-93 plus GQA ratios and the config-3
shape."""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import hadamard as oh
from oracle import quant as oq
from tests.gpu_util import assert_bitexact, to_dev, to_np

pytestmark = pytest.mark.gpu

ATOL = RTOL = 1e-2


@pytest.fixture(scope="module")
def C():
    from signrot_amd import _CUDA
    return _CUDA


def _close(got, ref, what, atol=ATOL, rtol=RTOL):
    got = np.asarray(got, np.float64)
    d = np.abs(got - ref)
    bad = d > atol + rtol * np.abs(ref)
    assert not bad.any(), (f"{what}: {bad.sum()} / {bad.size} outside tolerance, max |d| "
                           f"{d.max():.3e}")
    return d.max()


def _filled_cache(rng, B, T, H, page, L=2, spare=2):
    """A cache holding T tokens per request.  Small cases: N(0,1) K/V
    quantized by the oracle and laid out by the oracle's append (prefill
    form).  Large cases: random codes and [scale, zero] pairs everywhere
    (the layout is then exercised through the page table alone)."""
    pages_per = (T + page - 1) // page
    P = pages_per * B + spare
    indptr, indices, last = oa.page_table(B, T, page)
    if B * T * H > 200000:
        data = rng.integers(0, 256, (P, L, 2, H, page, 64), dtype=np.uint8)
        param = np.empty((P, L, 2, H, page, 2), np.float16)
        param[..., 0] = rng.uniform(0.1, 0.5, param.shape[:-1]).astype(np.float16)
        param[..., 1] = rng.uniform(0.5, 3.5, param.shape[:-1]).astype(np.float16)
        return data, param, indptr, indices, last
    data = np.zeros((P, L, 2, H, page, 64), np.uint8)
    param = np.zeros((P, L, 2, H, page, 2), np.float16)
    for layer in range(L):
        kv = rng.standard_normal((2, B * T, H, 128)).astype(np.float16)
        kq, kp = oq.kv_quant_pack(kv[0])
        vq, vp = oq.kv_quant_pack(kv[1])
        seq = (np.arange(B + 1) * T).astype(np.int32)
        oa.append(data, param, indptr, indices, last, layer, kq, vq, kp, vp, seq)
    return data, param, indptr, indices, last


@pytest.mark.parametrize("B,T,H,page", [(2, 37, 3, 16), (4, 513, 8, 128), (1, 1000, 2, 256)])
def test_init_and_append_bitexact(C, B, T, H, page):
    rng = np.random.default_rng(B * 1000 + T)
    L, layer = 3, 1
    P = ((T + 1 + page - 1) // page) * B + 1
    data = np.zeros((P, L, 2, H, page, 64), np.uint8)
    param = np.zeros((P, L, 2, H, page, 2), np.float16)
    d_data, d_param = to_dev(data), to_dev(param)
    k = rng.integers(0, 256, (B * T, H, 64), dtype=np.uint8)
    v = rng.integers(0, 256, (B * T, H, 64), dtype=np.uint8)
    kp = rng.standard_normal((B * T, H, 2)).astype(np.float16)
    vp = rng.standard_normal((B * T, H, 2)).astype(np.float16)
    seq = (np.arange(B + 1) * T).astype(np.int32)
    indptr, indices, last = oa.page_table(B, T, page)
    C.init_kv_i4(d_data, d_param, to_dev(indptr), to_dev(indices), to_dev(last), to_dev(k),
                 to_dev(v), to_dev(kp), to_dev(vp), to_dev(seq), layer)
    oa.append(data, param, indptr, indices, last, layer, k, v, kp, vp, seq)
    # one decode step
    indptr, indices, last = oa.page_table(B, T + 1, page)
    k1 = rng.integers(0, 256, (B, H, 64), dtype=np.uint8)
    v1 = rng.integers(0, 256, (B, H, 64), dtype=np.uint8)
    kp1 = rng.standard_normal((B, H, 2)).astype(np.float16)
    vp1 = rng.standard_normal((B, H, 2)).astype(np.float16)
    C.append_kv_i4(d_data, d_param, to_dev(indptr), to_dev(indices), to_dev(last), to_dev(k1),
                   to_dev(v1), to_dev(kp1), to_dev(vp1), layer)
    oa.append(data, param, indptr, indices, last, layer, k1, v1, kp1, vp1)
    torch.cuda.synchronize()
    assert_bitexact(to_np(d_data), data, "kv_data")
    assert_bitexact(to_np(d_param), param, "kv_param")


def test_init_ragged_requests(C):
    """Prefill with per-request lengths (the attention-mask path): request b
    holds lens[b] tokens, all requests share the page count."""
    rng = np.random.default_rng(77)
    B, H, page, lens = 3, 2, 16, [40, 33, 48]
    pages_per = 3
    P = pages_per * B
    data = np.zeros((P, 1, 2, H, page, 64), np.uint8)
    param = np.zeros((P, 1, 2, H, page, 2), np.float16)
    indptr = (np.arange(B + 1) * pages_per).astype(np.int32)
    indices = (np.arange(pages_per)[None, :] * B + np.arange(B)[:, None]).reshape(-1)
    indices = indices.astype(np.int32)
    last = np.array([(n - 1) % page + 1 for n in lens], np.int32)
    seq = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    tot = int(seq[-1])
    k = rng.integers(0, 256, (tot, H, 64), dtype=np.uint8)
    v = rng.integers(0, 256, (tot, H, 64), dtype=np.uint8)
    kp = rng.standard_normal((tot, H, 2)).astype(np.float16)
    d_data, d_param = to_dev(data), to_dev(param)
    C.init_kv_i4(d_data, d_param, to_dev(indptr), to_dev(indices), to_dev(last), to_dev(k),
                 to_dev(v), to_dev(kp), to_dev(kp), to_dev(seq), 0)
    oa.append(data, param, indptr, indices, last, 0, k, v, kp, kp, seq)
    torch.cuda.synchronize()
    assert_bitexact(to_np(d_data), data, "kv_data")
    assert_bitexact(to_np(d_param), param, "kv_param")


CASES = [  # B, T, Hkv, G, page
    (1, 1024, 32, 1, 256), (1, 1000, 32, 1, 256), (4, 513, 32, 1, 128), (2, 256, 32, 1, 256),
    (1, 2048, 32, 1, 256), (3, 1, 8, 4, 16), (2, 31, 8, 4, 16), (2, 100, 4, 2, 64),
    (2, 77, 2, 8, 32), (2, 65, 3, 3, 16), (32, 4096, 8, 4, 256),
]


@pytest.mark.parametrize("B,T,H,G,page", CASES)
def test_decode_vs_oracle_and_split(C, B, T, H, G, page):
    rng = np.random.default_rng(B * 7919 + T * 31 + H * G)
    data, param, indptr, indices, last = _filled_cache(rng, B, T, H, page)
    q = rng.standard_normal((B, H * G, 128)).astype(np.float16)
    ref = oa.decode(q, data, param, indptr, indices, last, 1)
    dev = [to_dev(a) for a in (data, param, indptr, indices, last)]
    dq = to_dev(q)
    o = torch.empty_like(dq)
    C.batch_decode_i4(o, dq, *dev, 1)
    unsplit = to_np(o)
    _close(unsplit, ref, "unsplit")
    for nc in sorted({2, 4, 8, 16, (T + page - 1) // page}):
        tmp = torch.empty((B, H * G, nc, 132), dtype=torch.float32, device="cuda")
        o2 = torch.empty_like(dq)
        C.batch_decode_i4(o2, dq, *dev, 1, tmp, nc)
        split = to_np(o2)
        _close(split, ref, f"chunks={nc} vs oracle")
        _close(split, unsplit.astype(np.float64), f"chunks={nc} vs unsplit", atol=2e-3,
               rtol=2e-3)


def test_decode_empty_request_gives_zeros(C):
    """A request with no pages (length 0) yields zeros; the others are unaffected."""
    rng = np.random.default_rng(4)
    data, param, indptr, indices, last = _filled_cache(rng, 2, 40, 2, 16)
    # request 0 keeps its pages, request 1 gets none
    indptr2 = np.array([0, 3, 3], np.int32)
    q = rng.standard_normal((2, 2, 128)).astype(np.float16)
    ref = oa.decode(q, data, param, indptr2, indices, last, 1)
    dq = to_dev(q)
    o = torch.full_like(dq, 7.0)
    C.batch_decode_i4(o, dq, to_dev(data), to_dev(param), to_dev(indptr2), to_dev(indices),
                      to_dev(last), 1)
    got = to_np(o)
    assert np.all(got[1] == 0)
    _close(got, ref, "empty request")


def test_decode_large_logits(C):
    """Large |q·k| (one dominant token) stays finite and picks that value."""
    rng = np.random.default_rng(8)
    data, param, indptr, indices, last = _filled_cache(rng, 1, 300, 1, 64)
    q = (rng.standard_normal((1, 4, 128)) * 40).astype(np.float16)
    ref = oa.decode(q, data, param, indptr, indices, last, 1)
    dq = to_dev(q)
    o = torch.empty_like(dq)
    C.batch_decode_i4(o, dq, *[to_dev(a) for a in (data, param, indptr, indices, last)], 1)
    got = to_np(o)
    assert np.isfinite(got.astype(np.float64)).all()
    _close(got, ref, "large logits")


def test_cache_module_prefill_then_decode():
    """MultiLayerPagedKVCache4Bit end to end: prefill update (init), one decode
    update (append) and the returned stub, against the oracle on the same
    rotated + quantized K/V (kv_cache.py:291-415)."""
    from signrot_amd.transformers import MultiLayerPagedKVCache4Bit
    rng = np.random.default_rng(12)
    B, T, H, G, L = 2, 70, 2, 4, 2
    cache = MultiLayerPagedKVCache4Bit(B, 32, 128, "cuda", L, H, 128, group_size=G)
    ks = rng.standard_normal((L, B, T + 1, H, 128)).astype(np.float16)
    vs = rng.standard_normal((L, B, T + 1, H, 128)).astype(np.float16)
    for layer in range(L):
        cache.update(to_dev(ks[layer, :, :T]), to_dev(vs[layer, :, :T]), layer, {})
    q = rng.standard_normal((B, 1, H * G, 128)).astype(np.float16)
    outs = []
    for layer in range(L):
        stub = cache.update(to_dev(ks[layer, :, T:]), to_dev(vs[layer, :, T:]), layer, {})
        outs.append(to_np(stub(to_dev(q))))
    assert cache.length == T + 1
    # oracle: rotate K (head-dim Hadamard, fp16), quantize, lay out, decode
    P = ((T + 1 + 31) // 32) * B
    data = np.zeros((P, L, 2, H, 32, 64), np.uint8)
    param = np.zeros((P, L, 2, H, 32, 2), np.float16)
    indptr, indices, last = oa.page_table(B, T + 1, 32)
    for layer in range(L):
        kr = oh.rotate(ks[layer].reshape(-1, 128)).reshape(B * (T + 1), H, 128)
        kq, kp = oq.kv_quant_pack(kr)
        vq, vp = oq.kv_quant_pack(vs[layer].reshape(B * (T + 1), H, 128))
        seq = (np.arange(B + 1) * (T + 1)).astype(np.int32)
        oa.append(data, param, indptr, indices, last, layer, kq, vq, kp, vp, seq)
    qr = oh.rotate(q.reshape(-1, 128)).reshape(B, H * G, 128)
    for layer in range(L):
        ref = oa.decode(qr, data, param, indptr, indices, last, layer)
        _close(outs[layer][:, 0], ref, f"layer {layer}")


@pytest.mark.parametrize("shape", [(1, 1, 32, 128), (1, 2048, 32, 128), (16, 1, 32, 128),
                                   (4, 37, 8, 128)])
def test_asym_quantize_and_pack_i4_equals_kv_quant_pack(shape):
    """The reference's torch KV quantizer against the fused kernel
    (benchmarks/test_fused_equivalence.py:76-90): codes, scales and zeros
    bit for bit, also for constant rows (the 1e-5 clamp)."""
    from signrot_amd import _CUDA
    from signrot_amd.transformers import asym_quantize_and_pack_i4
    g = torch.Generator(device="cuda").manual_seed(sum(shape))
    x = torch.randn(shape, device="cuda", generator=g).half() * 2
    x[..., 0, :, :] = 1.5
    q_f, param = _CUDA.kv_quant_pack(x)
    q_r, s_r, z_r = asym_quantize_and_pack_i4(x)
    assert torch.equal(q_f, q_r)
    assert torch.equal(param[..., 0:1], s_r)
    assert torch.equal(param[..., 1:2], z_r)


def test_hf_cache_adapter_over_the_paged_cache():
    """HFCacheAdapter around MultiLayerPagedKVCache4Bit: prefill and decode
    updates through the adapter return what the same calls on a bare cache
    return (bit for bit), and the lengths track."""
    from transformers.cache_utils import Cache
    from signrot_amd.transformers import HFCacheAdapter, MultiLayerPagedKVCache4Bit
    B, T, H, G, L = 2, 70, 2, 4, 2
    g = torch.Generator(device="cuda").manual_seed(5)
    ks = torch.randn((L, B, T + 1, H, 128), device="cuda", generator=g).half()
    vs = torch.randn((L, B, T + 1, H, 128), device="cuda", generator=g).half()
    q = torch.randn((B, 1, H * G, 128), device="cuda", generator=g).half()
    outs = []
    for wrap in (False, True):
        inner = MultiLayerPagedKVCache4Bit(B, 32, 128, "cuda", L, H, 128, group_size=G)
        cache = HFCacheAdapter(inner) if wrap else inner
        assert isinstance(cache, Cache) and len(inner) == L and bool(inner)
        for layer in range(L):
            k_ret, v_ret = cache.update(ks[layer, :, :T], vs[layer, :, :T], layer, {})
            assert torch.equal(k_ret, ks[layer, :, :T]) and torch.equal(v_ret, vs[layer, :, :T])
        assert cache.get_seq_length() == T and cache.get_usable_length(1, 0) == T
        res = [cache.update(ks[layer, :, T:], vs[layer, :, T:], layer, {})(q)
               for layer in range(L)]
        assert cache.get_seq_length() == T + 1
        outs.append(torch.stack(res))
    assert torch.equal(outs[0], outs[1])
