"""CPU tests of the signrot_amd.transformers surface (the reference's
signrot/transformers/kv_cache.py): asym_quantize_and_pack_i4 against the
oracle's KV quantizer (the fused kv_quant_pack's arithmetic, pinned in
tests/test_oracle_quant.py) bit for bit, its quantize=False and lac
branches by hand-worked values, HFCacheAdapter's delegation, and both
cache classes being transformers Caches."""
import numpy as np
import pytest
import torch
from transformers.cache_utils import Cache

from oracle import quant as oq
from signrot_amd.transformers import (HFCacheAdapter, MultiLayerPagedKVCache4Bit,
                                      asym_quantize_and_pack_i4)


@pytest.mark.parametrize("shape", [(1, 1, 32, 128), (1, 64, 32, 128), (4, 37, 8, 128),
                                   (3, 10)])
def test_asym_quantize_and_pack_matches_kv_quant_pack(shape):
    rng = np.random.default_rng(sum(shape))
    x = (rng.standard_normal(shape) * 2).astype(np.float16)
    x[..., 0, :] = 1.5 if len(shape) > 2 else x[..., 0, :]   # constant rows: the 1e-5 clamp
    q, s, z = asym_quantize_and_pack_i4(torch.from_numpy(x))
    qw, pw = oq.kv_quant_pack(x)
    assert np.array_equal(q.numpy(), qw)
    assert np.array_equal(s.numpy().view(np.uint16), pw[..., 0:1].view(np.uint16))
    assert np.array_equal(z.numpy().view(np.uint16), pw[..., 1:2].view(np.uint16))


def test_asym_quantize_known_answers():
    """One row [-1, 0, 0.5, 2] in fp16 worked by hand (every op rounds to
    fp16).  Default branch: scale = fp16(3 / 15) = 0.199951..., zero = 1,
    codes round((x + 1) / scale) = [0, 5, 8, 15] (1.5 / 0.19995 = 7.5018
    rounds to fp16 7.5, half to even -> 8); quantize=False gives scale *
    (codes - zero).  lac branch: the range [-1, 2] already holds 0, scale =
    0.19995, zero = round(1 / 0.19995 = 5.0012) = 5, codes round(x / scale) +
    5 = [0, 5, 7, 15] (0.5 / 0.19995 = 2.5006 rounds to fp16 2.5, half to
    even -> 2)."""
    x = torch.tensor([[-1.0, 0.0, 0.5, 2.0]], dtype=torch.float16)
    q, s, z = asym_quantize_and_pack_i4(x)
    s16 = torch.tensor(0.2, dtype=torch.float16)
    assert s.item() == s16.item() and z.item() == 1.0
    assert q.tolist() == [[0 | (5 << 4), 8 | (15 << 4)]]
    dq, _, _ = asym_quantize_and_pack_i4(x, quantize=False)
    codes = torch.tensor([[0, 5, 8, 15]], dtype=torch.float16)
    assert torch.equal(dq, s16 * (codes - 1))
    ql, sl, zl = asym_quantize_and_pack_i4(x, lac=True)
    assert sl.item() == s16.item() and zl.item() == 5.0
    assert ql.tolist() == [[0 | (5 << 4), 7 | (15 << 4)]]
    # an all-zero row: the range becomes [-1, 1]
    zr = torch.zeros(1, 4, dtype=torch.float16)
    qz, sz, zz = asym_quantize_and_pack_i4(zr, lac=True)
    s2 = (torch.tensor(2.0, dtype=torch.float16) / 15)
    assert sz.item() == s2.item() and zz.item() == torch.round(1 / s2).item()
    # clip factors scale the lac range
    _, sc, _ = asym_quantize_and_pack_i4(x, clip_factor_a_max=0.5, clip_factor_a_min=0.5,
                                        lac=True)
    assert sc.item() == (torch.tensor(1.5, dtype=torch.float16) / 15).item()


class _Inner:
    def __init__(self):
        self.calls = []

    def update(self, k, v, layer_idx, kw):
        self.calls.append(("update", k, v, layer_idx, kw))
        return "attn"

    def get_seq_length(self):
        return 11

    def get_max_length(self):
        return None

    def get_usable_length(self, n, layer_idx):
        self.calls.append(("usable", n, layer_idx))
        return 9

    def to_legacy_cache(self):
        return "legacy"


def test_hf_cache_adapter_delegates():
    inner = _Inner()
    a = HFCacheAdapter(inner)
    assert isinstance(a, Cache)
    assert a.update("k", "v", 3, {"x": 1}) == "attn"
    assert inner.calls[-1] == ("update", "k", "v", 3, {"x": 1})
    assert a.get_seq_length() == 11 and a.get_max_length() is None
    assert a.get_usable_length(5, 2) == 9 and inner.calls[-1] == ("usable", 5, 2)
    assert a.to_legacy_cache() == "legacy"
    plain = HFCacheAdapter(object())
    assert plain.to_legacy_cache() is plain


def test_cache_is_a_transformers_cache():
    assert issubclass(MultiLayerPagedKVCache4Bit, Cache)
