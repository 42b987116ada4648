"""CPU tests of the host-side module API (construction, buffers, packing,
Hadamard factor selection, fusion rewrite) -- no device compute."""
import numpy as np
import pytest
import torch

from oracle import hadamard as oh
from oracle import quant as oq


def test_get_hadK_matches_oracle():
    from signrot_amd.functional.hadamard import get_hadK
    for n in (4096, 14336, 28672, 11008, 128, 32, 3072, 5120, 18432, 13824):
        h, k = get_hadK(n)
        hw, kw = oh.get_hadK(n)
        assert k == kw
        if k > 1:
            assert np.array_equal(h.numpy().astype(np.int8), hw)


def test_pack_unpack_match_oracle():
    from signrot_amd.functional.quantization import pack_i4, unpack_i4
    rng = np.random.default_rng(0)
    q = rng.integers(-8, 8, (7, 64)).astype(np.int8)
    p = pack_i4(torch.from_numpy(q))
    assert np.array_equal(p.numpy(), oq.pack_i4(q))
    assert np.array_equal(unpack_i4(p).numpy(), q)
    with pytest.raises(AssertionError):
        pack_i4(torch.tensor([[8, 0]], dtype=torch.int8))


def test_linear4bit_from_float_codes():
    from signrot_amd.nn import Linear4bit
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((32, 64)) * 0.02).astype(np.float16)
    codes, s, wfq = oq.rtn_weight(w)
    lin = torch.nn.Linear(64, 32, bias=False).half()
    lin.weight.data = torch.from_numpy(wfq)
    q = Linear4bit.from_float(lin, torch.from_numpy(s))
    assert q.weight.shape == (32, 32) and q.weight.dtype == torch.uint8
    assert np.array_equal(q.weight.numpy(), oq.pack_i4(codes))
    assert q.weight_scales.dtype == torch.float16
    assert set(q.state_dict()) == {"weight", "weight_scales"}


def test_online_hadamard_buffers():
    from signrot_amd.nn import OnlineHadamard
    m = OnlineHadamard(14336, had_adj=True)
    assert m.rem_dim == 28 and m.had_rem_dim.dtype == torch.float16
    assert m.had_adj_sign.dtype == torch.int8 and m.had_adj_sign.shape == (14336,)
    assert set(m.state_dict()) == {"had_rem_dim", "had_adj_sign"}
    m2 = OnlineHadamard(4096)
    assert m2.rem_dim == 1 and m2.had_rem_dim is None
    m3 = OnlineHadamard(14336, force_fp32=True)
    assert m3.had_rem_dim.dtype == torch.float32


def test_fuse_online_hadamard_rewrites_pairs():
    from signrot_amd.nn import (HadamardQuantizer, Linear4bit, OnlineHadamard, Quantizer,
                                fuse_online_hadamard)
    lin = Linear4bit(14336, 64)
    block = torch.nn.Module()
    block.down_proj = torch.nn.Sequential(OnlineHadamard(14336, lin, had_adj=True),
                                          Quantizer(), lin)
    keys = set(block.state_dict())
    fuse_online_hadamard(block)
    assert isinstance(block.down_proj[0], HadamardQuantizer)
    assert block.down_proj[1] is lin
    # state-dict keys move under the fused module, values unchanged
    assert len(block.state_dict()) == len(keys)


def test_fuse_online_hadamard_rewrites_asym_pairs():
    from signrot_amd.nn import (AsymQuantizer, HadamardQuantizer, Linear4bit, OnlineHadamard,
                                fuse_online_hadamard)
    lin = Linear4bit(14336, 64)
    block = torch.nn.Module()
    block.down_proj = torch.nn.Sequential(OnlineHadamard(14336, lin, had_adj=True),
                                          AsymQuantizer(clip_ratio=0.9), lin)
    fuse_online_hadamard(block)
    assert isinstance(block.down_proj[0], HadamardQuantizer)
    assert isinstance(block.down_proj[0].quantizer, AsymQuantizer)
    assert block.down_proj[1] is lin
