"""Pins of oracle.glue against artefacts independent of its own formulas:
HF transformers' apply_rotary_pos_emb and torch's SiLU evaluated in fp16 on
the CPU (the functions the reference's kernels replace, compared the same way
in benchmarks/test_fused_equivalence.py:102-122), and closed forms /
invariants of RMSNorm."""
import numpy as np
import pytest
import torch

from oracle import glue


def _bits(a):
    return np.asarray(a, np.float16).view(np.uint16)


@pytest.mark.parametrize("b,t,hq,hk,d", [(1, 1, 32, 32, 128), (16, 1, 32, 32, 128),
                                         (4, 3, 32, 8, 128), (2, 5, 4, 2, 64)])
def test_rope_matches_hf_apply_rotary_pos_emb(b, t, hq, hk, d):
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    g = torch.Generator().manual_seed(b * 7 + t)
    q = torch.randn(b, t, hq, d, generator=g).half()
    k = torch.randn(b, t, hk, d, generator=g).half()
    for cb in sorted({1, b}):
        c = torch.randn(cb, t, d, generator=g).half()
        s = torch.randn(cb, t, d, generator=g).half()
        qr, kr = apply_rotary_pos_emb(q, k, c, s, unsqueeze_dim=2)
        qo, ko = glue.rope_qk(q.numpy(), k.numpy(), c.numpy(), s.numpy())
        assert np.array_equal(_bits(qo), _bits(qr.numpy()))
        assert np.array_equal(_bits(ko), _bits(kr.numpy()))


def test_rope_signed_zeros_match_hf():
    """Signed zeros in x, cos and sin (the products that are exactly -0 or
    +0, their sums, and fp16 underflow) bit for bit as HF's fp16 expression
    gives them: the sign of a zero output is part of the bit-exact contract
    (x1 = +0 with sin < 0 and x0 * cos = -0 gives +0)."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    vals = torch.tensor([0.0, -0.0, 1e-7, -1e-7, 6e-8, -6e-8, 0.5, -0.5, 3.0, -3.0],
                        dtype=torch.float16)
    n = len(vals)
    # every (x0, x1, cos, sin) combination of the values, one pair per row
    x0, x1, c, s = torch.meshgrid(vals, vals, vals, vals, indexing="ij")
    q = torch.stack([x0.reshape(-1), x1.reshape(-1)], dim=-1).view(1, n ** 4, 1, 2)
    cos = torch.stack([c.reshape(-1), c.reshape(-1)], dim=-1).view(1, n ** 4, 2)
    sin = torch.stack([s.reshape(-1), s.reshape(-1)], dim=-1).view(1, n ** 4, 2)
    qr, _ = apply_rotary_pos_emb(q, q, cos, sin, unsqueeze_dim=2)
    qo, _ = glue.rope_qk(q.numpy(), q.numpy(), cos.numpy(), sin.numpy())
    assert np.array_equal(_bits(qo), _bits(qr.numpy()))
    neg_zero = _bits(qr.numpy()) == 0x8000
    assert neg_zero.any() and (_bits(qr.numpy()) == 0).any()


def test_rope_identity_and_quarter_turn():
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 2, 3, 8)).astype(np.float16)
    one = np.ones((1, 2, 8), np.float16)
    zero = np.zeros((1, 2, 8), np.float16)
    qo, _ = glue.rope_qk(q, q, one, zero)
    assert np.array_equal(_bits(qo), _bits(q))
    # cos 0, sin 1: (x0, x1) -> (-x1, x0)
    qo, _ = glue.rope_qk(q, q, zero, one)
    assert np.array_equal(_bits(qo[..., :4]), _bits(-q[..., 4:]))
    assert np.array_equal(_bits(qo[..., 4:]), _bits(q[..., :4]))


@pytest.mark.parametrize("shape", [(1, 11008), (16, 11008), (3, 4096)])
def test_swiglu_matches_torch_silu(shape):
    g = torch.Generator().manual_seed(shape[0])
    gate = (torch.randn(*shape, generator=g) * 4).half()
    up = (torch.randn(*shape, generator=g) * 4).half()
    ref = (torch.nn.SiLU()(gate) * up).numpy()
    got = glue.swiglu(gate.numpy(), up.numpy())
    assert np.array_equal(_bits(got), _bits(ref))


def test_swiglu_special_values():
    gate = np.array([0.0, 20.0, -20.0, 1.0], np.float16)
    up = np.array([5.0, 1.0, 1.0, 1.0], np.float16)
    got = glue.swiglu(gate, up).astype(np.float64)
    assert got[0] == 0.0
    assert got[1] == 20.0                     # silu(20) rounds to 20 in fp16
    assert abs(got[2]) < 1e-6                 # silu(-20) ~ -4e-8
    assert abs(got[3] - 1 / (1 + np.exp(-1))) < 1e-3


def test_rmsnorm_closed_forms():
    # constant row c: out = c / sqrt(c^2 * cols / mean_dim + eps)
    x = np.full((1, 4096), 3.0, np.float16)
    out = glue.rmsnorm(x, 1e-5, 4096).astype(np.float64)
    np.testing.assert_allclose(out, 3.0 / np.sqrt(9.0 + 1e-5), rtol=2 ** -11)
    # mean_dim differs from cols (the o_proj / head-axis use): factor sqrt(mean_dim / cols)
    out2 = glue.rmsnorm(x, 0.0, 1024).astype(np.float64)
    np.testing.assert_allclose(out2, 3.0 / np.sqrt(9.0 * 4), rtol=2 ** -11)


def test_rmsnorm_invariants():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((8, 4096)).astype(np.float16)
    out = glue.rmsnorm(x, 0.0, 4096).astype(np.float64)
    # unit RMS rows, same signs, scale invariance
    np.testing.assert_allclose(np.sqrt((out ** 2).mean(-1)), 1.0, rtol=1e-3)
    assert np.array_equal(np.sign(out), np.sign(x.astype(np.float64)))
    out4 = glue.rmsnorm((x.astype(np.float32) * 4).astype(np.float16), 0.0, 4096)
    assert np.array_equal(_bits(out4), _bits(out.astype(np.float16)))
    # eps matters for tiny rows: all 2^-14 -> 2^-14 / sqrt(2^-28 + 1e-5)
    t = np.full((1, 128), 2.0 ** -14, np.float16)
    o = glue.rmsnorm(t, 1e-5, 128).astype(np.float64)
    np.testing.assert_allclose(o, 2.0 ** -14 / np.sqrt(2.0 ** -28 + 1e-5), rtol=2 ** -11)
