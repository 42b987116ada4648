"""GPU parity of the prefill attention (the flash-attn 2 call of
e2e/quantized_llama/modeling_llama.py:81-90) against the float64 oracle,
tolerance 1e-2 abs + rel (fp16 inputs and output, P rounded to fp16 as in
flash-attn); masked query rows are exactly zero."""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from tests.gpu_util import to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def C():
    from signrot_amd import _CUDA
    return _CUDA


def _inputs(B, T, Hq, Hkv, seed, mag=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, T, Hq, 128, generator=g) * mag).half()
    k = (torch.randn(B, T, Hkv, 128, generator=g) * mag).half()
    v = torch.randn(B, T, Hkv, 128, generator=g).half()
    return q, k, v


def _check(got, q, k, v, mask, causal, what):
    want = oa.prefill(q.numpy(), k.numpy(), v.numpy(), None if mask is None else mask.numpy(),
                      causal)
    got = to_np(got).astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2, err_msg=what)
    if mask is not None:
        dead = mask.numpy() == 0
        assert np.all(got[dead] == 0), what


@pytest.mark.parametrize("B,T,Hq,Hkv,causal,masked", [
    (1, 1, 4, 4, True, False), (2, 77, 8, 2, True, True), (1, 128, 4, 1, True, False),
    (1, 129, 2, 2, True, False), (1, 300, 32, 8, True, False), (2, 200, 4, 4, False, True),
    (1, 1031, 8, 8, True, False), (3, 65, 6, 3, False, False),
    # GQA groups of 8, 4 and 2 in 8-wave blocks of 32 / 64 / 128 query rows
    # (enough blocks for one per CU), and of 3 (4-wave blocks)
    (4, 333, 64, 8, True, False), (2, 1100, 64, 8, True, True), (4, 700, 32, 8, True, False),
    (8, 600, 16, 8, False, False), (3, 1031, 32, 16, True, True), (2, 70, 9, 3, True, True)])
def test_prefill_matches_oracle(C, B, T, Hq, Hkv, causal, masked):
    q, k, v = _inputs(B, T, Hq, Hkv, seed=T * 7 + B)
    mask = None
    if masked:
        mask = torch.ones(B, T, dtype=torch.int64)
        mask[0, : T // 3] = 0                   # left padding
        if B > 1:
            mask[1, 1::5] = 0                   # holes
    dev = "cuda:0"
    out = C.prefill_attention(q.to(dev), k.to(dev), v.to(dev),
                              None if mask is None else mask.to(dev), causal)
    torch.cuda.synchronize()
    _check(out, q, k, v, mask, causal, f"B={B} T={T} Hq={Hq} Hkv={Hkv} causal={causal}")


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_padded_positions_hold_nan_and_inf(C, causal):
    """Whatever a padded position holds never reaches a live row: NaN and
    ±inf in the masked q, K and V rows leave the live rows equal to the
    attention over the unpadded tokens, and the masked rows zero."""
    B, T, Hq, Hkv = 2, 150, 8, 2
    q, k, v = _inputs(B, T, Hq, Hkv, seed=91)
    mask = torch.ones(B, T, dtype=torch.int64)
    mask[0, :40] = 0                          # left padding
    mask[1, 3::7] = 0                         # holes
    dead = mask == 0
    want = oa.prefill(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), causal)
    qn, kn, vn = q.clone(), k.clone(), v.clone()
    for t, fill in ((qn, float("nan")), (kn, float("inf")), (vn, float("nan"))):
        t[dead] = fill
    kn[1, 3, 0, :5] = float("-inf")
    vn[0, 7, 1, 9] = float("inf")
    out = C.prefill_attention(qn.cuda(), kn.cuda(), vn.cuda(), mask.cuda(), causal)
    torch.cuda.synchronize()
    got = to_np(out).astype(np.float64)
    assert np.all(np.isfinite(got)), "a padded position leaked into the output"
    np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2)
    assert np.all(got[dead.numpy()] == 0)


def test_prefill_large_logits(C):
    """Logits far above 1 (|q.k| * scale in the hundreds): the running max
    keeps exp2 in range."""
    q, k, v = _inputs(1, 333, 4, 2, seed=5, mag=6.0)
    out = C.prefill_attention(q.cuda(), k.cuda(), v.cuda())
    torch.cuda.synchronize()
    _check(out, q, k, v, None, True, "large logits")


@pytest.mark.parametrize("step", [0.004, 0.01, 0.03, -0.01])
def test_prefill_rising_logits(C, step):
    """Logits that rise along the keys by about 2, 5 or 16 (log2 units) per
    64-key tile, or fall: the running max moves by less than its rescale
    threshold on many tiles, so probabilities above 1 go through the fp16 PV
    product and the row sum, and by more on others."""
    B, T, Hq, Hkv = 1, 600, 4, 2
    g = torch.Generator().manual_seed(17)
    q = torch.full((B, T, Hq, 128), 0.5).half()
    ramp = torch.arange(T, dtype=torch.float32) * step
    k = (ramp[None, :, None, None] + 0.05 * torch.randn(B, T, Hkv, 128, generator=g)).half()
    v = torch.randn(B, T, Hkv, 128, generator=g).half()
    out = C.prefill_attention(q.cuda(), k.cuda(), v.cuda())
    torch.cuda.synchronize()
    _check(out, q, k, v, None, True, f"ramp step {step}")


@pytest.mark.parametrize("scale", [0.3, -0.05, 0.0])
def test_prefill_softmax_scale(C, scale):
    """Any finite softmax_scale: larger than 1/sqrt(128), negative (the
    softmax then favours the smallest q.k), and zero (the mean of the visible
    V rows)."""
    B, T, Hq, Hkv = 2, 260, 8, 2
    q, k, v = _inputs(B, T, Hq, Hkv, seed=23)
    mask = torch.ones(B, T, dtype=torch.int64)
    mask[1, :50] = 0
    out = C.prefill_attention(q.cuda(), k.cuda(), v.cuda(), mask.cuda(), softmax_scale=scale)
    torch.cuda.synchronize()
    want = oa.prefill(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), True, sm_scale=scale)
    np.testing.assert_allclose(to_np(out).astype(np.float64), want, rtol=1e-2, atol=1e-2)


def test_prefill_rejects_nonfinite_scale(C):
    q = torch.zeros(1, 4, 4, 128, dtype=torch.float16, device="cuda:0")
    with pytest.raises(RuntimeError, match="sm_scale"):
        C.prefill_attention(q, q, q, softmax_scale=float("nan"))


def test_prefill_strided_qkv_slices(C):
    """q/k/v as column slices of one fused projection output."""
    B, T, Hq, Hkv = 2, 150, 8, 2
    g = torch.Generator().manual_seed(9)
    qkv = torch.randn(B, T, (Hq + 2 * Hkv) * 128, generator=g).half().cuda()
    q = qkv[..., : Hq * 128].view(B, T, Hq, 128)
    k = qkv[..., Hq * 128:(Hq + Hkv) * 128].view(B, T, Hkv, 128)
    v = qkv[..., (Hq + Hkv) * 128:].view(B, T, Hkv, 128)
    got = C.prefill_attention(q, k, v)
    want = C.prefill_attention(q.contiguous(), k.contiguous(), v.contiguous())
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    _check(got, q.cpu(), k.cpu(), v.cpu(), None, True, "strided")


@pytest.mark.parametrize("B,T,masked", [(1, 2048, False), (1, 8192, False), (2, 3000, True)])
def test_prefill_full_size_vs_fp32(C, B, T, masked):
    """Llama-70B heads at full size (T = 2048 and 8192: the grids whose
    blocks go out heaviest causal q tile first across the head groups; two
    left-padded sequences at T = 3000) against a float32 torch reference on
    the GPU (per kv-head group, explicit matmuls), tolerance 1e-2."""
    Hq, Hkv = 64, 8
    g = torch.Generator(device="cuda:0").manual_seed(T + B)
    q = torch.randn(B, T, Hq, 128, device="cuda:0", generator=g).half()
    k = torch.randn(B, T, Hkv, 128, device="cuda:0", generator=g).half()
    v = torch.randn(B, T, Hkv, 128, device="cuda:0", generator=g).half()
    mask = None
    if masked:
        mask = torch.ones(B, T, dtype=torch.int64, device="cuda:0")
        mask[1, : T // 4] = 0
    out = C.prefill_attention(q, k, v, mask).float()
    causal = torch.ones(T, T, dtype=torch.bool, device="cuda:0").tril()
    G = Hq // Hkv
    for bb in range(B):
        keep = causal if mask is None else causal & (mask[bb] != 0)[None, :]
        live = torch.ones(T, dtype=torch.bool, device="cuda:0") if mask is None else mask[bb] != 0
        for h in range(bb, Hq, 9):
            qh = q[bb, :, h].float()
            kh = k[bb, :, h // G].float()
            vh = v[bb, :, h // G].float()
            s = (qh @ kh.t().contiguous()) * 128 ** -0.5
            s = s.masked_fill(~keep, float("-inf"))
            ref = torch.softmax(s[live], dim=-1) @ vh
            torch.testing.assert_close(out[bb, live, h], ref, rtol=1e-2, atol=1e-2)
            assert torch.all(out[bb, ~live, h] == 0)


def test_prefill_rejects_bad_shapes(C):
    q = torch.zeros(1, 4, 4, 64, dtype=torch.float16, device="cuda:0")
    with pytest.raises(RuntimeError, match="head_dim"):
        C.prefill_attention(q, q, q)
    q = torch.zeros(1, 4, 6, 128, dtype=torch.float16, device="cuda:0")
    k = torch.zeros(1, 4, 4, 128, dtype=torch.float16, device="cuda:0")
    with pytest.raises(RuntimeError, match="multiple"):
        C.prefill_attention(q, k, k)
