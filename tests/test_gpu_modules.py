"""GPU parity of the reference consumer's symmetric module chains
(e2e/quantized_llama/modeling_llama.py:94-142) built from this package's
modules, against the oracle:

* q/k/v and o_proj: Quantizer -> Linear4bit.from_float (103-117);
* o_proj's head-axis OnlineHadamard(num_heads) on the transposed attention
  output, then Sequential(Quantizer, Linear4bit) (94-96, 116-117);
* the MLP: Quantizer -> gate/up Linear4bit -> SiLU(g) * u (torch, as
  LlamaMLP.forward) -> Sequential(OnlineHadamard(ffn, had_adj=True),
  Quantizer, Linear4bit) (119-142), with the sign calibrated by the
  product's OnlineHadamard.calibrate_adj_sign and folded into the fp16
  down_proj weight before RTN, as the fake-quant pipeline does
  (quant_utils.py:362-367, gptq_utils.py:438-457).

int4 codes, scales and int32 products are bit-exact against the oracle on
the GPU's own rotated fp16 values (the rotation's fp16 bits are fixed only to
tolerance, 1e-2 abs + rel, as the reference's fast_hadamard_transform is not
available); fp16 outputs of the fused GEMM + dequant are bit-exact too."""
import numpy as np
import pytest
import torch

from oracle import hadamard as oh
from oracle import quant as oq
from tests.gpu_util import assert_bitexact, outlier_input, to_dev, to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rtn_linear(rng, in_f, out_f, bias=False, sign=None, std=0.02):
    """An fp16 Linear with N(0, std) weights, the sign folded by column, RTN
    per channel (symmetric grid when a sign is folded), and its Linear4bit."""
    from signrot_amd.functional.quantization import rtn_weight_pack
    from signrot_amd.nn import Linear4bit
    fp = torch.nn.Linear(in_f, out_f, bias=bias).half().to(DEV)
    with torch.no_grad():
        fp.weight.copy_(to_dev((rng.standard_normal((out_f, in_f)) * std).astype(np.float16)))
        if bias:
            fp.bias.copy_(to_dev((rng.standard_normal(out_f) * 0.1).astype(np.float16)))
        if sign is not None:
            fp.weight.mul_(sign.to(torch.float16))
        _, s16, wfq = rtn_weight_pack(fp.weight.data, symmetric_grid=sign is not None)
        fp.weight.copy_(wfq)
    return Linear4bit.from_float(fp, s16.view(-1, 1)).to(DEV), fp


@torch.no_grad()
@pytest.mark.parametrize("bias,clip", [(False, 1.0), (True, 1.0), (False, 0.9)])
def test_quantizer_then_linear4bit(bias, clip):
    from signrot_amd.nn import Quantizer
    rng = np.random.default_rng(1 + int(bias))
    K, N = 4096, 1024
    lin, _ = _rtn_linear(rng, K, N, bias=bias)
    x = to_dev(outlier_input(rng, 10, K, n_out=4, mag=100.0)).view(2, 5, K)
    chain = torch.nn.Sequential(Quantizer(clip_ratio=clip), lin)
    out = chain(x)
    assert out.shape == (2, 5, N) and out.dtype == torch.float16
    qw, sw = oq.sym_quant_dynamic(to_np(x).reshape(-1, K), clip)
    want = oq.w4a4_linear(qw, sw, to_np(lin.weight), to_np(lin.weight_scales).reshape(-1),
                          to_np(lin.bias) if bias else None)
    assert_bitexact(to_np(out).reshape(-1, N), want, "Quantizer -> Linear4bit")
    # the module's unfused reference path gives the same codes and scales
    p = chain[0](x)
    pr = chain[0].forward_reference(x.view(-1, K))
    assert torch.equal(p.quantized_x.view(-1, K // 2), pr.quantized_x)
    if clip == 1.0:
        assert torch.equal(p.scales_x.view(-1), pr.scales_x.view(-1))


@torch.no_grad()
def test_o_proj_head_axis_hadamard_chain():
    from signrot_amd.nn import OnlineHadamard, Quantizer
    rng = np.random.default_rng(3)
    B, T, H, D = 3, 2, 32, 128
    o_proj, _ = _rtn_linear(rng, H * D, H * D)
    had = OnlineHadamard(H, o_proj).to(DEV)
    chain = torch.nn.Sequential(Quantizer(), o_proj)
    attn = to_dev((rng.standard_normal((B, T, H, D)) * 2).astype(np.float16))
    rot = had(attn.transpose(-1, -2)).transpose(-1, -2)
    flat = rot.reshape(B, T, H * D).contiguous()
    out = chain(flat)
    # rotation over the head axis: FWHT-32 / sqrt(32), within fp16 tolerance
    want_rot = np.swapaxes(oh.online_hadamard(np.swapaxes(to_np(attn), -1, -2)), -1, -2)
    np.testing.assert_allclose(to_np(rot).astype(np.float32), want_rot.astype(np.float32),
                               rtol=1e-2, atol=1e-2)
    qw, sw = oq.sym_quant_dynamic(to_np(flat).reshape(-1, H * D))
    want = oq.w4a4_linear(qw, sw, to_np(o_proj.weight), to_np(o_proj.weight_scales).reshape(-1))
    assert_bitexact(to_np(out).reshape(-1, H * D), want, "o_proj chain")


@torch.no_grad()
@pytest.mark.parametrize("hidden,ffn,tokens", [(4096, 14336, 6), (1024, 14336, 40),
                                               (1024, 28672, 3)])
def test_mlp_chain_with_calibrated_sign(hidden, ffn, tokens):
    from signrot_amd.nn import OnlineHadamard, Quantizer, fuse_online_hadamard
    rng = np.random.default_rng(hidden + ffn + tokens)
    gate, _ = _rtn_linear(rng, hidden, ffn)
    up, _ = _rtn_linear(rng, hidden, ffn)
    quant_in = Quantizer()
    x = to_dev(outlier_input(rng, tokens, hidden, n_out=4, mag=100.0)).view(1, tokens, hidden)

    # LlamaMLP.forward on the quantized input: act(gate(x)) * up(x) in torch
    px = quant_in(x)
    g, u = gate(px), up(px)
    act = torch.nn.functional.silu(g) * u
    qw, sw = oq.sym_quant_dynamic(to_np(x).reshape(-1, hidden))
    assert_bitexact(to_np(g).reshape(tokens, ffn),
                    oq.w4a4_linear(qw, sw, to_np(gate.weight),
                                   to_np(gate.weight_scales).reshape(-1)), "gate_proj")
    assert_bitexact(to_np(u).reshape(tokens, ffn),
                    oq.w4a4_linear(qw, sw, to_np(up.weight),
                                   to_np(up.weight_scales).reshape(-1)), "up_proj")

    # calibrate the SignRot sign on this batch, fold it into the fp16
    # down_proj weight, then RTN on the symmetric grid
    had = OnlineHadamard(ffn, had_adj=True).to(DEV)
    down_fp = torch.nn.Linear(ffn, hidden, bias=False).half().to(DEV)
    down_fp.weight.copy_(to_dev((rng.standard_normal((hidden, ffn)) * 0.02).astype(np.float16)))
    w_before = down_fp.weight.clone()
    sign = had.calibrate_adj_sign(act, fold_into=down_fp)
    assert torch.equal(down_fp.weight, w_before * sign.half())
    # the rule on the unsigned rotation (had(act) now applies the sign: undo it)
    want_sign = oh.sign_calibration(to_np(had(act) * sign.half()))
    assert np.array_equal(to_np(sign), want_sign)
    from signrot_amd.functional.quantization import rtn_weight_pack
    from signrot_amd.nn import Linear4bit
    _, s16, wfq = rtn_weight_pack(down_fp.weight.data, symmetric_grid=True)
    down_fp.weight.copy_(wfq)
    down = Linear4bit.from_float(down_fp, s16.view(-1, 1)).to(DEV)
    had.module = down

    chain = torch.nn.Sequential(had, Quantizer(), down)
    out = chain(act)
    rot = had(act)
    want_rot = oh.online_hadamard(to_np(act).reshape(-1, ffn), to_np(sign))
    np.testing.assert_allclose(to_np(rot).reshape(-1, ffn).astype(np.float32),
                               want_rot.astype(np.float32), rtol=1e-2, atol=1e-2)
    qd, sd = oq.sym_quant_dynamic(to_np(rot).reshape(-1, ffn))
    want = oq.w4a4_linear(qd, sd, to_np(down.weight), to_np(down.weight_scales).reshape(-1))
    assert_bitexact(to_np(out).reshape(-1, hidden), want, "down_proj chain")

    # fuse_online_hadamard (after loading) keeps the output bit for bit
    holder = torch.nn.Module()
    holder.down_proj = chain
    fuse_online_hadamard(holder)
    assert torch.equal(holder.down_proj(act), out)
