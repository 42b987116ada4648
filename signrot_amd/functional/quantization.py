"""Pure-torch quantization helpers of the reference's
signrot/functional/quantization.py (lines 5-101): int4 two's-complement
packing and the fake quant/dequant formulas used by module constructors and
fallbacks.  These run on whatever device their inputs live on; they are
host-side plumbing, not the kernel path."""
import torch


def two_compl(x, bits: int):
    """x < 0 -> 2**bits + x (quantization.py:5-6)."""
    return torch.where(x < 0, 2 ** bits + x, x)


def get_minq_maxq(bits: int, sym: bool):
    """(minq, maxq): sym -> (-(2^(b-1)), 2^(b-1)-1); asym -> (0, 2^b-1)
    (quantization.py:8-16)."""
    if sym:
        maxq = torch.tensor(2 ** (bits - 1) - 1)
        minq = -maxq - 1
    else:
        maxq = torch.tensor(2 ** bits - 1)
        minq = torch.tensor(0)
    return minq, maxq


def asym_quant(x, scale, zero, maxq):
    scale = scale.to(x.device)
    zero = zero.to(x.device)
    q = torch.clamp(torch.round(x / scale) + zero, 0, maxq)
    return q, scale, zero


def asym_dequant(q, scale, zero):
    return scale * (q - zero)


def asym_quant_dequant(x, scale, zero, maxq):
    return asym_dequant(*asym_quant(x, scale, zero, maxq))


def sym_quant(x, scale, maxq, minq=None):
    scale = scale.to(x.device)
    if minq is None:
        minq = -(maxq + 1)
    q = torch.clamp(torch.round(x / scale), minq, maxq)
    return q, scale


def sym_dequant(q, scale):
    return scale * q


def sym_quant_dequant(x, scale, maxq, minq=None):
    return sym_dequant(*sym_quant(x, scale, maxq, minq=minq))


def pack_i4(q):
    """Signed int tensor [..., K] in [-8, 7] -> uint8 [..., K/2], element 2j in
    the low nibble (quantization.py:45-52).  Raises AssertionError when a
    value is out of range, as the reference does."""
    assert torch.is_signed(q), "The tensor to be packed should be signed int"
    assert bool(torch.all((q >= -8) & (q <= 7))), "int4 values must lie in [-8, 7]"
    u = (q.to(torch.int16) & 0xF).to(torch.uint8)
    return u[..., 0::2] | (u[..., 1::2] << 4)


def unpack_i4(x: torch.Tensor, dtype=torch.int32):
    """uint8 [..., K/2] -> sign-extended ints [..., K] (quantization.py:55-77)."""
    assert x.dtype == torch.uint8, "The tensor to be unpacked should be stored in uint8"
    lo = (x & 0x0F).to(torch.int16)
    hi = (x >> 4).to(torch.int16)
    lo = torch.where(lo >= 8, lo - 16, lo)
    hi = torch.where(hi >= 8, hi - 16, hi)
    return torch.stack((lo, hi), dim=-1).reshape(*x.shape[:-1], x.shape[-1] * 2).to(dtype)


def unpack_ui4(x: torch.Tensor):
    """uint8 [..., K/2] -> unsigned ints [..., K] (quantization.py:80-101)."""
    assert x.dtype == torch.uint8, "The tensor to be unpacked should be stored in uint8"
    lo = (x & 0x0F).to(torch.int32)
    hi = (x >> 4).to(torch.int32)
    return torch.stack((lo, hi), dim=-1).reshape(*x.shape[:-1], x.shape[-1] * 2)


def rtn_weight_pack(w: torch.Tensor, symmetric_grid: bool = False):
    """Per-output-channel symmetric int4 RTN of an fp16 weight [N, K] and its
    kernel form (fake_quant/quant_utils.py:453-529 WeightQuantizer
    find_params/quantize, then nn/linear.py:52-73 Linear4bit.from_float):
      s = max(|min(W, 0)|, max(W, 0)).clamp(1e-5) / 7      (fp32)
      W_fq = fp16(clamp(round(W / s), qmin, 7) * s)         qmin = -8, or -7 on
                                                            the symmetric grid
      codes = round(W_fq / fp16(s)) in fp16, packed; scale = fp16(s).
    Returns (packed u8 [N, K/2], scale f16 [N], W_fq f16 [N, K])."""
    wf = w.float()
    xmax = torch.maximum(wf.min(1)[0].clamp(max=0).abs(), wf.max(1)[0].clamp(min=0))
    s = (xmax.clamp(min=1e-5) / 7).unsqueeze(1)
    wfq = (torch.clamp(torch.round(wf / s), -7 if symmetric_grid else -8, 7) * s).half()
    s16 = s.half()
    codes = (wfq / s16).round().to(torch.int8)
    return pack_i4(codes).contiguous(), s16.view(-1).contiguous(), wfq
