"""Oracle for the int4 quantizers, packing, GEMM and dequant -- test
infrastructure only.

Each function restates one reference routine; fp32 steps use numpy float32
(IEEE-754 single, round-to-nearest-even) and fp16 steps numpy float16 (RNE),
so every rounding point of the reference appears explicitly.
"""
import numpy as np

F16 = np.float16
F32 = np.float32


def half2int_rn(h):
    """__half2int_rn: round half to even; NaN -> 0; ±inf saturate (they are
    clamped to the int4 range right after, so only the sign matters)."""
    v = np.asarray(h, dtype=np.float32)
    r = np.rint(v)
    r = np.where(np.isnan(r), 0.0, r)
    r = np.clip(r, -2.0 ** 31, 2.0 ** 31 - 1)
    return r.astype(np.int64)


def sym_scale(x_f16, clip_ratio=1.0):
    """Per-row scale of sym_quant_dynamic_kernel (signrot/kernels/fused.cu:
    80-95): amax = max|x| (exact), scale = fp16(amax / 7.f); if clip != 1,
    scale = fp16(float(scale) * clip).  The reduction is fmaxf from 0.f
    (fused.cu:83-88, 17-21): NaN values are skipped, so an all-NaN row has
    amax 0 and scale 0, and an inf makes the scale inf."""
    x = np.asarray(x_f16, dtype=F16)
    amax = np.fmax.reduce(np.abs(x.astype(F32)), axis=-1, initial=F32(0.0))
    with np.errstate(over="ignore"):
        scale = (amax.astype(F32) / F32(7.0)).astype(F16)
    if clip_ratio != 1.0:
        scale = (scale.astype(F32) * F32(clip_ratio)).astype(F16)
    return scale


def sym_codes(x_f16, scale_f16, qmin=-8, qmax=7):
    """q = clamp(__half2int_rn(__hdiv(x, scale)), -8, 7) (fused.cu:102-104,
    quant.cu:38-40).  __hdiv is taken as the correctly rounded fp16 quotient,
    computed as fp16(fp32(x) / fp32(s)): fp32 division is correctly rounded
    and the second rounding to fp16 is innocuous (24 >= 2*11 + 2)."""
    x = np.asarray(x_f16, dtype=F16).astype(F32)
    s = np.asarray(scale_f16, dtype=F16).astype(F32)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        quot = (x / s).astype(F16)
    return np.clip(half2int_rn(quot), qmin, qmax).astype(np.int8)


def pack_i4(q):
    """pack_i4 (signrot/functional/quantization.py:45-52) and the kernels'
    Int4Subbyte packing (int4.h): two's-complement nibbles, column 2j in the
    low nibble and 2j+1 in the high nibble; an odd last column leaves the
    high nibble 0 (fused.cu:97-110 zero-fills the storage)."""
    q = np.asarray(q, dtype=np.int64)
    cols = q.shape[-1]
    if cols % 2:
        q = np.concatenate([q, np.zeros(q.shape[:-1] + (1,), np.int64)], axis=-1)
    u = (q & 0xF).astype(np.uint8)
    return (u[..., 0::2] | (u[..., 1::2] << 4)).astype(np.uint8)


def unpack_i4(p):
    """unpack_i4 (quantization.py:55-77): sign-extend both nibbles and
    interleave low, high."""
    p = np.asarray(p, dtype=np.uint8)
    lo = (p & 0xF).astype(np.int64)
    hi = (p >> 4).astype(np.int64)
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), np.int64)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


def sym_quant_dynamic(x_f16, clip_ratio=1.0):
    """_CUDA.sym_quant_dynamic (bindings.cpp:316-335, fused.cu:68-112):
    returns (packed u8 [rows, ceil(cols/2)], scale f16 [rows, 1])."""
    scale = sym_scale(x_f16, clip_ratio)
    q = sym_codes(x_f16, scale)
    return pack_i4(q), scale[..., None]


def sym_quant(x_f16, scale_f16):
    """_CUDA.sym_quant (bindings.cpp:208-225, quant.cu:13-47): given scale."""
    return pack_i4(sym_codes(x_f16, np.asarray(scale_f16, F16).reshape(-1)))


def matmul_s4s4(a_u8, b_u8):
    """_CUDA.matmul (bindings.cpp:13-29 -> gemm.cu:7-45): C = A · Bᵀ over the
    unpacked int4 codes, int32.  Evaluated as a float64 matmul, which is exact
    here: every partial sum is an integer below 2^53."""
    a = unpack_i4(a_u8).astype(np.float64)
    b = unpack_i4(b_u8).astype(np.float64)
    c = a @ b.T
    return c.astype(np.int64).astype(np.int32)


def sym_dequant(c_i32, scale_row_f16, scale_col_f16):
    """sym_dequant_i32_f16_kernel (quant.cu:66-87):
    out = __float2half_rn(((float)q * float(s_row)) * float(s_col))."""
    c = np.asarray(c_i32).astype(F32)
    r = np.asarray(scale_row_f16, F16).reshape(-1).astype(F32)[:, None]
    s = np.asarray(scale_col_f16, F16).reshape(-1).astype(F32)[None, :]
    return ((c * r) * s).astype(F16)


def add_bias(out_f16, bias_f16):
    """`sym_dequant(...) + self.bias` (signrot/nn/linear.py:47-48): fp16 + fp16
    in torch, i.e. an fp32 add rounded to fp16."""
    return (np.asarray(out_f16, F16).astype(F32) + np.asarray(bias_f16, F16).astype(F32)).astype(F16)


def w4a4_linear(a_u8, a_scale_f16, b_u8, b_scale_f16, bias_f16=None):
    """Linear4bit.forward on a PackedQuantizedTensor (nn/linear.py:30-50):
    matmul_si4_si4 then sym_dequant (then + bias)."""
    out = sym_dequant(matmul_s4s4(a_u8, b_u8), a_scale_f16, b_scale_f16)
    if bias_f16 is not None:
        out = add_bias(out, bias_f16)
    return out


def kv_quant_pack(x_f16):
    """kv_quant_pack_kernel (fused.cu:213-266), the fused form of the
    torch.jit asym_quantize_and_pack_i4 (kv_cache.py:12-58, lac=False):
      hmin, hmax exact; diff = fp16(hmax - hmin); diff = fp16(max(diff, 1e-5));
      scale = fp16(diff / 15); zero = -hmin;
      q = clamp(rne(fp16(fp16(x + zero) / scale)), 0, 15), packed low-first.
    The row max / min are fmaxf / fminf from -FLT_MAX / FLT_MAX
    (fused.cu:236-245, 17-28): NaN values are skipped (an all-NaN row gives
    hmax = fp16(-FLT_MAX) = -inf, hmin = +inf), the 1e-5 clamp is fmaxf too
    (a NaN difference becomes 1e-5), and a NaN quotient gives code 0.
    Returns (u8 [..., D/2], f16 param [..., 2] = [scale, zero])."""
    x = np.asarray(x_f16, dtype=F16)
    xf = x.astype(F32)
    fmax32 = np.finfo(F32).max
    with np.errstate(over="ignore", invalid="ignore"):
        hmax = np.fmax.reduce(xf, axis=-1, keepdims=True, initial=-fmax32).astype(F16)
        hmin = np.fmin.reduce(xf, axis=-1, keepdims=True, initial=fmax32).astype(F16)
        diff = (hmax.astype(F32) - hmin.astype(F32)).astype(F16).astype(F32)
        diff = np.fmax(diff, F32(1e-5)).astype(F16).astype(F32)
        scale = (diff / F32(15.0)).astype(F16)
    zero = -hmin
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        shifted = (xf + zero.astype(F32)).astype(F16).astype(F32)
        scaled = (shifted / scale.astype(F32)).astype(F16)
    q = np.clip(half2int_rn(scaled), 0, 15).astype(np.uint8)
    packed = (q[..., 0::2] | (q[..., 1::2] << 4)).astype(np.uint8)
    param = np.concatenate([scale, zero], axis=-1)
    return packed, param


def kv_unpack(p_u8):
    """uint4 unpack (kv_cache.py:60-63): low nibble first, no sign extension."""
    p = np.asarray(p_u8, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), np.int64)
    out[..., 0::2] = p & 0xF
    out[..., 1::2] = p >> 4
    return out


def kv_dequant(p_u8, param_f16):
    """Dequant inside the decode kernel (flashinfer quantization.cuh:59-84):
    x̂ = float(q) * scale - zero, in fp32."""
    q = kv_unpack(p_u8).astype(F32)
    prm = np.asarray(param_f16, F16).astype(F32)
    return q * prm[..., 0:1] - prm[..., 1:2]


def rtn_weight(w_f16, bits=4, symmetric_grid=False):
    """Per-output-channel symmetric RTN for the config weights
    (fake_quant/quant_utils.py:453-529 WeightQuantizer.find_params/quantize,
    gptq_utils.py:412-465 rtn_fwrd, nn/linear.py:52-73 Linear4bit.from_float):
      xmin = min(row, 0), xmax = max(row, 0)   (extend_zero, fp32)
      s = max(|xmin|, xmax).clamp(1e-5) / maxq   (fp32, maxq = 7)
      W_fq = fp16(clamp(round(W / s), -8, 7) * s)
      kernel scale = fp16(s); codes = round(W_fq / fp16(s)) in fp16.
    symmetric_grid=True uses [-7, 7] (quant_utils.py:445-448, set by rtn_fwrd
    when a sign vector is folded, gptq_utils.py:444-452).
    Returns (codes int8 [N, K], scale f16 [N, 1], W_fq f16 [N, K])."""
    maxq = F32(2 ** (bits - 1) - 1)
    minq = -maxq if symmetric_grid else -(maxq + 1)
    w = np.asarray(w_f16, dtype=F16).astype(F32)
    xmin = np.minimum(w.min(axis=1), F32(0))
    xmax = np.maximum(w.max(axis=1), F32(0))
    s = np.maximum(np.maximum(np.abs(xmin), xmax), F32(1e-5)) / maxq
    s = s.astype(F32)[:, None]
    q = np.clip(np.rint(w / s), minq, maxq)
    w_fq = (q * s).astype(F16)
    s16 = s.astype(F16)
    codes = np.rint((w_fq.astype(F32) / s16.astype(F32)).astype(F16).astype(F32))
    codes = np.clip(codes, -8, 7).astype(np.int8)
    return codes, s16, w_fq


# ------------------------------------------------- asymmetric activations

def wrap_i32(v):
    """Two's-complement int32 wrap of an integer array (the reference's int
    additions overflow this way on the GPU)."""
    v = np.asarray(v, np.int64)
    return ((v + 2 ** 31) % 2 ** 32) - 2 ** 31


def asym_params(x_f16, clip_ratio=1.0):
    """Per-row scale and zero of asym_quant_dynamic_kernel
    (signrot/kernels/fused.cu:155-179): vmin, vmax exact; hmin = fp16(vmin),
    hmax = fp16(vmax); if clip != 1 each is fp16(float(h) * clip);
    diff = fp16(hmax - hmin); scale = fp16(diff / 15.f);
    ratio = fp16(-hmin / scale) (fp32 division); zero = fp16(nearbyint(ratio))
    (round half to even).  The reductions are fminf / fmaxf from ±FLT_MAX
    (fused.cu:155-163): NaN values are skipped, an all-NaN row gives
    hmin = +inf, hmax = -inf.  Returns (scale f16 [rows], zero f16 [rows])."""
    x = np.asarray(x_f16, dtype=F16).astype(F32)
    fmax32 = np.finfo(F32).max
    with np.errstate(over="ignore"):  # ±FLT_MAX -> ±inf in fp16, as __float2half
        hmin = np.fmin.reduce(x, axis=-1, initial=fmax32).astype(F16)
        hmax = np.fmax.reduce(x, axis=-1, initial=-fmax32).astype(F16)
    if clip_ratio != 1.0:
        hmin = (hmin.astype(F32) * F32(clip_ratio)).astype(F16)
        hmax = (hmax.astype(F32) * F32(clip_ratio)).astype(F16)
    diff = (hmax.astype(F32) - hmin.astype(F32)).astype(F16)
    scale = (diff.astype(F32) / F32(15.0)).astype(F16)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        ratio = (-hmin.astype(F32) / scale.astype(F32)).astype(F16)
    zero = np.rint(ratio.astype(F32)).astype(F16)
    return scale, zero


def asym_codes(x_f16, scale_f16, zero_f16, qmin=0, qmax=15):
    """q = clamp(__half2int_rn(__hdiv(x, scale)) + __half2int_rn(zero), qmin,
    qmax) (fused.cu:183-193; quant.cu:156-158, 201-203), the int addition
    in int32 (wrapping: ±inf quotients saturate to INT_MAX / INT_MIN)."""
    x = np.asarray(x_f16, dtype=F16).astype(F32)
    s = np.asarray(scale_f16, dtype=F16).reshape(-1).astype(F32)[:, None]
    z = half2int_rn(np.asarray(zero_f16, dtype=F16).reshape(-1))[:, None]
    with np.errstate(divide="ignore", invalid="ignore"):
        quot = (x / s).astype(F16)
    return np.clip(wrap_i32(half2int_rn(quot) + z), qmin, qmax).astype(np.int64)


def pack_u4(q):
    """UInt4Subbyte packing: unsigned nibbles, column 2j low, 2j+1 high (an
    odd last column leaves the high nibble 0)."""
    return pack_i4(np.asarray(q, np.int64) & 0xF)


def unpack_u4(p):
    """The unsigned nibbles of a packed u8 tensor, low then high."""
    p = np.asarray(p, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), np.int64)
    out[..., 0::2] = p & 0xF
    out[..., 1::2] = p >> 4
    return out


def asym_quant_dynamic(x_f16, clip_ratio=1.0):
    """_CUDA.asym_quant_dynamic (bindings.cpp:337-358, fused.cu:143-195):
    returns (packed u8 [rows, ceil(cols/2)] of uint4 codes, scale f16
    [rows, 1], zero f16 [rows, 1])."""
    scale, zero = asym_params(x_f16, clip_ratio)
    q = asym_codes(x_f16, scale, zero)
    return pack_u4(q), scale[:, None], zero[:, None]


def asym_quant_f16_ui4(x_f16, scale_f16, zero_f16):
    """_CUDA.asym_quant_f16_ui4 (quant.cu:182-207): uint4 codes for a given
    per-row scale and zero."""
    return pack_u4(asym_codes(x_f16, scale_f16, zero_f16, 0, 15))


def asym_quant_f16_si4(x_f16, scale_f16, zero_f16):
    """_CUDA.asym_quant_f16_si4 (quant.cu:133-162): the same arithmetic
    clamped to [-8, 7], two's-complement nibbles."""
    return pack_i4(asym_codes(x_f16, scale_f16, zero_f16, -8, 7))


def sum_i4(x_u8, is_signed=True):
    """_CUDA.sum_i4 (bindings.cpp:437-451, quant.cu:233-321): per row, the
    sum of both nibbles of every byte, sign-extended when is_signed.
    int32 [rows, 1]."""
    v = unpack_i4(x_u8) if is_signed else unpack_u4(x_u8)
    return wrap_i32(v.sum(axis=-1))[:, None].astype(np.int32)


def matmul_colrow_i8_i32(a_col_i8, b_row_i32):
    """_CUDA.matmul_colrow_i8_i32 (bindings.cpp:453-477, quant.cu:341-383):
    out[r, c] = int32(a[r]) * b[c] (int32, wrapping)."""
    a = np.asarray(a_col_i8, np.int64).reshape(-1, 1)
    b = np.asarray(b_row_i32, np.int64).reshape(1, -1)
    return wrap_i32(a * b).astype(np.int32)


def matmul_u4s4(a_u8, b_u8):
    """_CUDA.matmul_ui4_si4 (bindings.cpp:31-47 -> gemm.cu:47-85): C = A · Bᵀ
    with A's nibbles unsigned (0..15) and B's two's complement, int32 (a
    float64 matmul, exact: every partial sum is an integer below 2^53)."""
    a = unpack_u4(a_u8).astype(np.float64)
    b = unpack_i4(b_u8).astype(np.float64)
    return wrap_i32((a @ b.T).astype(np.int64)).astype(np.int32)


def w4a4_linear_asym(a_u8, a_scale_f16, a_zero_i8, b_u8, b_scale_f16, bias_f16=None):
    """Linear4bit.forward on an asymmetric PackedQuantizedTensor
    (nn/linear.py:35-50): x = matmul_ui4_si4(A, W); x -= matmul_colrow_i8_i32(
    zeros_x, sum_i4(W)ᵀ) (int32); sym_dequant(x, scales_x, weight_scales)
    (+ bias)."""
    c = matmul_u4s4(a_u8, b_u8).astype(np.int64)
    ws = sum_i4(b_u8).reshape(-1)
    c = wrap_i32(c - matmul_colrow_i8_i32(a_zero_i8, ws).astype(np.int64))
    out = sym_dequant(c, a_scale_f16, b_scale_f16)
    if bias_f16 is not None:
        out = add_bias(out, bias_f16)
    return out
