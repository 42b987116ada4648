"""Oracle for the decode-layer glue (RMSNorm, RoPE, SwiGLU) -- test
infrastructure only.

Restates signrot/kernels/fused.cu:278-390 (rmsnorm_kernel, rope_qk_kernel,
swiglu_kernel) and signrot/nn/normalization.py:19-30.
"""
import numpy as np

F16 = np.float16
F32 = np.float32


def rmsnorm(x_f16, eps, mean_dim):
    """fused.cu:279-302: inv = rsqrt(sum(x^2) / mean_dim + eps) with an fp32
    sum, out = fp16(x * inv).  Computed in float64 (the reference's fp32
    accumulation order is not fixed), so the kernel is compared within an
    fp16 ulp of this value."""
    x = np.asarray(x_f16, F16).astype(np.float64)
    var = (x * x).sum(axis=-1, keepdims=True) / float(mean_dim)
    inv = 1.0 / np.sqrt(var + float(eps))
    return (x * inv).astype(F16)


def rope_qk(q_f16, k_f16, cos_f16, sin_f16):
    """fused.cu:316-350 = HF apply_rotary_pos_emb(unsqueeze_dim=2) in fp16:
    x' = fp16(fp16(x * cos) + fp16(rotate_half(x) * sin)), each op rounded to
    fp16 (a product of two fp16 values is exact in fp32, and an fp32 sum of
    two fp16 values rounds to fp16 as the exact sum would).
    q [B, T, Hq, D], k [B, T, Hk, D], cos/sin [B or 1, T, D]; returns new
    arrays."""
    c = np.asarray(cos_f16, F16).astype(F32)[:, :, None, :]
    s = np.asarray(sin_f16, F16).astype(F32)[:, :, None, :]

    def apply(x):
        x = np.asarray(x, F16).astype(F32)
        half = x.shape[-1] // 2
        rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
        a = (x * c).astype(F16).astype(F32)
        b = (rot * s).astype(F16).astype(F32)
        return (a + b).astype(F16)

    return apply(q_f16), apply(k_f16)


def swiglu(gate_f16, up_f16):
    """fused.cu:367-383: fp16(fp16(g / (1 + exp(-g))) * up); silu in float64
    here (the device expf is within an ulp of it), the product of two fp16
    values exact in fp32 and rounded once."""
    g = np.asarray(gate_f16, F16).astype(np.float64)
    with np.errstate(over="ignore"):
        silu = (g / (1.0 + np.exp(-g))).astype(F16)
    return (silu.astype(F32) * np.asarray(up_f16, F16).astype(F32)).astype(F16)
