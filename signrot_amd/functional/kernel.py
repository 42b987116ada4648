"""Python wrappers over the HIP op table, mirroring
signrot/functional/kernel.py:15-227 (flatten / view handling, the
PackedQuantizedTensor carrier, dtype asserts)."""
import torch

from .. import _CUDA

__all__ = [
    "matmul_si4_si4",
    "sym_quant",
    "sym_quant_dynamic",
    "sym_dequant",
    "kv_quant_pack",
    "w4a4_linear",
    "had_sign_quant",
    "rope_qk",
    "swiglu",
    "rmsnorm",
    "matmul_grouped",
    "sym_quant_dynamic_moe",
    "asym_quant_dynamic_moe",
    "sym_dequant_moe",
    "w4a4_linear_moe",
    "matmul_ui4_si4",
    "asym_quant_dynamic",
    "asym_quant_f16_si4",
    "asym_quant_f16_ui4",
    "sum_i4",
    "matmul_colrow_i8_i32",
    "w4a4_linear_asym",
    "w4a4_linear_moe_asym",
    "PackedQuantizedTensor",
]


class ShapeHandler:
    def __init__(self, x: torch.Tensor):
        self.size_excl_last = x.numel() // x.shape[-1]
        self.shape_excl_last = tuple(x.shape[:-1])

    def flatten(self, x: torch.Tensor):
        return x.view(self.size_excl_last, -1)

    def unflatten(self, x: torch.Tensor):
        return x.view(self.shape_excl_last + (-1,))

    def unflatten_scale(self, x: torch.Tensor):
        return x.view(self.shape_excl_last)


class PackedQuantizedTensor:
    """Quantized-activation carrier (kernel.py:32-52): packed int4 codes
    [..., K/2] u8, per-token fp16 scales [..., 1], zeros (asym only)."""

    def __init__(self, quantized_x: torch.Tensor, scales_x: torch.Tensor,
                 zeros_x: torch.Tensor | None = None):
        self.quantized_x = quantized_x
        self.scales_x = scales_x
        self.zeros_x = zeros_x

    def size(self):
        return self.quantized_x.size()

    @property
    def device(self):
        return self.quantized_x.device

    @property
    def dtype(self):
        return self.quantized_x.dtype


def flatten_last_dim_and_return_shape(x: torch.Tensor):
    shape_excl_last = x.shape[:-1]
    x = x.view(-1, x.shape[-1])
    return x, shape_excl_last


def flatten_last_two_dim_and_return_shape(x: torch.Tensor):
    shape_excl_last_two, shape_last_two = x.shape[:-2], x.shape[-2:]
    x = x.view(-1, x.shape[-2], x.shape[-1])
    return x, shape_excl_last_two, shape_last_two


def matmul_si4_si4(A, B):
    """int4 x int4 -> int32 over the last dim (kernel.py:67-73)."""
    assert A.shape[-1] % 32 == 0, "A.shape[-1]: {} must be multiplication of 32".format(
        A.shape[-1])
    A, A_shape_excl_last = flatten_last_dim_and_return_shape(A)
    B, B_shape_excl_last = flatten_last_dim_and_return_shape(B)
    return _CUDA.matmul(A, B).view(*A_shape_excl_last, *B_shape_excl_last)


def w4a4_linear(A, a_scale, B, b_scale, bias=None):
    """Fused matmul_si4_si4 + sym_dequant (+ bias): fp16 [..., N]."""
    A, A_shape_excl_last = flatten_last_dim_and_return_shape(A)
    out = _CUDA.w4a4_linear(A, a_scale.reshape(-1), B, b_scale.reshape(-1),
                            None if bias is None else bias.reshape(-1))
    return out.view(*A_shape_excl_last, B.shape[0])


def matmul_ui4_si4(A, B):
    """uint4 x int4 -> int32 over the last dim (kernel.py:75-81)."""
    assert A.shape[-1] % 32 == 0, "A.shape[-1]: {} must be multiplication of 32".format(
        A.shape[-1])
    A, A_shape_excl_last = flatten_last_dim_and_return_shape(A)
    B, B_shape_excl_last = flatten_last_dim_and_return_shape(B)
    return _CUDA.matmul_ui4_si4(A, B).view(*A_shape_excl_last, *B_shape_excl_last)


def w4a4_linear_asym(A, a_scale, a_zero, B, b_scale, b_sum, bias=None):
    """Fused matmul_ui4_si4 - zeros ⊗ weight_sum + sym_dequant (+ bias):
    fp16 [..., N] (the zeros_x branch of Linear4bit.forward in one launch)."""
    A, A_shape_excl_last = flatten_last_dim_and_return_shape(A)
    out = _CUDA.w4a4_linear_asym(A, a_scale.reshape(-1), a_zero.reshape(-1), B,
                                 b_scale.reshape(-1), b_sum.reshape(-1),
                                 None if bias is None else bias.reshape(-1))
    return out.view(*A_shape_excl_last, B.shape[0])


def asym_quant_dynamic(x, clip_ratio=1.0):
    """Fused per-row amin/amax + scale/zero + asymmetric uint4 quantize/pack
    (kernel.py:113-120): (q, scale, zero), scale and zero shaped
    (*x.shape[:-1], 1)."""
    assert x.dtype == torch.float16
    x, shape_excl_last = flatten_last_dim_and_return_shape(x.contiguous())
    q, scale, zero = _CUDA.asym_quant_dynamic(x, clip_ratio)
    return (q.view(*shape_excl_last, -1), scale.view(*shape_excl_last, 1),
            zero.view(*shape_excl_last, 1))


def asym_quant_f16_si4(q, scale, zero):
    """(kernel.py:188-194)"""
    assert q.dtype == torch.float16
    assert scale.dtype == zero.dtype == torch.float16
    q, q_shape_excl_last = flatten_last_dim_and_return_shape(q)
    return _CUDA.asym_quant_f16_si4(q, scale.reshape(-1), zero.reshape(-1)).view(
        *q_shape_excl_last, -1)


def asym_quant_f16_ui4(q, scale, zero):
    """(kernel.py:197-203)"""
    assert q.dtype == torch.float16
    assert scale.dtype == zero.dtype == torch.float16
    q, q_shape_excl_last = flatten_last_dim_and_return_shape(q)
    return _CUDA.asym_quant_f16_ui4(q, scale.reshape(-1), zero.reshape(-1)).view(
        *q_shape_excl_last, -1)


def sum_i4(x, is_signed=True, dtype=torch.int32):
    """(kernel.py:206-212)"""
    assert x.dtype == torch.uint8, "packed int4 tensor must be torch.uint8"
    x, x_shape_excl_last = flatten_last_dim_and_return_shape(x)
    out = _CUDA.sum_i4(x, is_signed).view(*x_shape_excl_last, 1)
    if dtype is not None and out.dtype != dtype:
        out = out.to(dtype=dtype)
    return out


def matmul_colrow_i8_i32(a_col, b_row):
    """(kernel.py:215-227)"""
    assert a_col.dtype == torch.int8, "a_col must be torch.int8"
    assert b_row.dtype == torch.int32, "b_row must be torch.int32"
    a_col, a_shape_excl_last = flatten_last_dim_and_return_shape(a_col)
    assert a_col.shape[1] == 1, "a_col must have last dimension == 1"
    if b_row.dim() == 1:
        b_row = b_row.view(1, -1)
    assert b_row.dim() == 2 and b_row.shape[0] == 1, "b_row must have shape [1, C]"
    out = _CUDA.matmul_colrow_i8_i32(a_col.contiguous(), b_row.contiguous())
    return out.view(*a_shape_excl_last, b_row.shape[1])


def sym_quant(x, scale):
    assert x.dtype == scale.dtype == torch.float16
    x, x_shape_excl_last = flatten_last_dim_and_return_shape(x)
    return _CUDA.sym_quant(x, scale.view(-1)).view(*x_shape_excl_last, -1)


def sym_quant_dynamic(x, clip_ratio=1.0):
    """Fused per-row amax + scale + symmetric int4 quantize/pack
    (kernel.py:101-110).  Returns (packed_q, scale) with scale shaped
    (*x.shape[:-1], 1)."""
    assert x.dtype == torch.float16
    x, shape_excl_last = flatten_last_dim_and_return_shape(x.contiguous())
    q, scale = _CUDA.sym_quant_dynamic(x, clip_ratio)
    return q.view(*shape_excl_last, -1), scale.view(*shape_excl_last, 1)


def had_sign_quant(x, hadK, K, sign=None, clip_ratio=1.0, fp32_had=False):
    """Fused OnlineHadamard -> sign -> sym_quant_dynamic (one launch)."""
    assert x.dtype == torch.float16
    x, shape_excl_last = flatten_last_dim_and_return_shape(x.contiguous())
    q, scale = _CUDA.had_sign_quant(x, hadK, K, sign, clip_ratio, fp32_had)
    return q.view(*shape_excl_last, -1), scale.view(*shape_excl_last, 1)


def kv_quant_pack(x):
    """Fused KV-cache asymmetric uint4 quantize + pack (kernel.py:148-155):
    (packed_q, param) with param[..., 0] the scale and param[..., 1] the zero."""
    assert x.dtype == torch.float16
    return _CUDA.kv_quant_pack(x.contiguous())


def rope_qk(q, k, cos, sin):
    """In-place rotary embedding of q [B, T, Hq, D] and k [B, T, Hk, D], as
    HF apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=2) with per-op fp16
    rounding (signrot/functional/kernel.py:158-165)."""
    _CUDA.rope_qk(q, k, cos.contiguous(), sin.contiguous())
    return q, k


def swiglu(gate, up):
    """silu(gate) * up in one launch (signrot/functional/kernel.py:168-170)."""
    return _CUDA.swiglu(gate.contiguous(), up.contiguous())


def rmsnorm(x, eps, mean_dim):
    """RMSNorm over the last dim, fp32 sum, fp16 in/out
    (signrot/functional/kernel.py:173-176)."""
    assert x.dtype == torch.float16
    return _CUDA.rmsnorm(x.contiguous(), eps, mean_dim)


def sym_dequant(q, scale_row, scale_col, bits=32):
    """(kernel.py:179-185)"""
    assert q.dtype == torch.int32
    assert scale_row.dtype == scale_col.dtype == torch.float16
    q, q_shape_excl_last = flatten_last_dim_and_return_shape(q)
    return _CUDA.sym_dequant(q, scale_row.view(-1), scale_col.view(-1), bits).view(
        *q_shape_excl_last, -1)


def matmul_grouped(problem_sizes, ptr_a, ptr_b, ptr_c, lda, ldb, ldc, signed_a=True):
    """Grouped 4-bit GEMM, C_i = A_i @ B_i^T per problem in one launch
    (signrot/functional/kernel.py:83-92).  All arguments are device tensors:
    problem_sizes int32 [P, 3] rows (m, n, k), the rest int64 [P] device
    addresses / leading dims; per-element output identical to matmul_si4_si4
    on each problem; nothing is read on the host (graph-capturable)."""
    _CUDA.matmul_grouped(problem_sizes, ptr_a, ptr_b, ptr_c, lda, ldb, ldc, signed_a)


def sym_quant_dynamic_moe(x, sign, expert_ids, clip_ratio=1.0):
    """sym_quant_dynamic over expert-sorted rows with the per-expert had_adj
    sign fused: row r is multiplied by sign[expert_ids[r]] (exact for +-1)
    before quantization; sign may be None (kernel.py:123-128)."""
    assert x.dtype == torch.float16
    return _CUDA.sym_quant_dynamic_moe(x.contiguous(), sign, expert_ids, clip_ratio)


def asym_quant_dynamic_moe(x, sign, expert_ids, clip_ratio=1.0):
    """asym_quant_dynamic variant of sym_quant_dynamic_moe -> (q, scale,
    zero) (kernel.py:131-134)."""
    assert x.dtype == torch.float16
    return _CUDA.asym_quant_dynamic_moe(x.contiguous(), sign, expert_ids, clip_ratio)


def sym_dequant_moe(q, scale_row, w_scales, expert_ids, zero_row=None, w_sum=None):
    """Expert-indexed dequant with the asym zero correction fused in
    (kernel.py:137-145): out[r, c] = (q[r, c] - zero_row[r] * w_sum[e, c]) *
    scale_row[r] * w_scales[e, c], e = expert_ids[r]."""
    assert q.dtype == torch.int32
    return _CUDA.sym_dequant_moe(q, scale_row.contiguous(), w_scales, expert_ids, zero_row,
                                 w_sum)


def w4a4_linear_moe(A, a_scale, B, b_scale, expert_offsets):
    """Fused grouped int4 GEMM + expert-indexed dequant over expert-sorted
    rows (one launch; bit-identical to matmul_grouped + sym_dequant_moe)."""
    return _CUDA.w4a4_linear_moe(A, a_scale.reshape(-1), B, b_scale, expert_offsets)


def w4a4_linear_moe_asym(A, a_scale, a_zero, B, b_scale, b_sum, expert_offsets):
    """w4a4_linear_moe for asymmetric activation codes (one launch;
    bit-identical to matmul_grouped(signed_a=False) + sym_dequant_moe with
    zero_row and w_sum)."""
    return _CUDA.w4a4_linear_moe_asym(A, a_scale.reshape(-1), a_zero.reshape(-1), B, b_scale,
                                      b_sum, expert_offsets)
