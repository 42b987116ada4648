"""Oracle for the MoE kernels (expert-indexed quantizer and dequant, grouped
GEMM) -- test infrastructure only.

Restates signrot/kernels/moe.cu:60-101 (sym_quant_dynamic_moe_kernel),
202-226 (sym_dequant_moe_kernel) and the grouped GEMM contract of
signrot/kernels/gemm_grouped.cu:54-107 (per problem, the dense int4 GEMM of
gemm.cu:7-45), plus the expert-sorted row bookkeeping of
signrot/nn/moe.py:161-236.
"""
import numpy as np

from . import quant as oq

F16 = np.float16
F32 = np.float32


def apply_sign(x_f16, sign_i8, expert_ids):
    """signed_load (moe.cu:51-56): row r times sign[expert_ids[r]]; an fp16
    times ±1 is exact (a flip of the sign bit).  sign None -> x."""
    x = np.asarray(x_f16, F16)
    if sign_i8 is None:
        return x.copy()
    s = np.asarray(sign_i8, np.int8)[np.asarray(expert_ids, np.int64)]
    return np.where(s < 0, -x, x).astype(F16)


def sym_quant_dynamic_moe(x_f16, sign_i8, expert_ids, clip_ratio=1.0):
    """sym_quant_dynamic_moe_kernel (moe.cu:60-101): sym_quant_dynamic of the
    sign-flipped rows.  Returns (packed u8 [rows, ceil(cols/2)], scale f16
    [rows, 1])."""
    return oq.sym_quant_dynamic(apply_sign(x_f16, sign_i8, expert_ids), clip_ratio)


def asym_quant_dynamic_moe(x_f16, sign_i8, expert_ids, clip_ratio=1.0):
    """asym_quant_dynamic_moe_kernel (moe.cu:104-152): asym_quant_dynamic of
    the sign-flipped rows.  Returns (packed uint4 u8, scale f16 [rows, 1],
    zero f16 [rows, 1])."""
    return oq.asym_quant_dynamic(apply_sign(x_f16, sign_i8, expert_ids), clip_ratio)


def sym_dequant_moe(c_i32, scale_row_f16, w_scales_f16, expert_ids, zero_row=None,
                    w_sum=None):
    """sym_dequant_moe_kernel (moe.cu:202-226): qval = q - zero_row[r] *
    w_sum[e, c] in int32 (two's-complement), then
    fp16((float(qval) * float(scale_row[r])) * float(w_scales[e, c]))."""
    e = np.asarray(expert_ids, np.int64)
    q = np.asarray(c_i32, np.int64)
    if zero_row is not None:
        z = np.asarray(zero_row, np.int64)[:, None]
        ws = np.asarray(w_sum, np.int64)[e]
        q = q - z * ws
        q = ((q + 2 ** 31) % 2 ** 32) - 2 ** 31  # int32 wrap
    r = np.asarray(scale_row_f16, F16).reshape(-1).astype(F32)[:, None]
    w = np.asarray(w_scales_f16, F16)[e].astype(F32)
    return ((q.astype(F32) * r) * w).astype(F16)


def matmul_grouped(problems):
    """Grouped GEMM contract (gemm_grouped.cu:54-107): for each (a_u8 [m,
    k/2], b_u8 [n, k/2]) the dense int32 product matmul_s4s4(a, b)."""
    return [oq.matmul_s4s4(a, b) for a, b in problems]


def expert_offsets(counts):
    """Row offsets of expert-sorted rows: [0, c0, c0 + c1, ...] (the
    reference's row_off, moe.py:204-205, with the total appended)."""
    c = np.asarray(counts, np.int64)
    return np.concatenate([[0], np.cumsum(c)]).astype(np.int32)


def w4a4_linear_moe(a_u8, a_scale_f16, b_u8, b_scale_f16, offsets):
    """matmul_grouped + sym_dequant_moe over expert-sorted rows
    (moe.py:126-136): expert e's rows offsets[e] .. offsets[e+1] of A times
    B[e]ᵀ, dequantized with the row scale and w_scales[e]."""
    a = np.asarray(a_u8, np.uint8)
    b = np.asarray(b_u8, np.uint8)
    out = np.zeros((a.shape[0], b.shape[1]), F16)
    for e in range(b.shape[0]):
        r0, r1 = int(offsets[e]), int(offsets[e + 1])
        if r1 <= r0:
            continue
        c = oq.matmul_s4s4(a[r0:r1], b[e])
        out[r0:r1] = oq.sym_dequant(c, np.asarray(a_scale_f16, F16).reshape(-1)[r0:r1],
                                    np.asarray(b_scale_f16, F16)[e])
    return out
