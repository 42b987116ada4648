"""Operator table of the HIP library -- the drop-in for the reference's
pybind11 module `signrot._CUDA` (signrot/kernels/bindings.cpp:785-909) and
for `fast_hadamard_transform.hadamard_transform`.

Same op names, argument order, output shapes/dtypes and error behaviour as
the reference: tensors must be contiguous CUDA(HIP) tensors on one device
with the documented dtypes, otherwise RuntimeError is raised (the
reference's torch::checkAllContiguous / checkDeviceType / TORCH_CHECK raise
c10::Error, which surfaces as RuntimeError).  Outputs are allocated with
torch's caching allocator on the input's device; every launch goes to the
current torch stream of that device, nothing synchronises, so every op is
graph-capturable.

Added ops (no reference counterpart, fused forms of reference chains):
  w4a4_linear     = matmul + sym_dequant (+ bias)            nn/linear.py:45-50
  online_hadamard = matmul_hadU_cuda + sign multiply          nn/hadamard.py:26-42
  had_sign_quant  = online_hadamard + sym_quant_dynamic       modeling_llama.py:134-138
  w4a4_linear_moe = matmul_grouped + sym_dequant_moe          nn/moe.py:126-136
  w4a4_linear_residual  = w4a4_linear + residual add          modeling_llama.py:19-137
  rmsnorm_quant         = rmsnorm + sym_quant_dynamic          fused.cu:68-138, 278-309
  head_had_quant        = head-axis Hadamard + sym_quant_dynamic  modeling_llama.py:94, 117
  swiglu_had_sign_quant = swiglu + had_sign_quant              modeling_llama.py:125-137
  qkv_rope_had_append   = rope_qk + K/q Hadamard + kv_quant_pack + append_kv_i4
                                                              kv_cache.py:144-170, 295-415
  qkv_decode_i4         = qkv_rope_had_append + batch_decode_i4 kv_cache.py:144-170, 295-415
"""
import functools

import torch

from . import _native

_call = _native.call


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _check(name, tensors, dtypes=None, contiguous=True):
    dev = None
    for i, (t, tname) in enumerate(tensors):
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise RuntimeError(f"{name}: argument '{tname}' must be a tensor")
        if t.device.type != "cuda":
            raise RuntimeError(
                f"{name}: expected '{tname}' on a GPU device, got {t.device}")
        if contiguous and not t.is_contiguous():
            raise RuntimeError(f"{name}: expected contiguous tensor for argument '{tname}'")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(
                f"{name}: expected all tensors on the same GPU, but '{tname}' is on {t.device}")
        if dtypes is not None and dtypes[i] is not None and t.dtype != dtypes[i]:
            raise RuntimeError(
                f"{name}: expected {dtypes[i]} for argument '{tname}', got {t.dtype}")


def _ptr(t):
    return None if t is None else t.data_ptr()


# ------------------------------------------------------------------- GEMM

def matmul(A, B):
    """C i32 [M, N] = A · Bᵀ for packed int4 A u8 [M, K/2], B u8 [N, K/2]
    (bindings.cpp:13-29)."""
    _check("matmul", [(A, "A"), (B, "B")], [torch.uint8, torch.uint8])
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[1]:
        raise RuntimeError(f"matmul: expected A [M, K/2] and B [N, K/2], got {tuple(A.shape)} "
                           f"and {tuple(B.shape)}")
    M, N, K = A.shape[0], B.shape[0], A.shape[1] * 2
    C = torch.empty((M, N), dtype=torch.int32, device=A.device)
    _call("srq_matmul_s4s4", _ptr(A), _ptr(B), M, N, K, _ptr(C), _stream(A))
    return C


def matmul_ui4_si4(A, B):
    """C i32 [M, N] = A · Bᵀ with A's codes unsigned (uint4) and B's int4
    (bindings.cpp:31-47)."""
    _check("matmul_ui4_si4", [(A, "A"), (B, "B")], [torch.uint8, torch.uint8])
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[1]:
        raise RuntimeError(f"matmul_ui4_si4: expected A [M, K/2] and B [N, K/2], got "
                           f"{tuple(A.shape)} and {tuple(B.shape)}")
    M, N, K = A.shape[0], B.shape[0], A.shape[1] * 2
    C = torch.empty((M, N), dtype=torch.int32, device=A.device)
    _call("srq_matmul_u4s4", _ptr(A), _ptr(B), M, N, K, _ptr(C), _stream(A))
    return C


def w4a4_linear_asym(A, a_scale, a_zero, B, b_scale, b_sum, bias=None):
    """Fused W4A4 linear for asymmetric activations: (A·Bᵀ - a_zero ⊗ b_sum)
    (int32) -> sym_dequant (+ bias); A uint4 codes [M, K/2], a_zero int8
    [M], b_sum int32 [N] (sum_i4 of B).  The zeros_x branch of
    Linear4bit.forward (linear.py:35-50) in one launch."""
    _check("w4a4_linear_asym", [(A, "A"), (a_scale, "a_scale"), (a_zero, "a_zero"), (B, "B"),
                                (b_scale, "b_scale"), (b_sum, "b_sum"), (bias, "bias")],
           [torch.uint8, torch.float16, torch.int8, torch.uint8, torch.float16, torch.int32,
            torch.float16])
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[1]:
        raise RuntimeError(f"w4a4_linear_asym: expected A [M, K/2] and B [N, K/2], got "
                           f"{tuple(A.shape)} and {tuple(B.shape)}")
    M, N, K = A.shape[0], B.shape[0], A.shape[1] * 2
    if a_scale.numel() != M or a_zero.numel() != M:
        raise RuntimeError("w4a4_linear_asym: a_scale and a_zero must have M elements")
    if b_scale.numel() != N or b_sum.numel() != N:
        raise RuntimeError("w4a4_linear_asym: b_scale and b_sum must have N elements")
    if bias is not None and bias.numel() != N:
        raise RuntimeError("w4a4_linear_asym: bias must have N elements")
    out = torch.empty((M, N), dtype=torch.float16, device=A.device)
    _call("srq_w4a4_linear_asym", _ptr(A), _ptr(a_scale), _ptr(a_zero), _ptr(B), _ptr(b_scale),
          _ptr(b_sum), _ptr(bias), M, N, K, _ptr(out), _stream(A))
    return out


def w4a4_linear(A, a_scale, B, b_scale, bias=None):
    """Fused matmul + sym_dequant (+ fp16 bias): out f16 [M, N]."""
    _check("w4a4_linear", [(A, "A"), (a_scale, "a_scale"), (B, "B"), (b_scale, "b_scale"),
                           (bias, "bias")],
           [torch.uint8, torch.float16, torch.uint8, torch.float16, torch.float16])
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[1]:
        raise RuntimeError(f"w4a4_linear: expected A [M, K/2] and B [N, K/2], got "
                           f"{tuple(A.shape)} and {tuple(B.shape)}")
    M, N, K = A.shape[0], B.shape[0], A.shape[1] * 2
    if a_scale.numel() != M or b_scale.numel() != N:
        raise RuntimeError("w4a4_linear: a_scale must have M and b_scale N elements")
    if bias is not None and bias.numel() != N:
        raise RuntimeError("w4a4_linear: bias must have N elements")
    out = torch.empty((M, N), dtype=torch.float16, device=A.device)
    ws = _splitk_workspace(M, N, K, A.device)
    if ws is None:
        _call("srq_w4a4_linear", _ptr(A), _ptr(a_scale), _ptr(B), _ptr(b_scale), _ptr(bias),
              M, N, K, _ptr(out), _stream(A))
    else:
        _call("srq_w4a4_linear_ws", _ptr(A), _ptr(a_scale), _ptr(B), _ptr(b_scale), _ptr(bias),
              M, N, K, _ptr(out), _ptr(ws), ws.numel(), _stream(A))
    return out


def interleave_gate_up(w, s, ffn):
    """Gate/up rows [gate (ffn); up (ffn)] (weights [2 ffn, K/2] or scales
    [2 ffn] / [2 ffn, 1]) rearranged into blocks of 8 gate rows then 8 up
    rows, the layout w4a4_linear_swiglu reads.  A copy (weight preparation,
    done once)."""
    if ffn % 8 or w.shape[0] != 2 * ffn or s.shape[0] != 2 * ffn:
        raise RuntimeError("interleave_gate_up: expects [2 ffn, ...] rows with ffn % 8 == 0")

    def il(t):
        rest = t.shape[1:]
        return t.reshape(2, ffn // 8, 8, *rest).transpose(0, 1).reshape(2 * ffn, *rest).contiguous()
    return il(w), il(s)


def w4a4_linear_swiglu(A, a_scale, B_il, b_scale_il):
    """swiglu(gate, up) of the gate/up projection in one launch (any M):
    B_il / b_scale_il from interleave_gate_up; out f16 [M, N/2]."""
    _check("w4a4_linear_swiglu", [(A, "A"), (a_scale, "a_scale"), (B_il, "B"),
                                  (b_scale_il, "b_scale")],
           [torch.uint8, torch.float16, torch.uint8, torch.float16])
    if A.dim() != 2 or B_il.dim() != 2 or A.shape[1] != B_il.shape[1]:
        raise RuntimeError("w4a4_linear_swiglu: expected A [M, K/2] and B [N, K/2]")
    M, N, K = A.shape[0], B_il.shape[0], A.shape[1] * 2
    if a_scale.numel() != M or b_scale_il.numel() != N:
        raise RuntimeError("w4a4_linear_swiglu: a_scale must have M and b_scale N elements")
    out = torch.empty((M, N // 2), dtype=torch.float16, device=A.device)
    _call("srq_w4a4_linear_swiglu", _ptr(A), _ptr(a_scale), _ptr(B_il), _ptr(b_scale_il), M, N, K,
          _ptr(out), _stream(A))
    return out


@functools.lru_cache(maxsize=512)
def _splitk_bytes(M, N, K):
    return int(_native.lib().srq_w4a4_linear_ws_bytes(M, N, K))


def _splitk_workspace(M, N, K, device):
    """The int32 split-K partials' workspace the library asks for at this
    shape (mid-size M with too few output tiles to fill the GPU), from
    torch's caching allocator (graph-capture safe), or None."""
    n = _splitk_bytes(M, N, K)
    return torch.empty(n, dtype=torch.uint8, device=device) if n else None


# ------------------------------------------------------------- bf6 GEMM
# The same W4A4 products on the 6-bit-operand MFMA (twice the int8 rate),
# from operands in the bf6 block layout (srq_i4_to_bf6 in
# include/signrot_hip.h): a weight is converted once, the product is
# bit-identical to matmul / w4a4_linear on the packed int4 operands.

def bf6_bytes(rows, K):
    """Bytes of the bf6 block layout of a [rows, K] code matrix (K % 128 == 0)."""
    if K % 128:
        raise RuntimeError(f"bf6_bytes: K={K} must be a multiple of 128")
    return -(-rows // 32) * (K // 128) * 3072


def i4_to_bf6(W):
    """Packed int4 rows u8 [R, K/2] -> the bf6 block layout, u8 [bf6_bytes(R, K)]."""
    _check("i4_to_bf6", [(W, "W")], [torch.uint8])
    if W.dim() != 2:
        raise RuntimeError(f"i4_to_bf6: expected [R, K/2], got {tuple(W.shape)}")
    R, K = W.shape[0], W.shape[1] * 2
    out = torch.empty(bf6_bytes(R, K), dtype=torch.uint8, device=W.device)
    _call("srq_i4_to_bf6", _ptr(W), R, K, _ptr(out), _stream(W))
    return out


def had_sign_quant_bf6(x, hadK, K, sign=None, clip_ratio=1.0):
    """had_sign_quant with the codes in the bf6 block layout: (q6 u8
    [bf6_bytes(rows, n)], scale f16 [..., 1]); the same codes and scales."""
    _check("had_sign_quant_bf6", [(x, "x"), (hadK, "hadK"), (sign, "sign")],
           [torch.float16, torch.float16, torch.int8])
    n = x.shape[-1]
    _check_had("had_sign_quant_bf6", n, hadK, K, sign, False)
    rows = x.numel() // n if n else 0
    q6 = torch.empty(bf6_bytes(rows, n), dtype=torch.uint8, device=x.device)
    scale = torch.empty((*x.shape[:-1], 1), dtype=torch.float16, device=x.device)
    if rows:
        _call("srq_had_sign_quant_bf6", _ptr(x), rows, n, int(K), _ptr(hadK), _ptr(sign),
              float(clip_ratio), _ptr(q6), _ptr(scale), _stream(x))
    return q6, scale


def _bf6_operands(name, A6, B6, M, N, K):
    _check(name, [(A6, "A6"), (B6, "B6")], [torch.uint8, torch.uint8])
    if A6.numel() < bf6_bytes(M, K) or B6.numel() < bf6_bytes(N, K):
        raise RuntimeError(f"{name}: A6 / B6 hold fewer bytes than bf6_bytes(M or N, K)")


def matmul_bf6(A6, B6, M, N, K):
    """int32 [M, N] = A @ B^T from bf6-layout operands (== matmul on int4)."""
    _bf6_operands("matmul_bf6", A6, B6, M, N, K)
    C = torch.empty((M, N), dtype=torch.int32, device=A6.device)
    _call("srq_matmul_bf6", _ptr(A6), _ptr(B6), M, N, K, _ptr(C), _stream(A6))
    return C


def w4a4_linear_bf6(A6, a_scale, B6, b_scale, M, N, K, bias=None):
    """w4a4_linear from bf6-layout operands: out f16 [M, N], bit-identical."""
    _bf6_operands("w4a4_linear_bf6", A6, B6, M, N, K)
    _check("w4a4_linear_bf6", [(a_scale, "a_scale"), (b_scale, "b_scale"), (bias, "bias")],
           [torch.float16, torch.float16, torch.float16])
    if a_scale.numel() != M or b_scale.numel() != N:
        raise RuntimeError("w4a4_linear_bf6: a_scale must have M and b_scale N elements")
    if bias is not None and bias.numel() != N:
        raise RuntimeError("w4a4_linear_bf6: bias must have N elements")
    out = torch.empty((M, N), dtype=torch.float16, device=A6.device)
    _call("srq_w4a4_linear_bf6", _ptr(A6), _ptr(a_scale), _ptr(B6), _ptr(b_scale), _ptr(bias),
          M, N, K, _ptr(out), _stream(A6))
    return out


# ------------------------------------------------------------------ quant

def w4a4_linear_residual(A, a_scale, B, b_scale, residual, bias=None, out=None):
    """w4a4_linear with `+ residual` fused into the epilogue: out f16 [M, N] =
    fp16(linear + residual).  `out` may be `residual` itself (in place)."""
    _check("w4a4_linear_residual", [(A, "A"), (a_scale, "a_scale"), (B, "B"),
                                    (b_scale, "b_scale"), (residual, "residual"), (bias, "bias"),
                                    (out, "out")],
           [torch.uint8, torch.float16, torch.uint8, torch.float16, torch.float16, torch.float16,
            torch.float16])
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[1]:
        raise RuntimeError(f"w4a4_linear_residual: expected A [M, K/2] and B [N, K/2], got "
                           f"{tuple(A.shape)} and {tuple(B.shape)}")
    M, N, K = A.shape[0], B.shape[0], A.shape[1] * 2
    if a_scale.numel() != M or b_scale.numel() != N:
        raise RuntimeError("w4a4_linear_residual: scale sizes do not match M / N")
    if residual.numel() != M * N:
        raise RuntimeError(f"w4a4_linear_residual: residual must have {M} x {N} elements")
    if bias is not None and bias.numel() != N:
        raise RuntimeError("w4a4_linear_residual: bias must have N elements")
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=A.device)
    elif out.numel() != M * N:
        raise RuntimeError(f"w4a4_linear_residual: out must have {M} x {N} elements")
    ws = _splitk_workspace(M, N, K, A.device)
    if ws is None:
        _call("srq_w4a4_linear_residual", _ptr(A), _ptr(a_scale), _ptr(B), _ptr(b_scale),
              _ptr(bias), _ptr(residual), M, N, K, _ptr(out), _stream(A))
    else:
        _call("srq_w4a4_linear_residual_ws", _ptr(A), _ptr(a_scale), _ptr(B), _ptr(b_scale),
              _ptr(bias), _ptr(residual), M, N, K, _ptr(out), _ptr(ws), ws.numel(),
              _stream(A))
    return out


def sym_quant(x, scale):
    """Packed int4 codes of fp16 x [M, N] with given fp16 scale [M]
    (bindings.cpp:208-225)."""
    _check("sym_quant", [(x, "x"), (scale, "scale")], [torch.float16, torch.float16])
    if x.dim() != 2:
        raise RuntimeError("sym_quant: expected a 2D [rows, cols] tensor")
    rows, cols = x.shape
    if scale.shape[0] != rows:
        raise RuntimeError(f"sym_quant: expected scale to have size {rows} at dimension 0, "
                           f"but got {scale.shape[0]}")
    q = torch.empty((rows, (cols + 1) // 2), dtype=torch.uint8, device=x.device)
    _call("srq_sym_quant", _ptr(x), _ptr(scale), rows, cols, _ptr(q), _stream(x))
    return q


def sym_dequant(q, scale_row, scale_col, bits=32):
    """fp16 [M, N] = fp16((float(q) * float(scale_row)) * float(scale_col))
    (bindings.cpp:228-268)."""
    _check("sym_dequant", [(q, "q"), (scale_row, "scale_row"), (scale_col, "scale_col")],
           [torch.int32, None, None])
    if bits != 32:
        raise RuntimeError("Unsupported data type")
    if scale_row.dtype != torch.float16 or scale_col.dtype != torch.float16:
        raise RuntimeError("sym_dequant: scales must be float16")
    rows, cols = q.shape
    if scale_row.shape[0] != rows:
        raise RuntimeError(f"sym_dequant: expected scale_row to have size {rows} at dimension "
                           f"0, but got {scale_row.shape[0]}")
    if scale_col.shape[0] != cols:
        raise RuntimeError(f"sym_dequant: expected scale_col to have size {cols} at dimension "
                           f"0, but got {scale_col.shape[0]}")
    out = torch.empty(q.shape, dtype=torch.float16, device=q.device)
    _call("srq_sym_dequant", _ptr(q), _ptr(scale_row), _ptr(scale_col), rows, cols, _ptr(out),
          _stream(q))
    return out


def sym_quant_dynamic(x, clip_ratio=1.0):
    """(q u8 [rows, ceil(cols/2)], scale f16 [rows, 1]) (bindings.cpp:316-335)."""
    _check("sym_quant_dynamic", [(x, "x")])
    if x.dim() != 2:
        raise RuntimeError("sym_quant_dynamic expects a 2D [rows, cols] tensor")
    if x.dtype != torch.float16:
        raise RuntimeError("sym_quant_dynamic expects fp16 input")
    rows, cols = x.shape
    q = torch.empty((rows, (cols + 1) // 2), dtype=torch.uint8, device=x.device)
    scale = torch.empty((rows, 1), dtype=torch.float16, device=x.device)
    _call("srq_sym_quant_dynamic", _ptr(x), rows, cols, float(clip_ratio), _ptr(q), _ptr(scale),
          _stream(x))
    return q, scale


def sym_quant_dynamic_rows(x, src_row, clip_ratio=1.0):
    """sym_quant_dynamic(x[src_row]) in one launch (no gathered copy): x f16
    [rows, cols], src_row int32 [R] -> (q u8 [R, cols/2], scale f16 [R, 1]).
    Indices outside [0, rows) give zero codes and scale 0."""
    _check("sym_quant_dynamic_rows", [(x, "x"), (src_row, "src_row")],
           [torch.float16, torch.int32])
    if x.dim() != 2 or src_row.dim() != 1:
        raise RuntimeError("sym_quant_dynamic_rows expects x [rows, cols] and src_row [R]")
    R, cols = src_row.shape[0], x.shape[1]
    q = torch.empty((R, cols // 2), dtype=torch.uint8, device=x.device)
    scale = torch.empty((R, 1), dtype=torch.float16, device=x.device)
    _call("srq_sym_quant_dynamic_rows", _ptr(x), x.shape[0], _ptr(src_row), R, cols,
          float(clip_ratio), _ptr(q), _ptr(scale), _stream(x))
    return q, scale


# ------------------------------------------------- asymmetric activations

def asym_quant_dynamic(x, clip_ratio=1.0):
    """(q u8 [rows, ceil(cols/2)] of uint4 codes, scale f16 [rows, 1], zero
    f16 [rows, 1]) (bindings.cpp:337-358)."""
    _check("asym_quant_dynamic", [(x, "x")])
    if x.dim() != 2:
        raise RuntimeError("asym_quant_dynamic expects a 2D [rows, cols] tensor")
    if x.dtype != torch.float16:
        raise RuntimeError("asym_quant_dynamic expects fp16 input")
    rows, cols = x.shape
    q = torch.empty((rows, (cols + 1) // 2), dtype=torch.uint8, device=x.device)
    scale = torch.empty((rows, 1), dtype=torch.float16, device=x.device)
    zero = torch.empty((rows, 1), dtype=torch.float16, device=x.device)
    _call("srq_asym_quant_dynamic", _ptr(x), rows, cols, float(clip_ratio), _ptr(q),
          _ptr(scale), _ptr(zero), _stream(x))
    return q, scale, zero


def _asym_given(name, x, scale, zero, is_signed):
    _check(name, [(x, "x"), (scale, "scale"), (zero, "zeros")],
           [torch.float16, torch.float16, torch.float16])
    if x.dim() != 2:
        raise RuntimeError(f"{name} expects a 2D [rows, cols] tensor")
    rows, cols = x.shape
    if scale.numel() != rows or zero.numel() != rows:
        raise RuntimeError(f"{name}: scale and zeros need one entry per row")
    q = torch.empty((rows, (cols + 1) // 2), dtype=torch.uint8, device=x.device)
    _call("srq_asym_quant", _ptr(x), _ptr(scale), _ptr(zero), rows, cols, int(is_signed),
          _ptr(q), _stream(x))
    return q


def asym_quant_f16_ui4(x, scale, zero):
    """uint4 codes for a given per-row scale and zero (bindings.cpp:292-312)."""
    return _asym_given("asym_quant_f16_ui4", x, scale, zero, False)


def asym_quant_f16_si4(x, scale, zero):
    """The same arithmetic clamped to [-8, 7], int4 codes (bindings.cpp:270-290)."""
    return _asym_given("asym_quant_f16_si4", x, scale, zero, True)


def sum_i4(x, is_signed=True):
    """int32 [rows, 1] sum of each packed row's nibbles (bindings.cpp:437-451)."""
    _check("sum_i4", [(x, "x")], [torch.uint8])
    if x.dim() != 2:
        raise RuntimeError("sum_i4 expects a 2D tensor of shape [rows, packed_cols]")
    rows, pc = x.shape
    out = torch.empty((rows, 1), dtype=torch.int32, device=x.device)
    _call("srq_sum_i4", _ptr(x), rows, pc, 1 if is_signed else 0, _ptr(out), _stream(x))
    return out


def matmul_colrow_i8_i32(a_col, b_row):
    """out int32 [N, C] = a_col int8 [N, 1] x b_row int32 [1, C]
    (bindings.cpp:453-477)."""
    _check("matmul_colrow_i8_i32", [(a_col, "a_col"), (b_row, "b_row")],
           [torch.int8, torch.int32])
    if a_col.dim() != 2 or a_col.shape[1] != 1:
        raise RuntimeError("a_col must be 2D with shape [N, 1]")
    if b_row.dim() != 2 or b_row.shape[0] != 1:
        raise RuntimeError("b_row must be 2D with shape [1, C]")
    rows, cols = a_col.shape[0], b_row.shape[1]
    out = torch.empty((rows, cols), dtype=torch.int32, device=a_col.device)
    _call("srq_matmul_colrow_i8_i32", _ptr(a_col), _ptr(b_row), rows, cols, _ptr(out),
          _stream(a_col))
    return out


def kv_quant_pack(x):
    """(q u8 [..., D/2], param f16 [..., 2]) (bindings.cpp:359-381)."""
    _check("kv_quant_pack", [(x, "x")])
    if x.dtype != torch.float16:
        raise RuntimeError("kv_quant_pack expects fp16 input")
    cols = x.shape[-1]
    if cols % 2:
        raise RuntimeError("kv_quant_pack expects an even last dimension")
    rows = x.numel() // cols if cols else 0
    q = torch.empty((*x.shape[:-1], cols // 2), dtype=torch.uint8, device=x.device)
    param = torch.empty((*x.shape[:-1], 2), dtype=torch.float16, device=x.device)
    _call("srq_kv_quant_pack", _ptr(x), rows, cols, _ptr(q), _ptr(param), _stream(x))
    return q, param


# --------------------------------------------------------------- Hadamard

def hadamard_transform(x, scale=1.0):
    """fast_hadamard_transform.hadamard_transform(x, scale): Sylvester-order
    WHT over the last dim (power of two, <= 32768), fp16 or fp32, times scale."""
    _check("hadamard_transform", [(x, "x")])
    if x.dtype not in (torch.float16, torch.float32):
        raise RuntimeError("hadamard_transform: only float16 and float32 are supported")
    n = x.shape[-1]
    rows = x.numel() // n if n else 0
    out = torch.empty_like(x)
    _call("srq_hadamard_transform", _ptr(x), _ptr(out), rows, n, float(scale),
          0 if x.dtype == torch.float16 else 1, _stream(x))
    return out


def online_hadamard(x, hadK, K, sign=None, fp32_had=False):
    """matmul_hadU_cuda(x, hadK, K) then `* sign`, fp16 in/out."""
    _check("online_hadamard", [(x, "x"), (hadK, "hadK"), (sign, "sign")],
           [torch.float16, None, torch.int8])
    n = x.shape[-1]
    _check_had("online_hadamard", n, hadK, K, sign, fp32_had)
    rows = x.numel() // n if n else 0
    out = torch.empty_like(x)
    _call("srq_online_hadamard", _ptr(x), _ptr(out), rows, n, int(K), _ptr(hadK), _ptr(sign),
          1 if fp32_had else 0, _stream(x))
    return out


def had_sign_quant(x, hadK, K, sign=None, clip_ratio=1.0, fp32_had=False):
    """online_hadamard followed by sym_quant_dynamic, one launch:
    (q u8 [..., n/2], scale f16 [..., 1])."""
    _check("had_sign_quant", [(x, "x"), (hadK, "hadK"), (sign, "sign")],
           [torch.float16, None, torch.int8])
    n = x.shape[-1]
    _check_had("had_sign_quant", n, hadK, K, sign, fp32_had)
    rows = x.numel() // n if n else 0
    q = torch.empty((*x.shape[:-1], n // 2), dtype=torch.uint8, device=x.device)
    scale = torch.empty((*x.shape[:-1], 1), dtype=torch.float16, device=x.device)
    _call("srq_had_sign_quant", _ptr(x), rows, n, int(K), _ptr(hadK), _ptr(sign),
          1 if fp32_had else 0, float(clip_ratio), _ptr(q), _ptr(scale), _stream(x))
    return q, scale


def had_asym_fusable(n, K):
    """Whether had_sign_asym_quant has a one-launch kernel for n = K x 2^k."""
    return K % 4 == 0 and 9 <= K <= 32 and n in (K * 512, K * 1024)


def had_sign_asym_quant(x, hadK, K, sign=None, clip_ratio=1.0):
    """online_hadamard followed by asym_quant_dynamic: (q u8 [..., n/2] uint4
    codes, scale f16 [..., 1], zero f16 [..., 1]).  One launch where the
    rotation has an MFMA form (had_asym_fusable), else the two ops in turn
    (the same results)."""
    _check("had_sign_asym_quant", [(x, "x"), (hadK, "hadK"), (sign, "sign")],
           [torch.float16, torch.float16, torch.int8])
    n = x.shape[-1]
    _check_had("had_sign_asym_quant", n, hadK, K, sign, False)
    rows = x.numel() // n if n else 0
    if not had_asym_fusable(n, K):
        rot = online_hadamard(x.reshape(rows, n), hadK, K, sign)
        q, s, z = asym_quant_dynamic(rot, clip_ratio)
        return (q.view(*x.shape[:-1], -1), s.view(*x.shape[:-1], 1),
                z.view(*x.shape[:-1], 1))
    q = torch.empty((*x.shape[:-1], n // 2), dtype=torch.uint8, device=x.device)
    scale = torch.empty((*x.shape[:-1], 1), dtype=torch.float16, device=x.device)
    zero = torch.empty((*x.shape[:-1], 1), dtype=torch.float16, device=x.device)
    if rows:
        _call("srq_had_sign_asym_quant", _ptr(x), rows, n, int(K), _ptr(hadK), _ptr(sign),
              float(clip_ratio), _ptr(q), _ptr(scale), _ptr(zero), _stream(x))
    return q, scale, zero


def _check_had(name, n, hadK, K, sign, fp32_had):
    if K > 1:
        if hadK is None or tuple(hadK.shape[-2:]) != (K, K) or hadK.numel() != K * K:
            raise RuntimeError(f"{name}: hadK must be [{K}, {K}]")
        want = torch.float32 if fp32_had else torch.float16
        if hadK.dtype != want:
            raise RuntimeError(f"{name}: hadK must be {want}")
    if sign is not None and sign.numel() != n:
        raise RuntimeError(f"{name}: sign must have {n} elements")


# ------------------------------------------------------ paged int4 KV cache

def _check_cache(name, kv_data, kv_param, kv_indptr, kv_indices, last_page_offset):
    _check(name, [(kv_data, "kv_data"), (kv_param, "kv_param"), (kv_indptr, "kv_indptr"),
                  (kv_indices, "kv_indices"), (last_page_offset, "last_page_offset")],
           [torch.uint8, torch.float16, torch.int32, torch.int32, torch.int32])
    if kv_data.dim() != 6 or kv_param.dim() != 6:
        raise RuntimeError(f"{name}: kv_data and kv_param must be 6D [pages, L, 2, H, P, *]")
    if tuple(kv_param.shape[:5]) != tuple(kv_data.shape[:5]) or kv_param.shape[5] != 2:
        raise RuntimeError(f"{name}: kv_param must be {tuple(kv_data.shape[:5]) + (2,)}")
    if kv_indptr.dim() != 1 or kv_indices.dim() != 1 or last_page_offset.dim() != 1:
        raise RuntimeError(f"{name}: index tensors must be 1D")
    head_dim = kv_data.shape[5] * 2
    if head_dim != 128:
        raise RuntimeError(f"CHECK_EQ(head_dim, 128) failed. {head_dim} vs 128")
    return kv_data.shape[1], kv_data.shape[3], kv_data.shape[4], head_dim


def init_kv_i4(kv_data, kv_param, kv_indptr, kv_indices, last_page_offset, k, v, k_param,
               v_param, seqlen_indptr, layer_idx):
    """Prefill fill of one layer of the paged int4 cache (bindings.cpp:561-604)."""
    L, H, P, D = _check_cache("init_kv_i4", kv_data, kv_param, kv_indptr, kv_indices,
                              last_page_offset)
    _check("init_kv_i4", [(k, "k"), (v, "v"), (k_param, "k_param"), (v_param, "v_param"),
                          (seqlen_indptr, "seqlen_indptr"), (kv_data, "kv_data")],
           [torch.uint8, torch.uint8, torch.float16, torch.float16, torch.int32, None])
    B = last_page_offset.shape[0]
    if kv_indptr.shape[0] != B + 1 or seqlen_indptr.shape[0] != B + 1:
        raise RuntimeError("init_kv_i4: kv_indptr and seqlen_indptr must have batch + 1 entries")
    if k.dim() != 3 or tuple(k.shape[1:]) != (H, D // 2) or v.shape != k.shape:
        raise RuntimeError(f"init_kv_i4: k and v must be [tokens, {H}, {D // 2}]")
    if tuple(k_param.shape) != (k.shape[0], H, 2) or v_param.shape != k_param.shape:
        raise RuntimeError(f"init_kv_i4: k_param and v_param must be [tokens, {H}, 2]")
    _call("srq_init_kv_i4", _ptr(kv_data), _ptr(kv_param), _ptr(kv_indptr), _ptr(kv_indices),
          _ptr(last_page_offset), _ptr(k), _ptr(v), _ptr(k_param), _ptr(v_param),
          _ptr(seqlen_indptr), B, k.shape[0], L, int(layer_idx), H, P, D, _stream(kv_data))


def append_kv_i4(kv_data, kv_param, kv_indptr, kv_indices, last_page_offset, k, v, k_param,
                 v_param, layer_idx):
    """Decode append of one token per request (bindings.cpp:606-645)."""
    L, H, P, D = _check_cache("append_kv_i4", kv_data, kv_param, kv_indptr, kv_indices,
                              last_page_offset)
    _check("append_kv_i4", [(k, "k"), (v, "v"), (k_param, "k_param"), (v_param, "v_param"),
                            (kv_data, "kv_data")],
           [torch.uint8, torch.uint8, torch.float16, torch.float16, None])
    if k.dim() != 3 or tuple(k.shape[1:]) != (H, D // 2) or v.shape != k.shape:
        raise RuntimeError(f"append_kv_i4: k and v must be [batch, {H}, {D // 2}]")
    B = k.shape[0]
    if kv_indptr.shape[0] != B + 1 or last_page_offset.shape[0] != B:
        raise RuntimeError("append_kv_i4: index tensors do not match the batch")
    if tuple(k_param.shape) != (B, H, 2) or v_param.shape != k_param.shape:
        raise RuntimeError(f"append_kv_i4: k_param and v_param must be [{B}, {H}, 2]")
    _call("srq_append_kv_i4", _ptr(kv_data), _ptr(kv_param), _ptr(kv_indptr), _ptr(kv_indices),
          _ptr(last_page_offset), _ptr(k), _ptr(v), _ptr(k_param), _ptr(v_param), B, L,
          int(layer_idx), H, P, D, _stream(kv_data))


def qkv_rope_had_append(qkv, cos, sin, n_q_heads, n_kv_heads, kv_data, kv_param, kv_indptr,
                        kv_indices, last_page_offset, layer_idx, had_scale, rotate=True):
    """Decode-step q/k/v post-processing of qkv f16 [B, (Hq + 2 Hk) * 128]:
    RoPE of q and k, head-dim Hadamard (times had_scale) of q and k when
    `rotate`, int4 quantize-and-append of k and v into the cache slot of the
    new token; returns q f16 [B, Hq, 128] (ready for batch_decode_i4)."""
    L, H, P, D = _check_cache("qkv_rope_had_append", kv_data, kv_param, kv_indptr, kv_indices,
                              last_page_offset)
    _check("qkv_rope_had_append", [(qkv, "qkv"), (cos, "cos"), (sin, "sin"),
                                   (kv_data, "kv_data")],
           [torch.float16, torch.float16, torch.float16, None])
    if H != n_kv_heads:
        raise RuntimeError(f"qkv_rope_had_append: the cache holds {H} KV heads, not {n_kv_heads}")
    B = qkv.shape[0]
    if qkv.numel() != B * (n_q_heads + 2 * n_kv_heads) * D:
        raise RuntimeError(f"qkv_rope_had_append: qkv must be [B, {(n_q_heads + 2 * n_kv_heads) * D}]")
    if kv_indptr.shape[0] != B + 1 or last_page_offset.shape[0] != B:
        raise RuntimeError("qkv_rope_had_append: index tensors do not match the batch")
    cb = cos.numel() // D
    if cos.numel() != sin.numel() or cos.numel() % D or cb not in (1, B):
        raise RuntimeError(f"qkv_rope_had_append: cos/sin must be [1 or {B}, {D}]")
    q = torch.empty((B, n_q_heads, D), dtype=torch.float16, device=qkv.device)
    _call("srq_qkv_rope_had_append", _ptr(qkv), _ptr(cos), _ptr(sin), cb, B, int(n_q_heads),
          int(n_kv_heads), D, float(had_scale), 1 if rotate else 0, _ptr(q), _ptr(kv_data),
          _ptr(kv_param), _ptr(kv_indptr), _ptr(kv_indices), _ptr(last_page_offset), L,
          int(layer_idx), P, _stream(qkv))
    return q


def batch_decode_i4(o, q, kv_data, kv_param, kv_indptr, kv_indices, last_page_offset,
                    layer_idx, tmp=None, num_chunks=1):
    """Single-query attention over the int4 cache into o [B, Hq, 128]
    (bindings.cpp:508-559).  Hq may be 1..8 times the cache's head count.
    o=None with a split (tmp, num_chunks > 1) leaves the partial states in
    tmp unmerged (see merge_head_had_quant)."""
    L, H, P, D = _check_cache("batch_decode_i4", kv_data, kv_param, kv_indptr, kv_indices,
                              last_page_offset)
    if o is None and (tmp is None or num_chunks <= 1):
        raise RuntimeError("batch_decode_i4: o may be None only with a split (tmp, num_chunks > 1)")
    _check("batch_decode_i4", [(q if o is None else o, "o"), (q, "q"), (kv_data, "kv_data")],
           [torch.float16, torch.float16, None])
    if o is not None and (o.dim() != 3 or q.dim() != 3 or o.shape != q.shape):
        raise RuntimeError("batch_decode_i4: o and q must be the same [B, N, D] shape")
    if q.dim() != 3:
        raise RuntimeError("batch_decode_i4: q must be [B, N, D]")
    B, Hq = q.shape[0], q.shape[1]
    if q.shape[2] != D:
        raise RuntimeError(f"batch_decode_i4: q head_dim {q.shape[2]} != cache head_dim {D}")
    if kv_indptr.shape[0] != B + 1 or last_page_offset.shape[0] != B:
        raise RuntimeError("batch_decode_i4: index tensors do not match the batch")
    tmp_ptr, chunks = None, 1
    if tmp is not None and num_chunks > 1:
        _check("batch_decode_i4", [(tmp, "tmp"), (q, "q")], [torch.float32, None])
        if tmp.numel() != B * Hq * num_chunks * (D + 4):
            raise RuntimeError("batch_decode_i4: tmp must be [B, N, num_chunks, head_dim + 4]")
        tmp_ptr, chunks = _ptr(tmp), int(num_chunks)
    _call("srq_batch_decode_i4", _ptr(o), _ptr(q), _ptr(kv_data), _ptr(kv_param),
          _ptr(kv_indptr), _ptr(kv_indices), _ptr(last_page_offset), B, Hq, H, L,
          int(layer_idx), P, D, tmp_ptr, chunks, _stream(q))


def qkv_decode_i4(o, qkv, cos, sin, kv_data, kv_param, kv_indptr, kv_indices, last_page_offset,
                  layer_idx, n_q_heads, had_scale, rotate=True, tmp=None, num_chunks=1):
    """qkv_rope_had_append followed by batch_decode_i4 in one launch: the
    new token's k / v are quantized into the cache and attended together
    with the context, q is rotated on chip.  qkv f16 [B, (Hq + 2 Hk) * 128],
    cos / sin [1 or B, 128]; o f16 [B, Hq, 128] (None with a split: the
    partial states stay in tmp for merge_head_had_quant).  The cache bytes
    and o are bit-identical to the two calls."""
    L, H, P, D = _check_cache("qkv_decode_i4", kv_data, kv_param, kv_indptr, kv_indices,
                              last_page_offset)
    _check("qkv_decode_i4", [(qkv, "qkv"), (cos, "cos"), (sin, "sin"), (o, "o")],
           [torch.float16, torch.float16, torch.float16, torch.float16])
    B = qkv.shape[0]
    if qkv.numel() != B * (n_q_heads + 2 * H) * D:
        raise RuntimeError(f"qkv_decode_i4: qkv must be [B, {(n_q_heads + 2 * H) * D}]")
    if n_q_heads % H or n_q_heads // H > 8:
        raise RuntimeError(f"qkv_decode_i4: {n_q_heads} query heads for {H} KV heads")
    if kv_indptr.shape[0] != B + 1 or last_page_offset.shape[0] != B:
        raise RuntimeError("qkv_decode_i4: index tensors do not match the batch")
    cb = cos.numel() // D
    if cos.numel() != sin.numel() or cos.numel() % D or cb not in (1, B):
        raise RuntimeError(f"qkv_decode_i4: cos/sin must be [1 or {B}, {D}]")
    tmp_ptr, chunks = None, 1
    if tmp is not None and num_chunks > 1:
        if tmp.dtype != torch.float32 or tmp.numel() < B * n_q_heads * num_chunks * (D + 4):
            raise RuntimeError("qkv_decode_i4: tmp must be float32 [B, Hq, chunks, D + 4]")
        tmp_ptr, chunks = _ptr(tmp), int(num_chunks)
    if o is None and chunks <= 1:
        raise RuntimeError("qkv_decode_i4: o may be None only with a split (tmp, num_chunks > 1)")
    if o is not None and tuple(o.shape) != (B, n_q_heads, D):
        raise RuntimeError(f"qkv_decode_i4: o must be [{B}, {n_q_heads}, {D}]")
    _call("srq_qkv_decode_i4", _ptr(o), _ptr(qkv), _ptr(cos), _ptr(sin), cb, float(had_scale),
          1 if rotate else 0, _ptr(kv_data), _ptr(kv_param), _ptr(kv_indptr), _ptr(kv_indices),
          _ptr(last_page_offset), B, int(n_q_heads), H, L, int(layer_idx), P, D, tmp_ptr, chunks,
          _stream(qkv))
    return o


def batch_decode_i4_noalloc(o, q, kv_data, kv_param, kv_indptr, kv_indices, last_page_offset,
                            layer_idx, num_chunks=1):
    """batch_decode_i4 split into num_chunks chunks whose partial states go
    to the library's fixed per-GPU scratch (no workspace, no allocation);
    same results as batch_decode_i4 with a tmp of that many chunks.  Calls
    that overlap on one GPU race on the scratch."""
    L, H, P, D = _check_cache("batch_decode_i4_noalloc", kv_data, kv_param, kv_indptr,
                              kv_indices, last_page_offset)
    _check("batch_decode_i4_noalloc", [(o, "o"), (q, "q"), (kv_data, "kv_data")],
           [torch.float16, torch.float16, None])
    if o.dim() != 3 or q.dim() != 3 or o.shape != q.shape:
        raise RuntimeError("batch_decode_i4_noalloc: o and q must be the same [B, N, D] shape")
    B, Hq = q.shape[0], q.shape[1]
    if q.shape[2] != D:
        raise RuntimeError(f"batch_decode_i4_noalloc: q head_dim {q.shape[2]} != {D}")
    if kv_indptr.shape[0] != B + 1 or last_page_offset.shape[0] != B:
        raise RuntimeError("batch_decode_i4_noalloc: index tensors do not match the batch")
    _call("srq_batch_decode_i4_noalloc", _ptr(o), _ptr(q), _ptr(kv_data), _ptr(kv_param),
          _ptr(kv_indptr), _ptr(kv_indices), _ptr(last_page_offset), B, Hq, H, L,
          int(layer_idx), P, D, int(num_chunks), _stream(q))


# ------------------------------------------------------- decode-layer glue

def rmsnorm(x, eps, mean_dim):
    """fp16 RMSNorm without gamma over the last dim (bindings.cpp:423-435)."""
    _check("rmsnorm", [(x, "x")])
    if x.dtype != torch.float16:
        raise RuntimeError("rmsnorm expects fp16 input")
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    out = torch.empty_like(x)
    _call("srq_rmsnorm", _ptr(x), rows, cols, float(eps), int(mean_dim), _ptr(out), _stream(x))
    return out


def rmsnorm_quant(x, eps, mean_dim, clip_ratio=1.0, return_norm=False):
    """rmsnorm followed by sym_quant_dynamic in one launch: (q u8 [..., cols/2],
    scale f16 [..., 1]) and, with return_norm, the fp16 normalized x."""
    _check("rmsnorm_quant", [(x, "x")], [torch.float16])
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    q = torch.empty((*x.shape[:-1], cols // 2), dtype=torch.uint8, device=x.device)
    scale = torch.empty((*x.shape[:-1], 1), dtype=torch.float16, device=x.device)
    h = torch.empty_like(x) if return_norm else None
    _call("srq_rmsnorm_quant", _ptr(x), rows, cols, float(eps), int(mean_dim), float(clip_ratio),
          _ptr(h), _ptr(q), _ptr(scale), _stream(x))
    return (q, scale, h) if return_norm else (q, scale)


# H * num_chunks limit of merge_head_had_quant (its records are staged in 64 KiB of LDS)
MERGE_HHQ_MAX_RECORDS = 65536 // (132 * 4)


def merge_head_had_quant(tmp, scale, clip_ratio=1.0, return_rot=False):
    """head_had_quant of the attention output merged from split-KV partial
    states tmp f32 [B, H, num_chunks, 132] (batch_decode_i4 with o=None), in
    one launch: bit-identical to batch_decode_i4's merge then
    head_had_quant.  H * num_chunks <= MERGE_HHQ_MAX_RECORDS."""
    _check("merge_head_had_quant", [(tmp, "tmp")], [torch.float32])
    if tmp.dim() != 4 or tmp.shape[3] != 132:
        raise RuntimeError("merge_head_had_quant expects tmp [B, H, num_chunks, 132]")
    B, H, chunks = tmp.shape[:3]
    D = 128
    q = torch.empty((B, H * D // 2), dtype=torch.uint8, device=tmp.device)
    qs = torch.empty((B, 1), dtype=torch.float16, device=tmp.device)
    rot = torch.empty((B, H * D), dtype=torch.float16, device=tmp.device) if return_rot else None
    _call("srq_merge_head_had_quant", _ptr(tmp), B, H, D, chunks, float(scale),
          float(clip_ratio), _ptr(q), _ptr(qs), _ptr(rot), _stream(tmp))
    return (q, qs, rot) if return_rot else (q, qs)


def head_had_quant(x, scale, clip_ratio=1.0, return_rot=False):
    """Head-axis Hadamard of x f16 [B, H, D] (times `scale`) then per-row
    sym_quant_dynamic of the [B, H * D] result: (q u8 [B, H*D/2], scale f16
    [B, 1]) and, with return_rot, the rotated fp16 rows."""
    _check("head_had_quant", [(x, "x")], [torch.float16])
    if x.dim() != 3:
        raise RuntimeError("head_had_quant expects x [B, H, D]")
    B, H, D = x.shape
    q = torch.empty((B, H * D // 2), dtype=torch.uint8, device=x.device)
    qs = torch.empty((B, 1), dtype=torch.float16, device=x.device)
    rot = torch.empty((B, H * D), dtype=torch.float16, device=x.device) if return_rot else None
    _call("srq_head_had_quant", _ptr(x), B, H, D, float(scale), float(clip_ratio), _ptr(q),
          _ptr(qs), _ptr(rot), _stream(x))
    return (q, qs, rot) if return_rot else (q, qs)


def prefill_attention(q, k, v, attention_mask=None, causal=True, softmax_scale=None):
    """Prefill attention over fp16 q [B, T, Hq, 128], k/v [B, T, Hkv, 128]
    -> out fp16 [B, T, Hq, 128]: the flash-attn 2 call of the layer's first
    update (e2e/quantized_llama/modeling_llama.py:81-90).  q/k/v may be
    strided views (dense last two dims, e.g. slices of a fused q/k/v
    projection).  attention_mask [B, T] (HF layout, any integer or bool
    dtype) drops the keys at 0 entries and zeroes those output rows."""
    _check("prefill_attention", [(q, "q"), (k, "k"), (v, "v")],
           [torch.float16, torch.float16, torch.float16], contiguous=False)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise RuntimeError("prefill_attention expects [B, T, H, D] q/k/v")
    B, T, Hq, D = q.shape
    if tuple(k.shape) != tuple(v.shape) or k.shape[0] != B or k.shape[1] != T or k.shape[3] != D:
        raise RuntimeError("prefill_attention: k and v must be [B, T, Hkv, D] matching q")
    if k.stride() != v.stride():
        raise RuntimeError("prefill_attention: k and v must have the same strides")
    for t, name in ((q, "q"), (k, "k")):
        if t.stride(3) != 1 or t.stride(2) != D:
            raise RuntimeError(f"prefill_attention: {name} must be dense in its last two dims")
    mask = None
    if attention_mask is not None:
        if tuple(attention_mask.shape) != (B, T):
            raise RuntimeError("prefill_attention: attention_mask must be [B, T]")
        if attention_mask.device != q.device:
            raise RuntimeError("prefill_attention: attention_mask is on another device")
        mask = attention_mask.to(torch.int32).contiguous()
    out = torch.empty(B, T, Hq, D, dtype=torch.float16, device=q.device)

    def strides(t):
        # a size-1 dim's stride is never used to address; give it the dense value
        tok = t.stride(1) if T > 1 else t.shape[2] * D
        return tok, (t.stride(0) if B > 1 else T * tok)

    (q_tok, q_seq), (kv_tok, kv_seq) = strides(q), strides(k)
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    _call("srq_prefill_attention", _ptr(q), _ptr(k), _ptr(v), _ptr(mask), B, T, Hq, k.shape[2],
          D, q_tok, q_seq, kv_tok, kv_seq, scale, 1 if causal else 0,
          _ptr(out), _stream(q))
    return out


def rope_qk(q, k, cos, sin):
    """In-place rotary embedding of q, k [B, T, H, D] (bindings.cpp:383-409)."""
    _check("rope_qk", [(q, "q"), (k, "k"), (cos, "cos"), (sin, "sin")])
    if q.dim() != 4 or k.dim() != 4:
        raise RuntimeError("rope_qk expects [B, T, H, D] q/k")
    if cos.dim() != 3:
        raise RuntimeError("rope_qk expects [B or 1, T, D] cos/sin")
    if cos.shape != sin.shape:
        raise RuntimeError("cos and sin must have the same shape")
    if q.dtype != torch.float16 or k.dtype != torch.float16:
        raise RuntimeError("rope_qk expects fp16 q/k")
    if cos.dtype != torch.float16 or sin.dtype != torch.float16:
        raise RuntimeError("rope_qk expects fp16 cos/sin")
    if k.shape[0] != q.shape[0] or k.shape[1] != q.shape[1] or k.shape[3] != q.shape[3]:
        raise RuntimeError("q and k must agree on batch, sequence and head_dim")
    if cos.shape[1] != q.shape[1] or cos.shape[2] != q.shape[3]:
        raise RuntimeError("cos/sin must be [B or 1, T, head_dim]")
    if cos.shape[0] not in (1, q.shape[0]):
        raise RuntimeError("cos/sin batch must be 1 or match q")
    if q.shape[3] % 2:
        raise RuntimeError("rope_qk expects an even head_dim")
    _call("srq_rope_qk", _ptr(q), _ptr(k), _ptr(cos), _ptr(sin), q.shape[0], q.shape[1],
          cos.shape[0], q.shape[2], k.shape[2], q.shape[3], _stream(q))


def swiglu(gate, up):
    """fp16(fp16(silu(gate)) * up) (bindings.cpp:411-421)."""
    _check("swiglu", [(gate, "gate"), (up, "up")])
    if gate.shape != up.shape:
        raise RuntimeError("gate and up must have the same shape")
    if gate.dtype != torch.float16 or up.dtype != torch.float16:
        raise RuntimeError("swiglu expects fp16 input")
    out = torch.empty_like(gate)
    _call("srq_swiglu", _ptr(gate), _ptr(up), gate.numel(), _ptr(out), _stream(gate))
    return out


# -------------------------------------------------------------------- MoE

def swiglu_had_fusable(n, K):
    """Whether swiglu_had_sign_quant has a kernel for rotation size n = K x
    2^k (the MFMA rotation's shapes: H_512 chunks with 9 <= K <= 32, H_1024
    chunks with 9 <= K <= 28; K a multiple of 4)."""
    if K % 4:
        return False
    return (9 <= K <= 32 and n == K * 512) or (9 <= K <= 28 and n == K * 1024)


def swiglu_had_sign_quant(gu, hadK, K, sign=None, clip_ratio=1.0):
    """swiglu(gu[..., :n], gu[..., n:]) followed by had_sign_quant, one launch,
    for a gate/up projection output gu f16 [..., 2n]: (q u8 [..., n/2], scale
    f16 [..., 1])."""
    _check("swiglu_had_sign_quant", [(gu, "gu"), (hadK, "hadK"), (sign, "sign")],
           [torch.float16, torch.float16, torch.int8])
    if gu.shape[-1] % 2:
        raise RuntimeError("swiglu_had_sign_quant: the last dim must be 2n")
    n = gu.shape[-1] // 2
    _check_had("swiglu_had_sign_quant", n, hadK, K, sign, False)
    rows = gu.numel() // (2 * n) if n else 0
    q = torch.empty((*gu.shape[:-1], n // 2), dtype=torch.uint8, device=gu.device)
    scale = torch.empty((*gu.shape[:-1], 1), dtype=torch.float16, device=gu.device)
    if rows:
        gate = gu.view(rows, 2 * n)
        _call("srq_swiglu_had_sign_quant", _ptr(gate), gate[:, n:].data_ptr(), 2 * n, rows, n,
              int(K), _ptr(hadK), _ptr(sign), float(clip_ratio), _ptr(q), _ptr(scale),
              _stream(gu))
    return q, scale


def matmul_grouped(problem_sizes, ptr_A, ptr_B, ptr_C, lda, ldb, ldc, signed_a=True):
    """Grouped int4 GEMM, C_p = A_p · B_pᵀ (int32) per problem, all problem
    descriptors in device memory (bindings.cpp:49-91): problem_sizes int32
    [P, 3] rows (m, n, k); ptr_* int64 [P] device addresses; ld* int64 [P]
    row strides (codes for A/B, int32 elements for C).  Writes through ptr_C;
    returns None.  signed_a=False: A holds unsigned (asymmetric) codes, as
    matmul_ui4_si4."""
    name = "matmul_grouped"
    _check(name, [(problem_sizes, "problem_sizes"), (ptr_A, "ptr_A"), (ptr_B, "ptr_B"),
                  (ptr_C, "ptr_C"), (lda, "lda"), (ldb, "ldb"), (ldc, "ldc")])
    if problem_sizes.dtype != torch.int32 or problem_sizes.dim() != 2 or \
            problem_sizes.shape[1] != 3:
        raise RuntimeError("problem_sizes must be int32 [problem_count, 3] (m, n, k) rows")
    P = problem_sizes.shape[0]
    for t in (ptr_A, ptr_B, ptr_C, lda, ldb, ldc):
        if t.dtype != torch.int64 or t.numel() != P:
            raise RuntimeError("pointer/ld arrays must be int64 with one entry per problem")
    _call("srq_matmul_grouped", _ptr(problem_sizes), _ptr(ptr_A), _ptr(ptr_B), _ptr(ptr_C),
          _ptr(lda), _ptr(ldb), _ptr(ldc), P, 1 if signed_a else 0, _stream(problem_sizes))


def _moe_sign(name, sign, cols):
    if sign is None:
        return None
    _check(name, [(sign, "sign")])
    if sign.dtype != torch.int8 or sign.dim() != 2 or sign.shape[1] != cols:
        raise RuntimeError(f"{name}: sign must be int8 [num_experts, cols]")
    return sign


def sym_quant_dynamic_moe(x, sign, expert_ids, clip_ratio=1.0):
    """sym_quant_dynamic of expert-sorted rows with the per-expert sign fused:
    row r is multiplied by sign[expert_ids[r]] first (bindings.cpp:108-132).
    Returns (q u8 [rows, ceil(cols/2)], scale f16 [rows, 1])."""
    name = "sym_quant_dynamic_moe"
    _check(name, [(x, "x"), (expert_ids, "expert_ids")])
    if x.dim() != 2 or x.dtype != torch.float16:
        raise RuntimeError("sym_quant_dynamic_moe expects a 2D fp16 [rows, cols] tensor")
    if expert_ids.dtype != torch.int32 or expert_ids.numel() != x.shape[0]:
        raise RuntimeError("expert_ids must be int32 with one entry per row")
    rows, cols = x.shape
    sign = _moe_sign(name, sign, cols)
    if sign is not None:
        _check(name, [(x, "x"), (sign, "sign")])
    E = sign.shape[0] if sign is not None else 0
    q = torch.empty((rows, (cols + 1) // 2), dtype=torch.uint8, device=x.device)
    scale = torch.empty((rows, 1), dtype=torch.float16, device=x.device)
    _call("srq_sym_quant_dynamic_moe", _ptr(x), _ptr(sign), _ptr(expert_ids), E, rows, cols,
          float(clip_ratio), _ptr(q), _ptr(scale), _stream(x))
    return q, scale


def swiglu_had_sign_quant_moe(gate, up, hadK, K, sign, expert_ids, clip_ratio=1.0):
    """swiglu(gate, up) -> online Hadamard (had_K x H_{n/K}) -> per-expert
    sign -> per-token int4 quantizer, one launch, for the expert-sorted rows
    of the MoE down projection: gate, up f16 [rows, n], sign int8
    [num_experts, n] or None, expert_ids int32 [rows].  Bit-identical to
    swiglu, matmul_hadU_cuda, sym_quant_dynamic_moe.  Returns (q u8
    [rows, n/2], scale f16 [rows, 1])."""
    name = "swiglu_had_sign_quant_moe"
    _check(name, [(gate, "gate"), (up, "up"), (hadK, "hadK"), (expert_ids, "expert_ids")],
           [torch.float16, torch.float16, torch.float16, torch.int32])
    if gate.dim() != 2 or up.shape != gate.shape:
        raise RuntimeError(f"{name}: gate and up must be 2D and of one shape")
    rows, n = gate.shape
    if expert_ids.numel() != rows:
        raise RuntimeError(f"{name}: expert_ids must have one entry per row")
    _check_had(name, n, hadK, K, None, False)
    sign = _moe_sign(name, sign, n)
    E = sign.shape[0] if sign is not None else 0
    q = torch.empty((rows, n // 2), dtype=torch.uint8, device=gate.device)
    scale = torch.empty((rows, 1), dtype=torch.float16, device=gate.device)
    if rows:
        _call("srq_swiglu_had_sign_quant_moe", _ptr(gate), _ptr(up), n, rows, n, int(K),
              _ptr(hadK), _ptr(sign), _ptr(expert_ids), E, float(clip_ratio), _ptr(q),
              _ptr(scale), _stream(gate))
    return q, scale


def asym_quant_dynamic_moe(x, sign, expert_ids, clip_ratio=1.0):
    """asym_quant_dynamic of expert-sorted rows with the per-expert sign fused
    (bindings.cpp:134-159).  Returns (q u8 [rows, ceil(cols/2)] uint4 codes,
    scale f16 [rows, 1], zero f16 [rows, 1])."""
    name = "asym_quant_dynamic_moe"
    _check(name, [(x, "x"), (expert_ids, "expert_ids")])
    if x.dim() != 2 or x.dtype != torch.float16:
        raise RuntimeError("asym_quant_dynamic_moe expects a 2D fp16 [rows, cols] tensor")
    if expert_ids.dtype != torch.int32 or expert_ids.numel() != x.shape[0]:
        raise RuntimeError("expert_ids must be int32 with one entry per row")
    rows, cols = x.shape
    sign = _moe_sign(name, sign, cols)
    E = sign.shape[0] if sign is not None else 0
    q = torch.empty((rows, (cols + 1) // 2), dtype=torch.uint8, device=x.device)
    scale = torch.empty((rows, 1), dtype=torch.float16, device=x.device)
    zero = torch.empty((rows, 1), dtype=torch.float16, device=x.device)
    _call("srq_asym_quant_dynamic_moe", _ptr(x), _ptr(sign), _ptr(expert_ids), E, rows, cols,
          float(clip_ratio), _ptr(q), _ptr(scale), _ptr(zero), _stream(x))
    return q, scale, zero


def sym_dequant_moe(q, scale_row, w_scales, expert_ids, zero_row=None, w_sum=None):
    """Expert-indexed dequant (bindings.cpp:161-206): out f16 [rows, cols] =
    fp16((float(q - zero_row * w_sum[e]) * float(scale_row)) * float(w_scales[e]))
    with e = expert_ids[row]; the zero term only when zero_row/w_sum given."""
    name = "sym_dequant_moe"
    _check(name, [(q, "q"), (scale_row, "scale_row"), (w_scales, "w_scales"),
                  (expert_ids, "expert_ids"), (zero_row, "zero_row"), (w_sum, "w_sum")])
    if q.dim() != 2 or q.dtype != torch.int32:
        raise RuntimeError("q must be int32 [rows, cols]")
    rows, cols = q.shape
    if scale_row.dtype != torch.float16 or scale_row.numel() != rows:
        raise RuntimeError("scale_row must be fp16 with one entry per row")
    if w_scales.dtype != torch.float16 or w_scales.dim() != 2 or w_scales.shape[1] != cols:
        raise RuntimeError("w_scales must be fp16 [num_experts, cols]")
    if expert_ids.dtype != torch.int32 or expert_ids.numel() != rows:
        raise RuntimeError("expert_ids must be int32 with one entry per row")
    if (zero_row is None) != (w_sum is None):
        raise RuntimeError("zero_row and w_sum must be given together")
    if zero_row is not None:
        if zero_row.dtype != torch.int8 or zero_row.numel() != rows:
            raise RuntimeError("zero_row must be int8 with one entry per row")
        if w_sum.dtype != torch.int32 or w_sum.dim() != 2 or w_sum.shape[1] != cols or \
                w_sum.shape[0] != w_scales.shape[0]:
            raise RuntimeError("w_sum must be int32 [num_experts, cols]")
    out = torch.empty((rows, cols), dtype=torch.float16, device=q.device)
    _call("srq_sym_dequant_moe", _ptr(q), _ptr(scale_row), _ptr(w_scales), _ptr(expert_ids),
          _ptr(zero_row), _ptr(w_sum), w_scales.shape[0], rows, cols, _ptr(out), _stream(q))
    return out


def w4a4_linear_moe(A, a_scale, B, b_scale, expert_offsets):
    """Fused grouped GEMM + expert-indexed dequant over expert-sorted rows:
    expert e owns rows expert_offsets[e] .. expert_offsets[e + 1] (int32
    [E + 1], device) of A u8 [R, K/2]; B u8 [E, N, K/2]; b_scale f16 [E, N];
    returns fp16 [R, N] (rows owned by no expert are left uninitialised)."""
    name = "w4a4_linear_moe"
    _check(name, [(A, "A"), (a_scale, "a_scale"), (B, "B"), (b_scale, "b_scale"),
                  (expert_offsets, "expert_offsets")],
           [torch.uint8, torch.float16, torch.uint8, torch.float16, torch.int32])
    if A.dim() != 2 or B.dim() != 3 or B.shape[2] != A.shape[1]:
        raise RuntimeError(f"{name}: expected A [R, K/2] and B [E, N, K/2], got "
                           f"{tuple(A.shape)} and {tuple(B.shape)}")
    R, E, N, K = A.shape[0], B.shape[0], B.shape[1], A.shape[1] * 2
    if a_scale.numel() != R or tuple(b_scale.shape) != (E, N):
        raise RuntimeError(f"{name}: a_scale must have R entries and b_scale be [E, N]")
    if expert_offsets.numel() != E + 1:
        raise RuntimeError(f"{name}: expert_offsets must have num_experts + 1 entries")
    out = torch.empty((R, N), dtype=torch.float16, device=A.device)
    _call("srq_w4a4_linear_moe", _ptr(A), _ptr(a_scale), _ptr(B), _ptr(b_scale),
          _ptr(expert_offsets), E, R, N, K, _ptr(out), _stream(A))
    return out


def w4a4_linear_moe_gate_up(A, a_scale, B_gate, s_gate, B_up, s_up, expert_offsets):
    """The MoE block's gate and up projections in one launch: (out_gate,
    out_up), each bit-identical to w4a4_linear_moe with its B / scales (the
    two _gemm_dequant_grouped calls of moe.py:187-190)."""
    name = "w4a4_linear_moe_gate_up"
    _check(name, [(A, "A"), (a_scale, "a_scale"), (B_gate, "B_gate"), (s_gate, "s_gate"),
                  (B_up, "B_up"), (s_up, "s_up"), (expert_offsets, "expert_offsets")],
           [torch.uint8, torch.float16, torch.uint8, torch.float16, torch.uint8, torch.float16,
            torch.int32])
    if A.dim() != 2 or B_gate.dim() != 3 or B_gate.shape[2] != A.shape[1]:
        raise RuntimeError(f"{name}: expected A [R, K/2] and B [E, N, K/2], got "
                           f"{tuple(A.shape)} and {tuple(B_gate.shape)}")
    if tuple(B_up.shape) != tuple(B_gate.shape) or tuple(s_up.shape) != tuple(s_gate.shape):
        raise RuntimeError(f"{name}: gate and up weights must have the same shapes")
    R, E, N, K = A.shape[0], B_gate.shape[0], B_gate.shape[1], A.shape[1] * 2
    if a_scale.numel() != R or tuple(s_gate.shape) != (E, N):
        raise RuntimeError(f"{name}: a_scale must have R entries and the scales be [E, N]")
    if expert_offsets.numel() != E + 1:
        raise RuntimeError(f"{name}: expert_offsets must have num_experts + 1 entries")
    out_g = torch.empty((R, N), dtype=torch.float16, device=A.device)
    out_u = torch.empty((R, N), dtype=torch.float16, device=A.device)
    _call("srq_w4a4_linear_moe_gate_up", _ptr(A), _ptr(a_scale), _ptr(B_gate), _ptr(s_gate),
          _ptr(B_up), _ptr(s_up), _ptr(expert_offsets), E, R, N, K, _ptr(out_g), _ptr(out_u),
          _stream(A))
    return out_g, out_u


def interleave_gate_up_experts(w_gate, s_gate, w_up, s_up):
    """Per-expert gate and up weights [E, ffn, K/2] (scales [E, ffn]) as one
    [E, 2 ffn, K/2] tensor with the rows interleaved in blocks of 8 (gate
    rows 8 c .. then up rows 8 c ..), the layout w4a4_linear_moe_swiglu
    reads; scales likewise.  A copy (weight preparation, done once)."""
    E, ffn = w_gate.shape[0], w_gate.shape[1]
    if ffn % 8 or tuple(w_up.shape) != tuple(w_gate.shape):
        raise RuntimeError("interleave_gate_up_experts: gate/up [E, ffn, ...], ffn % 8 == 0")

    def il(g, u):
        rest = g.shape[2:]
        return torch.stack([g.reshape(E, ffn // 8, 8, *rest), u.reshape(E, ffn // 8, 8, *rest)],
                           dim=2).reshape(E, 2 * ffn, *rest).contiguous()
    return il(w_gate, w_up), il(s_gate, s_up)


def w4a4_linear_moe_swiglu(A, a_scale, B_il, s_il, expert_offsets):
    """swiglu(gate, up) of the MoE block's gate/up projections in one
    launch, B_il / s_il from interleave_gate_up_experts: out f16 [R, ffn],
    bit-identical to w4a4_linear_moe_gate_up then swiglu."""
    name = "w4a4_linear_moe_swiglu"
    _check(name, [(A, "A"), (a_scale, "a_scale"), (B_il, "B"), (s_il, "b_scale"),
                  (expert_offsets, "expert_offsets")],
           [torch.uint8, torch.float16, torch.uint8, torch.float16, torch.int32])
    if A.dim() != 2 or B_il.dim() != 3 or B_il.shape[2] != A.shape[1]:
        raise RuntimeError(f"{name}: expected A [R, K/2] and B [E, N, K/2]")
    R, E, N, K = A.shape[0], B_il.shape[0], B_il.shape[1], A.shape[1] * 2
    if a_scale.numel() != R or tuple(s_il.shape) != (E, N):
        raise RuntimeError(f"{name}: a_scale must have R entries and the scales be [E, N]")
    if expert_offsets.numel() != E + 1:
        raise RuntimeError(f"{name}: expert_offsets must have num_experts + 1 entries")
    out = torch.empty((R, N // 2), dtype=torch.float16, device=A.device)
    _call("srq_w4a4_linear_moe_swiglu", _ptr(A), _ptr(a_scale), _ptr(B_il), _ptr(s_il),
          _ptr(expert_offsets), E, R, N, K, _ptr(out), _stream(A))
    return out


def had_sign_quant_moe(x, hadK, K, sign, expert_ids, clip_ratio=1.0):
    """swiglu_had_sign_quant_moe for an input already through the SwiGLU:
    x f16 [rows, n] -> online Hadamard (had_K x H_{n/K}) -> per-expert sign
    -> per-token int4 quantizer, one launch; bit-identical to
    matmul_hadU_cuda then sym_quant_dynamic_moe.  Returns (q u8 [rows, n/2],
    scale f16 [rows, 1])."""
    name = "had_sign_quant_moe"
    _check(name, [(x, "x"), (hadK, "hadK"), (expert_ids, "expert_ids")],
           [torch.float16, torch.float16, torch.int32])
    if x.dim() != 2:
        raise RuntimeError(f"{name}: x must be 2D")
    rows, n = x.shape
    if expert_ids.numel() != rows:
        raise RuntimeError(f"{name}: expert_ids must have one entry per row")
    _check_had(name, n, hadK, K, None, False)
    sign = _moe_sign(name, sign, n)
    E = sign.shape[0] if sign is not None else 0
    q = torch.empty((rows, n // 2), dtype=torch.uint8, device=x.device)
    scale = torch.empty((rows, 1), dtype=torch.float16, device=x.device)
    if rows:
        _call("srq_had_sign_quant_moe", _ptr(x), rows, n, int(K), _ptr(hadK), _ptr(sign),
              _ptr(expert_ids), E, float(clip_ratio), _ptr(q), _ptr(scale), _stream(x))
    return q, scale


def moe_route(logits, top_k, norm_topk_prob):
    """Routing of the MoE block in one launch (moe.py:168-185): returns
    (weights fp16 [T, k], order, inv, expert, token int32 [T k], counts int32
    [E], offsets int32 [E + 1]); see srq_moe_route."""
    name = "moe_route"
    _check(name, [(logits, "logits")], [torch.float16])
    if logits.dim() != 2:
        raise RuntimeError(f"{name}: logits must be [tokens, num_experts]")
    T, E = logits.shape
    dev = logits.device
    R = T * top_k
    weights = torch.empty((T, top_k), dtype=torch.float16, device=dev)
    ints = torch.empty((5, R), dtype=torch.int32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    choice, order, inv, expert, token = ints.unbind(0)
    _call("srq_moe_route", _ptr(logits), T, E, top_k, 1 if norm_topk_prob else 0, _ptr(weights),
          _ptr(choice), _ptr(order), _ptr(inv), _ptr(expert), _ptr(token), _ptr(counts),
          _ptr(offsets), _stream(logits))
    return weights, order, inv, expert, token, counts, offsets


def moe_combine(y, inv, weights):
    """out [T, H] = sum_j fp16(y[inv[t k + j]] * weights[t, j]) in fp32,
    rounded to fp16 (moe.py:226-230)."""
    name = "moe_combine"
    _check(name, [(y, "y"), (inv, "inv"), (weights, "weights")],
           [torch.float16, torch.int32, torch.float16])
    T, k = weights.shape
    if y.dim() != 2 or y.shape[0] != T * k or inv.numel() != T * k:
        raise RuntimeError(f"{name}: y must be [T k, H] and inv [T k] for weights [T, k]")
    out = torch.empty((T, y.shape[1]), dtype=torch.float16, device=y.device)
    _call("srq_moe_combine", _ptr(y), _ptr(inv), _ptr(weights), T, k, y.shape[1], _ptr(out),
          _stream(y))
    return out


def w4a4_linear_moe_asym(A, a_scale, a_zero, B, b_scale, b_sum, expert_offsets):
    """w4a4_linear_moe for asymmetric (uint4) activation codes: the int32
    product minus a_zero[row] * b_sum[e, col] before the dequant; a_zero int8
    [R], b_sum int32 [E, N].  Bit-identical to matmul_grouped(signed_a=False)
    + sym_dequant_moe(zero_row, w_sum)."""
    name = "w4a4_linear_moe_asym"
    _check(name, [(A, "A"), (a_scale, "a_scale"), (a_zero, "a_zero"), (B, "B"),
                  (b_scale, "b_scale"), (b_sum, "b_sum"), (expert_offsets, "expert_offsets")],
           [torch.uint8, torch.float16, torch.int8, torch.uint8, torch.float16, torch.int32,
            torch.int32])
    if A.dim() != 2 or B.dim() != 3 or B.shape[2] != A.shape[1]:
        raise RuntimeError(f"{name}: expected A [R, K/2] and B [E, N, K/2], got "
                           f"{tuple(A.shape)} and {tuple(B.shape)}")
    R, E, N, K = A.shape[0], B.shape[0], B.shape[1], A.shape[1] * 2
    if a_scale.numel() != R or a_zero.numel() != R or tuple(b_scale.shape) != (E, N):
        raise RuntimeError(f"{name}: a_scale / a_zero must have R entries, b_scale be [E, N]")
    if tuple(b_sum.shape) != (E, N):
        raise RuntimeError(f"{name}: b_sum must be [E, N]")
    if expert_offsets.numel() != E + 1:
        raise RuntimeError(f"{name}: expert_offsets must have num_experts + 1 entries")
    out = torch.empty((R, N), dtype=torch.float16, device=A.device)
    _call("srq_w4a4_linear_moe_asym", _ptr(A), _ptr(a_scale), _ptr(a_zero), _ptr(B),
          _ptr(b_scale), _ptr(b_sum), _ptr(expert_offsets), E, R, N, K, _ptr(out), _stream(A))
    return out
