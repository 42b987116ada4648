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
"""
import torch

from . import _native

_call = _native.call


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _check(name, tensors, dtypes=None):
    dev = None
    for i, (t, tname) in enumerate(tensors):
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise RuntimeError(f"{name}: argument '{tname}' must be a tensor")
        if t.device.type != "cuda":
            raise RuntimeError(
                f"{name}: expected '{tname}' on a GPU device, got {t.device}")
        if not t.is_contiguous():
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
    _call("srq_w4a4_linear", _ptr(A), _ptr(a_scale), _ptr(B), _ptr(b_scale), _ptr(bias),
          M, N, K, _ptr(out), _stream(A))
    return out


# ------------------------------------------------------------------ quant

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


def batch_decode_i4(o, q, kv_data, kv_param, kv_indptr, kv_indices, last_page_offset,
                    layer_idx, tmp=None, num_chunks=1):
    """Single-query attention over the int4 cache into o [B, Hq, 128]
    (bindings.cpp:508-559).  Hq may be 1..8 times the cache's head count."""
    L, H, P, D = _check_cache("batch_decode_i4", kv_data, kv_param, kv_indptr, kv_indices,
                              last_page_offset)
    _check("batch_decode_i4", [(o, "o"), (q, "q"), (kv_data, "kv_data")],
           [torch.float16, torch.float16, None])
    if o.dim() != 3 or q.dim() != 3 or o.shape != q.shape:
        raise RuntimeError("batch_decode_i4: o and q must be the same [B, N, D] shape")
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
