"""ctypes binding of libsignrot_hip.so (the C ABI declared in include/signrot_hip.h).

The library is loaded once, from signrot_amd/_lib/.  There is no fallback:
if the library is missing the import of the op table raises, so a GPU run
can never silently use a CPU or PyTorch path instead of the HIP kernels.
"""
import ctypes
import pathlib

LIB_PATH = pathlib.Path(__file__).resolve().parent / "_lib" / "libsignrot_hip.so"

_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_p = ctypes.c_void_p

# name -> argtypes (restype is int for all compute entry points)
SIGNATURES = {
    "srq_sym_quant_dynamic": [_p, _i64, _i64, _f32, _p, _p, _p],
    "srq_sym_quant_dynamic_rows": [_p, _i64, _p, _i64, _i64, _f32, _p, _p, _p],
    "srq_sym_quant": [_p, _p, _i64, _i64, _p, _p],
    "srq_sym_dequant": [_p, _p, _p, _i64, _i64, _p, _p],
    "srq_kv_quant_pack": [_p, _i64, _i64, _p, _p, _p],
    "srq_matmul_s4s4": [_p, _p, _i64, _i64, _i64, _p, _p],
    "srq_w4a4_linear": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p],
    "srq_w4a4_linear_swiglu": [_p, _p, _p, _p, _i64, _i64, _i64, _p, _p],
    "srq_w4a4_linear_residual": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p],
    "srq_w4a4_linear_ws": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p, _i64, _p],
    "srq_w4a4_linear_residual_ws": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p, _i64,
                                    _p],
    "srq_matmul_u4s4": [_p, _p, _i64, _i64, _i64, _p, _p],
    "srq_w4a4_linear_asym": [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p],
    "srq_w4a4_linear_moe_asym": [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _p],
    "srq_had_sign_asym_quant": [_p, _i64, _i64, _i64, _p, _p, _f32, _p, _p, _p, _p],
    "srq_asym_quant_dynamic": [_p, _i64, _i64, _f32, _p, _p, _p, _p],
    "srq_asym_quant_dynamic_moe": [_p, _p, _p, _i64, _i64, _i64, _f32, _p, _p, _p, _p],
    "srq_asym_quant": [_p, _p, _p, _i64, _i64, _i32, _p, _p],
    "srq_sum_i4": [_p, _i64, _i64, _i32, _p, _p],
    "srq_matmul_colrow_i8_i32": [_p, _p, _i64, _i64, _p, _p],
    "srq_i4_to_bf6": [_p, _i64, _i64, _p, _p],
    "srq_had_sign_quant_bf6": [_p, _i64, _i64, _i64, _p, _p, _f32, _p, _p, _p],
    "srq_matmul_bf6": [_p, _p, _i64, _i64, _i64, _p, _p],
    "srq_w4a4_linear_bf6": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p],
    "srq_swiglu_had_sign_quant_moe": [_p, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _i64, _f32,
                                      _p, _p, _p],
    "srq_hadamard_transform": [_p, _p, _i64, _i64, _f32, _i32, _p],
    "srq_online_hadamard": [_p, _p, _i64, _i64, _i64, _p, _p, _i32, _p],
    "srq_had_sign_quant": [_p, _i64, _i64, _i64, _p, _p, _i32, _f32, _p, _p, _p],
    "srq_swiglu_had_sign_quant": [_p, _p, _i64, _i64, _i64, _i64, _p, _p, _f32, _p, _p, _p],
    "srq_append_kv_i4": [_p, _p, _p, _p, _p, _p, _p, _p, _p,
                         _i64, _i64, _i64, _i64, _i64, _i64, _p],
    "srq_init_kv_i4": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                       _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p],
    "srq_batch_decode_i4": [_p, _p, _p, _p, _p, _p, _p,
                            _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "srq_qkv_decode_i4": [_p, _p, _p, _p, _i64, _f32, _i32, _p, _p, _p, _p, _p,
                          _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "srq_batch_decode_i4_noalloc": [_p, _p, _p, _p, _p, _p, _p,
                                    _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p],
    "srq_prefill_attention": [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                              _i64, _i64, _f32, _i32, _p, _p],
    "srq_rmsnorm": [_p, _i64, _i64, _f32, _i64, _p, _p],
    "srq_rmsnorm_quant": [_p, _i64, _i64, _f32, _i64, _f32, _p, _p, _p, _p],
    "srq_head_had_quant": [_p, _i64, _i64, _i64, _f32, _f32, _p, _p, _p, _p],
    "srq_merge_head_had_quant": [_p, _i64, _i64, _i64, _i64, _f32, _f32, _p, _p, _p, _p],
    "srq_qkv_rope_had_append": [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _i32,
                                _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p],
    "srq_rope_qk": [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p],
    "srq_swiglu": [_p, _p, _i64, _p, _p],
    "srq_matmul_grouped": [_p, _p, _p, _p, _p, _p, _p, _i64, _i32, _p],
    "srq_w4a4_linear_moe": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _p],
    "srq_w4a4_linear_moe_gate_up": [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _p,
                                    _p],
    "srq_w4a4_linear_moe_swiglu": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _p],
    "srq_had_sign_quant_moe": [_p, _i64, _i64, _i64, _p, _p, _p, _i64, _f32, _p, _p, _p],
    "srq_moe_route": [_p, _i64, _i64, _i64, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _p],
    "srq_moe_combine": [_p, _p, _p, _i64, _i64, _i64, _p, _p],
    "srq_sym_quant_dynamic_moe": [_p, _p, _p, _i64, _i64, _i64, _f32, _p, _p, _p],
    "srq_sym_dequant_moe": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p],
}


class NativeError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


_lib = None


def lib():
    """The loaded library (raises RuntimeError if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"signrot_amd: HIP library not found at {LIB_PATH}; build it with "
                "`python -m signrot_amd.csrc.build` (no CPU fallback exists)")
        handle = ctypes.CDLL(str(LIB_PATH))
        handle.srq_last_error.restype = ctypes.c_char_p
        handle.srq_last_error.argtypes = []
        handle.srq_abi_version.restype = ctypes.c_int
        handle.srq_abi_version.argtypes = []
        handle.srq_bf6_bytes.restype = ctypes.c_int64
        handle.srq_bf6_bytes.argtypes = [_i64, _i64]
        handle.srq_w4a4_linear_ws_bytes.restype = ctypes.c_int64
        handle.srq_w4a4_linear_ws_bytes.argtypes = [_i64, _i64, _i64]
        for name, args in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        _lib = handle
    return _lib


def call(name, *args):
    """Call entry point `name`; raise NativeError (a RuntimeError) on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().srq_last_error().decode(errors="replace")
        raise NativeError(f"{name} failed ({rc}): {msg}")
