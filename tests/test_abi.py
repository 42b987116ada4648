"""CPU checks of the C-ABI library: it loads, exports every symbol that
include/signrot_hip.h declares, and rejects bad arguments with an error code
and message before touching a device (no compute call is made here)."""
import ctypes
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "signrot_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(srq_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from signrot_amd import _native
    return _native.lib()


def test_exports_every_declared_symbol(lib):
    names = _declared()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), f"missing export {n}"


def test_python_signatures_cover_header():
    from signrot_amd import _native
    declared = set(_declared()) - {"srq_last_error", "srq_abi_version", "srq_bf6_bytes",
                                   "srq_w4a4_linear_ws_bytes"}
    assert declared == set(_native.SIGNATURES), declared ^ set(_native.SIGNATURES)


def test_abi_version(lib):
    assert lib.srq_abi_version() >= 1


@pytest.mark.parametrize("call,msg", [
    (lambda L: L.srq_sym_quant_dynamic(None, -1, 4, 1.0, None, None, None), "negative"),
    (lambda L: L.srq_kv_quant_pack(None, 4, 7, None, None, None), "even"),
    (lambda L: L.srq_matmul_s4s4(None, None, 4, 4, 48, None, None), "multiple of 32"),
    (lambda L: L.srq_matmul_s4s4(None, None, 4, 4, 262144, None, None), "131072"),
    # 2^14 * 131072 = 2^31 wraps the int32 accumulator: the bound is strict
    (lambda L: L.srq_matmul_s4s4(None, None, 4, 4, 131072, None, None), "131072"),
    (lambda L: L.srq_w4a4_linear_moe(None, None, None, None, None, 8, 16, 64, 131072, None,
                                     None), "131072"),
    (lambda L: L.srq_hadamard_transform(None, None, 4, 24, 1.0, 0, None), "power of two"),
    (lambda L: L.srq_online_hadamard(None, None, 4, 14336, 28, None, None, 0, None), "hadK"),
    (lambda L: L.srq_had_sign_quant(None, 4, 21 * 64, 3, None, None, 0, 1.0, None, None,
                                    None), "power of two"),
    (lambda L: L.srq_w4a4_linear(ctypes.c_void_p(8), None, ctypes.c_void_p(16), None, None, 4,
                                 4, 64, None, None), "aligned"),
    (lambda L: L.srq_matmul_grouped(None, None, None, None, None, None, None, 3, 1, None),
     "null"),
    (lambda L: L.srq_w4a4_linear_moe(None, None, None, None, None, 8, 16, 64, 48, None, None),
     "multiple of 32"),
    (lambda L: L.srq_sym_quant_dynamic_moe(None, None, None, 4, -1, 8, 1.0, None, None, None),
     "negative"),
    (lambda L: L.srq_sym_dequant_moe(None, None, None, None, ctypes.c_void_p(8), None, 4, 4, 4,
                                     None, None), "together"),
    # split-K workspaces are read and written 16 bytes at a time
    (lambda L: L.srq_w4a4_linear_ws(*[ctypes.c_void_p(256)] * 4, None, 256, 256, 1024,
                                    ctypes.c_void_p(256), ctypes.c_void_p(264), 64, None),
     "16-byte aligned"),
    (lambda L: L.srq_w4a4_linear_residual_ws(*[ctypes.c_void_p(256)] * 4, None,
                                             ctypes.c_void_p(256), 256, 256, 1024,
                                             ctypes.c_void_p(256), ctypes.c_void_p(8), 64, None),
     "16-byte aligned"),
    # the fused q/k/v + decode entry point checks its rotary-table batch
    (lambda L: L.srq_qkv_decode_i4(None, None, None, None, 3, ctypes.c_float(1.0), 1,
                                   *[ctypes.c_void_p(256)] * 5, 2, 8, 2, 1, 0, 16, 128, None, 1,
                                   None), "cos/sin batch"),
    # the scale goes into the exponent with its sign applied to q: it must be finite
    (lambda L: L.srq_prefill_attention(None, None, None, None, 1, 4, 4, 4, 128, 512, 2048, 512,
                                       2048, ctypes.c_float(float("nan")), 1, None, None),
     "sm_scale"),
    # the prefill kernel's linear block id over (q tile, head group) is 32-bit
    (lambda L: L.srq_prefill_attention(*[ctypes.c_void_p(256)] * 3, None, 1, 1 << 30, 65528,
                                       8191, 128, 65528 * 128, (1 << 30) * 65528 * 128,
                                       8191 * 128, (1 << 30) * 8191 * 128,
                                       ctypes.c_float(0.088), 1, ctypes.c_void_p(256), None),
     "too large"),
    # the no-allocation decode has nowhere to leave unmerged split-KV states
    (lambda L: L.srq_batch_decode_i4_noalloc(None, *[ctypes.c_void_p(256)] * 6, 2, 32, 8, 1, 0,
                                             64, 128, 4, None), "null output"),
])
def test_argument_errors(lib, call, msg):
    rc = call(lib)
    assert rc == -1
    assert msg in lib.srq_last_error().decode()


def test_empty_inputs_are_noops(lib):
    assert lib.srq_sym_quant_dynamic(None, 0, 4096, 1.0, None, None, None) == 0
    assert lib.srq_matmul_s4s4(None, None, 0, 16, 64, None, None) == 0
    assert lib.srq_kv_quant_pack(None, 0, 128, None, None, None) == 0
    assert lib.srq_matmul_grouped(None, None, None, None, None, None, None, 0, 1, None) == 0
    assert lib.srq_sym_dequant_moe(None, None, None, None, None, None, 8, 0, 16, None, None) == 0


def test_asym_argument_errors(lib):
    z = ctypes.c_void_p(16)
    assert lib.srq_asym_quant_dynamic(z, 4, 0, 1.0, z, z, z, None) == -1
    assert "empty rows" in lib.srq_last_error().decode()
    assert lib.srq_asym_quant_dynamic_moe(z, z, None, 4, 4, 8, 1.0, z, z, z, None) == -1
    assert "expert_ids" in lib.srq_last_error().decode()
    assert lib.srq_matmul_u4s4(None, None, 4, 4, 48, None, None) == -1
    assert "multiple of 32" in lib.srq_last_error().decode()
    assert lib.srq_w4a4_linear_asym(z, z, None, z, z, z, None, 4, 4, 64, z, None) == -1
    assert "null" in lib.srq_last_error().decode()
    # empty inputs are no-ops
    assert lib.srq_sum_i4(None, 0, 16, 1, None, None) == 0
    assert lib.srq_matmul_colrow_i8_i32(None, None, 0, 8, None, None) == 0
    assert lib.srq_asym_quant(None, None, None, 0, 8, 0, None, None) == 0
