"""CPU checks of the bf6 block layout statement used by the GPU tests, and
of the bf6 entry points' argument checks (no compute call)."""
import ctypes

import numpy as np
import pytest

from tests.bf6_layout import BLOCK, e3m2_code, e3m2_value, encode


def test_e3m2_codes_are_exact_integers():
    c = np.arange(-8, 8)
    assert np.array_equal(e3m2_value(e3m2_code(c)), c)
    # distinct patterns, zero is all-zero bits, sign is bit 5
    assert len(set(e3m2_code(c).tolist())) == 16
    assert e3m2_code(0) == 0
    assert np.all((e3m2_code(c[c < 0]) & 32) == 32)


def test_layout_places_each_code_in_its_lane_field():
    R, K = 70, 256
    rng = np.random.default_rng(3)
    base = rng.integers(-8, 8, (R, K))
    enc = encode(base)
    assert enc.size == -(-R // 32) * (K // 128) * BLOCK
    for (r, k) in [(0, 0), (31, 63), (32, 64), (69, 255), (5, 33), (40, 100), (7, 200)]:
        rb, kb, q, h, j = r // 32, k // 128, (k % 128) // 64, (k % 64) // 32, k % 32
        lane = r % 32 + 32 * h
        blk = enc[(rb * (K // 128) + kb) * BLOCK:][:BLOCK]
        lane_bytes = np.concatenate([blk[1024 * q + 16 * lane:][:16],
                                     blk[2048 + 16 * lane + 8 * q:][:8]])
        bits = np.unpackbits(lane_bytes, bitorder="little")
        field = int(sum(int(bits[6 * j + b]) << b for b in range(6)))
        assert field == e3m2_code(base[r, k]), (r, k)
    # padded rows are zero codes
    pad = encode(np.zeros((R, K), np.int64))
    assert not pad.any()


def test_bf6_bytes_formula():
    from signrot_amd import _native
    lib = _native.lib()
    for rows, K in [(1, 128), (32, 128), (33, 256), (2048, 14336), (0, 128)]:
        assert lib.srq_bf6_bytes(rows, K) == -(-rows // 32) * (K // 128) * BLOCK
    assert lib.srq_bf6_bytes(4, 64) == -1


@pytest.mark.parametrize("M,N,K", [(4, 4, 64), (4, 4, 100), (4, 4, 131072)])
def test_bf6_gemm_rejects_bad_k(M, N, K):
    from signrot_amd import _native
    lib = _native.lib()
    buf = ctypes.create_string_buffer(64)
    rc = lib.srq_matmul_bf6(ctypes.addressof(buf), ctypes.addressof(buf), M, N, K,
                            ctypes.addressof(buf), None)
    assert rc != 0
    assert b"K=" in lib.srq_last_error()


def test_i4_to_bf6_rejects_bad_k():
    from signrot_amd import _native
    lib = _native.lib()
    buf = ctypes.create_string_buffer(64)
    assert lib.srq_i4_to_bf6(ctypes.addressof(buf), 4, 64, ctypes.addressof(buf), None) != 0
    assert lib.srq_i4_to_bf6(None, 0, 128, None, None) == 0  # empty: no-op
