"""Pins of oracle/quant.py against exact arithmetic (fractions, Python
ints, binary32 rounding through struct) and the reference test suite's
cases (benchmarks/test_fused_equivalence.py:33-90)."""
import struct
from fractions import Fraction

import numpy as np
import pytest

from oracle import quant as oq
from tests.exact import f32, round_half_even, to_f16, to_f32


def _exact_code(x16, s16):
    """clamp(round_half_even(fp16(x / s)), -8, 7) from exact rationals."""
    x, s = Fraction(float(x16)), Fraction(float(s16))
    if s == 0:
        if x == 0:
            return 0  # 0/0 = NaN -> 0
        return 7 if x > 0 else -8
    q16 = to_f16(x / s)
    if q16 in (np.inf, -np.inf):
        return 7 if q16 > 0 else -8
    return max(-8, min(7, round_half_even(q16)))


def test_codes_match_exact_rational_division():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(3000) * 3).astype(np.float16)
    s = np.abs(rng.standard_normal(3000)).astype(np.float16) + np.float16(0.05)
    for xi, si in zip(x, s):
        assert oq.sym_codes(np.array([[xi]]), np.array([si]))[0, 0] == _exact_code(xi, si)


def test_codes_at_half_integer_ties():
    # x / s landing exactly on, or within an fp16 ulp of, k + 0.5: the fp16
    # quotient rounds first, then ties go to even
    cases = []
    for s in [np.float16(0.25), np.float16(0.1), np.float16(1.0 / 7), np.float16(3.3)]:
        for k in range(-8, 8):
            for d in (-2, -1, 0, 1, 2):
                t = Fraction(2 * k + 1, 2) * Fraction(float(s))
                x = np.float16(float(t))
                x = np.nextafter(x, np.float16(np.inf if d > 0 else -np.inf), dtype=np.float16) \
                    if d else x
                if d in (-2, 2):
                    x = np.nextafter(x, np.float16(np.inf if d > 0 else -np.inf),
                                     dtype=np.float16)
                cases.append((x, s))
    for x, s in cases:
        assert oq.sym_codes(np.array([[x]]), np.array([s]))[0, 0] == _exact_code(x, s), (x, s)


def test_scale_matches_exact_rule():
    rng = np.random.default_rng(1)
    for _ in range(500):
        row = (rng.standard_normal(64) * 10 ** rng.uniform(-5, 3)).astype(np.float16)
        amax = Fraction(float(np.abs(row.astype(np.float64)).max()))
        want = to_f16(to_f32(amax / 7))
        assert float(oq.sym_scale(row[None])[0]) == float(want)
    # clip != 1: fp16(float(scale) * clip)
    row = np.array([[3.0, -5.5, 1.0]], np.float16)
    s0 = to_f16(to_f32(Fraction(5.5) / 7))
    want = to_f16(to_f32(s0 * Fraction(f32(0.9))))
    assert float(oq.sym_scale(row, 0.9)[0]) == float(want)


@pytest.mark.parametrize("name", ["zeros", "spike", "range", "tiny", "negative"])
def test_reference_edge_cases(name):
    rng = np.random.default_rng(5)
    if name == "zeros":
        x = np.zeros((4, 4096), np.float16)
    elif name == "spike":
        x = np.zeros((4, 4096), np.float16)
        x[1, 7] = 100.0
    elif name == "range":
        x = (rng.standard_normal((4, 4096)) * 1e3).astype(np.float16)
    elif name == "tiny":
        x = (rng.standard_normal((4, 4096)) * 1e-4).astype(np.float16)
    else:
        x = -(rng.random((4, 4096)) + 1).astype(np.float16)
    q, s = oq.sym_quant_dynamic(x)
    codes = oq.unpack_i4(q)
    assert codes.min() >= -7 and codes.max() <= 7  # clip 1: |x| <= amax -> |code| <= 7
    if name == "zeros":
        assert np.all(s == 0) and np.all(codes == 0)
    if name == "spike":
        assert float(s[1, 0]) == float(np.float16(100.0 / 7))
        assert codes[1, 7] == 7 and np.count_nonzero(codes) == 1
        assert np.all(s[[0, 2, 3]] == 0)
    if name == "negative":
        # the row minimum maps to -7 in every row
        assert np.all(codes[np.arange(4), np.argmin(x.astype(np.float32), axis=1)] == -7)
    # spot-check the exact rule on a sample of elements
    for r in range(4):
        for c in rng.integers(0, 4096, 32):
            assert codes[r, c] == _exact_code(x[r, c], s[r, 0])


def test_zero_scale_with_nonzero_input_saturates():
    # amax/7 underflows fp16 when amax is the smallest subnormals
    x = np.array([[np.float16(2 ** -24), -np.float16(2 ** -24), 0.0, 0.0]], np.float16)
    q, s = oq.sym_quant_dynamic(x)
    assert float(s[0, 0]) == 0.0
    assert oq.unpack_i4(q)[0].tolist() == [7, -8, 0, 0]


def test_pack_known_bytes_and_round_trip():
    q = np.array([[1, -1, -8, 7, 0, 3]], np.int8)
    p = oq.pack_i4(q)
    assert p.tolist() == [[0xF1, 0x78, 0x30]]
    rng = np.random.default_rng(2)
    q = rng.integers(-8, 8, (5, 64)).astype(np.int8)
    assert np.array_equal(oq.unpack_i4(oq.pack_i4(q)), q)
    # odd column count: high nibble of the last byte is zero
    assert oq.pack_i4(np.array([[-1, 2, -3]], np.int8)).tolist() == [[0x2F, 0x0D]]


def test_matmul_matches_python_triple_loop():
    rng = np.random.default_rng(3)
    M, N, K = 3, 5, 64
    a = rng.integers(0, 256, (M, K // 2)).astype(np.uint8)
    b = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)

    def nib(byte, hi):
        v = (int(byte) >> 4) if hi else (int(byte) & 0xF)
        return v - 16 if v >= 8 else v

    got = oq.matmul_s4s4(a, b)
    for i in range(M):
        for j in range(N):
            acc = 0
            for k in range(K):
                acc += nib(a[i, k // 2], k % 2) * nib(b[j, k // 2], k % 2)
            assert got[i, j] == acc


def test_matmul_extreme_accumulator():
    K = 28672
    a = np.full((2, K // 2), 0x88, np.uint8)  # all -8
    b = np.full((3, K // 2), 0x88, np.uint8)
    assert np.all(oq.matmul_s4s4(a, b) == 64 * K)


def test_dequant_matches_binary32_arithmetic():
    rng = np.random.default_rng(4)
    c = rng.integers(-2 ** 20, 2 ** 20, (6, 7)).astype(np.int32)
    sr = (rng.random(6) * 0.1).astype(np.float16)
    sc = (rng.random(7) * 0.01).astype(np.float16)
    got = oq.sym_dequant(c, sr, sc)
    for i in range(6):
        for j in range(7):
            a = f32(float(c[i, j]) * float(sr[i]))
            v = f32(a * float(sc[j]))
            want = to_f16(Fraction(v))
            assert float(got[i, j]) == float(want)


def test_kv_quant_constant_row_and_bound():
    x = np.full((1, 4, 32, 128), 1.5, np.float16)
    q, p = oq.kv_quant_pack(x)
    s = to_f16(to_f32(Fraction(float(to_f16(Fraction(f32(1e-5))))) / 15))
    assert np.all(p[..., 0] == np.float16(float(s)))
    assert np.all(p[..., 1] == np.float16(-1.5))
    assert np.all(q == 0)
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((64, 128)) * 2).astype(np.float16)
    q, p = oq.kv_quant_pack(x)
    codes = oq.kv_unpack(q)
    assert codes.min() >= 0 and codes.max() <= 15
    xr = oq.kv_dequant(q, p)
    scale = p[:, 0:1].astype(np.float32)
    # reconstruction within half a step plus the fp16 rounding slack
    assert np.all(np.abs(xr - x.astype(np.float32)) <= 0.5 * scale + 0.02 * np.abs(x) + 1e-3)
    # the row min maps to 0 and the row max to 15
    assert np.all(codes.min(axis=1) == 0) and np.all(codes.max(axis=1) == 15)


def test_kv_codes_match_exact_rule():
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((8, 128)) * 3).astype(np.float16)
    q, p = oq.kv_quant_pack(x)
    codes = oq.kv_unpack(q)
    for r in range(8):
        s, z = Fraction(float(p[r, 0])), Fraction(float(p[r, 1]))
        mx, mn = Fraction(float(x[r].max())), Fraction(float(x[r].min()))
        diff = to_f16(mx - mn)
        diff = to_f16(max(diff, Fraction(f32(1e-5))))
        assert s == to_f16(to_f32(diff / 15))
        assert z == -mn
        for c in range(0, 128, 5):
            shifted = to_f16(Fraction(float(x[r, c])) + z)
            want = max(0, min(15, round_half_even(to_f16(shifted / s))))
            assert codes[r, c] == want


def test_rtn_weight_grid():
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((16, 256)) * 0.02).astype(np.float16)
    codes, s, wfq = oq.rtn_weight(w)
    assert codes.min() >= -8 and codes.max() <= 7
    # W_fq sits on the grid: codes * fp16(s) reproduces it to fp16 rounding
    rec = (codes.astype(np.float32) * s.astype(np.float32)).astype(np.float16)
    assert np.max(np.abs(rec.astype(np.float32) - wfq.astype(np.float32))) <= \
        np.max(np.spacing(np.abs(wfq))).astype(np.float32) * 2
    # the largest |w| of each row maps to ±7 (or -8 never on the max side)
    am = np.argmax(np.abs(w.astype(np.float32)), axis=1)
    assert np.all(np.abs(codes[np.arange(16), am]) == 7)
    c2, _, _ = oq.rtn_weight(w, symmetric_grid=True)
    assert c2.min() >= -7
