"""CPU pins of the oracle's asymmetric-activation functions: hand-derived
known answers for the quantizer's rounding points, brute force for the
integer routines, and identities that an independent formula must satisfy
(u4 = (u ^ 8 as int4) + 8; dequant round trip within scale / 2)."""
import numpy as np
import pytest

from oracle import quant as oq

F16 = np.float16


def _q(x, clip=1.0):
    q, s, z = oq.asym_quant_dynamic(np.asarray(x, F16)[None, :], clip)
    return oq.unpack_u4(q)[0, : len(x)], float(s[0, 0]), float(z[0, 0])


def test_known_answers_exact_scale():
    # min -1, max 14: diff 15, scale 1, ratio 1, zero 1
    codes, s, z = _q([-1.0, 0.0, 14.0])
    assert (s, z) == (1.0, 1.0)
    assert codes.tolist() == [0, 1, 15]


def test_known_answers_half_even():
    # scale 1, ratio -0.5 -> zero = rint(-0.5) = 0 (half to even), codes
    # rne(0.5) = 0, rne(2.5) = 2, rne(3.5) = 4, rne(15.5) = 16 -> 15
    codes, s, z = _q([0.5, 2.5, 3.5, 15.5])
    assert s == 1.0 and z == 0.0
    assert codes.tolist() == [0, 2, 4, 15]


def test_known_answers_fp16_rounding_points():
    # fp16(-0.3) = -307/1024, fp16(0.7) = 717/1024: diff = 1, scale =
    # fp16(1/15) = 273/4096; ratio = 1228/273 = 4.498 -> fp16 4.5 -> zero 4;
    # codes: -4.498 -> fp16 -4.5 -> rne -4 -> 0; 10.505 -> fp16 10.5078125
    # -> 11 -> 15
    codes, s, z = _q([-0.3, 0.7])
    assert s == 273 / 4096 and z == 4.0
    assert codes.tolist() == [0, 15]


def test_clip_rounds_each_bound():
    # clip 0.5 on [-1, 14]: hmin = -0.5, hmax = 7, diff 7.5, scale =
    # fp16(0.5) = 0.5, ratio = 1, zero 1; codes rne(x / 0.5) + 1 clamped
    codes, s, z = _q([-1.0, 0.0, 3.0, 14.0], clip=0.5)
    assert (s, z) == (0.5, 1.0)
    assert codes.tolist() == [0, 1, 7, 15]


def test_degenerate_rows():
    x = np.zeros((3, 8), F16)
    x[1] = 3.0                      # constant row: scale 0, zero -inf
    x[2] = F16(2.0 ** -24)          # positive tiny row: scale underflows to 0
    x[2, 0] = F16(2.0 ** -23)       # (diff / 15 < 2^-25), ratio -hmin / 0 = -inf
    q, s, z = oq.asym_quant_dynamic(x)
    assert np.all(s == 0)
    assert np.isnan(z[0, 0]) and np.isneginf(z[1, 0]) and np.isneginf(z[2, 0])
    # x / 0: NaN -> 0, +inf -> INT_MAX; plus zero -inf -> INT_MIN; the int32
    # sum wraps to -1 (0 for the NaN case) -> clamp -> 0
    assert np.all(oq.unpack_u4(q) == 0)


def test_nan_values_are_skipped_by_the_row_reductions():
    # fminf / fmaxf skip NaN: [NaN, -1, 14] has the parameters of [-1, 14]
    # (scale 1, zero 1); the NaN's own code is clamp(0 + zero) = 1
    codes, s, z = _q([np.nan, -1.0, 14.0])
    assert (s, z) == (1.0, 1.0)
    assert codes.tolist() == [1, 0, 15]
    # an all-NaN row: hmin = +inf, hmax = -inf, diff = -inf, scale = -inf
    q, s2, z2 = oq.asym_quant_dynamic(np.full((1, 4), np.nan, F16))
    assert np.isneginf(s2[0, 0]) and np.isnan(z2[0, 0])


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_round_trip_within_half_scale(seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((16, 256)) * rng.uniform(0.1, 50, (16, 1))).astype(F16)
    x[:, :3] += F16(rng.uniform(-20, 20))  # shifted rows
    q, s, z = oq.asym_quant_dynamic(x)
    codes = oq.unpack_u4(q).astype(np.float64)
    assert codes.min() >= 0 and codes.max() <= 15
    deq = s.astype(np.float64) * (codes - z.astype(np.float64))
    err = np.abs(deq - x.astype(np.float64))
    # within half a step plus the fp16 rounding of the quotient and the
    # zero point (|q| <= 2^11 * ulp)
    assert np.all(err <= 0.5 * s.astype(np.float64) + 2 ** -10 * np.abs(x) + 1e-6)
    # the row minimum and maximum land at the ends of the grid
    assert np.all(codes.min(axis=1) <= 1) and np.all(codes.max(axis=1) >= 14)


def test_given_parameter_forms():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 33)).astype(F16)
    s = np.full(4, 0.25, F16)
    z = np.array([0, 8, -3, 20], F16)
    u = oq.unpack_u4(oq.asym_quant_f16_ui4(x, s, z))[:, :33]
    i = oq.unpack_i4(oq.asym_quant_f16_si4(x, s, z))[:, :33]
    raw = np.rint((x.astype(np.float32) / np.float32(0.25)).astype(F16).astype(np.float64))
    raw = raw + z.astype(np.float64)[:, None]
    assert np.array_equal(u, np.clip(raw, 0, 15))
    assert np.array_equal(i, np.clip(raw, -8, 7))


def _brute_sum(p, signed):
    out = []
    for row in p:
        t = 0
        for b in row.tolist():
            for nib in (b & 15, b >> 4):
                t += nib - 16 if signed and nib >= 8 else nib
        out.append(t)
    return np.array(out)


@pytest.mark.parametrize("signed", [True, False])
def test_sum_i4_brute_force(signed):
    rng = np.random.default_rng(4)
    p = rng.integers(0, 256, (5, 37)).astype(np.uint8)
    assert np.array_equal(oq.sum_i4(p, signed)[:, 0], _brute_sum(p, signed))
    full = np.full((1, 10), 0x88, np.uint8)
    assert oq.sum_i4(full, True)[0, 0] == -160 and oq.sum_i4(full, False)[0, 0] == 160


def test_colrow_brute_force_and_wrap():
    a = np.array([1, -2, 127, -128], np.int8)
    b = np.array([3, -7, 1 << 30, 0x7fffffff], np.int32)
    got = oq.matmul_colrow_i8_i32(a, b)
    for r in range(4):
        for c in range(4):
            v = (int(a[r]) * int(b[c]) + 2 ** 31) % 2 ** 32 - 2 ** 31
            assert got[r, c] == v


def test_matmul_u4s4_brute_force_and_identity():
    rng = np.random.default_rng(5)
    a = rng.integers(0, 256, (3, 16)).astype(np.uint8)   # K = 32
    b = rng.integers(0, 256, (4, 16)).astype(np.uint8)
    c = oq.matmul_u4s4(a, b)
    au, bs = oq.unpack_u4(a), oq.unpack_i4(b)
    for i in range(3):
        for j in range(4):
            assert c[i, j] == sum(int(au[i, k]) * int(bs[j, k]) for k in range(32))
    # u = (u ^ 8 read as int4) + 8, so A·B = (A ^ 0x88)·B + 8 * rowsum(B)
    a2 = rng.integers(0, 256, (40, 64)).astype(np.uint8)
    b2 = rng.integers(0, 256, (24, 64)).astype(np.uint8)
    alt = oq.matmul_s4s4(a2 ^ 0x88, b2).astype(np.int64) + 8 * oq.sum_i4(b2)[:, 0][None, :]
    assert np.array_equal(oq.matmul_u4s4(a2, b2), alt)


def test_w4a4_linear_asym_identity_and_accuracy():
    rng = np.random.default_rng(6)
    M, N, K = 12, 20, 128
    x = (rng.standard_normal((M, K)) * 3 + 1).astype(F16)
    q, s, z = oq.asym_quant_dynamic(x)
    zi = z[:, 0].astype(np.int8)
    w = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
    sw = (np.abs(rng.standard_normal(N)) * 0.05 + 0.01).astype(F16)
    bias = rng.standard_normal(N).astype(F16)
    out = oq.w4a4_linear_asym(q, s, zi, w, sw, bias)
    # independent integer path: signed GEMM of the re-centred codes
    ws = oq.sum_i4(w)[:, 0].astype(np.int64)
    c = oq.matmul_s4s4(q ^ 0x88, w).astype(np.int64) + (8 - zi.astype(np.int64))[:, None] * ws
    alt = oq.add_bias(oq.sym_dequant(c, s, sw), bias)
    assert np.array_equal(out, alt)
    # and close to the dequantized product in float64
    deq = s.astype(np.float64) * (oq.unpack_u4(q).astype(np.float64) - zi[:, None])
    ref = deq @ (oq.unpack_i4(w).astype(np.float64) * sw.astype(np.float64)[:, None]).T
    ref = ref + bias.astype(np.float64)
    np.testing.assert_allclose(out.astype(np.float64), ref, rtol=1e-2, atol=1e-2)
