"""Pins of the oracle's quantizers on rows holding NaN or ±inf.

The reference reduces the row with fmaxf / fminf (signrot/kernels/fused.cu:
17-28, 83-88, 236-245), which skip NaN, and converts quotients with
__half2int_rn / (int)nearbyintf, which map NaN to 0 and saturate ±inf.  The
expected values below are worked out by hand from those rules, not by
re-running the oracle's own formula."""
import numpy as np
import pytest

from oracle import quant as oq

NAN, INF = np.nan, np.inf


def _sym(row, clip=1.0):
    q, s = oq.sym_quant_dynamic(np.array([row], np.float16), clip)
    return oq.unpack_i4(q)[0, :len(row)].tolist(), float(s[0, 0])


def test_sym_nan_is_skipped_by_the_row_max():
    # amax over {1, 7, 3} = 7 -> scale 1.0; NaN -> code 0
    codes, scale = _sym([NAN, 1, -7, 3, 0, 0, 0, 0])
    assert scale == 1.0
    assert codes == [0, 1, -7, 3, 0, 0, 0, 0]


def test_sym_nan_with_clip():
    # scale = fp16(fp16(14 / 7) * 0.5) = 1.0; 2 / 1 = 2, -14 / 1 -> clamp -8
    codes, scale = _sym([2, NAN, -14, 0], clip=0.5)
    assert scale == 1.0
    assert codes == [2, 0, -8, 0]


def test_sym_all_nan_row_has_zero_scale():
    # fmaxf(0, NaN) = 0 -> scale 0; NaN / 0 = NaN -> 0
    codes, scale = _sym([NAN] * 6)
    assert scale == 0.0
    assert codes == [0] * 6


@pytest.mark.parametrize("inf", [INF, -INF])
def test_sym_inf_row(inf):
    # amax = inf -> scale inf; finite / inf = 0; inf / inf = NaN -> 0
    codes, scale = _sym([3, inf, -2, 0.5])
    assert scale == INF
    assert codes == [0, 0, 0, 0]


def test_sym_nan_and_inf_row():
    codes, scale = _sym([NAN, INF, 1, -1])
    assert scale == INF
    assert codes == [0, 0, 0, 0]


def _kv(row):
    q, p = oq.kv_quant_pack(np.array([row], np.float16))
    return oq.kv_unpack(q)[0].tolist(), float(p[0, 0]), float(p[0, 1])


def test_kv_nan_is_skipped():
    # max 15, min 0 -> diff 15, scale 1, zero -0; NaN + 0 = NaN -> code 0
    codes, scale, zero = _kv([NAN, 0, 1, 2, 3, 4, 5, 15])
    assert (scale, zero) == (1.0, 0.0)
    assert codes == [0, 0, 1, 2, 3, 4, 5, 15]


def test_kv_nan_does_not_move_the_min():
    # min -2 (not NaN), max 13 -> diff 15, scale 1, zero 2
    codes, scale, zero = _kv([-2, NAN, 13, 0])
    assert (scale, zero) == (1.0, 2.0)
    assert codes == [0, 0, 15, 2]


def test_kv_all_nan_row():
    # max = -FLT_MAX -> fp16 -inf, min = FLT_MAX -> +inf; diff = -inf,
    # fmaxf(-inf, 1e-5) = 1e-5 -> fp16 168 * 2^-24; / 15 -> fp16 11 * 2^-24;
    # zero = -inf; every code 0
    codes, scale, zero = _kv([NAN] * 4)
    assert scale == 11 * 2.0 ** -24
    assert zero == -INF
    assert codes == [0, 0, 0, 0]


def test_kv_plus_inf_row():
    # max inf, min -1: diff inf, scale inf, zero 1; finite: (x + 1) / inf = 0;
    # inf: inf / inf = NaN -> 0
    codes, scale, zero = _kv([-1, 2, INF, 0])
    assert (scale, zero) == (INF, 1.0)
    assert codes == [0, 0, 0, 0]


def test_kv_both_infinities():
    # diff = inf - (-inf) = inf, zero = inf; x + inf = inf, -inf + inf = NaN;
    # inf / inf = NaN -> 0 everywhere
    codes, scale, zero = _kv([-INF, 3, INF, 0])
    assert (scale, zero) == (INF, INF)
    assert codes == [0, 0, 0, 0]


def test_kv_plus_inf_only_row():
    # max = min = inf: diff = inf - inf = NaN -> fmaxf(NaN, 1e-5) = 1e-5
    codes, scale, zero = _kv([INF, INF])
    assert scale == 11 * 2.0 ** -24
    assert zero == -INF
    assert codes == [0, 0]
