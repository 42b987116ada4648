"""CPU checks of the product's offline helpers and of the CPU fake-quant
restatement timed as bench.py's baseline:

* matmul_hadU (signrot/functional/hadamard.py:43-65) -- the product copy and
  the baseline copy -- against the Kronecker closed form built from
  scipy.linalg.hadamard (float64: exact up to the final division);
* rtn_weight_pack (quant_utils.py:453-529, linear.py:52-73) against
  oracle.rtn_weight, and both against exact rational arithmetic;
* adj_sign_from_rotated (quant_utils.py:362-367) against hand-worked known
  answers and oracle.sign_calibration;
* the baseline's per-token fake quantizer (quant_utils.py:90-145) against the
  exact per-element rule."""
import math
from fractions import Fraction

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import fakequant
from oracle import hadamard as oh
from oracle import quant as oq
from signrot_amd.functional.hadamard import (adj_sign_from_rotated, fold_adj_sign_into_linear,
                                             get_hadK, matmul_hadU, matmul_hadUt)
from signrot_amd.functional.quantization import pack_i4, rtn_weight_pack, unpack_i4
from tests.exact import round_half_even, to_f16, to_f32


def _kron_closed_form(x, transpose=False):
    """(H_K ⊗ H_{n/K}) x / sqrt(n) with H_{n/K} = scipy's Sylvester matrix; the
    divisor is torch.tensor(n).sqrt(), the correctly rounded fp32 sqrt."""
    n = x.shape[-1]
    had, k = get_hadK(n)
    hk = np.eye(1) if had is None else had.numpy().astype(np.float64)
    if transpose:
        hk = hk.T
    full = np.kron(hk, scipy.linalg.hadamard(n // k))
    return x @ full.T / float(np.float32(math.sqrt(n)))


@pytest.mark.parametrize("impl", ["product", "baseline"])
@pytest.mark.parametrize("n", [2, 8, 64, 12 * 4, 20 * 8, 28 * 16, 28 * 512, 4096])
def test_matmul_hadU_matches_kronecker_closed_form(impl, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((3, n))
    xt = torch.from_numpy(x)
    if impl == "product":
        got = matmul_hadU(xt).numpy()
    else:
        had, k = get_hadK(n)
        got = fakequant.matmul_hadU(xt, had, k).numpy()
    want = _kron_closed_form(x)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_matmul_hadUt_uses_the_transposed_factor():
    n = 20 * 8
    x = np.random.default_rng(1).standard_normal((2, n))
    got = matmul_hadUt(torch.from_numpy(x)).numpy()
    np.testing.assert_allclose(got, _kron_closed_form(x, transpose=True), rtol=1e-12, atol=1e-12)
    # H_20 is not symmetric (H_28 is), so the transposed factor gives another result
    assert not np.allclose(got, _kron_closed_form(x))


def test_matmul_hadU_fp16_rounds_each_stage():
    """In fp16 the butterfly rounds at every stage: the result stays within
    the stage count times half an ulp of the running magnitude."""
    n = 1024
    x = np.random.default_rng(2).standard_normal((4, n)).astype(np.float16)
    got = matmul_hadU(torch.from_numpy(x)).numpy().astype(np.float64)
    want = _kron_closed_form(x.astype(np.float64))
    bound = 10 * np.abs(x.astype(np.float64)).sum(-1, keepdims=True) * 2.0 ** -11 / math.sqrt(n)
    assert np.all(np.abs(got - want) <= bound + np.spacing(np.abs(want).astype(np.float16)))
    assert np.mean(got.astype(np.float16) != want.astype(np.float16)) > 0  # not exact


# ------------------------------------------------------------------ RTN

def _exact_rtn_row(w_row, symmetric_grid):
    """find_params + quantize + from_float for one fp16 row, in rationals
    with explicit binary32 / binary16 roundings."""
    vals = [Fraction(float(v)) for v in w_row]
    xmax = max(max(vals), Fraction(0))
    xmin = min(min(vals), Fraction(0))
    m = max(abs(xmin), xmax, Fraction(np.float32(1e-5).item()))
    s = to_f32(m / 7)
    lo = -7 if symmetric_grid else -8
    wfq, codes = [], []
    s16 = to_f16(s)
    for v in vals:
        q = max(lo, min(7, round_half_even(to_f32(v / s))))
        f = to_f16(to_f32(q * s))
        wfq.append(f)
        codes.append(max(-8, min(7, round_half_even(to_f16(f / s16)))))
    return codes, s16, wfq


@pytest.mark.parametrize("symmetric_grid", [False, True])
def test_rtn_oracle_and_product_match_exact_arithmetic(symmetric_grid):
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((6, 40)) * 0.02).astype(np.float16)
    w[2] = 0                                   # clamp(1e-5) branch
    w[3, :] = np.abs(w[3, :])                  # all positive: min extends to 0
    w[4, 7] = np.float16(-0.5)                 # a negative extreme: exactly -7 * s
    codes_o, s_o, wfq_o = oq.rtn_weight(w, symmetric_grid=symmetric_grid)
    packed_p, s_p, wfq_p = rtn_weight_pack(torch.from_numpy(w), symmetric_grid=symmetric_grid)
    for r in range(w.shape[0]):
        codes, s16, wfq = _exact_rtn_row(w[r], symmetric_grid)
        assert float(s_o[r, 0]) == float(s16) == float(s_p[r])
        assert codes_o[r].tolist() == codes
        assert [float(v) for v in wfq_o[r]] == [float(v) for v in wfq]
        assert [float(v) for v in wfq_p[r].numpy()] == [float(v) for v in wfq]
    assert torch.equal(unpack_i4(packed_p, torch.int8), torch.from_numpy(codes_o))
    # |w| <= 7 s for every entry, so neither grid reaches -8
    assert codes_o[4, 7] == -7 and codes_o.min() >= -7


def test_rtn_product_matches_oracle_at_config_width():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((64, 14336)) * 0.02).astype(np.float16)
    for sg in (False, True):
        codes_o, s_o, wfq_o = oq.rtn_weight(w, symmetric_grid=sg)
        packed_p, s_p, wfq_p = rtn_weight_pack(torch.from_numpy(w), symmetric_grid=sg)
        assert np.array_equal(packed_p.numpy(), oq.pack_i4(codes_o))
        assert np.array_equal(s_p.numpy().view(np.uint16), s_o.reshape(-1).view(np.uint16))
        assert np.array_equal(wfq_p.numpy().view(np.uint16), wfq_o.view(np.uint16))


def test_rtn_symmetric_grid_survives_a_sign_fold():
    """Folding ±1 after quantizing on [-7, 7] keeps every code representable
    (gptq_utils.py:438-457)."""
    rng = np.random.default_rng(5)
    w = torch.from_numpy((rng.standard_normal((8, 256)) * 0.02).astype(np.float16))
    sign = torch.from_numpy(rng.choice([-1, 1], 256).astype(np.int8))
    packed, _, _ = rtn_weight_pack(w * sign, symmetric_grid=True)
    flipped = unpack_i4(packed, torch.int16) * sign
    pack_i4(flipped.to(torch.int8))  # asserts the range


# --------------------------------------------------------- sign calibration

def test_adj_sign_known_answer():
    x = torch.tensor([[0.5, -1.0, 2.0],
                      [-3.0, 9.0, 0.0],      # the massive token: max |x| = 9
                      [4.0, -8.5, 1.0]])
    assert adj_sign_from_rotated(x).tolist() == [-1, 1, 1]   # 0 counts as +1
    # [B, T, n]: batch 0 only
    xb = torch.stack([x, -x * 10])
    assert adj_sign_from_rotated(xb).tolist() == [-1, 1, 1]
    # ties: the first token with the largest magnitude
    t = torch.tensor([[1.0, -5.0], [5.0, 1.0]])
    assert adj_sign_from_rotated(t).tolist() == [1, -1]
    assert adj_sign_from_rotated(x).dtype == torch.int8


def test_adj_sign_matches_oracle_on_outlier_rows():
    rng = np.random.default_rng(6)
    for n in (4096, 14336):
        x = rng.standard_normal((64, n)).astype(np.float16)
        x[17, rng.permutation(n)[:8]] *= 50
        rot = oh.online_hadamard(x)
        got = adj_sign_from_rotated(torch.from_numpy(rot)).numpy()
        assert np.array_equal(got, oh.sign_calibration(rot))


def test_fold_adj_sign_flips_input_columns():
    lin = torch.nn.Linear(4, 3, bias=False).half()
    w0 = lin.weight.data.clone()
    sign = torch.tensor([1, -1, -1, 1], dtype=torch.int8)
    fold_adj_sign_into_linear(lin, sign)
    assert torch.equal(lin.weight.data[:, 0], w0[:, 0])
    assert torch.equal(lin.weight.data[:, 1], -w0[:, 1])
    # x·s against W·s gives back x·W exactly
    x = torch.randn(2, 4).half()
    assert torch.equal((x * sign.half()).float() @ lin.weight.data.float().T,
                       x.float() @ w0.float().T)


# ---------------------------------------------------- baseline fake quant

def test_baseline_act_fake_quant_is_the_exact_per_token_rule():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((5, 32)) * 3
    x[1] = 0                                    # xmax == 0 -> scale 1
    x[2, 4] = -40.0                             # negative extreme -> q = -7
    got = fakequant.act_fake_quant(torch.from_numpy(x)).numpy()
    for r in range(5):
        row = [Fraction(v) for v in x[r]]
        m = max(abs(min(row)), max(row))
        s = m / 7 if m != 0 else Fraction(1)
        for c in range(32):
            q = max(-8, min(7, round_half_even(row[c] / s)))
            assert abs(Fraction(got[r, c]) - q * s) <= abs(q * s) * Fraction(1, 2 ** 50)
