"""Pins of oracle/hadamard.py against what the mathematics fixes:
Hadamard-ness and the committed digest of the tables, the selection rule's
known answers, scipy's Sylvester matrix, and the Kronecker closed form."""
import hashlib
import pathlib

import numpy as np
import pytest
import scipy.linalg

from oracle import hadamard as oh

ROOT = pathlib.Path(__file__).resolve().parents[1]
REF_TABLES = pathlib.Path("/root/reference/signrot/functional/hadamard_matrices.py")


def test_tables_are_hadamard_and_match_digest():
    h = hashlib.sha256()
    for k in sorted(oh.KNOWN_ORDER):
        t = oh.had_table(k).astype(np.int64)
        assert t.shape == (k, k)
        assert np.all(np.abs(t) == 1)
        assert np.array_equal(t @ t.T, k * np.eye(k, dtype=np.int64))
        h.update(str(k).encode())
        h.update(np.ascontiguousarray(t, dtype=np.int8).tobytes())
    want = (ROOT / "tests" / "golden" / "had_tables.sha256").read_text().strip()
    assert h.hexdigest() == want


@pytest.mark.skipif(not REF_TABLES.exists(), reason="reference tree not mounted")
def test_tables_match_reference_text():
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "mk", ROOT / "tests" / "golden" / "make_had_tables.py")
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    ref = mk.parse(REF_TABLES.read_text())
    for k, t in ref.items():
        assert np.array_equal(t, oh.had_table(k).astype(np.int64)), k


@pytest.mark.parametrize("n,k", [(4096, 1), (14336, 28), (28672, 28), (11008, 172),
                                 (128, 1), (32, 1), (12 * 256, 12), (5120, 40), (20, 20),
                                 (13824, 108), (8192, 1), (18432, 36)])
def test_get_hadK_known_answers(n, k):
    assert oh.get_hadK(n)[1] == k


def test_get_hadK_rejects_unknown():
    with pytest.raises(ValueError):
        oh.get_hadK(21 * 64)


@pytest.mark.parametrize("n", [2, 4, 8, 16, 64, 512, 4096])
def test_fwht_is_sylvester_matrix(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((3, n))
    want = x @ scipy.linalg.hadamard(n).T
    np.testing.assert_allclose(oh.fwht(x), want, rtol=1e-12, atol=1e-9)


def test_fwht_pairs_adjacent_elements_first():
    # matmul_hadU's first stage maps (x0, x1) -> (x0 + x1, x0 - x1); for n = 4
    # the rows are [1,1,1,1], [1,-1,1,-1], [1,1,-1,-1], [1,-1,-1,1]
    e = np.eye(4)
    got = np.stack([oh.fwht(r) for r in e], axis=1)
    want = np.array([[1, 1, 1, 1], [1, -1, 1, -1], [1, 1, -1, -1], [1, -1, -1, 1]], float)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("n", [4096, 14336, 28 * 64, 12 * 32])
def test_rotate_matches_kronecker_closed_form(n):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((4, n)).astype(np.float16)
    had, k = oh.get_hadK(n)
    m = n // k
    hk = np.ones((1, 1)) if had is None else had.astype(np.float64)
    dense = np.kron(hk, scipy.linalg.hadamard(m)) / np.sqrt(n)
    want = x.astype(np.float64) @ dense.T
    got = oh.rotate(x).astype(np.float64)
    # two fp16 rounding points when K > 1 (each <= half an ulp, the first one
    # amplified by the ±1 mix over K terms)
    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    # K == 1: one rounding, half an ulp.  K > 1: the first rounding's error
    # (<= half an ulp of each |y| <= max|y|) passes through the ±1 mix of K
    # terms, bounded by K/2 ulp(max|y|) / 1 plus the final half ulp
    if k == 1:
        assert np.all(np.abs(got - want) <= 0.5 * ulp)
    else:
        y = oh.fwht(x.astype(np.float64).reshape(-1, k, m)) / np.sqrt(n)
        ymax = np.abs(y).max(axis=1).reshape(4, 1, m)
        first = 0.5 * np.spacing(ymax.astype(np.float16)).astype(np.float64) * k
        first = np.broadcast_to(first, (4, k, m)).reshape(4, n)
        assert np.all(np.abs(got - want) <= 0.5 * ulp + first)
    # and the rotation is not trivially wrong: error far below the signal
    assert np.abs(got - want).max() < 1e-2 * np.abs(want).max()


def test_rotation_is_orthonormal():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 14336))
    y = oh.matmul_hadU_f64(x)
    np.testing.assert_allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=1e-12)


def test_scale_constants():
    # 1/sqrt(n) in fp32, bit patterns for the config widths
    assert oh.scale_f32(4096).view(np.uint32) == 0x3C800000
    assert oh.scale_f32(14336).view(np.uint32) == 0x3C08D677
    assert oh.scale_f32(28672).view(np.uint32) == 0x3BC18490


def test_sign_calibration_rule():
    x = np.array([[0.5, -1.0, 2.0], [-9.0, 0.0, 3.0], [1.0, 1.0, -1.0]], np.float16)
    s = oh.sign_calibration(x)
    # token 1 holds the largest magnitude; sign of 0 is +1
    assert s.dtype == np.int8
    assert s.tolist() == [-1, 1, 1]


def test_online_hadamard_rejects_zero_sign():
    x = np.ones((1, 8), np.float16)
    with pytest.raises(RuntimeError):
        oh.online_hadamard(x, np.array([1, 0, 1, 1, 1, 1, 1, 1], np.int8))
