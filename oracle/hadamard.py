"""Oracle for the online Hadamard rotation -- test infrastructure only.

Restates signrot/functional/hadamard.py:14-87 (get_hadK, matmul_hadU,
matmul_hadU_cuda) and signrot/nn/hadamard.py:26-42 (OnlineHadamard.forward).
"""
import json
import math
import pathlib

import numpy as np

_TABLES = pathlib.Path(__file__).resolve().parents[1] / "signrot_amd" / "functional" / "had_tables.json"

# Order in which the reference walks KNOWN_HADAMARD_MATRICES
# (signrot/functional/hadamard.py:14-29): largest factor first.
KNOWN_ORDER = (172, 156, 148, 140, 108, 60, 52, 40, 36, 28, 20, 12)

_cache = {}


def had_table(k):
    """±1 int8 [k, k] table for a known factor k (hadamard_matrices.py)."""
    if not _cache:
        raw = json.loads(_TABLES.read_text())
        for key, rows in raw.items():
            kk = int(key)
            m = np.empty((kk, kk), dtype=np.int8)
            for i, h in enumerate(rows):
                bits = int(h, 16)
                m[i] = [1 if (bits >> j) & 1 else -1 for j in range(kk)]
            _cache[kk] = m
    return _cache[k]


def is_pow2(n):
    return n > 0 and (n & (n - 1)) == 0


def get_hadK(n):
    """hadamard.py:30-40: first known K (in KNOWN_ORDER) with n % K == 0 and
    n/K a power of two, else (None, 1) for a power-of-two n."""
    for k in KNOWN_ORDER:
        if n % k == 0 and is_pow2(n // k):
            return had_table(k), k
    if not is_pow2(n):
        raise ValueError("No known Hadamard matrix factor found and n is not a power of 2!")
    return None, 1


def sylvester(n):
    """Sylvester H_n (H_2n = [[H, H], [H, -H]]), float64."""
    h = np.ones((1, 1))
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def fwht(x):
    """Unnormalised Walsh-Hadamard transform in Sylvester order over the last
    axis, float64 (the order fast_hadamard_transform and matmul_hadU use:
    hadamard.py:50-57 pairs element 2i with 2i+1 at every stage)."""
    x = np.asarray(x, dtype=np.float64)
    n = x.shape[-1]
    assert is_pow2(n)
    shp = x.shape
    y = x.reshape(-1, n).copy()
    h = 1
    while h < n:
        y = y.reshape(-1, n // (2 * h), 2, h)
        a = y[:, :, 0, :].copy()
        b = y[:, :, 1, :].copy()
        y[:, :, 0, :] = a + b
        y[:, :, 1, :] = a - b
        y = y.reshape(-1, n)
        h *= 2
    return y.reshape(shp)


def scale_f32(n):
    """1.0 / torch.tensor(n).sqrt() evaluated in fp32 (hadamard.py:81,85)."""
    return np.float32(1.0) / np.sqrt(np.float32(n))


def rotate(x_f16, k=None, had=None):
    """matmul_hadU_cuda(X, hadK, K) (hadamard.py:78-87) on fp16 input.

    K == 1: fp16(FWHT_n(x) * s) with s = fp32(1/sqrt(n)).
    K  > 1: view x as [..., K, n/K]; y = fp16(FWHT_{n/K}(chunk) * s) (first
            rounding point), then out = fp16(hadK @ y) (second rounding point,
            the torch fp16 matmul).  The sums are carried out in float64, so
            the only roundings are the two the reference's code makes visible;
            the reference's own fp32 accumulation order is not pinnable.
    """
    x = np.asarray(x_f16, dtype=np.float16)
    n = x.shape[-1]
    if k is None:
        had, k = get_hadK(n)
    s = np.float64(scale_f32(n))
    if k == 1:
        return (fwht(x.astype(np.float64)) * s).astype(np.float16)
    m = n // k
    xv = x.astype(np.float64).reshape(-1, k, m)
    y = (fwht(xv) * s).astype(np.float16).astype(np.float64)
    out = np.einsum("ij,rjm->rim", had.astype(np.float64), y)
    return out.astype(np.float16).reshape(x.shape)


def online_hadamard(x_f16, sign=None):
    """OnlineHadamard.forward (nn/hadamard.py:26-42): rotate, then multiply by
    the ±1 had_adj_sign (exact), then cast back to fp16."""
    y = rotate(x_f16)
    if sign is not None:
        sign = np.asarray(sign)
        if np.any(sign == 0):
            raise RuntimeError("Dynamic hadamard adjustment not implemented yet.")
        y = (y.astype(np.float32) * sign.astype(np.float32)).astype(np.float16)
    return y


def sign_calibration(x_rot):
    """The ±1 sign-adjust vector (fake_quant/quant_utils.py:362-367): take the
    token whose largest |value| is the largest, and return the sign pattern
    of that rotated token ((x >= 0) * 2 - 1) as int8."""
    x = np.asarray(x_rot)
    if x.ndim == 3:
        x = x[0]
    t = int(np.argmax(np.abs(x.astype(np.float32)).max(axis=-1)))
    return ((x[t] >= 0).astype(np.int8) * 2 - 1).astype(np.int8)


def matmul_hadU_f64(x):
    """Exact rotation (H_K ⊗ H_{n/K}) x / sqrt(n) in float64 -- the closed form
    the rotation is checked against."""
    x = np.asarray(x, dtype=np.float64)
    n = x.shape[-1]
    had, k = get_hadK(n)
    if k == 1:
        return fwht(x) / math.sqrt(n)
    xv = x.reshape(-1, k, n // k)
    y = fwht(xv)
    out = np.einsum("ij,rjm->rim", had.astype(np.float64), y)
    return out.reshape(x.shape) / math.sqrt(n)
