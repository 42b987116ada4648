"""Hadamard helpers mirroring signrot/functional/hadamard.py:14-133.

`matmul_hadU_cuda` runs on the HIP kernels (srq_hadamard_transform /
srq_online_hadamard) instead of the CUDA-only fast_hadamard_transform +
cuBLAS pair; `matmul_hadU` is the reference's pure-torch butterfly (used
offline and by random_hadamard_matrix)."""
import math
from collections import OrderedDict

import torch

from .hadamard_matrices import (get_had12, get_had20, get_had28, get_had36, get_had40,
                                get_had52, get_had60, get_had108, get_had140, get_had148,
                                get_had156, get_had172)

# Largest factor first, as the reference walks it (hadamard.py:14-29).
KNOWN_HADAMARD_MATRICES = OrderedDict([
    (172, get_had172),
    (156, get_had156),
    (148, get_had148),
    (140, get_had140),
    (108, get_had108),
    (60, get_had60),
    (52, get_had52),
    (40, get_had40),
    (36, get_had36),
    (28, get_had28),
    (20, get_had20),
    (12, get_had12),
])


def is_pow2(n):
    return (n & (n - 1) == 0) and (n > 0)


def get_hadK(n, transpose=False):
    """(hadK fp32 [K, K] or None, K) for the first known K with n % K == 0 and
    n / K a power of two (hadamard.py:30-40)."""
    for K, fn in KNOWN_HADAMARD_MATRICES.items():
        if n % K == 0 and is_pow2(n // K):
            had = fn()
            return (had.T if transpose else had), K
    assert is_pow2(n), "No known Hadamard matrix factor found and n is not a power of 2!"
    return None, 1


def hadamard_transform(x, scale=1.0):
    """Drop-in for fast_hadamard_transform.hadamard_transform (HIP kernel)."""
    from .. import _CUDA
    return _CUDA.hadamard_transform(x, scale)


def _inv_sqrt_f32(n):
    # 1.0 / torch.tensor(n).sqrt(): fp32 sqrt, fp32 division (hadamard.py:81,85)
    return float(1.0 / torch.tensor(n).sqrt())


def matmul_hadU(X, transpose=False, hadK=None, K=None) -> torch.Tensor:
    """Pure-torch Sylvester butterfly in X's dtype, then hadK, then / sqrt(n)
    (hadamard.py:43-65)."""
    n = X.shape[-1]
    if K is None:
        hadK, K = get_hadK(n, transpose)
    inp = X.clone().view(-1, n, 1)
    out = inp.clone()
    while inp.shape[1] > K:
        inp = inp.view(inp.shape[0], inp.shape[1] // 2, 2, inp.shape[2])
        out = out.view(inp.shape)
        out[:, :, 0, :] = inp[:, :, 0, :] + inp[:, :, 1, :]
        out[:, :, 1, :] = inp[:, :, 0, :] - inp[:, :, 1, :]
        out = out.view(inp.shape[0], inp.shape[1], -1)
        inp, out = out, inp
    del out
    if K > 1:
        inp = hadK.view(1, K, K).to(inp) @ inp
    return inp.view(X.shape) / torch.tensor(n).sqrt()


def matmul_hadUt(X):
    return matmul_hadU(X, transpose=True)


def random_hadamard_matrix(size, device):
    """Randomised Hadamard matrix (hadamard.py:71-76)."""
    Q = torch.randint(low=0, high=2, size=(size,)).to(torch.float64)
    Q = Q * 2 - 1
    Q = torch.diag(Q)
    return matmul_hadU(Q).to(device)


def matmul_hadU_cuda(X, hadK, K):
    """Online rotation (hadamard.py:78-87) on the HIP kernels.

    fp16 X: one launch of srq_online_hadamard with the reference's two fp16
    rounding points.  fp32 X: the fp32 FWHT kernel, then (K > 1) the fp32
    hadK product."""
    from .. import _CUDA
    n = X.shape[-1]
    if K == 1:
        return _CUDA.hadamard_transform(X.contiguous(), _inv_sqrt_f32(n))
    if X.dtype == torch.float16:
        return _CUDA.online_hadamard(X.contiguous(), _had_on(hadK, X.device, torch.float16), K)
    inp = X.reshape(*X.shape[:-1], K, n // K).contiguous()
    inp = _CUDA.hadamard_transform(inp, _inv_sqrt_f32(n))
    inp = _had_on(hadK, X.device, inp.dtype) @ inp
    return inp.reshape(X.shape)


def matmul_hadUt_cuda(X, hadK, K):
    return matmul_hadU_cuda(X, hadK.T.contiguous() if hadK is not None else None, K)


def _had_on(hadK, device, dtype):
    h = hadK.reshape(hadK.shape[-2], hadK.shape[-1])
    if h.device != device or h.dtype != dtype or not h.is_contiguous():
        h = h.to(device=device, dtype=dtype).contiguous()
    return h


def adj_sign_from_rotated(x_rot: torch.Tensor) -> torch.Tensor:
    """The SignRot sign-adjust vector from one rotated calibration batch
    (fake_quant/quant_utils.py:362-367): the token whose largest |value| is
    the largest of the batch (the massive-outlier token; the first such token
    on ties), and the sign pattern of that token, with 0 counted as +1.

    x_rot [T, n] or [B, T, n] (only batch 0 is used, as the reference does);
    returns int8 [n] of ±1 on x_rot's device."""
    tokens = x_rot[0] if x_rot.dim() == 3 else x_rot
    if tokens.dim() != 2 or tokens.shape[0] == 0:
        raise ValueError("adj_sign_from_rotated expects [T, n] or [B, T, n] with T > 0")
    peak = tokens.abs().amax(dim=-1).argmax()
    return torch.where(tokens[peak] >= 0, 1, -1).to(torch.int8)


def fold_adj_sign_into_linear(linear: torch.nn.Linear, sign: torch.Tensor) -> None:
    """W <- W * sign by input column (quant_utils.py:367), in the weight's own
    dtype: a ±1 factor is exact.  Done before weight quantization, so the
    rotated-and-flipped activation meets the matching flipped weight."""
    w = linear.weight.data
    linear.weight.data = w * sign.to(device=w.device, dtype=w.dtype)


def apply_exact_had_to_linear(module, had_dim=-1, output=False):
    """Fold a Hadamard into a Linear's weight (hadamard.py:94-130); offline."""
    assert isinstance(module, torch.nn.Linear)
    in_features, out_features = module.in_features, module.out_features
    if had_dim != -1:
        assert is_pow2(had_dim), "Hadamard dimension must be a power of 2!"
    W_ = module.weight.data
    dtype, dev = W_.dtype, W_.device
    W_ = W_.float().cuda()
    if had_dim == -1:
        if output:
            had_K, K = get_hadK(out_features)
            W_ = matmul_hadU_cuda(W_.t(), had_K, K).t()
        else:
            had_K, K = get_hadK(in_features)
            W_ = matmul_hadU_cuda(W_, had_K, K)
    else:
        if not output:
            raise NotImplementedError("Not implemented (or tested) yet!")
        W_ = W_.t()
        shp = W_.shape
        W_ = hadamard_transform(W_.reshape(-1, shp[-1] // had_dim, had_dim).contiguous(),
                                scale=1 / math.sqrt(had_dim)).reshape(shp).t()
    module.weight.data = W_.to(device=dev, dtype=dtype)
