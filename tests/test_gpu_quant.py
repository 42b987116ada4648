"""GPU parity: quantizers, dequant and KV quant vs the CPU oracle, bit-exact
(cases restated from benchmarks/test_fused_equivalence.py:33-90)."""
import numpy as np
import pytest
import torch

from oracle import quant as oq
from tests.gpu_util import assert_bitexact, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def C():
    from signrot_amd import _CUDA
    return _CUDA


SHAPES = [(r, c) for r in (1, 8, 16, 2048) for c in (4096, 11008, 128)] + \
         [(3, 14336), (2048, 14336), (5, 28672), (7, 4095), (2, 6), (1, 1), (9, 33000)]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_sym_quant_dynamic_bitexact(C, rows, cols):
    rng = np.random.default_rng(rows * 100003 + cols)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float16)
    q, s = C.sym_quant_dynamic(to_dev(x))
    qw, sw = oq.sym_quant_dynamic(x)
    assert_bitexact(to_np(s), sw, "scale")
    assert_bitexact(to_np(q), qw, "codes")


@pytest.mark.parametrize("name", ["zeros", "spike", "range", "tiny", "negative", "subnormal"])
def test_sym_quant_dynamic_edge_cases(C, name):
    rng = np.random.default_rng(11)
    if name == "zeros":
        x = np.zeros((4, 4096), np.float16)
    elif name == "spike":
        x = np.zeros((4, 4096), np.float16)
        x[1, 7] = 100.0
    elif name == "range":
        x = (rng.standard_normal((4, 4096)) * 1e3).astype(np.float16)
    elif name == "tiny":
        x = (rng.standard_normal((4, 4096)) * 1e-4).astype(np.float16)
    elif name == "negative":
        x = -(rng.random((4, 4096)) + 1).astype(np.float16)
    else:
        x = np.zeros((2, 64), np.float16)
        x[0, 3] = np.float16(2 ** -24)
        x[0, 9] = -np.float16(2 ** -24)
        x[1, :] = np.float16(2 ** -20)
    q, s = C.sym_quant_dynamic(to_dev(x))
    qw, sw = oq.sym_quant_dynamic(x)
    assert_bitexact(to_np(s), sw, "scale")
    assert_bitexact(to_np(q), qw, "codes")


@pytest.mark.parametrize("clip", [0.9, 0.75])
def test_sym_quant_dynamic_clip(C, clip):
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((33, 4096)) * 2).astype(np.float16)
    q, s = C.sym_quant_dynamic(to_dev(x), clip)
    qw, sw = oq.sym_quant_dynamic(x, clip)
    assert_bitexact(to_np(s), sw, "scale")
    assert_bitexact(to_np(q), qw, "codes")


@pytest.mark.parametrize("rows,cols", [(16, 4096), (5, 1000), (3, 7)])
def test_sym_quant_given_scale(C, rows, cols):
    rng = np.random.default_rng(13)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float16)
    s = (np.abs(rng.standard_normal(rows)) + 0.1).astype(np.float16)
    q = C.sym_quant(to_dev(x), to_dev(s))
    assert_bitexact(to_np(q), oq.sym_quant(x, s), "codes")


@pytest.mark.parametrize("rows,cols", [(16, 4096), (2048, 4096), (3, 7), (1, 1)])
def test_sym_dequant(C, rows, cols):
    rng = np.random.default_rng(14)
    c = rng.integers(-2 ** 21, 2 ** 21, (rows, cols)).astype(np.int32)
    sr = (rng.random(rows) * 0.1).astype(np.float16)
    sc = (rng.random(cols) * 0.01).astype(np.float16)
    out = C.sym_dequant(to_dev(c), to_dev(sr), to_dev(sc))
    assert_bitexact(to_np(out), oq.sym_dequant(c, sr, sc), "dequant")


@pytest.mark.parametrize("shape", [(1, 1, 32, 128), (1, 2048, 32, 128), (16, 1, 32, 128),
                                   (4, 37, 8, 128), (2, 3, 4, 64), (2, 5, 6)])
def test_kv_quant_pack(C, shape):
    rng = np.random.default_rng(15)
    x = (rng.standard_normal(shape) * 2).astype(np.float16)
    q, p = C.kv_quant_pack(to_dev(x))
    qw, pw = oq.kv_quant_pack(x)
    assert_bitexact(to_np(p), pw, "param")
    assert_bitexact(to_np(q), qw, "codes")


def test_kv_quant_constant_row(C):
    x = np.full((1, 4, 32, 128), 1.5, np.float16)
    q, p = C.kv_quant_pack(to_dev(x))
    qw, pw = oq.kv_quant_pack(x)
    assert_bitexact(to_np(p), pw, "param")
    assert_bitexact(to_np(q), qw, "codes")


def test_errors_are_runtime_errors(C):
    x = torch.zeros(4, 8, dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError):
        C.sym_quant_dynamic(x)
    with pytest.raises(RuntimeError):
        C.sym_quant_dynamic(torch.zeros(4, 8, 2, dtype=torch.float16, device="cuda"))
    with pytest.raises(RuntimeError):
        C.kv_quant_pack(torch.zeros(4, 7, dtype=torch.float16, device="cuda"))
    with pytest.raises(RuntimeError):
        C.sym_dequant(torch.zeros(4, 8, dtype=torch.int32, device="cuda"),
                      torch.zeros(3, dtype=torch.float16, device="cuda"),
                      torch.zeros(8, dtype=torch.float16, device="cuda"))
