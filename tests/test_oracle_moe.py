"""Pins of oracle/moe.py by properties that do not restate its formulas:

* the sign-fused quantizer: flipping signs leaves the row max (hence the
  scale) unchanged and, with clip 1 (codes within [-7, 7], no clamp
  asymmetry), negates exactly the codes at flipped positions -- checked
  against the unsigned oracle quantizer, itself pinned by exact rational
  arithmetic in test_oracle_quant.py;
* the expert-indexed dequant: per row, the dense dequant with that expert's
  weight-scale row, with the zero correction done in Python ints (the
  reference test's own check, benchmarks/test_moe_kernels.py:53-74);
* the grouped GEMM: a Python-int triple loop per problem, zero-row problems
  included (benchmarks/test_grouped_gemm.py:28-59).
"""
import numpy as np
import pytest

from oracle import moe as om
from oracle import quant as oq


@pytest.mark.parametrize("rows,cols,experts", [(8, 768, 16), (33, 192, 4), (5, 2048, 128)])
def test_sign_flip_negates_codes(rows, cols, experts):
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float16)
    eid = rng.integers(0, experts, rows).astype(np.int32)
    sign = (rng.integers(0, 2, (experts, cols)) * 2 - 1).astype(np.int8)
    sign[-1] = 1
    q, s = om.sym_quant_dynamic_moe(x, sign, eid)
    q0, s0 = oq.sym_quant_dynamic(x)
    assert np.array_equal(s.view(np.uint16), s0.view(np.uint16))
    codes, codes0 = oq.unpack_i4(q), oq.unpack_i4(q0)
    assert np.abs(codes0).max() <= 7
    assert np.array_equal(codes, codes0 * sign[eid].astype(np.int64))


def test_sign_none_is_plain_quant():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((9, 96)) * 4).astype(np.float16)
    eid = rng.integers(0, 3, 9).astype(np.int32)
    q, s = om.sym_quant_dynamic_moe(x, None, eid, 0.9)
    q0, s0 = oq.sym_quant_dynamic(x, 0.9)
    assert np.array_equal(q, q0) and np.array_equal(s.view(np.uint16), s0.view(np.uint16))


@pytest.mark.parametrize("asym", [False, True])
def test_dequant_moe_is_per_row_dense_dequant(asym):
    rng = np.random.default_rng(11)
    rows, cols, experts = 12, 40, 5
    q = rng.integers(-(2 ** 20), 2 ** 20, (rows, cols)).astype(np.int32)
    s_row = ((rng.random(rows) + 0.1) / 64).astype(np.float16)
    w_scales = ((rng.random((experts, cols)) + 0.1) / 64).astype(np.float16)
    eid = rng.integers(0, experts, rows).astype(np.int32)
    zero_row = w_sum = None
    q_adj = [[int(v) for v in r] for r in q]
    if asym:
        zero_row = rng.integers(0, 16, rows).astype(np.int8)
        w_sum = rng.integers(-8 * cols, 7 * cols, (experts, cols)).astype(np.int32)
        for r in range(rows):
            for c in range(cols):
                q_adj[r][c] -= int(zero_row[r]) * int(w_sum[eid[r], c])
    out = om.sym_dequant_moe(q, s_row, w_scales, eid, zero_row, w_sum)
    for r in range(rows):
        want = oq.sym_dequant(np.array([q_adj[r]], np.int64), s_row[r:r + 1], w_scales[eid[r]])
        assert np.array_equal(out[r:r + 1].view(np.uint16), want.view(np.uint16))


def test_grouped_gemm_brute_force():
    rng = np.random.default_rng(5)
    k = 64
    problems = []
    for m, n in [(3, 5), (0, 4), (1, 7), (6, 2)]:
        a = rng.integers(0, 256, (m, k // 2)).astype(np.uint8)
        b = rng.integers(0, 256, (n, k // 2)).astype(np.uint8)
        problems.append((a, b))
    outs = om.matmul_grouped(problems)
    for (a, b), c in zip(problems, outs):
        ca, cb = oq.unpack_i4(a).tolist(), oq.unpack_i4(b).tolist()
        want = [[sum(x * y for x, y in zip(ra, rb)) for rb in cb] for ra in ca]
        assert c.shape == (a.shape[0], b.shape[0])
        assert c.tolist() == want


def test_w4a4_linear_moe_offsets():
    rng = np.random.default_rng(8)
    counts = [2, 0, 3, 1]
    off = om.expert_offsets(counts)
    assert off.tolist() == [0, 2, 2, 5, 6]
    k, n = 32, 6
    a = rng.integers(0, 256, (6, k // 2)).astype(np.uint8)
    b = rng.integers(0, 256, (4, n, k // 2)).astype(np.uint8)
    sa = ((rng.random(6) + 0.5) / 8).astype(np.float16)
    sb = ((rng.random((4, n)) + 0.5) / 8).astype(np.float16)
    out = om.w4a4_linear_moe(a, sa, b, sb, off)
    eid = np.repeat(np.arange(4), counts)
    c = np.concatenate([oq.matmul_s4s4(a[off[e]:off[e + 1]], b[e]) for e in range(4)])
    want = om.sym_dequant_moe(c, sa, sb, eid)
    assert np.array_equal(out.view(np.uint16), want.view(np.uint16))
