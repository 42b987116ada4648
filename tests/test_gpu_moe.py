"""GPU parity of the MoE path (the reference's benchmarks/test_moe_kernels.py,
test_grouped_gemm.py and test_moe_equivalence.py cases, restated):

* sym_quant_dynamic_moe == x * sign[eid] then quant: bit-exact vs the oracle
  and vs the unfused GPU composition;
* sym_dequant_moe (with and without the zero correction): bit-exact;
* matmul_grouped == the dense GEMM per problem, bit-exact, over decode
  (M = 1 per expert), ragged prefill with never-routed experts, heavy skew
  and a single problem; w4a4_linear_moe == matmul_grouped + sym_dequant_moe;
* SignRotMoEBlock: grouped path == per-expert loop bit for bit, stage-wise
  parity with the oracle, and a captured HIP graph replayed on inputs it
  never saw (routing is data-dependent) == eager.
"""
import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle import quant as oq
from tests.gpu_util import assert_bitexact, to_dev, to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def C():
    from signrot_amd import _CUDA
    return _CUDA


def _rows(rng, rows, cols, experts):
    x = rng.standard_normal((rows, cols)).astype(np.float16)
    eid = rng.integers(0, experts, rows).astype(np.int32)
    sign = (rng.integers(0, 2, (experts, cols)) * 2 - 1).astype(np.int8)
    sign[-1] = 1  # an identity (never-calibrated) expert
    return x, eid, sign


QUANT_CASES = [  # rows, cols, experts, clip, with_sign
    (8, 2048, 128, 1.0, True), (8, 768, 128, 1.0, True), (4096, 768, 128, 1.0, True),
    (33, 768, 128, 1.0, False), (128, 768, 128, 0.9, True), (5, 192, 16, 1.0, True),
    (1024, 14336, 8, 1.0, True), (7, 100, 3, 1.0, True), (3, 4104, 2, 1.0, True),
]


@pytest.mark.parametrize("rows,cols,experts,clip,with_sign", QUANT_CASES)
def test_sym_quant_dynamic_moe(C, rows, cols, experts, clip, with_sign):
    rng = np.random.default_rng(rows + cols + experts)
    x, eid, sign = _rows(rng, rows, cols, experts)
    s_arg = to_dev(sign) if with_sign else None
    q, s = C.sym_quant_dynamic_moe(to_dev(x), s_arg, to_dev(eid), clip)
    qw, sw = om.sym_quant_dynamic_moe(x, sign if with_sign else None, eid, clip)
    assert_bitexact(to_np(s), sw, "scale")
    assert_bitexact(to_np(q), qw, "codes")
    # the eager composition it replaces: x * sign[eid], then the plain kernel
    xd = to_dev(x)
    x_ref = xd * to_dev(sign)[to_dev(eid).long()] if with_sign else xd
    q2, s2 = C.sym_quant_dynamic(x_ref.contiguous(), clip)
    assert torch.equal(q, q2) and torch.equal(s, s2)


@pytest.mark.parametrize("rows,cols,experts", [(8, 768, 128), (8, 2048, 128), (200, 2048, 128),
                                               (37, 14336, 8)])
@pytest.mark.parametrize("asym", [False, True])
def test_sym_dequant_moe(C, rows, cols, experts, asym):
    rng = np.random.default_rng(rows * 3 + cols + asym)
    q = rng.integers(-(2 ** 20), 2 ** 20, (rows, cols)).astype(np.int32)
    s_row = ((rng.random(rows) + 0.1) / 64).astype(np.float16)
    w_scales = ((rng.random((experts, cols)) + 0.1) / 64).astype(np.float16)
    eid = rng.integers(0, experts, rows).astype(np.int32)
    z = ws = None
    if asym:
        z = rng.integers(0, 16, rows).astype(np.int8)
        ws = rng.integers(-8 * cols, 7 * cols, (experts, cols)).astype(np.int32)
    out = C.sym_dequant_moe(to_dev(q), to_dev(s_row), to_dev(w_scales), to_dev(eid),
                            None if z is None else to_dev(z), None if ws is None else to_dev(ws))
    assert_bitexact(to_np(out), om.sym_dequant_moe(q, s_row, w_scales, eid, z, ws), "dequant")


def _grouped_inputs(rng, counts, n, k):
    e = len(counts)
    m_total = int(sum(counts))
    a = torch.randint(0, 256, (max(m_total, 1), k // 2), dtype=torch.uint8, device=DEV)[:m_total]
    b = torch.randint(0, 256, (e, n, k // 2), dtype=torch.uint8, device=DEV)
    return a.contiguous(), b


def _run_grouped(C, a, b, counts, n, k):
    e = len(counts)
    c = torch.full((a.shape[0], n), -7, dtype=torch.int32, device=DEV)
    counts_t = torch.tensor(counts, dtype=torch.int32, device=DEV)
    offsets = torch.zeros(e, dtype=torch.int64, device=DEV)
    if e > 1:
        offsets[1:] = torch.cumsum(counts_t[:-1], 0)
    ps = torch.empty((e, 3), dtype=torch.int32, device=DEV)
    ps[:, 0] = counts_t
    ps[:, 1] = n
    ps[:, 2] = k
    ptr_a = a.data_ptr() + offsets * (k // 2)
    ptr_b = b.data_ptr() + torch.arange(e, dtype=torch.int64, device=DEV) * (n * k // 2)
    ptr_c = c.data_ptr() + offsets * (n * 4)
    lda = torch.full((e,), k, dtype=torch.int64, device=DEV)
    ldc = torch.full((e,), n, dtype=torch.int64, device=DEV)
    C.matmul_grouped(ps, ptr_a, ptr_b, ptr_c, lda, lda, ldc, True)
    return c


def _prefill_counts():
    g = np.random.default_rng(0)
    counts = g.integers(0, 40, 128).tolist()
    counts[::7] = [0] * len(counts[::7])
    return counts


GROUPED_CASES = [  # name, counts, n, k
    ("decode 8x(M=1)/128 gateup", [1] * 8 + [0] * 120, 768, 2048),
    ("decode 8x(M=1)/128 down", [1] * 8 + [0] * 120, 2048, 768),
    ("prefill random/128 gateup", _prefill_counts(), 768, 2048),
    ("prefill random/128 down", _prefill_counts(), 2048, 768),
    ("skew [4096,3,0,1]", [4096, 3, 0, 1], 768, 2048),
    ("single problem M=513", [513], 2048, 768),
    ("mixtral 8 experts", [130, 125, 140, 111, 128, 119, 135, 136], 1024, 4096),
    ("all empty", [0, 0, 0], 64, 64),
]


@pytest.mark.parametrize("name,counts,n,k", GROUPED_CASES, ids=[c[0] for c in GROUPED_CASES])
def test_matmul_grouped_vs_dense(C, name, counts, n, k):
    torch.manual_seed(len(counts) + n + k)
    a, b = _grouped_inputs(None, counts, n, k)
    c = _run_grouped(C, a, b, counts, n, k)
    row = 0
    for i, m in enumerate(counts):
        if m == 0:
            continue
        ref = C.matmul(a[row:row + m].contiguous(), b[i].contiguous())
        assert torch.equal(c[row:row + m], ref), f"problem {i} (m={m}) differs"
        row += m


def test_matmul_grouped_vs_oracle(C):
    counts, n, k = [3, 0, 17, 1], 40, 96
    torch.manual_seed(1)
    a, b = _grouped_inputs(None, counts, n, k)
    c = to_np(_run_grouped(C, a, b, counts, n, k))
    an, bn = to_np(a), to_np(b)
    off = om.expert_offsets(counts)
    want = om.matmul_grouped([(an[off[e]:off[e + 1]], bn[e]) for e in range(len(counts))])
    for e in range(len(counts)):
        assert_bitexact(c[off[e]:off[e + 1]], want[e], f"problem {e}")


# Experts past one 128-row tile with 1..64 rows left over compute those rows
# on their last full tile (one or two extra 32-row blocks of the grouped
# kernel's compute waves); 65+ left over, exact tiles and single tiles are
# tiled as they are.  The cases put
# every kind of expert side by side, at the MoE down shape too, with every
# expert taking extra rows, with many experts, at the fewest K steps that
# allow it (two) and with a ragged last K step, and at K <= 256 (one step:
# every row tiled).
REM_COUNTS = [160, 161, 257, 0, 100, 128, 140, 288, 33, 129, 1, 416, 170, 192, 193]


@pytest.mark.parametrize("counts,n,k", [([3, 0, 5, 1], 300, 768),
                                        ([130, 125, 140, 111, 128, 119, 135, 136], 14336, 4096),
                                        ([0, 0], 128, 128), ([1], 4096, 14336),
                                        (REM_COUNTS, 1000, 800), (REM_COUNTS, 4096, 14336),
                                        ([129, 0, 150], 16, 64), ([1025] * 4, 300, 2048),
                                        ([140] * 8, 14336, 4096), ([131] * 300, 40, 1024),
                                        ([131] * 1025, 16, 64), ([140, 129, 160], 200, 512),
                                        ([150, 33, 161, 288], 64, 288)],
                         ids=["small", "cfg5-gate", "empty", "one-row", "rem-kinds",
                              "rem-down", "rem-narrow", "rem-one-row", "rem-all-experts",
                              "rem-300-experts", "1025-experts", "rem-two-steps",
                              "rem-ragged-k"])
def test_w4a4_linear_moe(C, counts, n, k):
    torch.manual_seed(sum(counts) + n)
    a, b = _grouped_inputs(None, counts, n, k)
    e, rows = len(counts), a.shape[0]
    sa = (torch.rand(rows, device=DEV) * 0.05 + 1e-3).half()
    sb = (torch.rand(e, n, device=DEV) * 0.01 + 1e-4).half()
    off = torch.tensor(om.expert_offsets(counts), dtype=torch.int32, device=DEV)
    out = C.w4a4_linear_moe(a, sa, b, sb, off)
    eid = torch.repeat_interleave(torch.arange(e, device=DEV, dtype=torch.int32),
                                  torch.tensor(counts, device=DEV))
    c = _run_grouped(C, a, b, counts, n, k)
    ref = C.sym_dequant_moe(c, sa, sb, eid)
    assert torch.equal(out, ref)
    if rows and rows * n * k <= 64 * 1024 * 1024:
        want = om.w4a4_linear_moe(to_np(a), to_np(sa), to_np(b), to_np(sb), to_np(off))
        assert_bitexact(to_np(out), want, "fp16 out")


@pytest.mark.parametrize("counts,n,k", [([3, 0, 5, 1], 300, 768),
                                        ([123, 127, 123, 122, 123, 126, 136, 144], 14336, 4096),
                                        ([0, 0], 128, 128), ([1], 4096, 1024)])
def test_w4a4_linear_moe_gate_up_equals_two_calls(C, counts, n, k):
    """The paired launch gives each projection bit for bit what its own
    w4a4_linear_moe call gives (the oracle pins that call above)."""
    torch.manual_seed(sum(counts) + n + 1)
    a, bg = _grouped_inputs(None, counts, n, k)
    _, bu = _grouped_inputs(None, counts, n, k)
    e, rows = len(counts), a.shape[0]
    sa = (torch.rand(rows, device=DEV) * 0.05 + 1e-3).half()
    sg = (torch.rand(e, n, device=DEV) * 0.01 + 1e-4).half()
    su = (torch.rand(e, n, device=DEV) * 0.01 + 1e-4).half()
    off = torch.tensor(om.expert_offsets(counts), dtype=torch.int32, device=DEV)
    g, u = C.w4a4_linear_moe_gate_up(a, sa, bg, sg, bu, su, off)
    assert torch.equal(g, C.w4a4_linear_moe(a, sa, bg, sg, off))
    assert torch.equal(u, C.w4a4_linear_moe(a, sa, bu, su, off))
    if rows:
        assert not torch.equal(g, u)


@pytest.mark.parametrize("T,E,k,norm", [(512, 8, 2, True), (37, 8, 2, False),
                                        (300, 64, 8, True), (5, 4, 4, True),
                                        (1000, 60, 6, False), (700, 16, 1, True),
                                        (0, 8, 2, True), (5000, 8, 2, True),
                                        (2049, 9, 3, False), (900, 32, 4, True),
                                        (3, 1, 1, True), (4100, 64, 2, False)])
def test_moe_route_matches_torch(C, T, E, k, norm):
    """srq_moe_route against the reference's torch ops (moe.py:168-185):
    softmax in fp32, topk, renormalization and the fp16 cast bit for bit;
    the same experts chosen except where the k-th and (k+1)-th
    probabilities tie (then the lower expert wins); rows ordered by expert,
    stable; counts, offsets, inv and token consistent with the order."""
    g = torch.Generator(device=DEV).manual_seed(T + E + k)
    logits = torch.randn(T, E, generator=g, device=DEV).half()
    if T > 10:  # exact ties inside rows
        logits[::5, 1] = logits[::5, 0]
        logits[::7, E - 1] = logits[::7, E // 2]
    w, order, inv, expert, token, counts, offsets = C.moe_route(logits, k, norm)
    probs = torch.softmax(logits, dim=1, dtype=torch.float)
    tp, te = torch.topk(probs, k, dim=-1)
    if norm:
        tp = tp / tp.sum(dim=-1, keepdim=True)
    assert torch.equal(w, tp.half())
    # our choice per row: expert[inv] in (token, choice) order
    ours = expert[inv.long()].view(T, k).long() if T else te
    same = (torch.sort(ours, 1).values == torch.sort(te, 1).values).all(1)
    if T and not same.all():
        bad = (~same).nonzero().flatten()
        srt = torch.sort(probs[bad], 1, descending=True).values
        assert k < E and torch.equal(srt[:, k - 1], srt[:, k]), "choice differs without a tie"
    # our value order: descending, ties to the lower expert
    pv = probs.gather(1, ours) if T else tp
    assert (pv[:, :-1] >= pv[:, 1:]).all()
    tie = pv[:, :-1] == pv[:, 1:]
    assert (ours[:, :-1][tie] < ours[:, 1:][tie]).all()
    flat = ours.reshape(-1)
    assert torch.equal(expert.long(), torch.sort(flat, stable=True).values)
    assert torch.equal(flat[order.long()], expert.long())
    assert torch.equal(inv[order.long()], torch.arange(T * k, device=DEV, dtype=torch.int32))
    assert torch.equal(token, order // k)
    assert torch.equal(counts.long(), torch.bincount(flat, minlength=E))
    assert offsets[0] == 0 and torch.equal(offsets[1:] - offsets[:-1], counts)
    for e in range(E):
        r = order[offsets[e]:offsets[e + 1]]
        assert torch.all(r[1:] > r[:-1])


@pytest.mark.parametrize("E,k,norm", [(8, 2, True), (8, 2, False), (16, 4, True)])
def test_moe_route_nonfinite_rows(C, E, k, norm):
    """Rows whose logits hold a NaN, a +inf or only -inf have all-NaN fp32
    softmax probabilities in torch; torch.topk ranks NaN above every number,
    so such a token gets k distinct experts with NaN weights (and a NaN block
    output).  Here: NaN ranks first, NaN ties go to the lower expert, each
    expert at most once; finite rows (a partly -inf row among them) are
    unchanged and equal torch's ops bit for bit."""
    g = torch.Generator(device=DEV).manual_seed(E * 10 + k)
    T = 24
    logits = torch.randn(T, E, generator=g, device=DEV).half()
    nan, inf = float("nan"), float("inf")
    logits[3, 1] = nan
    logits[5, E - 1] = inf
    logits[7, :] = -inf
    logits[9, 2] = inf
    logits[9, 4] = -inf
    logits[11, ::2] = -inf  # partly -inf: finite probabilities
    bad = torch.tensor([3, 5, 7, 9], device=DEV)
    w, order, inv, expert, token, counts, offsets = C.moe_route(logits, k, norm)
    probs = torch.softmax(logits, dim=1, dtype=torch.float)
    assert torch.isnan(probs[bad]).all()  # the premise: torch's rows are all NaN
    ours = expert[inv.long()].view(T, k).long()
    wv = w.view(T, k)
    assert torch.isnan(wv[bad]).all(), "non-finite rows must carry NaN weights"
    for t in bad.tolist():
        assert ours[t].tolist() == list(range(k)), "NaN ties: the lower experts, once each"
    good = torch.ones(T, dtype=torch.bool, device=DEV)
    good[bad] = False
    tp, te = torch.topk(probs[good], k, dim=-1)
    if norm:
        tp = tp / tp.sum(dim=-1, keepdim=True)
    assert torch.equal(wv[good], tp.half())
    assert torch.isfinite(wv[good]).all()
    assert torch.equal(torch.sort(ours[good], 1).values, torch.sort(te, 1).values)
    flat = ours.reshape(-1)
    assert torch.equal(counts.long(), torch.bincount(flat, minlength=E))
    assert torch.equal(expert.long(), torch.sort(flat, stable=True).values)


@torch.no_grad()
def test_block_nan_token():
    """One token with a NaN activation through SignRotMoEBlock.forward: its
    router logits are NaN, so (as with torch's softmax / topk) its output row
    is all NaN; every other token's output equals the clean run's bit for
    bit (grouping by expert does not change a row's arithmetic)."""
    blk = _block(256, 768, 16, 4, True, seed=11)
    x = torch.randn(1, 37, 256, device=DEV, dtype=torch.float16)
    out, _ = blk(x)
    xn = x.clone()
    xn[0, 3, 5] = float("nan")
    outn, logits = blk(xn)
    assert torch.isnan(logits[3]).all()
    assert torch.isnan(outn[0, 3]).all()
    keep = torch.ones(37, dtype=torch.bool, device=DEV)
    keep[3] = False
    assert torch.equal(outn[0, keep], out[0, keep])


@pytest.mark.parametrize("T,k,H", [(512, 2, 4096), (33, 1, 64), (7, 2, 8), (100, 4, 256),
                                   (0, 2, 64), (20, 8, 128), (16, 10, 64)])
def test_moe_combine_matches_torch(C, T, k, H):
    """srq_moe_combine against (y[inv].view(T, k, H) * w.unsqueeze(-1)).sum(1)
    in torch fp16 (moe.py:226-230): bit for bit for k <= 2 (fp32 sums of
    two products are order-free); for k = 4, 8 and 10 (past the kernel's
    batched choices) within one fp16 ulp (torch's reduction order is its
    own)."""
    g = torch.Generator(device=DEV).manual_seed(T * k + H)
    y = torch.randn(T * k, H, generator=g, device=DEV).half()
    w = torch.rand(T, k, generator=g, device=DEV).half()
    inv = torch.randperm(T * k, generator=g, device=DEV).to(torch.int32)
    got = C.moe_combine(y, inv, w)
    want = (y[inv.long()].view(T, k, H) * w.unsqueeze(-1)).sum(dim=1)
    if k <= 2:
        assert torch.equal(got, want)
    else:
        ulp = torch.finfo(torch.float16).eps * want.float().abs().clamp(min=6.1e-5)
        assert ((got.float() - want.float()).abs() <= ulp).all()


# ------------------------------------------------------------------ block

def _block(hidden, inter, experts, top_k, norm, seed, with_sign=True):
    from signrot_amd.nn import SignRotMoEBlock
    g = torch.Generator(device=DEV).manual_seed(seed)
    gate = torch.nn.Linear(hidden, experts, bias=False, dtype=torch.float16, device=DEV)
    with torch.no_grad():
        gate.weight.normal_(0, 0.1, generator=g)

    def w(n, k):
        return torch.randint(0, 256, (experts, n, k // 2), dtype=torch.uint8, device=DEV,
                             generator=g)

    def s(n, k):
        # keep each stage's gain near one so activations stay finite in fp16
        return torch.full((experts, n), 1.0 / k, dtype=torch.float16, device=DEV)

    sign = None
    if with_sign:
        sign = (torch.randint(0, 2, (experts, inter), dtype=torch.int8, device=DEV,
                              generator=g) * 2 - 1)
    return SignRotMoEBlock(gate, top_k=top_k, norm_topk_prob=norm,
                           w_gate=w(inter, hidden), s_gate=s(inter, hidden),
                           w_up=w(inter, hidden), s_up=s(inter, hidden),
                           w_down=w(hidden, inter), s_down=s(hidden, inter),
                           sign_down=sign).eval()


BLOCKS = [  # hidden, inter, experts, top_k, norm, tokens
    (256, 768, 16, 4, True, 37),
    (512, 1536, 8, 2, False, 5),
    (4096, 14336, 8, 2, True, 64),
    (4096, 14336, 8, 2, True, 512),      # config 5 (Mixtral-8x7B shape, 512 tokens)
]


@pytest.mark.parametrize("hidden,inter,experts,top_k,norm,tokens", BLOCKS)
@torch.no_grad()
def test_block_grouped_equals_loop(hidden, inter, experts, top_k, norm, tokens):
    blk = _block(hidden, inter, experts, top_k, norm, seed=hidden + tokens)
    x = torch.randn(1, tokens, hidden, device=DEV, dtype=torch.float16)
    blk.use_grouped = True
    out, logits = blk(x)
    blk.use_grouped = False
    out_loop, logits_loop = blk(x)
    assert torch.equal(logits, logits_loop)
    assert torch.equal(out, out_loop)
    assert torch.isfinite(out).all()


def _check_moe_rows(got, q, s, w, s_w, eid, rows, what):
    """Oracle W4A4 linear of the given expert-ordered rows, each against its
    own expert's weights, bit-exact."""
    got, q, s, eid = to_np(got), to_np(q), to_np(s), to_np(eid)
    w, s_w = to_np(w), to_np(s_w)
    for e in np.unique(eid[rows]):
        r = rows[eid[rows] == e]
        assert_bitexact(got[r], oq.w4a4_linear(q[r], s[r].reshape(-1), w[e], s_w[e]),
                        f"{what} (expert {e})")


@pytest.mark.parametrize("hidden,inter,experts,top_k,norm,tokens", BLOCKS[:2] + BLOCKS[3:])
@torch.no_grad()
def test_block_stagewise_vs_oracle(C, hidden, inter, experts, top_k, norm, tokens):
    """Each stage of the grouped forward against the oracle on the previous
    stage's GPU output (the rotation's fp16 bits are tolerance-pinned, so it
    is checked against its own oracle separately)."""
    from signrot_amd.functional.hadamard import matmul_hadU_cuda
    from oracle import glue as og
    blk = _block(hidden, inter, experts, top_k, norm, seed=7 + tokens)
    x = torch.randn(tokens, hidden, device=DEV, dtype=torch.float16)
    route = blk.route(x)
    tok = route.order // top_k
    eid = route.expert
    off = route.offsets
    assert torch.equal(off[1:] - off[:-1], route.counts)
    # the routing rule itself (moe.py:168-185): fp32 softmax, top-k,
    # renormalised, rows ordered by expert, stable within an expert
    probs = torch.softmax(route.logits.float(), dim=1)
    tp, te = torch.topk(probs, top_k, dim=-1)
    if norm:
        tp = tp / tp.sum(dim=-1, keepdim=True)
    assert torch.equal(route.weights, tp.to(x.dtype))
    flat = te.reshape(-1)
    assert torch.equal(route.expert.long(), torch.sort(flat, stable=True).values)
    assert torch.equal(flat[route.order], route.expert.long())
    for e in range(experts):
        rows = route.order[off[e]:off[e + 1]]
        assert torch.all(rows[1:] > rows[:-1])   # stable: increasing within an expert
    q_tok, s_tok = C.sym_quant_dynamic(x, 1.0)
    qw, sw = oq.sym_quant_dynamic(to_np(x))
    assert_bitexact(to_np(q_tok), qw, "token codes")
    q_a, s_a = q_tok[tok], s_tok[tok]
    gate_h = C.w4a4_linear_moe(q_a, s_a.view(-1), blk.w_gate, blk.s_gate, off)
    up_h = C.w4a4_linear_moe(q_a, s_a.view(-1), blk.w_up, blk.s_up, off)
    offn = to_np(off)
    nrows = tokens * top_k
    big = nrows * inter * hidden > 1e9
    # every row for small blocks; the first, last and 16 random rows of
    # every expert at the config-5 shape (the float64 oracle is too slow
    # for all 1024 rows x 14336 x 4096 three times)
    rng = np.random.default_rng(tokens)
    rows = np.arange(nrows) if not big else np.unique(np.concatenate(
        [np.concatenate([[offn[e], offn[e + 1] - 1],
                         rng.integers(offn[e], offn[e + 1], 16)])
         for e in range(experts) if offn[e + 1] > offn[e]]).astype(np.int64))
    if not big:
        assert_bitexact(to_np(gate_h), om.w4a4_linear_moe(to_np(q_a), to_np(s_a),
                                                           to_np(blk.w_gate), to_np(blk.s_gate),
                                                           offn), "gate")
    _check_moe_rows(gate_h, q_a, s_a, blk.w_gate, blk.s_gate, eid, rows, "gate")
    _check_moe_rows(up_h, q_a, s_a, blk.w_up, blk.s_up, eid, rows, "up")
    inter_h = C.swiglu(gate_h, up_h)
    np.testing.assert_allclose(to_np(inter_h).astype(np.float32),
                               og.swiglu(to_np(gate_h), to_np(up_h)).astype(np.float32),
                               rtol=2e-3, atol=2e-3)
    h = matmul_hadU_cuda(inter_h, blk.had_K, blk.K)
    q_d, s_d = C.sym_quant_dynamic_moe(h, blk.sign_down, eid, 1.0)
    qdw, sdw = om.sym_quant_dynamic_moe(to_np(h), to_np(blk.sign_down), to_np(eid))
    assert_bitexact(to_np(s_d), sdw, "down scale")
    assert_bitexact(to_np(q_d), qdw, "down codes")
    y = C.w4a4_linear_moe(q_d, s_d.view(-1), blk.w_down, blk.s_down, off)
    _check_moe_rows(y, q_d, s_d, blk.w_down, blk.s_down, eid, rows, "down")
    # the block's own forward gives these stages' result after the combine
    out, _ = blk(x.view(1, tokens, hidden))
    slots = torch.empty_like(y)
    slots[route.order] = y
    want = (slots.view(tokens, top_k, hidden) * route.weights.unsqueeze(-1)).sum(dim=1)
    assert torch.equal(out.view(tokens, hidden), want), "block output"


@torch.no_grad()
def test_block_graph_replay_on_new_inputs():
    blk = _block(256, 768, 16, 4, True, seed=99)
    x_static = torch.randn(1, 24, 256, device=DEV, dtype=torch.float16)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            blk(x_static)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static, _ = blk(x_static)
    for i in range(4):
        x_new = torch.randn(1, 24, 256, device=DEV, dtype=torch.float16) * (1 + i)
        x_static.copy_(x_new)
        graph.replay()
        torch.cuda.synchronize()
        want, _ = blk(x_new)
        torch.cuda.synchronize()
        assert torch.equal(out_static, want), f"replay {i} differs from eager"


@pytest.mark.parametrize("rows,n,K,experts,clip,with_sign", [
    (600, 14336, 28, 8, 1.0, True), (37, 6144, 12, 16, 0.8, True), (5, 10240, 20, 4, 1.0, True),
    (300, 14336, 28, 8, 1.0, False)])
def test_swiglu_had_sign_quant_moe(C, rows, n, K, experts, clip, with_sign):
    """The fused MoE down-proj input op equals swiglu -> rotation (no sign) ->
    sym_quant_dynamic_moe bit for bit, with expert ids in random order, ids
    outside the sign table (sign +1), and more rows than persistent blocks
    (each row's sign masks are loaded for that row)."""
    from oracle import hadamard as oh
    rng = np.random.default_rng(rows + n)
    gate = to_dev((rng.standard_normal((rows, n)) * 2).astype(np.float16))
    up = to_dev((rng.standard_normal((rows, n)) * 2).astype(np.float16))
    eid_np = rng.integers(0, experts, rows).astype(np.int32)
    eid_np[: min(rows, 3)] = [-1, experts, 1 << 20][: min(rows, 3)]
    eid = to_dev(eid_np)
    sign = to_dev(rng.choice([-1, 1], (experts, n)).astype(np.int8)) if with_sign else None
    hk = to_dev(oh.had_table(K).astype(np.float32)).half()
    q, s = C.swiglu_had_sign_quant_moe(gate, up, hk, K, sign, eid, clip)
    inter = C.swiglu(gate, up)
    rot = C.online_hadamard(inter, hk, K, None)
    q2, s2 = C.sym_quant_dynamic_moe(rot, sign, eid, clip)
    assert torch.equal(s, s2), "scales"
    assert torch.equal(q, q2), "codes"


@pytest.mark.parametrize("counts,n,k", [([3, 0, 5, 1], 304, 768), ([0, 0], 64, 256),
                                       ([123, 127, 123, 122, 123, 126, 136, 144], 14336, 4096),
                                       ([700, 1], 1024, 2048), (REM_COUNTS, 1008, 800),
                                       ([130, 131, 160, 99], 14336, 4096),
                                       ([140] * 8, 14336, 4096), ([140, 161, 129], 48, 512),
                                       ([170, 192, 193, 224, 160], 2048, 1024)])
def test_w4a4_linear_moe_swiglu_equals_gate_up_then_swiglu(C, counts, n, k):
    """The SwiGLU epilogue of the grouped gate/up launch over interleaved
    weights: bit-identical to the two projections followed by srq_swiglu."""
    torch.manual_seed(sum(counts) + n)
    a, bg = _grouped_inputs(None, counts, n, k)
    _, bu = _grouped_inputs(None, counts, n, k)
    e, rows = len(counts), a.shape[0]
    sa = (torch.rand(rows, device=DEV) * 0.05 + 1e-3).half()
    sg = (torch.rand(e, n, device=DEV) * 0.01 + 1e-4).half()
    su = (torch.rand(e, n, device=DEV) * 0.01 + 1e-4).half()
    off = torch.tensor(om.expert_offsets(counts), dtype=torch.int32, device=DEV)
    g, u = C.w4a4_linear_moe_gate_up(a, sa, bg, sg, bu, su, off)
    want = C.swiglu(g, u) if rows else g
    w_il, s_il = C.interleave_gate_up_experts(bg, sg, bu, su)
    got = C.w4a4_linear_moe_swiglu(a, sa, w_il, s_il, off)
    assert torch.equal(got, want)


@pytest.mark.parametrize("rows,n,K,experts,with_sign", [
    (600, 14336, 28, 8, True), (37, 6144, 12, 16, True), (5, 20480, 20, 4, True),
    (300, 14336, 28, 8, False)])
def test_had_sign_quant_moe_equals_rotation_then_moe_quant(C, rows, n, K, experts, with_sign):
    """The plain MoE down-proj input op (input already through the SwiGLU)
    equals rotation (no sign) -> sym_quant_dynamic_moe bit for bit, H_512
    and H_1024 chunks, ids outside the sign table."""
    from oracle import hadamard as oh
    rng = np.random.default_rng(rows + n + 1)
    x = to_dev((rng.standard_normal((rows, n)) * 2).astype(np.float16))
    eid_np = rng.integers(0, experts, rows).astype(np.int32)
    eid_np[: min(rows, 3)] = [-1, experts, 1 << 20][: min(rows, 3)]
    eid = to_dev(eid_np)
    sign = to_dev(rng.choice([-1, 1], (experts, n)).astype(np.int8)) if with_sign else None
    hk = to_dev(oh.had_table(K).astype(np.float32)).half()
    q, s = C.had_sign_quant_moe(x, hk, K, sign, eid)
    rot = C.online_hadamard(x, hk, K, None)
    q2, s2 = C.sym_quant_dynamic_moe(rot, sign, eid)
    assert torch.equal(s, s2), "scales"
    assert torch.equal(q, q2), "codes"


@pytest.mark.parametrize("rows,cols,R", [(512, 4096, 1024), (37, 768, 100), (5, 8, 3),
                                        (64, 14336, 130)])
def test_sym_quant_dynamic_rows_equals_quant_then_gather(C, rows, cols, R):
    """Quantizing gathered rows in one launch: bit-identical to
    sym_quant_dynamic then the row gather; out-of-range indices give zero
    codes and scale 0."""
    rng = np.random.default_rng(rows + cols + R)
    x = to_dev((rng.standard_normal((rows, cols)) * 3).astype(np.float16))
    idx_np = rng.integers(0, rows, R).astype(np.int32)
    idx_np[: min(R, 2)] = [-1, rows][: min(R, 2)]
    idx = to_dev(idx_np)
    q, s = C.sym_quant_dynamic_rows(x, idx)
    qa, sa = C.sym_quant_dynamic(x)
    ok = torch.from_numpy((idx_np >= 0) & (idx_np < rows)).to(DEV)
    safe = torch.where(ok, idx.long(), torch.zeros_like(idx.long()))
    want_q = torch.where(ok[:, None], qa[safe], torch.zeros_like(qa[safe]))
    want_s = torch.where(ok[:, None], sa[safe], torch.zeros_like(sa[safe]))
    assert torch.equal(q, want_q), "codes"
    assert torch.equal(s, want_s), "scales"


@torch.no_grad()
def test_block_fused_down_equals_unfused():
    blk = _block(4096, 14336, 8, 2, True, seed=5)
    x = torch.randn(1, 96, 4096, device=DEV, dtype=torch.float16)
    blk.fuse_down = True
    out, _ = blk(x)
    blk.fuse_down = False
    out2, _ = blk(x)
    assert torch.equal(out, out2)
    assert torch.isfinite(out).all()
