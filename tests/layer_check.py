"""Stage-by-stage checks of the W4A4 Llama layer against the oracle, shared
by the decode-step and prefill tests.  Each stage's HIP output is compared
with the oracle applied to the HIP output of the previous stage, so integer
stages are checked bit-exactly on identical fp16 inputs (int4 codes flip on
one-ulp input changes, which end-to-end comparisons would amplify).
Arrays are host numpy copies of the layer's trace."""
import numpy as np

from oracle import attention as oa
from oracle import glue
from oracle import hadamard as oh
from oracle import quant as oq
from tests.gpu_util import assert_bitexact

D = 128


def ulps(got, want, what, n=1):
    g = np.asarray(got, np.float16).astype(np.float64)
    w = np.asarray(want, np.float16).astype(np.float64)
    tol = n * np.spacing(np.abs(np.asarray(want, np.float16))).astype(np.float64)
    bad = np.abs(g - w) > tol
    assert not bad.any(), f"{what}: {bad.sum()} / {bad.size} beyond {n} ulp"


def linear(x, w):
    q, s = oq.sym_quant_dynamic(x)
    return oq.w4a4_linear(q, s.reshape(-1), *w)


def page_table(lengths, page):
    """(indptr, indices, last) of the cache's page table for per-request
    lengths that need the same page count (physical page of (request b,
    page j) = j * B + b, kv_cache.py:417-433)."""
    lengths = np.asarray(lengths)
    B = len(lengths)
    pages = (lengths + page - 1) // page
    assert (pages == pages[0]).all()
    n = int(pages[0])
    indptr = (np.arange(B + 1) * n).astype(np.int32)
    indices = (np.arange(n)[None, :] * B + np.arange(B)[:, None]).reshape(-1).astype(np.int32)
    last = ((lengths - 1) % page + 1).astype(np.int32)
    return indptr, indices, last


def check_k_entry(got_data, got_param, pg, e, layer, k_rot, what):
    """A cached K entry: quantized from the rotated fp16 K, which the HIP
    FWHT reproduces within rounding: within half a step plus 2e-3."""
    kd = oq.kv_dequant(got_data[pg, layer, 0, :, e], got_param[pg, layer, 0, :, e])
    err = np.abs(kd - np.asarray(k_rot, np.float32))
    tol = got_param[pg, layer, 0, :, e, 0:1].astype(np.float32) * 0.51 + 2e-3
    assert (err <= tol).all(), what


def check_attn_out_and_mlp(tr, h, w, hidden, Hq, ffn, out, rows=None):
    """From the attention output on: head-axis Hadamard, o_proj + residual,
    RMSNorm, gate/up, SwiGLU, the down-proj rotation + quantizer, down_proj
    and the final residual.  tr["attn"] holds [R, ..., Hq, D]; h the layer
    input [R, hidden]; rows: the rows to compare (default all)."""
    R = h.shape[0]
    sel = np.arange(R) if rows is None else np.asarray(rows)
    attn = tr["attn"].reshape(R, Hq, D)
    a_rot = oh.rotate(np.ascontiguousarray(attn.transpose(0, 2, 1)).reshape(-1, Hq)
                      ).reshape(R, D, Hq).transpose(0, 2, 1).reshape(R, hidden)
    ulps(tr["attn_rot"][sel], a_rot[sel], "head-axis Hadamard")
    o = linear(tr["attn_rot"], w["o"])
    assert_bitexact(tr["resid1"][sel],
                    (h.astype(np.float32) + o.astype(np.float32)).astype(np.float16)[sel],
                    "o_proj + residual")
    ulps(tr["norm2"][sel], glue.rmsnorm(tr["resid1"], 1e-5, hidden)[sel], "post-attention rmsnorm")
    assert_bitexact(tr["gu"][sel], linear(tr["norm2"], w["gu"])[sel], "gate/up projection")
    sw = glue.swiglu(tr["gu"][:, :ffn], tr["gu"][:, ffn:])
    mism = (tr["act"][sel].view(np.uint16) != sw[sel].view(np.uint16)).mean()
    assert mism < 1e-3, mism
    qd, sd = oq.sym_quant_dynamic(oh.online_hadamard(tr["act"], w["down_sign"]))
    assert (tr["down_q"][sel] != qd[sel]).mean() < 0.01  # one-ulp rotation differences
    assert_bitexact(tr["down"][sel], oq.w4a4_linear(tr["down_q"], tr["down_s"].reshape(-1),
                                                    *w["down"])[sel], "down_proj")
    assert_bitexact(out.reshape(R, hidden)[sel],
                    (tr["resid1"].astype(np.float32) + tr["down"].astype(np.float32))
                    .astype(np.float16)[sel], "final residual")


def check_decode_step(tr, h, w, out, cos, sin, got_data, got_param, table, positions, layer,
                      hidden, Hq, Hkv, ffn, page):
    """One decode step (op-by-op trace) of a batch of B requests: h [B,
    hidden] the input, cos/sin [1 or B, 1, D] host arrays, got_data /
    got_param the cache after the step, table the page table after the step,
    positions[b] the appended token's position in request b."""
    B = h.shape[0]
    indptr, indices, last = table
    ulps(tr["norm1"], glue.rmsnorm(h, 1e-5, hidden), "input rmsnorm")
    assert_bitexact(tr["qkv"], linear(tr["norm1"], w["qkv"]), "q/k/v projection")
    q = tr["qkv"][:, : Hq * D].reshape(B, 1, Hq, D)
    k = tr["qkv"][:, Hq * D: (Hq + Hkv) * D].reshape(B, 1, Hkv, D)
    qw, kw = glue.rope_qk(q, k, cos, sin)
    assert_bitexact(tr["q_rope"], qw, "rope q")
    assert_bitexact(tr["k_rope"], kw, "rope k")
    # the appended token: V codes bit-exact, K within the FWHT tolerance
    kr = oh.rotate(tr["k_rope"].reshape(-1, D)).reshape(B, Hkv, D)
    vq, vp = oq.kv_quant_pack(tr["qkv"][:, (Hq + Hkv) * D:].reshape(B, Hkv, D))
    for b in range(B):
        pg, e = oa.slot(indptr, indices, page, b, int(positions[b]))
        assert_bitexact(got_data[pg, layer, 1, :, e], vq[b], f"appended V codes b={b}")
        assert_bitexact(got_param[pg, layer, 1, :, e], vp[b], f"appended V params b={b}")
        check_k_entry(got_data, got_param, pg, e, layer, kr[b], f"appended K b={b}")
    # attention over the cache as stored (incl. the appended token)
    qr = oh.rotate(tr["q_rope"].reshape(-1, D)).reshape(B, Hq, D)
    att = oa.decode(qr, got_data, got_param, indptr, indices, last, layer)
    d = np.abs(tr["attn"].reshape(B, Hq, D).astype(np.float64) - att)
    assert (d <= 1e-2 + 1e-2 * np.abs(att)).all(), d.max()
    check_attn_out_and_mlp(tr, h, w, hidden, Hq, ffn, out)
