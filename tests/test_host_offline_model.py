"""CPU tests of the offline model preparation (signrot_amd/offline.py: the
reference's rotation_utils / gptq_utils / adjust_hadamard / packed export)
on a small random HF Llama in float64.  Pins:

* function preservation: fusing the norms (with pre-centred embeddings)
  and rotating (with the deployed path's online rotations attached) leave
  the logits unchanged, for Hadamard and random orthogonal Q, with a
  had_28 Kronecker factor on the FFN axis;
* the sign calibration leaves the function unchanged and picks the sign of
  the rotated massive-outlier token, recorded independently;
* GPTQ: with H proportional to I it is RTN exactly; in float64 it matches
  a textbook restatement of the greedy OBS update with explicit inverses
  (the Cholesky form is a different computation of the same quantities);
  act-order is GPTQ on the permuted problem; its layer objective is never
  worse than RTN's on correlated inputs;
* the packed export: codes and scales read back through load_decode_layer
  reproduce the fake-quantized weights."""
import copy
import math

import numpy as np
import pytest
import torch

from signrot_amd import offline as off
from signrot_amd.functional.hadamard import adj_sign_from_rotated, matmul_hadU


def _model(seed=0, layers=2, ffn=112):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=97, hidden_size=64, intermediate_size=ffn,
                      num_hidden_layers=layers, num_attention_heads=4, num_key_value_heads=2,
                      head_dim=16, rms_norm_eps=1e-5, max_position_embeddings=64,
                      tie_word_embeddings=False)
    torch.manual_seed(seed)
    m = LlamaForCausalLM(cfg).double().eval()
    with torch.no_grad():  # non-trivial norm weights
        for layer in m.model.layers:
            layer.input_layernorm.weight.uniform_(0.5, 1.5)
            layer.post_attention_layernorm.weight.uniform_(0.5, 1.5)
        m.model.norm.weight.uniform_(0.5, 1.5)
    return m


def _logits(m, ids):
    with torch.no_grad():
        return m(ids, use_cache=False).logits


def _ids(seed=1, b=2, t=11):
    return torch.randint(0, 97, (b, t), generator=torch.Generator().manual_seed(seed))


def _close(a, b, rtol):
    scale = b.abs().max()
    assert (a - b).abs().max() <= rtol * scale, float((a - b).abs().max() / scale)


def test_fuse_layer_norms_preserves_function():
    m = _model()
    with torch.no_grad():  # centred rows: the embedding fusion is then exact
        e = m.model.embed_tokens.weight
        e -= e.mean(dim=-1, keepdim=True)
    ids = _ids()
    want = _logits(m, ids)
    off.fuse_layer_norms(m)
    assert isinstance(m.model.norm, off.WeightlessRMSNorm)
    # HF's RMSNorm computes in float32 even for a float64 model
    _close(_logits(m, ids), want, 1e-6)


def test_fuse_layer_norms_centres_the_embeddings():
    m = _model()
    off.fuse_layer_norms(m)
    e = m.model.embed_tokens.weight
    assert e.mean(dim=-1).abs().max() < 1e-12


@pytest.mark.parametrize("mode", ["hadamard", "random"])
def test_rotate_model_preserves_function(mode):
    m = _model(seed=3)
    off.fuse_layer_norms(m)
    ids = _ids(4)
    want = _logits(m, ids)
    Q = off.rotate_model(m, mode=mode, seed=5)
    assert torch.equal(m.Q, Q)
    # without the online rotations the function changes ...
    assert (_logits(m, ids) - want).abs().max() > 1e-3 * want.abs().max()
    # ... with them it is the same (matmul_hadU's fp32 1/sqrt(n) costs ~1e-7)
    hs = off.attach_online_rotations(m)
    _close(_logits(m, ids), want, 1e-6)
    for h in hs:
        h.remove()


def test_orthogonal_matrices():
    for n in (64, 112):
        H = off.orthogonal_matrix(n, "hadamard", seed=2)
        assert torch.allclose(H @ H.T, torch.eye(n, dtype=H.dtype), atol=1e-6)
        # ±1 entries up to the normalization
        assert torch.allclose(H.abs() * np.sqrt(n), torch.ones_like(H), atol=1e-5)
        R = off.orthogonal_matrix(n, "random", seed=2)
        assert torch.allclose(R @ R.T, torch.eye(n, dtype=R.dtype), atol=1e-12)
    assert torch.equal(off.orthogonal_matrix(64, "random", 7), off.orthogonal_matrix(64, "random", 7))
    assert not torch.equal(off.orthogonal_matrix(64, "random", 7),
                           off.orthogonal_matrix(64, "random", 8))
    with pytest.raises(ValueError):
        off.orthogonal_matrix(8, "bogus")


def test_calibrate_signs_preserves_function_and_follows_the_rule():
    m = _model(seed=6)
    off.fuse_layer_norms(m)
    off.rotate_model(m, seed=1)
    ids = _ids(7, b=1, t=16)
    hs = off.attach_online_rotations(m)
    want = _logits(m, ids)
    for h in hs:
        h.remove()
    # the rotated down_proj inputs of an untouched copy, recorded directly
    ref = copy.deepcopy(m)
    rec = {}
    hs = off.attach_online_rotations(ref)
    for i, layer in enumerate(ref.model.layers):
        layer.mlp.down_proj.register_forward_pre_hook(
            lambda _, inp, i=i: rec.setdefault(i, inp[0].clone()))
    _logits(ref, ids)
    before = [layer.mlp.down_proj.weight.clone() for layer in m.model.layers]
    signs = off.calibrate_down_proj_signs(m, ids)
    assert sorted(signs) == [0, 1]
    for i, s in signs.items():
        assert torch.equal(s, adj_sign_from_rotated(rec[i]))
        assert set(s.tolist()) <= {-1, 1}
        assert torch.equal(m.model.layers[i].mlp.down_proj.weight, before[i] * s.double())
    hs = off.attach_online_rotations(m, signs)
    _close(_logits(m, ids), want, 1e-12)


# ------------------------------------------------------------ quantizers


def test_weight_quantizer_sym_matches_rtn_weight_pack():
    from signrot_amd.functional.quantization import rtn_weight_pack
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(24, 64, generator=g) * 0.02).half()
    for grid in (False, True):
        q = off.WeightQuantizer(4, symmetric_grid=grid)
        q.find_params(w.float())
        _, s, wfq = rtn_weight_pack(w, symmetric_grid=grid)
        assert torch.equal(q.quantize(w.float()).half(), wfq)
        assert torch.equal(q.scale.view(-1).half(), s)


def test_weight_quantizer_asym_known_answer():
    w = torch.tensor([[-1.0, 0.0, 2.0, 0.5]], dtype=torch.float64)
    q = off.WeightQuantizer(4, sym=False)
    q.find_params(w)
    # range [-1, 2] over 15 steps: scale 0.2, zero round(5) = 5; 0.5 / 0.2
    # = 2.4999... in float64 (and round-half-even would give 2 as well)
    assert torch.allclose(q.scale, torch.tensor([[0.2]], dtype=torch.float64))
    assert q.zero.item() == 5
    assert torch.equal(q.codes(w), torch.tensor([[0.0, 5, 15, 7]], dtype=torch.float64))
    assert torch.allclose(q.quantize(w), torch.tensor([[-1.0, 0.0, 2.0, 0.4]],
                                                      dtype=torch.float64))


def test_weight_quantizer_mse_never_worse():
    g = torch.Generator().manual_seed(1)
    w = torch.randn(16, 128, generator=g, dtype=torch.float64)
    w[:, 0] *= 20  # a clipped outlier pays off
    plain, mse = off.WeightQuantizer(4), off.WeightQuantizer(4, mse=True)
    plain.find_params(w)
    mse.find_params(w)
    e_plain = (plain.quantize(w) - w).abs().pow(2.4).sum(1)
    e_mse = (mse.quantize(w) - w).abs().pow(2.4).sum(1)
    assert (e_mse <= e_plain + 1e-12).all() and (e_mse < e_plain).any()


def _obs_reference(W, H, quantizer, percdamp=0.01):
    """Greedy OBS in column order with explicit inverses: quantize column
    i, move its error onto the later columns through the inverse Hessian of
    the columns not yet quantized, then drop column i from that inverse."""
    W = W.clone().double()
    H = H.clone().double()
    n = W.shape[1]
    H += percdamp * torch.mean(torch.diagonal(H)) * torch.eye(n, dtype=H.dtype)
    Hinv = torch.linalg.inv(H)
    Q = torch.zeros_like(W)
    for i in range(n):
        q = quantizer.quantize(W[:, i:i + 1]).flatten()
        Q[:, i] = q
        err = (W[:, i] - q) / Hinv[i, i]
        W[:, i + 1:] -= err.unsqueeze(1) * Hinv[i, i + 1:].unsqueeze(0)
        Hinv = Hinv - Hinv[:, i:i + 1] @ Hinv[i:i + 1, :] / Hinv[i, i]
    return Q


def _problem(seed, rows=8, cols=24, n=64):
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(rows, cols, generator=g, dtype=torch.float64)
    mix = torch.randn(cols, cols, generator=g, dtype=torch.float64)
    X = torch.randn(n, cols, generator=g, dtype=torch.float64) @ mix  # correlated inputs
    return W, X


def _gptq(W, X, dtype=torch.float64, **kw):
    lin = torch.nn.Linear(W.shape[1], W.shape[0], bias=False).double()
    lin.weight.data = W.clone()
    q = off.WeightQuantizer(4)
    g = off.GPTQ(lin, q, dtype)
    g.add_batch(X.unsqueeze(0))
    H = g.H.clone()
    g.fasterquant(**kw)
    return lin.weight.data, H, g.quantizer


@pytest.mark.parametrize("blocksize", [1, 5, 128])
def test_gptq_matches_greedy_obs(blocksize):
    W, X = _problem(0)
    Q, H, q = _gptq(W, X, blocksize=blocksize)
    # one sample (the leading batch entry) of 64 tokens: H = 2 X^T X / 1
    assert torch.allclose(H, 2 * X.T @ X, rtol=1e-12)
    want = _obs_reference(W, H, q)
    assert torch.equal(Q, want)


def test_gptq_with_identity_hessian_is_rtn():
    W, _ = _problem(1, cols=32)
    X = torch.eye(32, dtype=torch.float64) * 3.0
    Q, _, q = _gptq(W, X, blocksize=8)
    rtn = off.WeightQuantizer(4)
    rtn.find_params(W)
    assert torch.equal(Q, rtn.quantize(W))
    # grouped: per-group RTN
    Qg, _, _ = _gptq(W, X, blocksize=8, groupsize=8)
    want = torch.cat([_rtn(W[:, c:c + 8]) for c in range(0, 32, 8)], 1)
    assert torch.equal(Qg, want)


def _rtn(w):
    q = off.WeightQuantizer(4)
    q.find_params(w)
    return q.quantize(w)


def test_gptq_actorder_is_gptq_of_the_permuted_problem():
    W, X = _problem(2)
    Q, H, _ = _gptq(W, X, actorder=True)
    perm = torch.argsort(torch.diagonal(H), descending=True)
    Qp, _, _ = _gptq(W[:, perm], X[:, perm])
    assert torch.equal(Q[:, perm], Qp)


def test_gptq_objective_beats_rtn():
    for seed in range(3):
        W, X = _problem(10 + seed, rows=16, cols=48, n=200)
        Q, H, _ = _gptq(W, X, dtype=torch.float32)
        R = _rtn(W)

        def obj(A):
            d = (A - W).double()
            return torch.trace(d @ H.double() @ d.T)

        assert obj(Q) < obj(R)


def test_gptq_quantize_model_runs_layerwise_and_changes_outputs_little():
    m = _model(seed=8)
    off.fuse_layer_norms(m)
    off.rotate_model(m, seed=3)
    hs = off.attach_online_rotations(m)
    calib = [_ids(20 + i, b=1, t=24) for i in range(4)]
    ids = _ids(30)
    want = _logits(m, ids)
    ref = copy.deepcopy(m)
    quant = off.gptq_quantize(m, calib, dtype=torch.float64)
    assert len(quant) == 2 * 7
    rtn_q = off.rtn_quantize(ref)
    for key, q in quant.items():  # every weight sits on its grid
        lin = m.get_submodule(key)
        assert torch.equal(lin.weight.data, q.quantize(lin.weight.data))
        assert torch.equal(ref.get_submodule(key).weight.data,
                           rtn_q[key].quantize(ref.get_submodule(key).weight.data))
    got = _logits(m, ids)
    assert (got - want).abs().max() < 0.5 * want.abs().max()
    for h in hs:
        h.remove()


# ------------------------------------------------------------------ export


def test_export_reads_back_through_load_decode_layer(tmp_path):
    from signrot_amd import checkpoint as ck
    from signrot_amd.functional.quantization import unpack_i4
    from signrot_amd.transformers.decode_layer import W4A4LlamaDecodeLayer
    m = _model(seed=9, layers=1)
    off.fuse_layer_norms(m)
    off.rotate_model(m, seed=4)
    signs = off.calibrate_down_proj_signs(m, _ids(5, b=1, t=16))
    quant = off.rtn_quantize(m, signs=signs)
    # the refolded down_proj stays on the symmetric grid
    assert quant["model.layers.0.mlp.down_proj"].symmetric_grid
    off.export_packed_checkpoint(m, quant, str(tmp_path), signs=signs)
    c = ck.PackedCheckpoint(str(tmp_path))
    assert c.quantization_config["format"] == "packed_int4"
    assert c.quantization_config["adj_layers"] == ["down_proj"]
    assert c.config["hidden_size"] == 64
    layer = W4A4LlamaDecodeLayer(64, 4, 2, 16, 112)
    ck.load_decode_layer(layer, c, "model.layers.0.")
    assert torch.equal(layer.down_sign, signs[0])
    parts = {"qkv": ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"],
             "o": ["self_attn.o_proj"], "gu": ["mlp.gate_proj", "mlp.up_proj"],
             "down": ["mlp.down_proj"]}
    for buf, names in parts.items():
        codes = unpack_i4(getattr(layer, f"w_{buf}")).double()
        scale = getattr(layer, f"s_{buf}").double().unsqueeze(1)
        want_w = torch.cat([m.get_submodule("model.layers.0." + n).weight.data for n in names])
        want_s = torch.cat([quant["model.layers.0." + n].scale for n in names]).half().double()
        want_codes = torch.cat([quant["model.layers.0." + n].codes(
            m.get_submodule("model.layers.0." + n).weight.data) for n in names])
        assert torch.equal(scale, want_s)
        assert torch.equal(codes, want_codes)
        assert codes.abs().max() <= 8
        # the fake-quantized weight is code x scale (scale in float64 here)
        s64 = torch.cat([quant["model.layers.0." + n].scale for n in names])
        assert torch.allclose(codes * s64, want_w, rtol=0, atol=1e-12)


# ----------------------------------------------------------------- MoE layers


class _Expert(torch.nn.Module):
    def __init__(self, hidden, ffn):
        super().__init__()
        self.gate_proj = torch.nn.Linear(hidden, ffn, bias=False)
        self.up_proj = torch.nn.Linear(hidden, ffn, bias=False)
        self.down_proj = torch.nn.Linear(ffn, hidden, bias=False)

    def forward(self, x):
        return self.down_proj(torch.nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))


class _SparseMoE(torch.nn.Module):
    """The sparse MoE block of the reference's target models (transformers
    4.57 Qwen3-MoE layout: router `gate`, `experts[e]` with gate/up/down
    Linears): fp32-style softmax over the router logits, top-k, optional
    renormalization, each expert called once per forward on the rows routed
    to it (and not at all when none is)."""

    def __init__(self, hidden, ffn, experts, top_k, norm=True):
        super().__init__()
        self.gate = torch.nn.Linear(hidden, experts, bias=False)
        # added to the router logits: -1e4 makes an expert unreachable (a
        # buffer, so the offline rotation leaves it alone)
        self.register_buffer("route_bias", torch.zeros(experts, dtype=torch.float64))
        self.experts = torch.nn.ModuleList(_Expert(hidden, ffn) for _ in range(experts))
        self.top_k, self.norm = top_k, norm

    def forward(self, x):
        shp = x.shape
        x2 = x.reshape(-1, shp[-1])
        p = torch.softmax(self.gate(x2) + self.route_bias, dim=-1)
        w, sel = torch.topk(p, self.top_k, dim=-1)
        if self.norm:
            w = w / w.sum(dim=-1, keepdim=True)
        out = torch.zeros_like(x2)
        for e, ex in enumerate(self.experts):
            tok, pos = torch.where(sel == e)
            if tok.numel() == 0:
                continue
            out.index_add_(0, tok, ex(x2[tok]) * w[tok, pos, None])
        return out.reshape(shp)


def _moe_model(seed=0, layers=1, ffn=112, experts=4, top_k=2, dead=None):
    """A small float64 Llama whose MLPs are sparse MoE blocks; expert `dead`
    (if given) has a router row that never wins a top-k slot."""
    m = _model(seed=seed, layers=layers, ffn=ffn)
    torch.manual_seed(seed + 100)
    for layer in m.model.layers:
        moe = _SparseMoE(64, ffn, experts, top_k).double()
        if dead is not None:
            moe.route_bias[dead] = -1e4   # never routed
        layer.mlp = moe
    return m.eval()


def test_moe_rotation_and_sign_calibration_per_expert():
    """Fusion, rotation and per-expert sign calibration of an MoE model:
    the function is unchanged with the online rotations and signs attached;
    each expert's sign follows the rule on the rows routed to it in the
    calibration forward (recorded independently on an untouched copy) and
    is folded into its down_proj only; an expert that receives no row keeps
    the all-ones sign, unfolded, and is reported as not calibrated."""
    m = _moe_model(seed=12, dead=3)
    ids = _ids(13, b=1, t=40)
    want0 = _logits(m, ids)
    off.fuse_layer_norms(m)
    # the embedding centring changes the function (reference behaviour);
    # compare the rotated model against the fused one
    want = _logits(m, ids)
    off.rotate_model(m, seed=2)
    hs = off.attach_online_rotations(m)
    # (matmul_hadU's fp32 1/sqrt(n) costs ~1e-7)
    _close(_logits(m, ids), want, 1e-6)
    want_rot = _logits(m, ids)
    for h in hs:
        h.remove()
    ref = copy.deepcopy(m)
    rec = {}
    hs = off.attach_online_rotations(ref)
    for e, ex in enumerate(ref.model.layers[0].mlp.experts):
        ex.down_proj.register_forward_pre_hook(
            lambda _, inp, e=e: rec.setdefault(e, inp[0].clone()))
    _logits(ref, ids)
    for h in hs:
        h.remove()
    assert 3 not in rec and sorted(rec) == [0, 1, 2]
    before = [ex.down_proj.weight.clone() for ex in m.model.layers[0].mlp.experts]
    signs = off.calibrate_down_proj_signs(m, ids)
    es = signs[0]
    assert isinstance(es, off.ExpertSigns) and es.sign.shape == (4, 112)
    assert es.calibrated.tolist() == [True, True, True, False]
    for e in range(3):
        assert torch.equal(es.sign[e], adj_sign_from_rotated(rec[e]))
        assert torch.equal(m.model.layers[0].mlp.experts[e].down_proj.weight,
                           before[e] * es.sign[e].double())
    assert torch.equal(es.sign[3], torch.ones(112, dtype=torch.int8))
    assert torch.equal(m.model.layers[0].mlp.experts[3].down_proj.weight, before[3])
    assert es.folded(3) is None and torch.equal(es.folded(1), es.sign[1])
    hs = off.attach_online_rotations(m, signs)
    _close(_logits(m, ids), want_rot, 1e-12)
    for h in hs:
        h.remove()
    # RTN: calibrated experts' down_proj on the symmetric grid, the others not
    quant = off.rtn_quantize(copy.deepcopy(m), signs=signs)
    grid = [quant[f"model.layers.0.mlp.experts.{e}.down_proj"].symmetric_grid for e in range(4)]
    assert grid == [True, True, True, False]
    assert want0.shape == want.shape


def test_moe_gptq_per_expert_hessians(monkeypatch):
    """GPTQ of an MoE layer (_quantize_moe_mlp, gptq_utils.py:161-255): each
    expert's gate_proj Hessian is 2/n sum x x^T over exactly the rows routed
    to it, one sample per forward (recomputed here from the block's recorded
    inputs by an independent softmax / top-k); up_proj is quantized with the
    same Hessian object, after the gate's in-place dead-column fix and
    damping; every weight ends on its quantizer's grid.  An expert that gets
    no row has all-zero Hessians: the dead-column rule zeroes its gate_proj
    and down_proj, while its up_proj, handed the gate's fixed and damped
    Hessian (1.01 I), is quantized as RTN -- what the reference's shared
    Hessian object does."""
    m = _moe_model(seed=14, dead=2)
    off.fuse_layer_norms(m)
    off.rotate_model(m, seed=5)
    hs = off.attach_online_rotations(m)
    calib = [_ids(40 + i, b=1, t=24) for i in range(3)]
    seen = {}
    orig = off.GPTQ.fasterquant

    def spy(self, *a, **k):
        seen[id(self.linear)] = (self.H.clone(), self.nsamples, id(self.H))
        return orig(self, *a, **k)

    monkeypatch.setattr(off.GPTQ, "fasterquant", spy)
    blk_in = []
    moe = m.model.layers[0].mlp
    up_before = [ex.up_proj.weight.data.clone() for ex in moe.experts]
    h_in = moe.register_forward_pre_hook(lambda _, inp: blk_in.append(inp[0].clone()))
    quant = off.gptq_quantize(m, calib, dtype=torch.float64)
    h_in.remove()
    for h in hs:
        h.remove()
    assert len(quant) == 4 + 3 * 4
    for key, q in quant.items():
        lin = m.get_submodule(key)
        assert torch.equal(lin.weight.data, q.quantize(lin.weight.data))
    # block inputs: the o stage's forwards, then the gate/up pass, the down
    # pass and the final pass: the gate/up pass is forwards 3 * 3 .. 3 * 4
    gate_up_inputs = blk_in[2 * len(calib):3 * len(calib)]
    for e, ex in enumerate(moe.experts):
        H = torch.zeros(64, 64, dtype=torch.float64)
        n = 0
        for x in gate_up_inputs:
            x2 = x.reshape(-1, 64)
            p = torch.softmax(moe.gate(x2) + moe.route_bias, dim=-1)
            _, sel = torch.topk(p, moe.top_k, dim=-1)
            rows = x2[(sel == e).any(-1)]
            if rows.shape[0] == 0:
                continue
            H *= n / (n + 1)
            n += 1
            r = math.sqrt(2 / n) * rows.T
            H += r @ r.T
        Hg, ng, idg = seen[id(ex.gate_proj)]
        Hu, nu, idu = seen[id(ex.up_proj)]
        assert idg == idu and ng == nu == n
        if n == 0:
            assert e == 2 and torch.count_nonzero(Hg) == 0
            assert torch.count_nonzero(ex.gate_proj.weight) == 0
            assert torch.count_nonzero(ex.down_proj.weight) == 0
            assert torch.equal(Hu, 1.01 * torch.eye(64, dtype=torch.float64))
            qu = quant[f"model.layers.0.mlp.experts.{e}.up_proj"]
            assert torch.equal(ex.up_proj.weight.data, qu.quantize(up_before[e]))
            continue
        assert torch.allclose(Hg, H, rtol=1e-12, atol=1e-12)
        fixed = Hg.clone()
        dead = torch.diagonal(fixed) == 0
        fixed[dead, dead] = 1
        damp = 0.01 * torch.mean(torch.diagonal(fixed))
        assert torch.equal(Hu, fixed + damp * torch.eye(64, dtype=torch.float64))


def test_packed_export_keys_and_config(tmp_path):
    """The exporter's reference steps (realquant_utils.py:17-142): every
    quantizer's scale, zero (zeros for symmetric) and maxq; the full
    quantization_config; an MoE layer's signs per expert; asymmetric codes
    (0..15) fail pack_i4's [-8, 7] range check as the reference's export
    does, while symmetric ones round-trip."""
    from signrot_amd import checkpoint as ck
    from signrot_amd.functional.quantization import unpack_i4
    m = _moe_model(seed=15, dead=1)
    off.fuse_layer_norms(m)
    off.rotate_model(m, seed=6)
    signs = off.calibrate_down_proj_signs(m, _ids(16, b=1, t=16))
    quant = off.rtn_quantize(m, signs=signs)
    qcfg = off.export_packed_checkpoint(m, quant, str(tmp_path), signs=signs,
                                        w_quantizer="rtn")
    c = ck.PackedCheckpoint(str(tmp_path))
    for key in ("w_quantizer", "a_groupsize", "a_clip_ratio", "k_bits", "k_asym",
                "k_groupsize", "k_clip_ratio", "v_bits", "v_asym", "v_groupsize",
                "v_clip_ratio", "fp32_had", "int8_down_proj", "adj_layers"):
        assert key in c.quantization_config and c.quantization_config[key] == qcfg[key]
    assert c.quantization_config["fp32_had"] is False
    assert c.quantization_config["int8_down_proj"] is False
    for layer, q in quant.items():
        assert int(c.get_tensor(f"quantizer.{layer}.maxq")) == 7
        assert torch.count_nonzero(c.get_tensor(f"quantizer.{layer}.zero")) == 0
        codes = unpack_i4(c.get_tensor(layer + ".weight")).double()
        assert torch.equal(codes, q.codes(m.get_submodule(layer).weight.data))
    for e in range(4):
        s = c.get_tensor(f"model.layers.0.mlp.experts.{e}.down_proj.had_adj_sign")
        assert torch.equal(s, signs[0].sign[e])
    assert torch.equal(c.get_tensor("model.layers.0.mlp.experts.1.down_proj.had_adj_sign"),
                       torch.ones(112, dtype=torch.int8))
    # asymmetric weights: codes 0..15 with zero points; pack_i4 refuses > 7
    m2 = _model(seed=17, layers=1)
    qa = off.rtn_quantize(m2, sym=False)
    some = next(iter(qa.values()))
    assert not some.sym and some.maxq == 15
    with pytest.raises(AssertionError):
        off.packed_checkpoint_tensors(m2, qa)
