"""Offline preparation of a Llama-like model for the W4A4 path: layer-norm
fusion, the global rotation, the SignRot sign calibration, weight
quantization (RTN or GPTQ) and export to the packed-int4 checkpoint.

This is the reference's fake_quant tooling (fake_quant/rotation_utils.py:
20-253, gptq_utils.py:23-158, 258-537, 539-638, quant_utils.py:326-368,
440-529, realquant_utils.py:17-142).  It runs once, offline, in float64 (or
the weights' dtype) on any torch device, and is not part of the measured
path: the deployed model runs the exported checkpoint on the HIP kernels.

Models are HF Llama-like causal LMs (`model.model.embed_tokens`,
`model.model.layers[i].{self_attn.{q,k,v,o}_proj, mlp.{gate,up,down}_proj,
input_layernorm, post_attention_layernorm}`, `model.model.norm`,
`model.lm_head`); an MoE layer has `mlp.gate` and `mlp.experts[e]` with the
three projections.

Function preservation: after `fuse_layer_norms` and `rotate_model`, the
model computes the same function as before provided the two online
rotations of the deployed path are applied at run time: the full Hadamard
on the down_proj input and the Hadamard over the head axis on the o_proj
input (`attach_online_rotations` installs both, plus the calibrated signs,
as forward pre-hooks for float evaluation).
"""
import copy
import json
import math

import torch

from .functional.hadamard import adj_sign_from_rotated, get_hadK, matmul_hadU
from .functional.quantization import pack_i4

# ----------------------------------------------------------------- access


def _layers(model):
    return list(model.model.layers)


def _is_moe(layer):
    return hasattr(layer.mlp, "experts")


def _qkv(layer):
    a = layer.self_attn
    return [a.q_proj, a.k_proj, a.v_proj]


def _mlp_inputs(layer):
    """Linears that read the post-attention norm's output
    (model_utils.py:146-157): the router and every expert's gate/up for an
    MoE layer."""
    if _is_moe(layer):
        out = [layer.mlp.gate]
        for ex in layer.mlp.experts:
            out += [ex.gate_proj, ex.up_proj]
        return out
    return [layer.mlp.up_proj, layer.mlp.gate_proj]


def _down_projs(layer):
    if _is_moe(layer):
        return [ex.down_proj for ex in layer.mlp.experts]
    return [layer.mlp.down_proj]


class WeightlessRMSNorm(torch.nn.Module):
    """RMSNorm with its weight folded away (model_utils.py:251-270):
    x * rsqrt(sum(x^2) / mean_dim + eps), fp16 inputs computed in fp32."""

    def __init__(self, mean_dim, eps=1e-5):
        super().__init__()
        self.mean_dim, self.eps = mean_dim, eps

    def forward(self, x):
        dt = x.dtype
        if dt == torch.float16:
            x = x.float()
        var = x.pow(2).sum(-1, keepdim=True) / self.mean_dim
        return (x * torch.rsqrt(var + self.eps)).to(dt)


# ------------------------------------------------------ layer-norm fusion


def _scale_columns(linear, g):
    """W <- W diag(g): a norm's per-channel weight moved into the linear that
    reads its output (rotation_utils.py:27-43), computed in float64."""
    w = linear.weight.data
    linear.weight.data = (w.double() * g.double()).to(w.dtype)


def fuse_layer_norms(model, eps=1e-5):
    """Fold every RMSNorm weight into the linears that follow it and replace
    the norms by weightless ones (rotation_utils.py:80-107); the embedding
    rows are mean-centred first, as the reference does for every model type
    (rotation_utils.py:72-77; for RMSNorm models this changes the function
    unless the rows already have zero mean).  eps is the weightless norm's
    (the reference's RMSN default, 1e-5)."""
    emb = model.model.embed_tokens.weight
    e = emb.data.double()
    emb.data = (e - e.mean(dim=-1, keepdim=True)).to(emb.dtype)
    hidden = model.config.hidden_size
    for layer in _layers(model):
        for lin in _qkv(layer):
            _scale_columns(lin, layer.input_layernorm.weight.data)
        for lin in _mlp_inputs(layer):
            _scale_columns(lin, layer.post_attention_layernorm.weight.data)
        layer.input_layernorm = WeightlessRMSNorm(hidden, eps)
        layer.post_attention_layernorm = WeightlessRMSNorm(hidden, eps)
    _scale_columns(model.lm_head, model.model.norm.weight.data)
    model.model.norm = WeightlessRMSNorm(hidden, eps)


# ---------------------------------------------------------------- rotation


def random_orthogonal_matrix(size, generator=None):
    """QR of a standard normal matrix with the signs of R's diagonal moved
    into Q, so Q is Haar-distributed (rotation_utils.py:110-126); float64."""
    a = torch.randn(size, size, dtype=torch.float64, generator=generator)
    q, r = torch.linalg.qr(a)
    return q * torch.sign(torch.diagonal(r)).unsqueeze(0)


def random_hadamard_matrix(size, generator=None):
    """H diag(s) / sqrt(n) with random signs s (hadamard_utils.py /
    functional/hadamard.py:71-76): the normalized Sylvester (or
    had_K-Kronecker) Hadamard applied to a random ±1 diagonal; float64."""
    s = torch.randint(0, 2, (size,), generator=generator).to(torch.float64) * 2 - 1
    return matmul_hadU(torch.diag(s))


def orthogonal_matrix(size, mode="hadamard", seed=0):
    """The global rotation Q (rotation_utils.py:129-137).  A seed >= 0
    seeds torch's global generator first, as the reference does, so the same
    seed gives the reference's Q on the same torch version; a negative seed
    draws from the generator's current state."""
    if seed >= 0:
        torch.random.manual_seed(seed)
    if mode == "random":
        return random_orthogonal_matrix(size)
    if mode == "hadamard":
        return random_hadamard_matrix(size)
    raise ValueError(f"unknown rotation mode {mode!r}")


def _right(linear, Q):
    """W <- W Q (the linear reads a rotated input)."""
    w = linear.weight.data
    linear.weight.data = (w.double() @ Q.to(w.device)).to(w.dtype)


def _left(linear, Q):
    """W <- Q^T W, b <- Q^T b (the linear's output is rotated)."""
    w = linear.weight.data
    linear.weight.data = (Q.to(w.device).T @ w.double()).to(w.dtype)
    if linear.bias is not None:
        b = linear.bias.data
        linear.bias.data = (Q.to(b.device).T @ b.double()).to(b.dtype)


def fold_hadamard(linear, head_dim=None, output=False):
    """Fold the exact normalized Hadamard into a Linear (hadamard.py:94-130),
    in float64 with the torch butterfly.  Input side (output=False): every
    row w becomes H w, for a linear whose input is rotated by H at run
    time.  Output side with head_dim: H over each head's head_dim output
    channels (the v_proj half of the o_proj head-axis rotation)."""
    w = linear.weight.data
    wd = w.double()
    if not output:
        if head_dim is not None:
            raise NotImplementedError("per-head input rotation")
        new = matmul_hadU(wd)
    else:
        t = wd.T.contiguous()                                   # [in, out]
        if head_dim is None:
            new = matmul_hadU(t).T
        else:
            if head_dim & (head_dim - 1):
                raise ValueError("head_dim must be a power of two")
            shp = t.shape
            new = matmul_hadU(t.reshape(-1, head_dim)).reshape(shp).T
    linear.weight.data = new.contiguous().to(w.dtype)


@torch.no_grad()
def rotate_model(model, mode="hadamard", seed=0):
    """Rotate the residual stream by Q (rotation_utils.py:229-253): the
    embeddings and every linear reading the stream get W Q, every linear
    writing it gets Q^T W; down_proj also gets the exact Hadamard on its
    input side and v_proj the per-head Hadamard on its output side (the
    online rotations of the deployed path undo them).  Q is registered as
    the model buffer `Q` and returned.  Run fuse_layer_norms first: a norm
    with a weight does not commute with Q."""
    cfg = model.config
    hidden = cfg.hidden_size
    head_dim = getattr(cfg, "head_dim", None) or hidden // cfg.num_attention_heads
    Q = orthogonal_matrix(hidden, mode, seed)
    model.register_buffer("Q", Q.clone())
    emb = model.model.embed_tokens.weight
    emb.data = (emb.data.double() @ Q.to(emb.device)).to(emb.dtype)
    _right(model.lm_head, Q)
    for layer in _layers(model):
        for lin in _qkv(layer):
            _right(lin, Q)
        _left(layer.self_attn.o_proj, Q)
        for lin in _mlp_inputs(layer):
            _right(lin, Q)
        for down in _down_projs(layer):
            _left(down, Q)
            fold_hadamard(down)
        fold_hadamard(layer.self_attn.v_proj, head_dim=head_dim, output=True)
        fold_hadamard(layer.self_attn.o_proj)
    return Q


# ------------------------------------------------ online rotations (float)


def head_axis_hadamard(x, num_heads):
    """The o_proj input rotation of the deployed path
    (modeling_llama.py:94, 117): [..., H * D] viewed as [..., H, D], the
    normalized Hadamard of size H over the head axis."""
    shp = x.shape
    d = shp[-1] // num_heads
    y = x.reshape(-1, num_heads, d).transpose(1, 2)
    return matmul_hadU(y.contiguous()).transpose(1, 2).reshape(shp)


def attach_online_rotations(model, signs=None):
    """Forward pre-hooks that apply the deployed path's online rotations in
    the model's float dtype: the full Hadamard on every down_proj input
    (then that layer's calibrated sign, if `signs` holds one; an MoE
    layer's entry is an ExpertSigns, one sign per expert) and the head-axis
    Hadamard on every o_proj input.  Returns the hook handles."""
    heads = model.config.num_attention_heads
    handles = []
    for i, layer in enumerate(_layers(model)):
        entry = None if signs is None else signs.get(i)

        def down_hook(_, inp, sign=None):
            x = matmul_hadU(inp[0])
            if sign is not None:
                x = x * sign.to(device=x.device, dtype=x.dtype)
            return (x,) + inp[1:]

        def o_hook(_, inp):
            return (head_axis_hadamard(inp[0], heads),) + inp[1:]

        for e, down in enumerate(_down_projs(layer)):
            sign = entry.sign[e] if isinstance(entry, ExpertSigns) else entry
            handles.append(down.register_forward_pre_hook(
                lambda m, inp, sign=sign: down_hook(m, inp, sign)))
        handles.append(layer.self_attn.o_proj.register_forward_pre_hook(o_hook))
    return handles


# --------------------------------------------------------- sign calibration


class ExpertSigns:
    """The SignRot signs of an MoE layer's expert down_projs: `sign` int8
    [E, n] (all ones for an expert that received no calibration token, the
    identity adjustment the reference leaves in place, quant_utils.py:
    225-236) and `calibrated` bool [E] (whether the expert's sign was taken
    from a token and folded into its weight).  `sign` is the sign_down
    tensor of SignRotMoEBlock."""

    def __init__(self, sign, calibrated):
        self.sign, self.calibrated = sign, calibrated

    def folded(self, e):
        """Expert e's folded sign, or None if it kept the identity."""
        return self.sign[e] if bool(self.calibrated[e]) else None


def _folded_sign(signs, i, name):
    """The sign folded into target `name` of layer i (a down_proj), or None."""
    if signs is None or i not in signs or not name.endswith("down_proj"):
        return None
    entry = signs[i]
    if isinstance(entry, ExpertSigns):
        return entry.folded(int(name.split(".")[2]))  # mlp.experts.<e>.down_proj
    return entry


@torch.no_grad()
def calibrate_down_proj_signs(model, input_ids):
    """The SignRot sign of every down_proj (adjust_hadamard, gptq_utils.py:
    539-638, with the rule of quant_utils.py:362-367): one calibration
    forward with the rotations of a rotated model attached; each down_proj
    takes the sign pattern of its first call's massive-outlier token (batch
    0 of a [B, T, n] input, all rows of an expert's [rows, n] input) and the
    sign is folded into its weight's columns (W <- W diag(s)).  With those
    signs applied to the rotated input at run time the function is
    unchanged.  MoE layers calibrate every expert separately on the rows
    routed to it; an expert that receives no row keeps the all-ones sign
    (nothing folded).  Returns {layer: int8 [n] sign} for dense layers and
    {layer: ExpertSigns} for MoE layers."""
    found = {}          # (layer, expert) -> sign
    handles = []
    heads = model.config.num_attention_heads
    for i, layer in enumerate(_layers(model)):
        for e, down in enumerate(_down_projs(layer)):
            def down_hook(mod, inp, key=(i, e)):
                x = matmul_hadU(inp[0])
                rows = x.reshape(-1, x.shape[-1]).shape[0]
                if key not in found and rows > 0:
                    found[key] = adj_sign_from_rotated(x).cpu()
                    w = mod.weight.data
                    mod.weight.data = w * found[key].to(device=w.device, dtype=w.dtype)
                if key in found:
                    x = x * found[key].to(device=x.device, dtype=x.dtype)
                return (x,) + inp[1:]

            handles.append(down.register_forward_pre_hook(down_hook))

        def o_hook(_, inp):
            return (head_axis_hadamard(inp[0], heads),) + inp[1:]

        handles.append(layer.self_attn.o_proj.register_forward_pre_hook(o_hook))
    try:
        model(input_ids, use_cache=False)
    finally:
        for h in handles:
            h.remove()
    signs = {}
    for i, layer in enumerate(_layers(model)):
        downs = _down_projs(layer)
        if not _is_moe(layer):
            if (i, 0) in found:
                signs[i] = found[(i, 0)]
            continue
        n = downs[0].weight.shape[1]
        sign = torch.ones(len(downs), n, dtype=torch.int8)
        cal = torch.zeros(len(downs), dtype=torch.bool)
        for e in range(len(downs)):
            if (i, e) in found:
                sign[e], cal[e] = found[(i, e)], True
        signs[i] = ExpertSigns(sign, cal)
    return signs


# ------------------------------------------------------ weight quantizers


class WeightQuantizer:
    """Per-channel (or per-tensor) weight quantizer (quant_utils.py:
    440-529).  Symmetric: scale = max(|min(w, 0)|, max(w, 0)).clamp(1e-5) /
    maxq, codes clamp(round(w / scale), -(maxq + 1), maxq) (or -maxq on the
    symmetric grid, used where a sign is refolded after quantization).
    Asymmetric: scale = (max - min).clamp(1e-5) / maxq, zero =
    round(-min / scale), codes clamp(round(w / scale) + zero, 0, maxq).
    With mse, the range is shrunk by p = 1 - i / grid for i < maxshrink *
    grid and the p with the least sum |w - q(w)|^norm is kept, per row."""

    def __init__(self, bits=4, perchannel=True, sym=True, mse=False, norm=2.4, grid=100,
                 maxshrink=0.8, extend_zero=True, symmetric_grid=False):
        self.bits, self.perchannel, self.sym, self.mse = bits, perchannel, sym, mse
        self.norm, self.grid, self.maxshrink = norm, grid, maxshrink
        self.extend_zero, self.symmetric_grid = extend_zero, symmetric_grid
        self.maxq = 2 ** (bits - 1) - 1 if sym else 2 ** bits - 1
        self.scale = self.zero = None

    def ready(self):
        return self.scale is not None

    def _minq(self):
        return -self.maxq if self.symmetric_grid else -(self.maxq + 1)

    def _qdq(self, x, scale, zero):
        if self.sym:
            return torch.clamp(torch.round(x / scale), self._minq(), self.maxq) * scale
        q = torch.clamp(torch.round(x / scale) + zero, 0, self.maxq)
        return scale * (q - zero)

    def find_params(self, w):
        if self.bits >= 16:
            return
        rows = w.shape[0]
        x = w.flatten(1) if self.perchannel else w.flatten().unsqueeze(0)
        lo, hi = x.min(1)[0], x.max(1)[0]
        if self.extend_zero:
            lo, hi = lo.clamp(max=0), hi.clamp(min=0)
        if self.sym:
            hi = torch.maximum(lo.abs(), hi).clamp(min=1e-5)
            scale = hi / self.maxq
            zero = torch.zeros_like(scale)
        else:
            both0 = (lo == 0) & (hi == 0)
            lo, hi = lo.masked_fill(both0, -1), hi.masked_fill(both0, 1)
            scale = (hi - lo).clamp(min=1e-5) / self.maxq
            zero = torch.round(-lo / scale)
        if self.mse:
            # errors in x's dtype against a float32 best, as the reference
            # compares them
            best = torch.full((x.shape[0],), float("inf"), device=x.device)
            for i in range(int(self.maxshrink * self.grid)):
                p = 1 - i / self.grid
                lo1, hi1 = p * lo, p * hi
                if self.sym:
                    s1, z1 = hi1 / self.maxq, torch.zeros_like(hi1)
                else:
                    s1 = (hi1 - lo1) / self.maxq
                    z1 = torch.round(-lo1 / s1)
                err = (self._qdq(x, s1.unsqueeze(1), z1.unsqueeze(1)) - x).abs_()
                err = err.pow_(self.norm).sum(1)
                better = err < best
                best = torch.where(better, err.to(best.dtype), best)
                scale = torch.where(better, s1, scale)
                zero = torch.where(better, z1, zero)
        if not self.perchannel:
            scale, zero = scale.repeat(rows), zero.repeat(rows)
        self.scale = scale.reshape(-1, 1)
        self.zero = zero.reshape(-1, 1)

    def quantize(self, w):
        """Fake-quantized w (w's dtype)."""
        if self.bits >= 16 or not self.ready():
            return w
        return self._qdq(w, self.scale.to(w.device), self.zero.to(w.device)).to(w.dtype)

    def codes(self, w):
        """Integer codes of w: signed for sym, unsigned for asym."""
        q = torch.round(w / self.scale.to(w.device))
        if self.sym:
            return torch.clamp(q, self._minq(), self.maxq)
        return torch.clamp(q + self.zero.to(w.device), 0, self.maxq)


class GPTQ:
    """GPTQ for one Linear (gptq_utils.py:23-158): the Hessian of the layer
    objective, H = 2/n sum x x^T over the calibration inputs, then columns
    quantized in order, each column's error spread over the columns not yet
    quantized through the upper Cholesky factor of H^-1 (lazy batches of
    `blocksize` columns).  dtype is the working precision of W and H (the
    reference's float32)."""

    def __init__(self, linear, quantizer, dtype=torch.float32):
        self.linear, self.quantizer, self.dtype = linear, quantizer, dtype
        cols = linear.weight.shape[1]
        self.H = torch.zeros(cols, cols, dtype=dtype, device=linear.weight.device)
        self.nsamples = 0

    def add_batch(self, inp):
        """Accumulate the running mean of 2 x x^T; inp [..., cols], each
        leading batch entry one sample."""
        if inp.dim() == 2:
            inp = inp.unsqueeze(0)
        n = inp.shape[0]
        x = inp.reshape(-1, inp.shape[-1]).T.to(self.dtype)
        self.H *= self.nsamples / (self.nsamples + n)
        self.nsamples += n
        x = math.sqrt(2 / self.nsamples) * x
        self.H += x @ x.T

    def fasterquant(self, blocksize=128, percdamp=0.01, groupsize=-1, actorder=False,
                    static_groups=False):
        lin = self.linear
        W = lin.weight.data.clone().to(self.dtype)
        cols = W.shape[1]
        q = self.quantizer
        if not q.ready():
            q.find_params(W)
        H = self.H
        self.H = None
        dead = torch.diagonal(H) == 0
        H[dead, dead] = 1
        W[:, dead] = 0
        groups = None
        if static_groups:
            groups = []
            for g0 in range(0, cols, groupsize):
                gq = copy.deepcopy(q)
                gq.find_params(W[:, g0:g0 + groupsize])
                groups.append(gq)
        perm = None
        if actorder:
            perm = torch.argsort(torch.diagonal(H), descending=True)
            W, H = W[:, perm], H[perm][:, perm]
        # in place, as the reference adds it (H[diag, diag] += damp): a
        # Hessian object shared with another linear (an MoE expert's gate and
        # up projections) is seen damped by the next one
        damp = percdamp * torch.mean(torch.diagonal(H))
        H.diagonal().add_(damp)
        Hinv = torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(H)), upper=True)
        Q = torch.zeros_like(W)
        for b0 in range(0, cols, blocksize):
            b1 = min(b0 + blocksize, cols)
            W1 = W[:, b0:b1].clone()
            Err = torch.zeros_like(W1)
            Hb = Hinv[b0:b1, b0:b1]
            for i in range(b1 - b0):
                col = b0 + i
                if groupsize != -1:
                    if static_groups:
                        idx = int(perm[col]) if actorder else col
                        q = groups[idx // groupsize]
                    elif col % groupsize == 0:
                        # the group's range is read from W, whose columns of
                        # the current block have not received this block's
                        # error updates yet (gptq_utils.py:113-118)
                        q.find_params(W[:, col:col + groupsize])
                w = W1[:, i]
                d = Hb[i, i]
                qc = q.quantize(w.unsqueeze(1)).flatten()
                Q[:, col] = qc
                e = (w - qc) / d
                W1[:, i:] -= e.unsqueeze(1) @ Hb[i, i:].unsqueeze(0)
                Err[:, i] = e
            W[:, b1:] -= Err @ Hinv[b0:b1, b1:]
        if actorder:
            Q = Q[:, torch.argsort(perm)]
        if torch.isnan(Q).any():
            raise ValueError("GPTQ produced NaN weights")
        lin.weight.data = Q.reshape(lin.weight.shape).to(lin.weight.dtype)
        self.quantizer = q
        return q


# ------------------------------------------------------- model quantization


def _quant_targets(layer):
    """(name, linear) of a decoder layer's quantized linears, in the
    reference's order (attention k/v/q, o, then the MLP)."""
    a = layer.self_attn
    out = [("self_attn.k_proj", a.k_proj), ("self_attn.v_proj", a.v_proj),
           ("self_attn.q_proj", a.q_proj), ("self_attn.o_proj", a.o_proj)]
    if _is_moe(layer):
        for e, ex in enumerate(layer.mlp.experts):
            for p in ("gate_proj", "up_proj", "down_proj"):
                out.append((f"mlp.experts.{e}.{p}", getattr(ex, p)))
    else:
        out += [("mlp.up_proj", layer.mlp.up_proj), ("mlp.gate_proj", layer.mlp.gate_proj),
                ("mlp.down_proj", layer.mlp.down_proj)]
    return out


def _make_quantizer(name, bits, sym, mse, folded_sign):
    # lm_head stays fp16 (create_quantizer, gptq_utils.py:521-536); a
    # down_proj with a folded sign is searched and rounded on [-7, 7], so
    # refolding the sign keeps every code representable (rtn_fwrd)
    return WeightQuantizer(bits, sym=sym, mse=mse, symmetric_grid=folded_sign and sym)


@torch.no_grad()
def rtn_quantize(model, bits=4, sym=True, mse=False, signs=None):
    """Round-to-nearest weight quantization of every decoder linear
    (rtn_fwrd, gptq_utils.py:412-465).  A down_proj whose calibrated sign
    was folded into its weight is quantized unfolded (W s), on the
    symmetric grid, and refolded.  Returns {"model.layers.i.<name>":
    quantizer}."""
    quantizers = {}
    for i, layer in enumerate(_layers(model)):
        for name, lin in _quant_targets(layer):
            sign = _folded_sign(signs, i, name)
            if sign is not None:
                sign = sign.to(device=lin.weight.device, dtype=lin.weight.dtype)
            w = lin.weight.data
            if sign is not None:
                w = w * sign
            q = _make_quantizer(name, bits, sym, mse, sign is not None)
            q.find_params(w)
            wq = q.quantize(w)
            if sign is not None:
                wq = wq * sign
            lin.weight.data = wq.to(lin.weight.dtype)
            quantizers[f"model.layers.{i}.{name}"] = q
    return quantizers


def _layer_inputs(model, input_ids):
    """The first decoder layer's positional and keyword inputs for each
    calibration batch (the Catcher of gptq_utils.py:283-304)."""
    caught = []

    class _Stop(Exception):
        pass

    def grab(_, args, kwargs):
        caught.append((args, kwargs))
        raise _Stop

    h = model.model.layers[0].register_forward_pre_hook(grab, with_kwargs=True)
    try:
        for ids in input_ids:
            try:
                model(ids, use_cache=False)
            except _Stop:
                pass
    finally:
        h.remove()
    return caught


@torch.no_grad()
def gptq_quantize(model, input_ids, bits=4, sym=True, mse=False, percdamp=0.01,
                  groupsize=-1, actorder=False, blocksize=128, dtype=torch.float32,
                  signs=None):
    """GPTQ of every decoder linear, layer by layer (gptq_fwrd,
    gptq_utils.py:258-410): the layer's calibration inputs are recorded,
    each group of linears that share an input (k/v/q; o; up/gate; down)
    gets the Hessian of that input and is quantized, then the inputs of the
    next layer are the quantized layer's outputs.  input_ids: a list of
    token batches.  A down_proj with a calibrated sign in `signs` is
    quantized on the symmetric grid.  For a rotated model, attach the
    online rotations first (attach_online_rotations): the Hessians are then
    those of the rotated inputs the deployed linears see, as the
    reference's hooks on the wrapped modules record them.  Returns
    {"model.layers.i.<name>": quantizer}."""
    quantizers = {}
    calls = _layer_inputs(model, input_ids)
    hidden = [args[0] if args else kw["hidden_states"] for args, kw in calls]

    def run_layer(layer):
        outs = []
        for x, (args, kw) in zip(hidden, calls):
            kw = {k: v for k, v in kw.items() if k != "hidden_states"}
            out = layer(x, *args[1:], **kw)
            outs.append(out[0] if isinstance(out, tuple) else out)
        return outs

    def quantize_group(i, layer, names, hooked):
        """GPTQ of the linears `names` of layer i, which share one input: the
        Hessian is recorded on `hooked` (the first of them) over the
        calibration batches, copied to the others, then each is quantized."""
        targets = dict(_quant_targets(layer))
        work = {n: GPTQ(targets[n], _make_quantizer(n, bits, sym, mse,
                                                    _folded_sign(signs, i, n) is not None),
                        dtype) for n in names}
        handles = [targets[h].register_forward_pre_hook(
            lambda _, inp, h=h: work[h].add_batch(inp[0])) for h in hooked]
        try:
            run_layer(layer)
        finally:
            for h in handles:
                h.remove()
        return work

    for i, layer in enumerate(_layers(model)):
        stages = [["self_attn.k_proj", "self_attn.v_proj", "self_attn.q_proj"],
                  ["self_attn.o_proj"]]
        if not _is_moe(layer):
            stages += [["mlp.up_proj", "mlp.gate_proj"], ["mlp.down_proj"]]
        for names in stages:
            work = quantize_group(i, layer, names, [names[0]])
            for n in names[1:]:
                work[n].H = work[names[0]].H.clone()
                work[n].nsamples = work[names[0]].nsamples
            for n in names:
                quantizers[f"model.layers.{i}.{n}"] = work[n].fasterquant(
                    blocksize=blocksize, percdamp=percdamp, groupsize=groupsize,
                    actorder=actorder)
        if _is_moe(layer):
            # _quantize_moe_mlp (gptq_utils.py:161-255): every expert's
            # gate_proj records the rows routed to it over the same forwards
            # (its Hessian is shared with up_proj); the down_projs record
            # their inputs in a second pass, after gate/up are quantized.  An
            # expert that receives no row has an all-zero Hessian, and GPTQ's
            # dead-column rule then zeroes its weight, as the reference's does.
            experts = range(len(layer.mlp.experts))
            gate_up = [f"mlp.experts.{e}.{p}" for e in experts for p in ("gate_proj", "up_proj")]
            work = quantize_group(i, layer, gate_up,
                                  [f"mlp.experts.{e}.gate_proj" for e in experts])
            for e in experts:
                # the same tensor, not a copy (gptq_utils.py:203): up_proj's
                # fasterquant sees the gate's in-place dead-column fix and
                # damping
                g, u = f"mlp.experts.{e}.gate_proj", f"mlp.experts.{e}.up_proj"
                work[u].H, work[u].nsamples = work[g].H, work[g].nsamples
            for n in gate_up:
                quantizers[f"model.layers.{i}.{n}"] = work[n].fasterquant(
                    blocksize=blocksize, percdamp=percdamp, groupsize=groupsize,
                    actorder=actorder)
            downs = [f"mlp.experts.{e}.down_proj" for e in experts]
            work = quantize_group(i, layer, downs, downs)
            for n in downs:
                quantizers[f"model.layers.{i}.{n}"] = work[n].fasterquant(
                    blocksize=blocksize, percdamp=percdamp, groupsize=groupsize,
                    actorder=actorder)
        hidden = run_layer(layer)
    return quantizers


# ------------------------------------------------------------------ export


def packed_checkpoint_tensors(model, quantizers, signs=None):
    """The packed-int4 checkpoint of a quantized model
    (realquant_utils.py:50-92), in the reference's steps: every quantized
    weight as its integer codes (sym: round(W / scale) clamped to the
    quantizer's range; asym: round(W / scale) + zero clamped to [0, maxq])
    packed two per byte by pack_i4, every other tensor in fp16; then under
    `quantizer.<layer>.` the quantizer's scale, zero (zeros for a symmetric
    one) and maxq.  pack_i4 accepts codes in [-8, 7] only (as the reference's
    does), so codes of an asymmetric or 8-bit quantizer pack only when every
    one of them lies in that range; otherwise its AssertionError propagates,
    as the reference's export raises there.  The calibrated signs go under
    `model.layers.<i>.mlp.down_proj.had_adj_sign` (an MoE layer: one per
    expert, `mlp.experts.<e>.down_proj.had_adj_sign`, all ones for an
    expert without a calibration token)."""
    out = {}
    for name, t in model.state_dict().items():
        layer = name.rsplit(".", 1)[0]
        q = quantizers.get(layer)
        if q is not None and name.endswith(".weight"):
            codes = q.codes(t.double() if t.dtype != torch.float16 else t.float())
            out[name] = pack_i4(codes.to(torch.int8)).contiguous()
        else:
            out[name] = t.to(torch.float16).contiguous()
    for layer, q in quantizers.items():
        out[f"quantizer.{layer}.scale"] = q.scale.to(torch.float16).contiguous()
        out[f"quantizer.{layer}.zero"] = q.zero.to(torch.float16).contiguous()
        out[f"quantizer.{layer}.maxq"] = torch.tensor(q.maxq)
    for i, s in (signs or {}).items():
        if isinstance(s, ExpertSigns):
            for e in range(s.sign.shape[0]):
                out[f"model.layers.{i}.mlp.experts.{e}.down_proj.had_adj_sign"] = \
                    s.sign[e].to(torch.int8).contiguous()
        else:
            out[f"model.layers.{i}.mlp.down_proj.had_adj_sign"] = s.to(torch.int8).contiguous()
    return out


def export_packed_checkpoint(model, quantizers, path, signs=None, rotate_mode="hadamard",
                             max_shard_bytes=5 * 2 ** 30, w_quantizer="rtn", a_clip_ratio=1.0,
                             kv_bits=4, kv_asym=True, kv_groupsize=128, kv_clip_ratio=1.0,
                             fp32_had=False, int8_down_proj=False):
    """Write the packed checkpoint directory (realquant_utils.py:17-142):
    the tensors of packed_checkpoint_tensors, and the quantization_config
    (the reference's keys: weight and activation settings, the K/V cache
    settings, format, rotation, fp32_had, adj_layers, int8_down_proj) as
    the first shard's metadata and in config.json.  Returns the config."""
    from .checkpoint import save_packed_checkpoint
    any_q = next(iter(quantizers.values()))
    qcfg = {"quant_method": "SignRot", "w_quantizer": w_quantizer,
            "w_bits": any_q.bits, "w_asym": not any_q.sym, "w_groupsize": -1,
            "w_clip": any_q.mse, "w_perchannel": True,
            "a_bits": 4, "a_asym": False, "a_groupsize": -1, "a_clip_ratio": a_clip_ratio,
            "k_bits": kv_bits, "k_asym": kv_asym, "k_groupsize": kv_groupsize,
            "k_clip_ratio": kv_clip_ratio,
            "v_bits": kv_bits, "v_asym": kv_asym, "v_groupsize": kv_groupsize,
            "v_clip_ratio": kv_clip_ratio,
            "format": "packed_int4",
            "rotate": hasattr(model, "Q"), "rotate_mode": rotate_mode, "fp32_had": fp32_had,
            "adj_layers": ["down_proj"] if signs else [],
            "int8_down_proj": int8_down_proj}
    cfg = json.loads(model.config.to_json_string()) if hasattr(model.config, "to_json_string") \
        else {}
    save_packed_checkpoint(path, packed_checkpoint_tensors(model, quantizers, signs), qcfg, cfg,
                           max_shard_bytes=max_shard_bytes)
    return qcfg
