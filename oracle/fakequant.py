"""CPU restatement of the reference's PyTorch fake-quant simulation of the
W4A4 linear path -- the `cpu_baseline` leg of bench.py and nothing else
(test infrastructure; never imported by the product).

ActQuantWrapper.forward (fake_quant/quant_utils.py:316-386) with an online
full Hadamard and a SignRot sign on CPU:
  x = matmul_hadU(x)                 signrot/functional/hadamard.py:43-65
                                     (the CPU substitute for the CUDA-only
                                     fast_hadamard_transform)
  x = x * had_adj_sign               quant_utils.py:365-367
  ActQuantizer.find_params + forward quant_utils.py:90-145, 41-48
  (per-token sym, 4 bits, maxq 7)
  x = F.linear(x, W_fq)              the RTN fake-quant weights
All in the model dtype (fp16), as the reference runs it.
"""
import torch


def matmul_hadU(X, hadK, K):
    """Pure-torch Sylvester butterfly in X's dtype (hadamard.py:43-65)."""
    n = X.shape[-1]
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


def act_fake_quant(x, bits=4, clip_ratio=1.0):
    """ActQuantizer per-token symmetric quant-dequant (quant_utils.py:90-145,
    41-48; sym_quant_dequant from signrot/functional/quantization.py:33-42)."""
    maxq = torch.tensor(2 ** (bits - 1) - 1)
    xr = x.reshape(-1, x.shape[-1])
    xmin = xr.min(1)[0] * clip_ratio
    xmax = xr.max(1)[0] * clip_ratio
    xmax = torch.maximum(torch.abs(xmin), xmax)
    tmp = xmax == 0
    scale = (xmax / maxq).unsqueeze(1).repeat(1, xr.shape[-1])
    scale[tmp] = 1
    scale = scale.reshape(x.shape)
    q = torch.clamp(torch.round(x / scale), -(maxq + 1), maxq)
    return (scale * q).to(x.dtype)


def qlinear(x, hadK, K, sign, w_fq):
    """One fake-quant W4A4 QLinear forward on CPU."""
    h = matmul_hadU(x, hadK, K)
    if sign is not None:
        h = h * sign
    h = act_fake_quant(h)
    return torch.nn.functional.linear(h, w_fq)
