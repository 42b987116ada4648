"""Online Hadamard module (signrot/nn/hadamard.py:7-56) and its fused form
with the following Quantizer."""
import torch

from .. import _CUDA
from ..functional import kernel
from ..functional.hadamard import (adj_sign_from_rotated, fold_adj_sign_into_linear, get_hadK,
                                   matmul_hadU_cuda)
from .quantization import AsymQuantizer, Quantizer


class OnlineHadamard(torch.nn.Module):
    """x -> (H_K ⊗ H_{n/K}) x / sqrt(n) -> * had_adj_sign -> x.dtype.

    Buffers as in the reference: had_rem_dim (hadK, fp16 unless
    force_fp32) and had_adj_sign (int8 ±1, initialised to ones when
    had_adj).  fp16 input runs as one launch of the HIP rotation kernel with
    the sign fused; a zero in had_adj_sign raises RuntimeError
    (hadamard.py:32-34), checked once and cached."""

    had_adj_sign: torch.Tensor | None

    def __init__(self, hadamard_dim, tied_module=None, force_fp32=False, had_adj=False,
                 dynamic_adj=False):
        super().__init__()
        self.fp32_had = force_fp32
        self.hadamard_dim = hadamard_dim
        had_rem_dim, self.rem_dim = get_hadK(hadamard_dim)
        if had_rem_dim is not None:
            self.register_buffer("had_rem_dim", had_rem_dim)
            if not self.fp32_had:
                self.had_rem_dim = self.had_rem_dim.to(torch.float16)
        else:
            self.had_rem_dim = None
        self.register_buffer("had_adj_sign", None)
        if had_adj:
            self.register_buffer("had_adj_sign", torch.ones(hadamard_dim, dtype=torch.int8))
        self.dynamic_adj = dynamic_adj
        self.module = tied_module

    def _sign(self):
        if self.had_adj_sign is None:
            return None
        if not self._had_adj_ready_cached:
            raise RuntimeError("Dynamic hadamard adjustment not implemented yet.")
        return self.had_adj_sign

    def _hadk(self, device):
        if self.rem_dim == 1:
            return None
        want = torch.float32 if self.fp32_had else torch.float16
        h = self.had_rem_dim
        if h.device != device or h.dtype != want:
            h = h.to(device=device, dtype=want)
        return h.reshape(self.rem_dim, self.rem_dim).contiguous()

    def forward(self, x: torch.Tensor):
        if x.dtype == torch.float16 and x.is_cuda:
            sign = self._sign()
            return _CUDA.online_hadamard(x.contiguous(), self._hadk(x.device), self.rem_dim,
                                         sign, self.fp32_had)
        # other dtypes: the reference's composition over the HIP FWHT
        x_dtype = x.dtype
        if self.fp32_had:
            x = x.float()
        x = matmul_hadU_cuda(x, self.had_rem_dim, self.rem_dim)
        sign = self._sign()
        if sign is not None:
            x = x * sign
        return x.to(x_dtype)

    @torch.no_grad()
    def calibrate_adj_sign(self, x: torch.Tensor, fold_into=None) -> torch.Tensor:
        """Set had_adj_sign from one calibration batch x (un-rotated, as it
        reaches this module) by the SignRot rule (fake_quant/quant_utils.py:
        362-367): rotate without a sign, take the sign pattern of the token
        with the largest |value|, and fold it into `fold_into` (a float
        torch.nn.Linear, before its weights are quantized), or into the tied
        module when that is a float Linear.  Returns the int8 sign."""
        if self.had_adj_sign is None:
            raise RuntimeError("calibrate_adj_sign needs a module built with had_adj=True")
        x_dtype = x.dtype
        h = x.float() if self.fp32_had else x
        rot = matmul_hadU_cuda(h, self.had_rem_dim, self.rem_dim).to(x_dtype)
        sign = adj_sign_from_rotated(rot)
        self.had_adj_sign.copy_(sign.to(self.had_adj_sign.device))
        self._had_adj_ready_flag = None
        target = fold_into if fold_into is not None else self.module
        if isinstance(target, torch.nn.Linear):
            fold_adj_sign_into_linear(target, sign)
        elif fold_into is not None:
            raise TypeError("the sign folds into a float torch.nn.Linear only (fold before "
                            "quantizing: a flipped int4 code -8 has no +8)")
        return sign

    @property
    def _had_adj_ready_cached(self):
        ready = getattr(self, "_had_adj_ready_flag", None)
        if ready is None:
            ready = self.had_adj_ready()
            self._had_adj_ready_flag = ready
        return ready

    def had_adj_ready(self):
        return bool(self.had_adj_sign is not None and torch.all(self.had_adj_sign != 0))


class HadamardQuantizer(torch.nn.Module):
    """Fused Sequential(OnlineHadamard, Quantizer or AsymQuantizer): rotation,
    sign and per-token int4 (or asymmetric uint4) quantization in one launch,
    bit-identical to running the two modules in sequence.  Holds the original
    modules (state_dict keys unchanged under `had.` / `quantizer.`)."""

    def __init__(self, had: OnlineHadamard, quantizer):
        super().__init__()
        self.had = had
        self.quantizer = quantizer

    def forward(self, x):
        h = self.had
        if x.dtype != torch.float16 or not x.is_cuda:
            return self.quantizer(h(x))
        if isinstance(self.quantizer, AsymQuantizer):
            if h.fp32_had:
                return self.quantizer(h(x))
            q, s, z = _CUDA.had_sign_asym_quant(x.contiguous(), h._hadk(x.device), h.rem_dim,
                                                h._sign(), self.quantizer.clip_ratio)
            return kernel.PackedQuantizedTensor(q, s, z.to(torch.int8))
        q, s = kernel.had_sign_quant(x, h._hadk(x.device), h.rem_dim, h._sign(),
                                     self.quantizer.clip_ratio, h.fp32_had)
        return kernel.PackedQuantizedTensor(q, s)



def fuse_online_hadamard(module: torch.nn.Module) -> torch.nn.Module:
    """Replace every (OnlineHadamard, Quantizer) pair inside a Sequential with
    one HadamardQuantizer, in place; returns the module."""
    for name, child in list(module.named_children()):
        if isinstance(child, torch.nn.Sequential):
            mods = list(child)
            out, i = [], 0
            while i < len(mods):
                if (i + 1 < len(mods) and isinstance(mods[i], OnlineHadamard)
                        and type(mods[i + 1]) in (Quantizer, AsymQuantizer)):
                    out.append(HadamardQuantizer(mods[i], mods[i + 1]))
                    i += 2
                else:
                    out.append(mods[i])
                    i += 1
            if len(out) != len(mods):
                setattr(module, name, torch.nn.Sequential(*out))
            else:
                fuse_online_hadamard(child)
        else:
            fuse_online_hadamard(child)
    return module
