"""GPU parity of one W4A4 Llama decoder layer decode step (the config-3
path), stage by stage: each stage's HIP output is compared with the oracle
applied to the HIP output of the previous stage, so integer stages are
checked bit-exactly on identical fp16 inputs (tests/layer_check.py).  Shapes: a
reduced layer (hidden 1024, 8 query / 2 or 4 KV heads of 128, FFN 896 =
28 x 32, so the down-proj rotation is had_28 x H_32), the config-3 head
layout (32 / 8 heads) with a reduced FFN, and config 3 itself (hidden 4096,
32 / 8 heads, FFN 14336, batch 32, 4096 cached tokens).
"""
import numpy as np
import pytest
import torch

from tests import layer_check as lc
from tests.gpu_util import to_dev, to_np

pytestmark = pytest.mark.gpu


def _run(B, T, hidden, Hq, Hkv, ffn, page, seed, ckpt_dir=None, layer=None):
    """One decode step of a random layer (or of `layer`), checked stage by
    stage.  With ckpt_dir, the layer is written as a packed checkpoint
    (save_packed_checkpoint), read back into a fresh layer
    (load_decode_layer) and that layer runs the step, while the oracle
    takes the original layer's weights."""
    from signrot_amd.transformers import MultiLayerPagedKVCache4Bit
    from signrot_amd.transformers.decode_layer import W4A4LlamaDecodeLayer, rope_cos_sin
    D = 128
    rng = np.random.default_rng(seed)
    if layer is None:
        layer = W4A4LlamaDecodeLayer.random(hidden, Hq, Hkv, D, ffn, layer_idx=1, seed=seed)
    w = layer.unpacked()
    if ckpt_dir is not None:
        from signrot_amd import checkpoint as ck
        prefix = "model.layers.1."
        ck.save_packed_checkpoint(str(ckpt_dir), ck.decode_layer_tensors(layer, prefix),
                                  {"quant_method": "SignRot", "w_bits": 4, "a_bits": 4,
                                   "format": "packed_int4"})
        layer = W4A4LlamaDecodeLayer(hidden, Hq, Hkv, D, ffn, layer_idx=1).to("cuda")
        ck.load_decode_layer(layer, ck.PackedCheckpoint(str(ckpt_dir)), prefix)
    cache = MultiLayerPagedKVCache4Bit(B, page, T + 1, "cuda", 2, Hkv, D, group_size=Hq // Hkv)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    for li in range(2):  # prefill both layers (init_kv_i4)
        kv = torch.randn((2, B, T, Hkv, D), device="cuda", generator=gen).half()
        cache.update(kv[0], kv[1], li, {})
    k0 = torch.zeros(B, 1, Hkv, D, dtype=torch.float16, device="cuda")
    cache.update(k0, k0, 0, {})  # layer 0's step: the cache now counts T + 1 tokens
    h = (rng.standard_normal((B, hidden)) * 0.5).astype(np.float16)
    cos, sin = rope_cos_sin([T], D, 500000.0, "cuda")
    tr = {}
    out = to_np(layer(to_dev(h).view(B, 1, hidden), cache, cos, sin, trace=tr)).reshape(B, hidden)
    tr = {k: to_np(v) for k, v in tr.items()}
    lc.check_decode_step(tr, h, w, out, to_np(cos), to_np(sin), to_np(cache.pages),
                         to_np(cache.scales), lc.page_table([T + 1] * B, page), [T] * B, 1,
                         hidden, Hq, Hkv, ffn, page)


@pytest.mark.parametrize("B,T,hidden,Hq,Hkv,ffn,page,seed", [
    (3, 70, 1024, 8, 2, 896, 32, 1),
    (4, 300, 1024, 8, 4, 896, 64, 2),
    (2, 200, 4096, 32, 8, 896, 64, 3),
    # config 3 at its full shape: Llama-3-8B layer, batch 32, 4096 cached
    # tokens in 256-token pages, FFN 14336 (had_28 x H_512)
    (32, 4096, 4096, 32, 8, 14336, 256, 4),
])
def test_decode_layer_stagewise(B, T, hidden, Hq, Hkv, ffn, page, seed):
    _run(B, T, hidden, Hq, Hkv, ffn, page, seed)


@pytest.mark.parametrize("B,T,hidden,Hq,Hkv,ffn,page,seed", [
    (3, 70, 1024, 8, 2, 896, 32, 5),
    (4, 130, 4096, 32, 8, 14336, 64, 6),
])
def test_decode_layer_from_checkpoint(tmp_path, B, T, hidden, Hq, Hkv, ffn, page, seed):
    """A layer saved as a packed-int4 checkpoint in the reference's layout
    (realquant_utils.py:85-142) and loaded back (modeling_llama.py:250-263
    key remap, fused into the decode layer's q/k/v and gate/up buffers)
    decodes one step as the oracle does with the original weights."""
    _run(B, T, hidden, Hq, Hkv, ffn, page, seed, ckpt_dir=tmp_path)


def test_offline_model_export_loads_and_decodes(tmp_path):
    """The whole offline -> deployed flow (the reference's rotate /
    adjust_hadamard / rtn_fwrd / realquant export, then modeling_llama.py's
    load): a float64 HF Llama layer (hidden 1024, 8 query / 2 KV heads of
    128, FFN 896 = had_28 x 32) has its norms fused, is rotated, has its
    down_proj sign calibrated and its weights RTN-quantized by offline.py,
    is exported with export_packed_checkpoint, loaded into the decode layer
    with load_decode_layer, and decodes one step on the HIP kernels, checked
    stage by stage against the oracle with the loaded codes and scales,
    which equal the offline model's fake-quantized weights."""
    from transformers import LlamaConfig, LlamaForCausalLM
    from signrot_amd import checkpoint as ck
    from signrot_amd import offline as off
    from signrot_amd.functional.quantization import unpack_i4
    from signrot_amd.transformers.decode_layer import W4A4LlamaDecodeLayer
    hidden, Hq, Hkv, ffn = 1024, 8, 2, 896
    cfg = LlamaConfig(vocab_size=128, hidden_size=hidden, intermediate_size=ffn,
                      num_hidden_layers=1, num_attention_heads=Hq, num_key_value_heads=Hkv,
                      head_dim=128, max_position_embeddings=64, tie_word_embeddings=False)
    torch.manual_seed(21)
    m = LlamaForCausalLM(cfg).double().eval()
    with torch.no_grad():
        m.model.layers[0].input_layernorm.weight.uniform_(0.5, 1.5)
        m.model.layers[0].post_attention_layernorm.weight.uniform_(0.5, 1.5)
    off.fuse_layer_norms(m)
    off.rotate_model(m, seed=7)
    ids = torch.randint(0, 128, (1, 24), generator=torch.Generator().manual_seed(3))
    signs = off.calibrate_down_proj_signs(m, ids)
    quant = off.rtn_quantize(m, signs=signs)
    off.export_packed_checkpoint(m, quant, str(tmp_path), signs=signs)
    c = ck.PackedCheckpoint(str(tmp_path))
    layer = W4A4LlamaDecodeLayer(hidden, Hq, Hkv, 128, ffn, layer_idx=1).to("cuda")
    ck.load_decode_layer(layer, c, "model.layers.0.")
    assert torch.equal(layer.down_sign.cpu(), signs[0])
    for buf, names in {"qkv": ["q_proj", "k_proj", "v_proj"], "o": ["o_proj"]}.items():
        codes = unpack_i4(getattr(layer, f"w_{buf}").cpu()).double()
        s64 = torch.cat([quant[f"model.layers.0.self_attn.{n}"].scale for n in names])
        want = torch.cat([m.get_submodule(f"model.layers.0.self_attn.{n}").weight.data
                          for n in names])
        assert torch.allclose(codes * s64, want, rtol=0, atol=1e-12)
    _run(3, 70, hidden, Hq, Hkv, ffn, 32, 8, layer=layer)
