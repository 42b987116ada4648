"""CPU tests of the packed-int4 checkpoint format (realquant_utils.py layout,
modeling_llama.py key remap): round trips, sharding, metadata, the remap,
and loading one decoder layer into the fused q/k/v and gate/up layout."""
import json
import os

import torch

from signrot_amd import checkpoint as ck

QCFG = {"quant_method": "SignRot", "w_bits": 4, "a_bits": 4, "a_asym": False,
        "format": "packed_int4", "rotate": True}


def _tensors(g):
    return {
        "model.layers.0.self_attn.q_proj.weight":
            torch.randint(0, 256, (64, 32), dtype=torch.uint8, generator=g),
        "quantizer.model.layers.0.self_attn.q_proj.scale":
            torch.rand(64, 1, generator=g).half(),
        "model.layers.0.mlp.down_proj.had_adj_sign":
            (torch.randint(0, 2, (96,), generator=g) * 2 - 1).to(torch.int8),
        "model.norm.weight": torch.randn(64, generator=g).half(),
    }


def test_round_trip_single_file(tmp_path):
    t = _tensors(torch.Generator().manual_seed(0))
    ck.save_packed_checkpoint(str(tmp_path), t, QCFG, {"hidden_size": 64})
    assert os.path.exists(tmp_path / "model.safetensors")
    c = ck.PackedCheckpoint(str(tmp_path))
    assert set(c.keys()) == set(t)
    for k, v in t.items():
        assert torch.equal(c.get_tensor(k), v) and c.get_tensor(k).dtype == v.dtype
    assert c.quantization_config == QCFG
    assert c.config["hidden_size"] == 64


def test_round_trip_sharded(tmp_path):
    t = _tensors(torch.Generator().manual_seed(1))
    ck.save_packed_checkpoint(str(tmp_path), t, QCFG, max_shard_bytes=1024)
    with open(tmp_path / "model.safetensors.index.json") as f:
        idx = json.load(f)
    assert len(set(idx["weight_map"].values())) >= 2
    c = ck.PackedCheckpoint(str(tmp_path))
    for k, v in t.items():
        assert torch.equal(c.get_tensor(k), v)
    assert c.quantization_config["format"] == "packed_int4"


def test_remap_known_answers():
    cases = {
        "quantizer.model.layers.3.self_attn.q_proj.scale":
            "model.layers.3.self_attn.q_proj.weight_scales",
        "quantizer.model.layers.3.self_attn.o_proj.scale":
            "model.layers.3.self_attn.o_proj.1.weight_scales",
        "model.layers.3.self_attn.o_proj.weight": "model.layers.3.self_attn.o_proj.1.weight",
        "model.layers.3.mlp.down_proj.weight": "model.layers.3.mlp.down_proj.2.weight",
        "quantizer.model.layers.3.mlp.down_proj.scale":
            "model.layers.3.mlp.down_proj.2.weight_scales",
        "model.layers.3.mlp.down_proj.had_adj_sign": "model.layers.3.mlp.down_proj.0.had_adj_sign",
        "model.layers.3.mlp.up_proj.weight": "model.layers.3.mlp.up_proj.weight",
    }
    for k, want in cases.items():
        assert ck.remap_key(k) == want


def test_load_decode_layer(tmp_path):
    from signrot_amd.transformers.decode_layer import W4A4LlamaDecodeLayer
    g = torch.Generator().manual_seed(2)
    hidden, heads, kv, hd, ffn = 256, 4, 2, 64, 512
    p = "model.layers.0."
    shapes = {"self_attn.q_proj": (heads * hd, hidden), "self_attn.k_proj": (kv * hd, hidden),
              "self_attn.v_proj": (kv * hd, hidden), "self_attn.o_proj": (hidden, hidden),
              "mlp.gate_proj": (ffn, hidden), "mlp.up_proj": (ffn, hidden),
              "mlp.down_proj": (hidden, ffn)}
    t = {}
    for name, (o, i) in shapes.items():
        t[p + name + ".weight"] = torch.randint(0, 256, (o, i // 2), dtype=torch.uint8,
                                                generator=g)
        t[f"quantizer.{p}{name}.scale"] = torch.rand(o, 1, generator=g).half()
    t[p + "mlp.down_proj.had_adj_sign"] = (torch.randint(0, 2, (ffn,), generator=g) * 2 - 1
                                           ).to(torch.int8)
    ck.save_packed_checkpoint(str(tmp_path), t, QCFG)
    layer = W4A4LlamaDecodeLayer(hidden, heads, kv, hd, ffn)
    ck.load_decode_layer(layer, ck.PackedCheckpoint(str(tmp_path)), p)
    qkv = [t[p + f"self_attn.{n}_proj.weight"] for n in "qkv"]
    assert torch.equal(layer.w_qkv, torch.cat(qkv))
    assert torch.equal(layer.s_qkv, torch.cat([t[f"quantizer.{p}self_attn.{n}_proj.scale"]
                                               for n in "qkv"]).reshape(-1))
    assert torch.equal(layer.w_gu, torch.cat([t[p + "mlp.gate_proj.weight"],
                                              t[p + "mlp.up_proj.weight"]]))
    assert torch.equal(layer.w_o, t[p + "self_attn.o_proj.weight"])
    assert torch.equal(layer.w_down, t[p + "mlp.down_proj.weight"])
    assert torch.equal(layer.down_sign, t[p + "mlp.down_proj.had_adj_sign"])


def test_decode_layer_export_round_trip(tmp_path):
    """decode_layer_tensors writes the reference's per-projection keys
    (q/k/v and gate/up split out of the fused buffers, scales as [out, 1]);
    saving them and loading them into a fresh layer restores every buffer."""
    from signrot_amd.transformers.decode_layer import W4A4LlamaDecodeLayer
    hidden, heads, kv, hd, ffn = 256, 4, 2, 64, 512
    src = W4A4LlamaDecodeLayer.random(hidden, heads, kv, hd, ffn, seed=3, device="cpu")
    p = "model.layers.5."
    t = ck.decode_layer_tensors(src, p)
    assert t[p + "self_attn.k_proj.weight"].shape == (kv * hd, hidden // 2)
    assert t[f"quantizer.{p}mlp.up_proj.scale"].shape == (ffn, 1)
    assert torch.equal(t[p + "mlp.up_proj.weight"], src.w_gu[ffn:])
    ck.save_packed_checkpoint(str(tmp_path), t, QCFG, max_shard_bytes=40000)
    dst = W4A4LlamaDecodeLayer(hidden, heads, kv, hd, ffn)
    ck.load_decode_layer(dst, ck.PackedCheckpoint(str(tmp_path)), p)
    want = dict(src.named_buffers())
    for name, b in dst.named_buffers():
        if b is not None:
            assert torch.equal(b, want[name]), name
