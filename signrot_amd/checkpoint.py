"""Packed-int4 checkpoint format of the reference's real-quant models
(fake_quant/realquant_utils.py:17-142 writer, 159-340 reader;
e2e/quantized_llama/modeling_llama.py:240-265 key remap).

Layout (kept so checkpoints move between the two builds unchanged):

* `model.safetensors`, or shards `model-0000i-of-0000n.safetensors` plus
  `model.safetensors.index.json` ({"metadata": ..., "weight_map": {key:
  file}});
* quantized linear weights under their module key (`...q_proj.weight`): u8
  [out, in/2], two's-complement int4 codes, column 2j in the low nibble;
* per-channel weight scales under `quantizer.<layer>.scale` (+ `.zero`,
  `.maxq` when present); every other tensor (norms, embeddings, the SignRot
  `down_proj.had_adj_sign`) in fp16 / its own dtype;
* the first shard's safetensors metadata holds `quantization_config` as
  JSON, and `config.json` holds the model config with the same
  `quantization_config` entry.

Only safetensors and JSON are read: nothing in a checkpoint is executed.
"""
import json
import os

import torch
from safetensors import safe_open
from safetensors.torch import save_file

INDEX = "model.safetensors.index.json"
SINGLE = "model.safetensors"


class PackedCheckpoint:
    """Read-only view of a packed-int4 checkpoint directory
    (realquant_utils.py:159-247 Safetensors): keys(), get_tensor(key),
    quantization_config, config."""

    def __init__(self, path, device="cpu"):
        self.path = path
        self.device = str(device)
        index = os.path.join(path, INDEX)
        if os.path.exists(index):
            with open(index) as f:
                idx = json.load(f)
            self.weight_map = dict(idx["weight_map"])
        else:
            with safe_open(os.path.join(path, SINGLE), framework="pt") as f:
                self.weight_map = {k: SINGLE for k in f.keys()}
        self.quantization_config = {}
        first = sorted(set(self.weight_map.values()))[0] if self.weight_map else None
        if first is not None:
            with safe_open(os.path.join(path, first), framework="pt") as f:
                meta = f.metadata() or {}
            if "quantization_config" in meta:
                self.quantization_config = json.loads(meta["quantization_config"])
        self.config = {}
        cfg = os.path.join(path, "config.json")
        if os.path.exists(cfg):
            with open(cfg) as f:
                self.config = json.load(f)
            self.quantization_config = self.config.get("quantization_config",
                                                       self.quantization_config)

    def keys(self):
        return self.weight_map.keys()

    def get_tensor(self, key):
        if key not in self.weight_map:
            raise KeyError(f"Key {key} not found in safetensors.")
        with safe_open(os.path.join(self.path, self.weight_map[key]), framework="pt",
                       device=self.device) as f:
            return f.get_tensor(key)


def save_packed_checkpoint(path, tensors, quantization_config, config=None,
                           max_shard_bytes=5 * 2 ** 30):
    """Write `tensors` (already packed: u8 weights, `quantizer.*` scales, the
    rest) in the reference's layout (realquant_utils.py:85-142): shards of at
    most max_shard_bytes, the quantization_config JSON as the first shard's
    metadata, an index when sharded, and config.json."""
    os.makedirs(path, exist_ok=True)
    shards, cur, size = [], {}, 0
    for k in tensors:  # insertion order, as the reference's splitter keeps it
        t = tensors[k].contiguous()
        nb = t.numel() * t.element_size()
        if cur and size + nb > max_shard_bytes:
            shards.append(cur)
            cur, size = {}, 0
        cur[k] = t
        size += nb
    if cur or not shards:
        shards.append(cur)
    meta = {"quantization_config": json.dumps(quantization_config)}
    names = ([SINGLE] if len(shards) == 1 else
             [f"model-{i + 1:05d}-of-{len(shards):05d}.safetensors" for i in range(len(shards))])
    for i, (name, shard) in enumerate(zip(names, shards)):
        save_file(shard, os.path.join(path, name), metadata=meta if i == 0 else None)
    if len(shards) > 1:
        wm = {k: name for name, shard in zip(names, shards) for k in shard}
        total = sum(t.numel() * t.element_size() for t in tensors.values())
        with open(os.path.join(path, INDEX), "w") as f:
            json.dump({"metadata": {"total_size": total}, "weight_map": wm}, f, indent=2)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump({**(config or {}), "quantization_config": quantization_config}, f, indent=2)


def remap_key(key):
    """The quantized Llama's key remap (modeling_llama.py:253-263):
    `quantizer.<layer>.scale` -> `<layer>.weight_scales`; o_proj / down_proj
    weights and scales move under their Sequential slots (o_proj.1,
    down_proj.2); had_adj_sign under down_proj.0."""
    if key.startswith("quantizer."):
        key = key.replace("quantizer.", "", 1).replace(".scale", ".weight_scales")
    return (key.replace("o_proj.weight", "o_proj.1.weight")
            .replace("o_proj.weight_scales", "o_proj.1.weight_scales")
            .replace("down_proj.weight", "down_proj.2.weight")
            .replace("down_proj.weight_scales", "down_proj.2.weight_scales")
            .replace("down_proj.had_adj_sign", "down_proj.0.had_adj_sign"))


def load_remapped_state_dict(path, device="cpu"):
    """The checkpoint as a state dict under the quantized Llama's module keys
    (what QuantizedLlama.from_pretrained feeds load_state_dict)."""
    ck = PackedCheckpoint(path, device)
    return {remap_key(k): ck.get_tensor(k) for k in ck.keys()}


def load_decode_layer(layer, ckpt, prefix):
    """Fill a W4A4LlamaDecodeLayer from checkpoint keys under `prefix`
    (e.g. "model.layers.0."): q/k/v and gate/up codes and scales are
    concatenated along the output dim (the layer's fused layout), o/down
    taken as stored, the SignRot down_proj sign copied.  The RMSNorms carry
    no weight (SignRot folds them into the following linears).  `ckpt` is a
    PackedCheckpoint (raw keys)."""
    def t(k):
        return ckpt.get_tensor(prefix + k)

    def scale(name):
        return ckpt.get_tensor(f"quantizer.{prefix}{name}.scale").reshape(-1).to(torch.float16)

    att, mlp = "self_attn.", "mlp."
    with torch.no_grad():
        layer.w_qkv.copy_(torch.cat([t(att + p + ".weight") for p in ("q_proj", "k_proj",
                                                                        "v_proj")]))
        layer.s_qkv.copy_(torch.cat([scale(att + p) for p in ("q_proj", "k_proj", "v_proj")]))
        layer.w_o.copy_(t(att + "o_proj.weight"))
        layer.s_o.copy_(scale(att + "o_proj"))
        layer.w_gu.copy_(torch.cat([t(mlp + p + ".weight") for p in ("gate_proj", "up_proj")]))
        layer.s_gu.copy_(torch.cat([scale(mlp + p) for p in ("gate_proj", "up_proj")]))
        layer.w_down.copy_(t(mlp + "down_proj.weight"))
        layer.s_down.copy_(scale(mlp + "down_proj"))
        if prefix + mlp + "down_proj.had_adj_sign" in ckpt.keys():
            layer.down_sign.copy_(t(mlp + "down_proj.had_adj_sign").to(torch.int8))
    return layer


def decode_layer_tensors(layer, prefix):
    """The inverse of load_decode_layer: a W4A4LlamaDecodeLayer's packed
    codes and scales under the reference's checkpoint keys
    (realquant_utils.py:85-142 writes `<prefix>self_attn.q_proj.weight` u8
    [out, in/2] and `quantizer.<prefix>self_attn.q_proj.scale` fp16
    [out, 1] per linear, plus `<prefix>mlp.down_proj.had_adj_sign`): the
    fused q/k/v and gate/up buffers are split back into their projections.
    Tensors are copied to the CPU."""
    hd = layer.head_dim
    nq, nkv = layer.n_heads * hd, layer.n_kv * hd
    att, mlp = prefix + "self_attn.", prefix + "mlp."
    parts = {
        att + "q_proj": (layer.w_qkv[:nq], layer.s_qkv[:nq]),
        att + "k_proj": (layer.w_qkv[nq:nq + nkv], layer.s_qkv[nq:nq + nkv]),
        att + "v_proj": (layer.w_qkv[nq + nkv:], layer.s_qkv[nq + nkv:]),
        att + "o_proj": (layer.w_o, layer.s_o),
        mlp + "gate_proj": (layer.w_gu[:layer.ffn], layer.s_gu[:layer.ffn]),
        mlp + "up_proj": (layer.w_gu[layer.ffn:], layer.s_gu[layer.ffn:]),
        mlp + "down_proj": (layer.w_down, layer.s_down),
    }
    out = {}
    for key, (w, s) in parts.items():
        out[key + ".weight"] = w.detach().cpu().contiguous()
        out[f"quantizer.{key}.scale"] = s.detach().cpu().reshape(-1, 1).contiguous()
    out[mlp + "down_proj.had_adj_sign"] = layer.down_sign.detach().cpu().contiguous()
    return out
