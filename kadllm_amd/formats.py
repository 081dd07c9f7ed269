"""Checkpoint and prefix-state formats (interop with transformers).

* ``load_checkpoint(path)`` reads a Qwen3.5 checkpoint written by transformers'
  ``save_pretrained`` -- the format of the reference's benchmark model
  (benchmarks/prepare_model.py:77-81: ``Qwen3_5ForConditionalGeneration`` in
  bf16 with ``config.json`` holding a ``text_config``), or a
  ``Qwen3_5ForCausalLM`` / bare text-model checkpoint -- from its safetensors
  files (single file or sharded with an index).  It returns the text config
  and a state dict in ``Qwen3_5TextModel`` naming plus ``lm_head.weight``
  (the embedding when the head is tied), ready for
  ``adapters.native_model`` or ``Qwen35GRBeamAdapter.from_pretrained``.
* ``prefix_layers_from_cache(cache, layer_types)`` takes the per-layer prefix
  tensors from a transformers cache as the reference adapter does
  (src/kadllm/adapters/qwen3_5.py:113-142): GDN layers (conv_states
  [B, C, 4], recurrent_states [B, HV, K, V] fp32), attention layers (keys and
  values [B, HK, L, D] exposed as [B, L, HK, D] transposed views).
* ``cache_from_prefix_layers(layers, layer_types, hf_config)`` builds the
  transformers ``DynamicCache`` holding the same state, so a prefix made here
  continues in a transformers forward (transformers cache_utils.py:1032-1086).

Nothing here is on the search's hot path.
"""

import json
import os

import torch

from .config import Qwen35Config

_TEXT_PREFIXES = ("model.language_model.", "model.", "")


def _read_safetensors(path):
    from safetensors.torch import load_file

    index = os.path.join(path, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            files = sorted(set(json.load(f)["weight_map"].values()))
    else:
        files = sorted(fn for fn in os.listdir(path) if fn.endswith(".safetensors"))
    if not files:
        raise FileNotFoundError(f"no safetensors files in {path}")
    tensors = {}
    for fn in files:
        tensors.update(load_file(os.path.join(path, fn)))
    return tensors


def load_checkpoint(path, device=None, dtype=torch.bfloat16):
    """(Qwen35Config, state_dict) of a transformers Qwen3.5 checkpoint directory."""
    with open(os.path.join(path, "config.json")) as f:
        raw = json.load(f)
    text = raw.get("text_config", raw)
    cfg = Qwen35Config.from_dict(text)
    tensors = _read_safetensors(path)
    prefix = next((p for p in _TEXT_PREFIXES if f"{p}embed_tokens.weight" in tensors), None)
    if prefix is None:
        raise KeyError("checkpoint holds no text-model embed_tokens.weight")
    sd = {}
    for name, t in tensors.items():
        if name.startswith(prefix) and not (prefix == "" and name.startswith("lm_head.")):
            key = name[len(prefix):]
            if prefix == "model." and key.startswith(("language_model.", "visual.")):
                continue
            if key.startswith(("visual.", "mtp.")):
                continue
            sd[key] = t
    head = tensors.get("lm_head.weight")
    sd["lm_head.weight"] = head if head is not None else sd["embed_tokens.weight"]
    sd = {k: v.to(device=device, dtype=dtype if v.is_floating_point() else v.dtype)
          for k, v in sd.items()}
    return cfg, sd


def _cache_tensor(value):
    if isinstance(value, dict):
        value = value[0]
    if not isinstance(value, torch.Tensor):
        raise TypeError("unsupported transformers linear-attention cache layout")
    return value.detach()


def prefix_layers_from_cache(cache, layer_types):
    """Per-layer prefix tensors of a transformers cache, in the reference's layout."""
    out = []
    for kind, layer in zip(layer_types, cache.layers, strict=True):
        if kind == "linear_attention":
            out.append((_cache_tensor(layer.conv_states), _cache_tensor(layer.recurrent_states)))
        else:
            out.append((layer.keys.transpose(1, 2).detach(), layer.values.transpose(1, 2).detach()))
    return tuple(out)


def cache_from_prefix_layers(layers, layer_types, hf_config):
    """A transformers DynamicCache holding the given prefix (any device/dtype)."""
    from transformers.cache_utils import DynamicCache

    cache = DynamicCache(config=hf_config)
    for kind, layer, (a, b) in zip(layer_types, cache.layers, layers, strict=True):
        if kind == "linear_attention":
            layer.update_conv_state(a.clone())
            layer.update_recurrent_state(b.clone())
        else:
            layer.update(a.transpose(1, 2).contiguous(), b.transpose(1, 2).contiguous())
    return cache
