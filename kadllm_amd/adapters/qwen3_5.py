"""GRBeam inference adapter for the dense Qwen3.5 text model (MI355X HIP path).

Drop-in for src/kadllm/adapters/qwen3_5.py: same constructor, validation,
exception types and messages, ``Qwen35Prefix`` layout and prefill/decode
contract.  Pass the transformers ``Qwen3_5TextModel`` and its LM head (for
``Qwen3_5ForConditionalGeneration``: ``model.model.language_model,
model.lm_head``), or the package's own ``Qwen35TextModel`` / ``LMHead``.

The wrapped model is not mutated: its weights are packed once, at
construction, into fused bf16 device buffers, and both prefill and decode run
the native HIP kernels (kadllm_amd.qwen35.Qwen35Runner).  The backend
arguments keep their reference names and validation; every accepted value
runs the single HIP implementation.  The prefix is request-sized and is never
written by decode.  Models must be on one ROCm device, in bf16 (the packed
bf16 kernels, with the transformers bf16 rounding points), fp32 (fp32
kernels throughout, kadllm_amd.qwen35_f32) or fp16 (the fp32 kernels on
weights widened once; fp32 logits and prefix).
"""

from dataclasses import dataclass

import torch

from ..config import Qwen35Config
from ..grbeam import PrefillResult
from ..ops import _gdn_launch
from ..qwen35 import LMHead, Qwen35Runner, Qwen35TextModel
from ..qwen35_f32 import Qwen35RunnerF16, Qwen35RunnerF32


@dataclass(frozen=True)
class Qwen35Prefix:
    length: int
    batch: int
    owner: object
    layers: tuple[tuple[torch.Tensor, torch.Tensor], ...]


def _is_transformers_text_model(obj):
    try:
        from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextModel
    except ImportError:
        return False
    return type(obj) is Qwen3_5TextModel


class Qwen35GRBeamAdapter:
    """Wrap an eval-mode Qwen3.5 text model and its matching LM head.

    gdn_backend / conv_backend accept torch/auto/triton and attention_backend
    torch/flash_attn, as in the reference; all run the HIP kernels.
    gdn_triton_config keeps its validation (tile_v, warps, stages[, beam_group])
    and its requirement of gdn_backend='triton'; the HIP kernel picks its own
    tiling.
    """

    def __init__(self, text_model, lm_head, *, gdn_backend="torch", conv_backend="torch",
                 attention_backend="torch", gdn_triton_config=None, head_tokens=None):
        native = isinstance(text_model, Qwen35TextModel)
        if not native and not _is_transformers_text_model(text_model):
            raise TypeError("pass the dense Qwen3_5TextModel explicitly")
        cfg = text_model.config
        rope = getattr(cfg, "rope_parameters", None) or {}
        if rope.get("rope_type", "default") != "default":
            raise ValueError("only default RoPE is supported")
        if cfg.hidden_act != "silu":
            raise ValueError("only SiLU convolution is supported")
        if gdn_backend not in ("torch", "auto", "triton") or conv_backend not in (
            "torch", "auto", "triton",
        ):
            raise ValueError("invalid GDN or convolution backend")
        if attention_backend not in ("torch", "flash_attn"):
            raise ValueError("invalid attention backend")
        if any(kind not in ("linear_attention", "full_attention") for kind in cfg.layer_types):
            raise ValueError("unsupported layer type")
        devices = {p.device for module in (text_model, lm_head) for p in module.parameters()}
        if len(devices) != 1:
            raise ValueError("only single-device models are supported")
        device = devices.pop()
        _gdn_launch(gdn_triton_config)
        if gdn_triton_config is not None and gdn_backend != "triton":
            raise ValueError("gdn_triton_config requires gdn_backend='triton'")
        dtypes = {p.dtype for module in (text_model, lm_head) for p in module.parameters()}
        if dtypes == {torch.bfloat16}:
            runner = Qwen35Runner
        elif dtypes == {torch.float32}:
            runner = Qwen35RunnerF32
        elif dtypes == {torch.float16}:
            runner = Qwen35RunnerF16
        else:
            raise TypeError("the HIP GRBeam path runs bf16, fp16 or fp32 models with one dtype; "
                            "convert with .to()")
        if device.type != "cuda":
            raise RuntimeError("the HIP GRBeam path needs the model on a ROCm device")
        self.layer_types = tuple(cfg.layer_types)
        self.model, self.lm_head = text_model, lm_head
        self.gdn_backend, self.conv_backend = gdn_backend, conv_backend
        self.attention_backend = attention_backend
        self.gdn_triton_config = gdn_triton_config
        self.config = cfg if native else Qwen35Config.from_hf(cfg)
        self.device = device
        self._runner = runner(self.config, text_model.state_dict(),
                              lm_head_weight=lm_head.weight, device=device,
                              head_tokens=head_tokens)
        if runner in (Qwen35RunnerF32, Qwen35RunnerF16):
            # fp32 and fp16 models replay the whole suffix at every level, as
            # the reference does
            self.decode_incremental = None
        # logits column -> token id for a SID-only head (None: the full vocabulary)
        self.vocab_ids = self._runner.head_ids
        self._owner = object()

    def _check(self, tokens):
        if self.model.training or self.lm_head.training:
            raise RuntimeError("call eval() before replay")
        if tokens.dtype not in (torch.int32, torch.int64):
            raise TypeError("token IDs must be integers")
        if tokens.device != self.device:
            raise ValueError("tokens and model must share a device")

    def _range_probe(self, tokens):
        """Start the check that every token id lies in the embedding table:
        the ids' (min, max) go to pinned host memory behind an event, so the
        call's own kernels are enqueued before the host waits for the result
        (the embedding kernel clamps ids, so nothing reads outside the table
        meanwhile).  _raise_out_of_range finishes the check."""
        lo_hi = torch.stack(torch.aminmax(tokens))
        host = torch.empty(2, dtype=lo_hi.dtype, pin_memory=True)
        host.copy_(lo_hi, non_blocking=True)
        done = torch.cuda.Event()
        done.record()
        return host, done

    def _raise_out_of_range(self, probe):
        """IndexError with torch's nn.Embedding message for any id outside
        [0, vocab_size)."""
        host, done = probe
        done.synchronize()
        lo, hi = host.tolist()
        if lo < 0 or hi >= self.config.vocab_size:
            raise IndexError("index out of range in self")

    @torch.no_grad()
    def prefill(self, input_ids):
        self._check(input_ids)
        if input_ids.ndim != 2 or min(input_ids.shape) < 1:
            raise ValueError("input_ids must be nonempty unpadded [B,L]")
        probe = self._range_probe(input_ids)
        logits, layers = self._runner.prefill(input_ids)
        self._raise_out_of_range(probe)
        state = Qwen35Prefix(input_ids.shape[1], input_ids.shape[0], self._owner, layers)
        return PrefillResult(logits, state)

    @torch.no_grad()
    def decode(self, history, state):
        self._check(history)
        if not isinstance(state, Qwen35Prefix) or state.owner is not self._owner:
            raise ValueError("prefix belongs to a different adapter")
        if history.ndim != 3 or min(history.shape) < 1 or history.shape[0] != state.batch:
            raise ValueError("history must be nonempty [B,W,T] matching the prefix")
        probe = self._range_probe(history)
        logits = self._runner.decode(history, state.layers, state.length)
        self._raise_out_of_range(probe)
        return logits

    @classmethod
    def from_pretrained(cls, path, device="cuda", **kwargs):
        """Adapter over a transformers Qwen3.5 checkpoint directory (safetensors +
        config.json, e.g. the reference's benchmark model), loaded natively."""
        from ..formats import load_checkpoint

        cfg, sd = load_checkpoint(path, device=device)
        return cls(*native_model(cfg, sd), **kwargs)

    def prefix_from_cache(self, cache, length):
        """A prefix owned by this adapter from a transformers cache of `length`
        prompt tokens (the layout src/kadllm/adapters/qwen3_5.py:113-142 reads)."""
        from ..formats import prefix_layers_from_cache

        layers = []
        act = self._runner.dtype
        for kind, (a, b) in zip(self.layer_types,
                                prefix_layers_from_cache(cache, self.layer_types)):
            if kind == "linear_attention":
                layers.append((a.to(self.device, act), b.to(self.device, torch.float32)))
            else:
                layers.append((a.to(self.device, act), b.to(self.device, act)))
        batch = layers[0][0].shape[0]
        return Qwen35Prefix(int(length), batch, self._owner, tuple(layers))

    def prefix_to_cache(self, state, hf_config=None):
        """A transformers DynamicCache holding this adapter's prefix."""
        from ..formats import cache_from_prefix_layers

        if not isinstance(state, Qwen35Prefix) or state.owner is not self._owner:
            raise ValueError("prefix belongs to a different adapter")
        return cache_from_prefix_layers(state.layers, self.layer_types,
                                        hf_config if hf_config is not None else self.config.to_hf())

    @torch.no_grad()
    def decode_incremental(self, history, parents, state, cache=None, *, keep_cache=True):
        """decode(history, state) for a level whose beams extend the previous
        level's beams by one token: history[b, w] = history_prev[b, parents[b, w]]
        followed by one new token.  ``cache`` is what the previous call returned
        (None for the first decode level).  Returns (logits, cache); the logits
        equal decode(history, state) while only the new token goes through the
        projections.  With ``keep_cache=False`` (a search's last level) the
        returned cache is None and each layer's per-token rows are released as
        soon as the layer is done.  grbeam_search uses it when the adapter
        offers it."""
        self._check(history)
        if not isinstance(state, Qwen35Prefix) or state.owner is not self._owner:
            raise ValueError("prefix belongs to a different adapter")
        if history.ndim != 3 or min(history.shape) < 1 or history.shape[0] != state.batch:
            raise ValueError("history must be nonempty [B,W,T] matching the prefix")
        T = history.shape[2]
        if (cache is None and T != 1) or (cache is not None and T != cache.T + 1):
            raise ValueError("history must extend the cached suffixes by exactly one token")
        if cache is not None and (parents.shape != history.shape[:2] or parents.device != history.device):
            raise ValueError("parents must be [B, W] on the history's device")
        tokens = history[:, :, -1].contiguous()
        probe = self._range_probe(tokens)
        out = self._runner.decode_step(tokens, parents, state.layers, state.length, cache,
                                       keep_cache=keep_cache)
        self._raise_out_of_range(probe)
        return out


def native_model(cfg, state_dict):
    """(Qwen35TextModel, LMHead) for a state dict in transformers naming."""
    head = state_dict.get("lm_head.weight", state_dict["embed_tokens.weight"])
    return Qwen35TextModel(cfg, state_dict), LMHead(head)
