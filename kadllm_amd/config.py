"""Qwen3.5 hybrid text-model configuration used by the native GRBeam path.

Attribute names follow transformers' Qwen3_5TextConfig so that either object
can be passed where a config is expected (the reference adapter reads these
fields from ``text_model.config``, src/kadllm/adapters/qwen3_5.py:57-73).
"""

from dataclasses import dataclass, field


@dataclass(frozen=True)
class Qwen35Config:
    vocab_size: int
    hidden_size: int
    num_hidden_layers: int
    intermediate_size: int
    linear_num_key_heads: int
    linear_num_value_heads: int
    linear_key_head_dim: int
    linear_value_head_dim: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    layer_types: tuple = field(default=None)
    linear_conv_kernel_dim: int = 4
    rope_theta: float = 10000.0
    partial_rotary_factor: float = 0.25
    rms_norm_eps: float = 1e-6
    tie_word_embeddings: bool = True
    hidden_act: str = "silu"

    def __post_init__(self):
        if self.layer_types is None:
            # every 4th layer is full attention, the rest Gated DeltaNet
            kinds = tuple("full_attention" if (i + 1) % 4 == 0 else "linear_attention"
                          for i in range(self.num_hidden_layers))
            object.__setattr__(self, "layer_types", kinds)
        else:
            object.__setattr__(self, "layer_types", tuple(self.layer_types))
        if len(self.layer_types) != self.num_hidden_layers:
            raise ValueError("layer_types must have one entry per layer")

    @property
    def conv_dim(self):
        return 2 * self.linear_num_key_heads * self.linear_key_head_dim + \
            self.linear_num_value_heads * self.linear_value_head_dim

    @property
    def rope_parameters(self):
        return {"rope_type": "default", "rope_theta": self.rope_theta,
                "partial_rotary_factor": self.partial_rotary_factor}

    @staticmethod
    def from_dict(d):
        """Read a Qwen3.5 text config dict (``config.json``'s ``text_config``, or a
        text-model config), with rope settings in ``rope_parameters`` or at the
        top level."""
        rope = dict(d.get("rope_parameters") or {})
        return Qwen35Config(
            vocab_size=d["vocab_size"],
            hidden_size=d["hidden_size"],
            num_hidden_layers=d["num_hidden_layers"],
            intermediate_size=d["intermediate_size"],
            linear_num_key_heads=d["linear_num_key_heads"],
            linear_num_value_heads=d["linear_num_value_heads"],
            linear_key_head_dim=d["linear_key_head_dim"],
            linear_value_head_dim=d["linear_value_head_dim"],
            num_attention_heads=d["num_attention_heads"],
            num_key_value_heads=d["num_key_value_heads"],
            head_dim=d["head_dim"],
            layer_types=tuple(d["layer_types"]) if d.get("layer_types") else None,
            linear_conv_kernel_dim=d.get("linear_conv_kernel_dim", 4),
            rope_theta=float(rope.get("rope_theta", d.get("rope_theta", 10000.0))),
            partial_rotary_factor=float(rope.get("partial_rotary_factor",
                                                 d.get("partial_rotary_factor", 0.25))),
            rms_norm_eps=d.get("rms_norm_eps", 1e-6),
            tie_word_embeddings=bool(d.get("tie_word_embeddings", False)),
            hidden_act=d.get("hidden_act", "silu"),
        )

    @staticmethod
    def from_hf(hf_config):
        """Read the fields of a transformers Qwen3_5TextConfig."""
        rope = dict(getattr(hf_config, "rope_parameters", None) or {})
        return Qwen35Config(
            vocab_size=hf_config.vocab_size,
            hidden_size=hf_config.hidden_size,
            num_hidden_layers=hf_config.num_hidden_layers,
            intermediate_size=hf_config.intermediate_size,
            linear_num_key_heads=hf_config.linear_num_key_heads,
            linear_num_value_heads=hf_config.linear_num_value_heads,
            linear_key_head_dim=hf_config.linear_key_head_dim,
            linear_value_head_dim=hf_config.linear_value_head_dim,
            num_attention_heads=hf_config.num_attention_heads,
            num_key_value_heads=hf_config.num_key_value_heads,
            head_dim=hf_config.head_dim,
            layer_types=tuple(hf_config.layer_types),
            linear_conv_kernel_dim=hf_config.linear_conv_kernel_dim,
            rope_theta=float(rope.get("rope_theta", 10000.0)),
            partial_rotary_factor=float(rope.get("partial_rotary_factor", 0.25)),
            rms_norm_eps=hf_config.rms_norm_eps,
            tie_word_embeddings=bool(getattr(hf_config, "tie_word_embeddings", False)),
            hidden_act=hf_config.hidden_act,
        )

    def to_hf(self):
        """Build a transformers Qwen3_5TextConfig with the same fields (needs transformers)."""
        from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig

        return Qwen3_5TextConfig(
            vocab_size=self.vocab_size,
            hidden_size=self.hidden_size,
            num_hidden_layers=self.num_hidden_layers,
            intermediate_size=self.intermediate_size,
            linear_num_key_heads=self.linear_num_key_heads,
            linear_num_value_heads=self.linear_num_value_heads,
            linear_key_head_dim=self.linear_key_head_dim,
            linear_value_head_dim=self.linear_value_head_dim,
            num_attention_heads=self.num_attention_heads,
            num_key_value_heads=self.num_key_value_heads,
            head_dim=self.head_dim,
            layer_types=list(self.layer_types),
            linear_conv_kernel_dim=self.linear_conv_kernel_dim,
            rope_parameters={"rope_type": "default", "rope_theta": self.rope_theta,
                             "partial_rotary_factor": self.partial_rotary_factor},
            rms_norm_eps=self.rms_norm_eps,
            tie_word_embeddings=self.tie_word_embeddings,
            hidden_act=self.hidden_act,
        )


def tiny_hybrid_config():
    """4 layers [GDN, GDN, GDN, attention], hidden 256, GDN 4/4 heads x 64,
    attention 4 Q / 1 KV heads x 64, SwiGLU 768, vocabulary 4096."""
    return Qwen35Config(vocab_size=4096, hidden_size=256, num_hidden_layers=4,
                        intermediate_size=768, linear_num_key_heads=4,
                        linear_num_value_heads=4, linear_key_head_dim=64,
                        linear_value_head_dim=64, num_attention_heads=4,
                        num_key_value_heads=1, head_dim=64)


def qwen35_08b_config():
    """Qwen3.5-0.8B text shape: 24 layers [3x GDN, 1x attention] x 6, hidden 1024,
    GDN 16/16 heads x 128, attention 8 Q / 2 KV heads x 256, SwiGLU 3584,
    vocabulary 248320, tied embeddings."""
    return Qwen35Config(vocab_size=248320, hidden_size=1024, num_hidden_layers=24,
                        intermediate_size=3584, linear_num_key_heads=16,
                        linear_num_value_heads=16, linear_key_head_dim=128,
                        linear_value_head_dim=128, num_attention_heads=8,
                        num_key_value_heads=2, head_dim=256)
