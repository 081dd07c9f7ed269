"""Deterministic random weights for Qwen3.5-shaped hybrid models.

The state dict uses transformers' Qwen3_5TextModel parameter names, so the
same tensors load into the native adapter or into a transformers model.
Initialisation follows the transformers defaults for the family
(modeling_qwen3_5.py:812-823: Linear/Embedding N(0, 0.02), dt_bias = 1,
A_log = log U(0, 16)), except that the RMSNorm weights are drawn N(0, 0.1)
around their centre instead of being exactly centred, so that the (1 + w)
and w scalings are exercised by parity tests.  Depthwise conv weights are
U(-1/2, 1/2) (the Conv1d fan-in bound for width 4).
"""

import torch


def _normal(shape, std, gen, device):
    return torch.randn(shape, generator=gen, device=device) * std


def random_state_dict(cfg, *, seed=0, dtype=torch.bfloat16, device="cpu"):
    """Draw every parameter of ``cfg`` from a torch generator seeded ``seed``.

    Draws are made in float32 on ``device`` in a fixed order and then cast to
    ``dtype`` (A_log and dt_bias keep ``dtype`` too, as in a bf16 checkpoint).
    """
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    sd = {}
    H = cfg.hidden_size

    def lin(name, n_out, n_in):
        sd[name] = _normal((n_out, n_in), 0.02, gen, device)

    sd["embed_tokens.weight"] = _normal((cfg.vocab_size, H), 0.02, gen, device)
    kd = cfg.linear_num_key_heads * cfg.linear_key_head_dim
    vd = cfg.linear_num_value_heads * cfg.linear_value_head_dim
    for i, kind in enumerate(cfg.layer_types):
        p = f"layers.{i}."
        sd[p + "input_layernorm.weight"] = _normal((H,), 0.1, gen, device)
        sd[p + "post_attention_layernorm.weight"] = _normal((H,), 0.1, gen, device)
        if kind == "linear_attention":
            a = p + "linear_attn."
            lin(a + "in_proj_qkv.weight", 2 * kd + vd, H)
            lin(a + "in_proj_z.weight", vd, H)
            lin(a + "in_proj_b.weight", cfg.linear_num_value_heads, H)
            lin(a + "in_proj_a.weight", cfg.linear_num_value_heads, H)
            k = cfg.linear_conv_kernel_dim
            sd[a + "conv1d.weight"] = (torch.rand((2 * kd + vd, 1, k), generator=gen,
                                                  device=device) - 0.5)
            sd[a + "dt_bias"] = torch.ones(cfg.linear_num_value_heads, device=device)
            sd[a + "A_log"] = torch.log(torch.rand(cfg.linear_num_value_heads, generator=gen,
                                                   device=device) * 16 + 1e-3)
            sd[a + "norm.weight"] = 1.0 + _normal((cfg.linear_value_head_dim,), 0.1, gen, device)
            lin(a + "out_proj.weight", H, vd)
        elif kind == "full_attention":
            a = p + "self_attn."
            hd = cfg.head_dim
            lin(a + "q_proj.weight", 2 * cfg.num_attention_heads * hd, H)
            lin(a + "k_proj.weight", cfg.num_key_value_heads * hd, H)
            lin(a + "v_proj.weight", cfg.num_key_value_heads * hd, H)
            lin(a + "o_proj.weight", H, cfg.num_attention_heads * hd)
            sd[a + "q_norm.weight"] = _normal((hd,), 0.1, gen, device)
            sd[a + "k_norm.weight"] = _normal((hd,), 0.1, gen, device)
        else:
            raise ValueError(f"unsupported layer type {kind}")
        m = p + "mlp."
        lin(m + "gate_proj.weight", cfg.intermediate_size, H)
        lin(m + "up_proj.weight", cfg.intermediate_size, H)
        lin(m + "down_proj.weight", H, cfg.intermediate_size)
    sd["norm.weight"] = _normal((H,), 0.1, gen, device)
    if not cfg.tie_word_embeddings:
        sd["lm_head.weight"] = _normal((cfg.vocab_size, H), 0.02, gen, device)
    return {k: v.to(dtype) for k, v in sd.items()}


def build_hf_text_model(cfg, state_dict):
    """A transformers Qwen3_5TextModel + lm_head holding ``state_dict`` (eval mode)."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextModel

    dtype = state_dict["embed_tokens.weight"].dtype
    device = state_dict["embed_tokens.weight"].device
    hf_cfg = cfg.to_hf()
    hf_cfg._attn_implementation = "sdpa"
    torch_default = torch.get_default_dtype()
    try:
        model = Qwen3_5TextModel(hf_cfg)
    finally:
        torch.set_default_dtype(torch_default)
    # as from_pretrained(dtype=...) leaves it: parameters in `dtype`, the
    # rotary inverse frequencies (a non-persistent buffer) in fp32
    inv, inv0 = model.rotary_emb.inv_freq.clone(), model.rotary_emb.original_inv_freq.clone()
    model = model.to(dtype=dtype, device=device)
    model.rotary_emb.inv_freq = inv.to(device)
    model.rotary_emb.original_inv_freq = inv0.to(device)
    missing, unexpected = model.load_state_dict(
        {k: v for k, v in state_dict.items() if k != "lm_head.weight"}, strict=False)
    missing = [m for m in missing if "rotary_emb" not in m]
    if missing or unexpected:
        raise RuntimeError(f"state dict mismatch: missing={missing} unexpected={unexpected}")
    head = torch.nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False).to(dtype=dtype, device=device)
    with torch.no_grad():
        head.weight.copy_(state_dict.get("lm_head.weight", state_dict["embed_tokens.weight"]))
    return model.eval(), head.eval()
