"""Checkpoint loading and prefix-state interop with transformers (no GPU).

Checkpoints are written by transformers' own save_pretrained in the format of
the reference benchmark model (benchmarks/prepare_model.py:77-81); prefixes are
exchanged with transformers caches both ways and continued by the other side
(the oracle restates the reference decode).
"""

import pytest
import torch

from kadllm_amd.config import Qwen35Config, tiny_hybrid_config
from kadllm_amd.formats import cache_from_prefix_layers, load_checkpoint, prefix_layers_from_cache
from kadllm_amd.weights import build_hf_text_model, random_state_dict
from oracle.qwen35_ref import OraclePrefix, Qwen35Oracle


def _tiny_text_dict():
    cfg = tiny_hybrid_config()
    d = cfg.to_hf().to_dict()
    return cfg, d


def test_load_conditional_generation_checkpoint(tmp_path):
    """Qwen3_5ForConditionalGeneration with a small vision tower, as the
    reference's prepare_model writes it: text weights, config and tied head."""
    from transformers import Qwen3_5Config, Qwen3_5ForConditionalGeneration

    _, text = _tiny_text_dict()
    full = Qwen3_5Config(text_config=text,
                         vision_config=dict(depth=1, hidden_size=32, intermediate_size=64,
                                            num_heads=1, out_hidden_size=text["hidden_size"],
                                            num_position_embeddings=16, patch_size=2))
    torch.manual_seed(0)
    model = Qwen3_5ForConditionalGeneration(full).eval().to(torch.bfloat16)
    model.save_pretrained(tmp_path)
    cfg, sd = load_checkpoint(str(tmp_path), dtype=torch.bfloat16)
    ref = model.model.language_model.state_dict()
    assert cfg.num_hidden_layers == text["num_hidden_layers"]
    assert tuple(cfg.layer_types) == tuple(text["layer_types"])
    assert set(sd) == set(ref) | {"lm_head.weight"}
    for k, v in ref.items():
        assert torch.equal(sd[k], v), k
    assert torch.equal(sd["lm_head.weight"], model.lm_head.weight)


def test_load_causal_lm_checkpoint(tmp_path):
    from transformers import Qwen3_5ForCausalLM
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig

    _, text = _tiny_text_dict()
    text = dict(text, tie_word_embeddings=False)
    torch.manual_seed(1)
    model = Qwen3_5ForCausalLM(Qwen3_5TextConfig(**text)).eval().to(torch.bfloat16)
    model.save_pretrained(tmp_path)
    cfg, sd = load_checkpoint(str(tmp_path))
    for k, v in model.model.state_dict().items():
        assert torch.equal(sd[k], v), k
    assert torch.equal(sd["lm_head.weight"], model.lm_head.weight)
    assert not torch.equal(sd["lm_head.weight"], sd["embed_tokens.weight"])


def test_config_from_dict_reads_rope_both_ways():
    _, text = _tiny_text_dict()
    a = Qwen35Config.from_dict(text)
    legacy = dict(text)
    rope = legacy.pop("rope_parameters")
    legacy.update(rope_theta=rope["rope_theta"], partial_rotary_factor=rope["partial_rotary_factor"])
    b = Qwen35Config.from_dict(legacy)
    assert a == b


@pytest.fixture(scope="module")
def tiny_models():
    cfg = tiny_hybrid_config()
    sd = random_state_dict(cfg, seed=3, dtype=torch.float32)
    model, head = build_hf_text_model(cfg, sd)
    return cfg, model, head, Qwen35Oracle(cfg, sd)


def test_prefix_from_transformers_cache_continues_in_the_oracle(tiny_models):
    """A transformers prefill's cache, read as a prefix, decodes to the logits of
    transformers' own next-token forward on that cache."""
    cfg, model, head, orc = tiny_models
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, cfg.vocab_size, (2, 30), generator=g)
    nxt = torch.randint(0, cfg.vocab_size, (2, 1), generator=g)
    with torch.no_grad():
        out = model(input_ids=ids, use_cache=True, return_dict=True)
        layers = prefix_layers_from_cache(out.past_key_values, cfg.layer_types)
        ours = orc.decode(nxt[:, None, :], OraclePrefix(30, 2, layers))[:, 0]
        hf = head(model(input_ids=nxt, past_key_values=out.past_key_values,
                        use_cache=True).last_hidden_state[:, -1])
    assert (ours - hf).abs().max().item() <= 1e-4 * hf.abs().max().item()


def test_prefix_to_transformers_cache_continues_in_transformers(tiny_models):
    """An oracle prefix, written into a transformers cache, continues in the
    transformers forward exactly as the oracle's own decode."""
    cfg, model, head, orc = tiny_models
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, cfg.vocab_size, (2, 25), generator=g)
    nxt = torch.randint(0, cfg.vocab_size, (2, 1), generator=g)
    with torch.no_grad():
        _, prefix = orc.prefill(ids)
        cache = cache_from_prefix_layers(prefix.layers, cfg.layer_types, model.config)
        assert cache.get_seq_length() == 25
        hf = head(model(input_ids=nxt, past_key_values=cache, use_cache=True).last_hidden_state[:, -1])
        ours = orc.decode(nxt[:, None, :], prefix)[:, 0]
    assert (ours - hf).abs().max().item() <= 1e-4 * hf.abs().max().item()
