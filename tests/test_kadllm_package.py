"""The ``kadllm`` package: the reference's import names for the GRBeam path
(src/kadllm/__init__.py:3-18, src/kadllm/adapters/__init__.py:3-6,
src/kadllm/ops.py, src/kadllm/grbeam.py) resolve to the HIP implementation."""

import kadllm
import kadllm.adapters
import kadllm.adapters.qwen3_5
import kadllm.adapters.reference
import kadllm.grbeam
import kadllm.ops
import kadllm_amd
from kadllm_amd import adapters as amd_adapters
from kadllm_amd import ops as amd_ops

# src/kadllm/__init__.py __all__ without the WideTuning training-time names
REFERENCE_GRBEAM_NAMES = ["GRBeamResult", "PrefillResult", "GRBeamAdapter", "grbeam_search",
                          "causal_conv1d", "gated_delta", "prefix_attention"]


def test_top_level_names_are_the_hip_implementation():
    for name in REFERENCE_GRBEAM_NAMES:
        assert getattr(kadllm, name) is getattr(kadllm_amd, name), name
        assert name in kadllm.__all__
    assert kadllm.conditional_search is kadllm_amd.conditional_search


def test_submodules_and_adapters():
    assert kadllm.grbeam.grbeam_search is kadllm_amd.grbeam_search
    for name in ("gated_delta", "causal_conv1d", "prefix_attention", "merge_attention"):
        assert getattr(kadllm.ops, name) is getattr(amd_ops, name), name
    for name in ("Qwen35GRBeamAdapter", "ReferenceHybridLM", "native_model", "Qwen35Prefix"):
        assert getattr(kadllm.adapters, name) is getattr(amd_adapters, name), name
    assert kadllm.adapters.qwen3_5.Qwen35GRBeamAdapter is amd_adapters.Qwen35GRBeamAdapter
    assert kadllm.adapters.reference.ReferenceHybridLM is amd_adapters.ReferenceHybridLM
