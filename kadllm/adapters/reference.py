"""``kadllm.adapters.reference`` (src/kadllm/adapters/reference.py) on the HIP path."""

from kadllm_amd.adapters.reference import GatedMLP, HybridPrefix, ReferenceHybridLM  # noqa: F401
