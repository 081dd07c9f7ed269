"""``kadllm.adapters.qwen3_5`` (src/kadllm/adapters/qwen3_5.py) on the HIP path."""

from kadllm_amd.adapters.qwen3_5 import Qwen35GRBeamAdapter, Qwen35Prefix  # noqa: F401
