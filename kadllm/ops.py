"""``kadllm.ops`` (src/kadllm/ops.py) on the HIP path: kadllm_amd.ops, including
the validation helpers the reference's benchmark imports (``_gdn_launch``,
benchmarks/grbeam.py:99)."""

from kadllm_amd.ops import (_backend, _gdn_launch, _same_device, _width,  # noqa: F401
                            causal_conv1d, gated_delta, merge_attention, prefix_attention)
