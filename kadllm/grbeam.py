"""``kadllm.grbeam`` (src/kadllm/grbeam.py) on the HIP path: kadllm_amd.grbeam."""

from kadllm_amd.grbeam import (Constraint, GRBeamAdapter, GRBeamResult, PrefillResult,  # noqa: F401
                               conditional_search, grbeam_search)
