"""``echokv_vllm.tiered_cache``: the module ``echokv_amd.tiered_cache`` under the reference's name."""

import sys

from echokv_amd import tiered_cache as _module

sys.modules[__name__] = _module
