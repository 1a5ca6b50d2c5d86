"""``echokv_vllm.write_plan``: the module ``echokv_amd.write_plan`` under the reference's name."""

import sys

from echokv_amd import write_plan as _module

sys.modules[__name__] = _module
