"""``echokv_vllm.canary``: the module ``echokv_amd.canary`` under the reference's name."""

import sys

from echokv_amd import canary as _module

sys.modules[__name__] = _module
