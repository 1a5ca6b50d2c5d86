"""``echokv_vllm.control``: the module ``echokv_amd.control`` under the reference's name."""

import sys

from echokv_amd import control as _module

sys.modules[__name__] = _module
