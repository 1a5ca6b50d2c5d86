"""``echokv_vllm.controller``: the module ``echokv_amd.controller`` under the reference's name."""

import sys

from echokv_amd import controller as _module

sys.modules[__name__] = _module
