"""``echokv_vllm.config``: the module ``echokv_amd.config`` under the reference's name."""

import sys

from echokv_amd import config as _module

sys.modules[__name__] = _module
