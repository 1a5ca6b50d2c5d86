"""``echokv_vllm.plugin``: the module ``echokv_amd.plugin`` under the reference's name."""

import sys

from echokv_amd import plugin as _module

sys.modules[__name__] = _module
