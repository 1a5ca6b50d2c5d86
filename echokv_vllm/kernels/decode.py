"""``echokv_vllm.kernels.decode``: the module ``echokv_amd.kernels.decode`` under the reference's name."""

import sys

from echokv_amd.kernels import decode as _module

sys.modules[__name__] = _module
