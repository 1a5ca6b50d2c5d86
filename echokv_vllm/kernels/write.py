"""``echokv_vllm.kernels.write``: the module ``echokv_amd.kernels.write`` under the reference's name."""

import sys

from echokv_amd.kernels import write as _module

sys.modules[__name__] = _module
