"""``echokv_vllm.kernels.prefill``: the module ``echokv_amd.kernels.prefill`` under the reference's name."""

import sys

from echokv_amd.kernels import prefill as _module

sys.modules[__name__] = _module
