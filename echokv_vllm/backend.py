"""``echokv_vllm.backend``: the module ``echokv_amd.backend`` under the reference's name."""

import sys

from echokv_amd import backend as _module

sys.modules[__name__] = _module
