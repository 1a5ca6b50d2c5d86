"""``echokv_vllm.host_slots``: the module ``echokv_amd.host_slots`` under the reference's name."""

import sys

from echokv_amd import host_slots as _module

sys.modules[__name__] = _module
