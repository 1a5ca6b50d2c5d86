"""vLLM general plugin: installs the EchoKV backend when ``ECHOKV_ENABLE=1``.

Interface of ``echokv_vllm/plugin.py:17-28``, registered under the reference's
``vllm.general_plugins`` entry point ``echokv = "echokv_vllm.plugin:register"``
(``pyproject.toml``; ``echokv_vllm`` is this package under the reference's
module path), so vLLM calls ``register`` in the engine process and every worker
before any model is built.
Select the backend with ``attention_config={"backend": "CUSTOM"}``. The kernels
run on the GPU only, so unlike the reference nothing is registered for vLLM's
CPU platform.
"""

from __future__ import annotations

import os

BACKEND_PATH = "echokv_vllm.backend.EchoKVAttentionBackend"


def register() -> None:
    if os.environ.get("ECHOKV_ENABLE", "0") != "1":
        return
    from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend

    from echokv_amd.host_slots import install

    install()
    register_backend(AttentionBackendEnum.CUSTOM, BACKEND_PATH)
