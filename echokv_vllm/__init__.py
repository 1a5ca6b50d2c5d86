"""The reference's module path, ``echokv_vllm``, over this build's implementation.

vLLM loads the plugin through the entry point ``echokv =
"echokv_vllm.plugin:register"`` and the backend through
``"echokv_vllm.backend.EchoKVAttentionBackend"``; the reference's harnesses
import ``from echokv_vllm import control``. Each submodule here is the
``echokv_amd`` module of the same name (the very module object, installed in
``sys.modules`` under this name), so callers written against the reference run
unchanged and both names share one state.
"""
