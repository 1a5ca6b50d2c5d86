"""MI355X-native (gfx950) EchoKV quantized KV-cache hot path.

Drop-in for the ``echokv_vllm`` plugin's store / write-plan / decode / prefill
/ canary path: the same classes and functions, with every device operation a
hand-written HIP kernel in ``libechokv.so`` (built by ``echokv_amd.build``).
"""

__all__ = ["config", "controller", "write_plan", "tiered_cache", "canary", "kernels"]
