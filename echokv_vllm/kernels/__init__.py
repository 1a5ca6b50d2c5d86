"""``echokv_vllm.kernels``: the kernel modules (``decode``, ``prefill``, ``write``) under the reference's names."""
