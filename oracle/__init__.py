"""CPU oracle of EchoKV's quantized KV-cache hot path (TEST INFRASTRUCTURE ONLY).

A from-scratch numpy restatement of the reference algorithm, used as the
checker by ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` -- never by the product path (``echokv_amd``), which
runs only the HIP kernels and fails loudly without them.

Modules (each function cites the reference file:line it restates):

* ``quant``     -- storage numerics (``echokv_vllm/quant.py``)
* ``store``     -- page layout, addressing, write / finalize / seal / demote
                   device effects, and ``gather`` (``echokv_vllm/tiered_cache.py``,
                   ``echokv_vllm/kernels/write.py:61-121``)
* ``attention`` -- decode and chunked-prefill attention over ``gather``
                   (``echokv_vllm/kernels/decode.py:95-129``,
                   ``echokv_vllm/kernels/prefill.py:210-236``)
* ``canary``    -- the per-tier attention-KL probe (``echokv_vllm/canary.py:59-89``)

Pinning (how each part is checked, so a plausible slip fails a test):

* quant: the reference's own outputs on seeded inputs
  (``tests/golden/quant.npz``, written by ``tests/golden/make_golden.py``),
  plus closed-form checks (codes within half a step, constant groups exact,
  pack/unpack inverse, partial K tail exact).
* store: whole page bytes, residual rows, residual map and K_ref ring after
  every golden write script, produced by the reference's store (its PyTorch
  path) and -- as hashes -- by its Triton kernels under the CPU interpreter.
* attention: the reference's ``decode_attention_torch`` /
  ``prefill_attention_torch`` outputs on the config-1 stores, and a brute-force
  per-token softmax on tiny inputs.
* canary: the reference's ``canary_kl`` outputs, and the manual-KL
  known-answer check of ``tests/echokv_vllm/test_canary_controller.py:35-47``.
"""
