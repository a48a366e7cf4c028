"""The oracle: a CPU restatement of the reference's segment-LoRA path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import this package, and only
to check results against (or as the timed CPU baseline); the product package
``multi_lora_amd`` never imports it and has no CPU path.

Modules and the reference code each one restates:

* ``lora_ref``     — ``TorchLoRABackend`` (multi_lora/backend/torch_backend.py:17-90),
                     ``lora_delta`` (multi_lora/layers.py:23-39), a float64
                     brute-force closed form, and a restatement of the GPU
                     kernels' rounding sequence (sgemm_lora_a.py:109,
                     sgemm_lora_b.py:84-89).
* ``metadata_ref`` — ``segment_lens`` / ``group_rows`` / the resident column
                     padding of ``write_kernel_input_metadata``
                     (multi_lora/batch_info.py:45-179), token -> slot maps and
                     slot-grouped gather order.
* ``pool_ref``     — slot allocation and LRU/FIFO eviction
                     (multi_lora/pool.py:382-473, multi_lora/eviction.py:12-50).
* ``rmsnorm_ref``  — the fused RMSNorm math (multi_lora/kernels/rmsnorm.py:38-45)
                     and the HF module it replaces (multi_lora/tests/test_fused_rmsnorm.py:19-32).

How each function is pinned (known answers from the reference's tests,
closed forms, brute force, invariants) is listed in the test files under
``tests/`` whose names start with ``test_oracle``.
"""
