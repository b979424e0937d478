"""CPU oracle for the RotateK decode hot path and its prefill producer.

TEST INFRASTRUCTURE ONLY.  This package is a numpy restatement of the
reference algorithm (beomseokg/rotatek), used as the checker for the HIP
library.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only to check or to
time the CPU baseline; the product path (``rotatek_amd``) never imports,
calls or falls back to it.

Modules
-------
``oracle.decode``   decode attention (fused_decode.py, gqa_decode.py,
                    full_channel_flash_decoding.py)
``oracle.prefill``  covariance, query weighting, eigenbasis, rotation,
                    channel top-k, delta-mu, power iteration
                    (kv_pruning_utils.py, rotation.py)
``oracle.numerics`` round-to-nearest-even emulation of fp16 / bf16 storage

Parity status of each function is stated in its docstring: "pinned by"
names the independent checks in ``tests/test_oracle_*.py``; a function with
no such check says "parity unpinned".
"""
