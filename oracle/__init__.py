"""CPU oracle for slm-turbo's fused 4-bit KV dequant + decode-attention path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import, call, link or execute anything
under ``oracle/`` -- and only as the checker (or the timed CPU baseline), never
as the thing measured or shipped.  The product package (``slm-turbo_amd/``)
never imports it and has no CPU fallback.

Modules
-------
``quant``      per-channel host quantizer (numpy fp16 semantics) and the
               per-token quantize-on-write store (C, IEEE fp32, via ctypes).
``attention``  dequantizers, paged-cache addressing and dequant-then-attend in
               float64.
``cpu_path``   the reference's CPU torch path (dequant -> fp16 -> GQA broadcast
               -> scaled_dot_product_attention), timed as the CPU baseline.

Every function cites the reference file:line it restates.  How each function is
pinned (golden vectors, known answers, library cross-checks, invariants) is
listed in the tests under ``tests/test_oracle_*.py``.
"""
