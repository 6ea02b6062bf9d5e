"""slm-turbo's fused 4-bit KV dequant + attention kernels for MI355X (gfx950).

The public functions live in :mod:`kernels.kv_dequant`, signature-compatible
with the reference's ``kernels/kv_dequant.py``.
"""
