"""CPU oracle for the full-attention KV-cache path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (``mi50grad_amd``) may import
this package. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker or as the
timed CPU baseline, never as the thing measured on the GPU.
"""
