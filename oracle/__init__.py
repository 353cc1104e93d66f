"""CPU oracle of the quantized DiT-block path -- TEST INFRASTRUCTURE ONLY.

A restatement, in torch-CPU and numpy, of the reference's arithmetic for the
path that the HIP library implements.  Each function cites the reference
file:line it follows.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only to check
the GPU results against or as the timed CPU baseline; the product
(``waveforcing_amd``) never imports it and has no CPU fallback.

Modules:
  fp8        e4m3fn cast (torch's cast) and an independent bit-level encoder
  kv         per-(token, head) FP8 KV pack, page scatter, gather-dequant
"""
