"""CPU oracle of the paged decode step — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or the timed
CPU baseline). The product path (``mini_vllm``) never imports it and has no
CPU fallback.

Contents
  paged_ref  — restatement of the reference's PyTorch path: the KV write
               (mini_vllm/cache/cache_write.py:25-140), the paged gather
               (mini_vllm/cache/cache_read.py:19-84) and the decode of
               AttentionBackendRef (mini_vllm/attention/paged_attention_ref.py:102-161),
               with the same per-sequence / per-token loops.
  brute      — independent float64 numpy brute force of the same maths
               (explicit softmax, explicit index arithmetic), used to pin
               paged_ref; it shares no code with paged_ref.

The reference is pure Python, so there is no C restatement and no build of
the reference itself (its files are read, never run).
"""
