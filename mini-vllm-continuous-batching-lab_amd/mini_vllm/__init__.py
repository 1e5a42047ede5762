"""MI355X-native decode hot path of mini-vLLM.

This package provides the pieces of ``mini_vllm`` that the paged decode step
touches, under the same import paths: the attention plugin API
(``mini_vllm.attention``), the physical KV pool (``mini_vllm.cache.pool``)
and the per-step metadata types (``mini_vllm.model_runner.base``). The
kernels are hand-written HIP for gfx950 in ``libmvattn.so``; importing this
package never imports triton.
"""
