"""CPU oracle for the speculative-verify hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy float64, the algorithms of the reference's
verify path:

* ``qmv``      4-bit affine group-wise quantized matmul
               (``mtplx/verify_kernels.py:69-88``, ``:372``; ``mtplx/verify_qmv.py:58-191``)
* ``sampler``  sampler law and the depth-K accept/reject loop
               (``mtplx/sampling.py:131-391``, ``mtplx/generation.py:15560-15790``,
               ``:16085-16110``, ``mtplx/qwen4_draft_device_chain.py:294-305``)
* ``attention`` ragged causal mask + GQA scaled-dot-product attention
               (``mtplx/ragged_attention.py:42-105``)
* ``kv_cache`` ragged KV cache scatter / restore
               (``mtplx/ragged_kv_cache.py:201-496``)
* ``moe``      expert sort, gathered quantized matmul, SwiGLU, unsort
               (``mtplx/moe_sorted_gather.py:170-328``, ``mtplx/models/qwen4_exp.py:1544-1577``)
* ``model``    one verify step of a dense or MoE decoder built from the above
               (``decoder_layer`` is the one-layer restatement both use).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import it, and only as the checker. The product package
``mtplx_amd`` never imports it: its kernels run on the GPU or raise.

Each public function names its parity pin in its docstring; the pins
themselves live in ``tests/test_oracle_*.py``.
"""
