"""CPU oracle for the W4 group-64 static-KV decode/prefill path.

TEST INFRASTRUCTURE ONLY. This package is the checker the HIP path is compared
against. It is imported by ``tests/``, by ``__graft_entry__.smoke()`` and by the
``cpu_baseline`` leg of ``bench.py`` - nowhere else. The product package
(``aotolith_amd``) never imports it and has no CPU fallback.

Every function restates, in NumPy, the arithmetic of one piece of the reference
(aotolith 0.68.0) and cites the file:line it follows. Paths are relative to the
reference's ``src/aotolith/`` unless they start with ``tests/``.

Pinning (what checks each function beyond a retyped formula):

* ``quant``: the reference's known-answer tests (``tests/test_quantize.py:66-74``
  nibble order, ``:94-100`` scale closed form, ``:103-107`` zero group,
  ``:110-115`` error bound), an exhaustive 16-code x bf16-scale dequant table, a
  pack -> unpack round trip, and idempotence of re-packing a dequantized grid.
* ``ops``: f64 brute force on tiny shapes, closed forms (softmax rows sum to 1,
  a one-key attention returns V, RoPE at position 0 is the identity, RoPE
  preserves the pairwise norm to bf16 precision, RMSNorm of a constant row),
  and an independent torch fp32 cross-check of each fused op's dequant->matmul
  semantics (``tests/test_oracle_ops.py``).
* ``decoder``: greedy tokens cross-checked against HuggingFace torch eager on
  round-tripped weights (``tests/test_oracle_decoder.py``), the pattern of
  ``tests/test_quantized_qwen2.py:107-123``.

Parity unpinned: the bitwise output of the reference's ``mlx-reference`` target
(MLX's own accumulation order) - MLX is not installable here, and the reference
refuses non-darwin hosts (``__init__.py:43-56``).
"""
