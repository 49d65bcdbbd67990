"""CPU oracle for the batch-1 W4A16 decode path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of the reference's numerical ground truth:

  * ``oracle.quant_ref``  — numpy restatement of the INT4 format producer (RTN group parameters, quantize,
                            dequantize, nibble pack/unpack, scale/zero interleave) of ``runtime/quant.py``.
  * ``oracle.ref_ops``    — torch-CPU fp32 restatement of every op in ``reference/ref_ops.py`` (GEMV, fused
                            residual+RMSNorm, SwiGLU, RoPE tables / RoPE + paged KV append, KV gather, GQA attention,
                            split-K softmax combine).
  * ``oracle.decode_ref`` — the ``backend="ref"`` decode-step composition of ``runtime/model.py:216-233`` on the CPU.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this package, and only
as the checker or as the timed CPU baseline. The product (``llm-decode-kernels_amd``) never imports it: the HIP path has
no CPU fallback and fails loudly when its extension is missing.

Each function cites the reference file:line it follows and is pinned by a check in ``tests/test_oracle.py``
(known-answer vectors from the reference's own tests, closed forms, brute force on tiny inputs, or library routines).
"""
