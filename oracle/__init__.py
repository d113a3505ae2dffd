"""CPU oracle for the decode hot path — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference algorithms, used as the checker by
``tests/``, by ``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg of
``bench.py``. Nothing in the product package imports it, and it is never the
thing measured as the product.

Modules and the reference code each one restates:
  paged_attention  paged gather + softmax attention, decode and bottom-right
                   causal verify (nanovllm/kernels/paged_decode_attn.py:472-495,
                   nanovllm/layers/attention.py:64-81,
                   nanovllm/engine/model_runner.py:492-584)
  kvcache          slot formula and the store_kvcache scatter
                   (nanovllm/layers/attention.py:10-40,
                   nanovllm/engine/model_runner.py:466-482,522-548)
  w8a16            quantize / dequantize / dequantize-then-matmul
                   (nanovllm/layers/quant.py:123-159,209-223)
  decoder_ops      the draft step's neighbour ops: RMSNorm (+ residual add),
                   q/k norm + rotate-half RoPE, SiLU*up, argmax and the
                   exponential-race sampler with Philox4x32-10 noise
                   (nanovllm/layers/layernorm.py:16-47, rotary_embedding.py:6-48,
                   models/qwen3.py:80-88, activation.py:6-11, sampler.py:6-12)
  bf16             bf16 <-> fp32 bit conversion (round to nearest even)
  torch_cpu        the same paged attention, dequantize-then-matmul and slot
                   scatter in torch fp32 on the host: the timed CPU baseline
                   of bench.py (pinned against the numpy modules above)

How each function is pinned (tests/test_oracle_*.py): against library
routines (torch scaled_dot_product_attention, torch.nn.functional.linear,
torch.round, rms_norm, silu) on the cases that reduce to them, published
known-answer vectors (Philox4x32-10), a chi-square test of the sampling law, closed forms (uniform keys,
one dominant key, identity weights), invariants (page placement, table
padding, GQA == repeated heads, verify with one row == decode) and brute-force
Python loops on tiny inputs, plus the committed fixtures in tests/golden/
(made by tests/golden/make_golden.py from torch library routines, not from
this package). The reference ships no golden vectors for this path.
"""
