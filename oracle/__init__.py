"""CPU oracle for the FlashAttention hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or, for bench.py, as the timed CPU
baseline). The product path (lightserve_amd) never imports it: with the HIP
library missing it raises instead of falling back to anything here.

Contents
  attention.py  closed-form attention in float64 (the reference's test oracle,
                kernels/tests/test_flash_attention.py:47), its autograd
                gradients, a line-by-line restatement of the reference's
                tiled forward/backward loops, varlen/GQA, paged-KV decode,
                paged-KV chunked prefill,
                and a pure-Python loop version for tiny inputs.
  model.py      the reference's model forward in plain torch (RoPE tables and
                rotation, RMSNorm, the fused add + RMSNorm's semantics,
                reference_llama_forward, with GQA).

How each function is pinned (tests/test_oracle.py):
  attention_reference   pure-Python loops (golden fixtures under tests/golden),
                        closed-form invariants, torch SDPA in float64.
  attention_grads       float64 gradcheck (calculus) and the restated backward.
  flash_forward_tiled   attention_reference (fp32 operands: 1e-6).
  flash_backward_tiled  attention_grads (fp32 operands: 1e-6).
  varlen_reference      pure-Python loops with GQA and bottom-right masking.
  paged_decode_reference  pure-Python loops over a hand-built cache, the
                        dense closed form through an identity block table,
                        and invariance under a permutation of the blocks.
  paged_prefill_reference  pure-Python loops (ragged chunks, GQA, empty
                        chunks), a block permutation, and the chunking
                        invariant (chunk-by-chunk prefill equals one causal
                        pass); a planted top-left mask fails it.
  model.apply_rope      RoPE as an element-by-element rotation (tests/test_oracle_model.py).
  model.add_rmsnorm_reference  h and out written out by hand per element
                        (pure-Python sums), with and without the residual; unit
                        RMS with a unit weight (tests/test_oracle_model.py).
  model.reference_llama_forward  a pure-Python float64 one-layer forward.
Every function has at least one check that a planted mistake (a dropped
scale, a transposed operand, a wrong mask offset) fails.
"""
