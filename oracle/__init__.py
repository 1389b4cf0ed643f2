"""CPU oracle for the GRPO rollout decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference's hot path
(eblancocabana/grpo-training-engine):

* ``oracle.bf16``        -- float32 <-> bfloat16 round-to-nearest-even.
* ``oracle.nf4``         -- NF4 codebook, blockwise quantizer (test-data
                            generator) and the dequantizer of
                            ``src/triton_kernels/lora_forward.py:171-206``.
* ``oracle.lora_linear`` -- ``Y = W_nf4(x) + bias + B(A(x))*scaling`` with the
                            rounding points of ``lora_forward.py:161-257``.
* ``oracle.paged``       -- block-table addressing, KV append
                            (``paged_kv.py:253-319``) and single-query paged
                            decode attention (``paged_kv.py:63-251``).
* ``oracle.decode``      -- greedy/top-p sampling (``paged_kv.py:418-450``),
                            the low-level decode loop (``paged_kv.py:840-985``)
                            and a Qwen2-shaped decode step
                            (``paged_kv.py:690-820``, ``fused_ops.py:34-251``).
* ``oracle.sampling``    -- the sampled-token rule of the device sampler for a
                            given uniform draw (temperature, top-p cut, ties),
                            and the SplitMix64 draw of (seed, row, step).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or as the timed
CPU baseline.  The product (``grpo_mi355x``) never imports it: when the HIP
extension is missing the product raises ``ImportError``; it never falls back to
this code.

Pinning (what each function is checked against, besides the GPU kernels):

* ``bf16.f32_to_bf16_bits``      -- torch's CPU ``.to(torch.bfloat16)`` (RNE).
* ``nf4.NF4_CODE``               -- the QLoRA closed form
                                    ``norm.ppf`` quantiles (scipy), <= 2e-7.
* ``nf4.dequantize_nf4``         -- hand-built known-answer bytes (nibble order,
                                    block index), quantize->dequantize error
                                    bound, all 256 byte values.
* ``paged.gather_kv`` / ``append_kv`` -- brute-force dense reconstruction on tiny
                                    shapes with permuted block tables.
* ``paged.paged_attention_decode`` -- torch ``scaled_dot_product_attention``
                                    (float64) on the gathered dense K/V;
                                    ``ctx=1 => v0``, ``q=0 => mean(v)``,
                                    ``ctx=0 => 0``, permutation invariance.
* ``lora_linear.nf4_lora_linear`` -- the closed-form KAT of the reference's
                                    ``tests/test_lora.py:69-91``; torch float64
                                    ``F.linear`` on the dequantized weight.
* ``decode.paged_kv_decode``     -- the dense recompute model of the
                                    reference's
                                    ``tests/test_triton_performance.py:152-219``.
* ``decode.Qwen2DecodeOracle``   -- per-op checks above, plus
                                    ``transformers``' ``Qwen2RMSNorm`` and
                                    ``apply_rotary_pos_emb`` on CPU.
* ``sampling`` (kept set, draw)  -- torch's CPU sort / softmax / cumsum on the
                                    same bf16 logits; closed-form edge cases
                                    (top_p 0 and 1, ties in index order, a
                                    two-of-four known answer); draw frequencies
                                    against the kept probabilities;
                                    ``exp_nonpos`` against float64 ``exp``;
                                    ``splitmix64`` against published vectors
                                    (``tests/test_oracle_sampling.py``).
"""

__all__ = ["bf16", "nf4", "lora_linear", "paged", "decode", "sampling"]
