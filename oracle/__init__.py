"""CPU oracle for the int4 LLM hot path -- TEST INFRASTRUCTURE ONLY.

A restatement, in PyTorch on the CPU, of the reference's LlamaQ4 path
(scripts/llm/llama_q4.py), its runner schedule (runner/llm_runner.c) and its GEMM data contract
(gemm/shapes.py). Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
it, and only as the checker or the CPU baseline: the product path (iree-adreno-genai-tuner_amd/)
never imports or calls anything here.

How each part is pinned (checks live in tests/test_oracle.py):
  quantize_q4 / unpack_q4 / dequantize_q4  hand-computed known answers (bit patterns, half-even
                                           rounding, bit 31, all 16 nibble values), invariants.
  gemv_fused / QLinearRef                  fp64 textbook matvec on the dequantized weight; the
                                           fused and eager forms agree (qgemv_test.py:13-19).
  attention                                closed forms (one valid key returns that V row bit for
                                           bit per GQA group; equal keys give the mean of V; two
                                           keys give sigmoid weights, which pins the scale); rows
                                           past pos changed to large values leave the output
                                           identical; fp64 brute force on a causal prefill chunk.
  rope_tables                              transformers' LlamaRotaryEmbedding (the reference's own
                                           source of the tables, llama_q4.py:184-192).
  LlamaQ4Ref.step (whole model)            transformers' LlamaForCausalLM on the same dequantized
                                           weights, the scripts/llm/test_tiny.py protocol: equal
                                           greedy tokens and |dlogit| < 1e-3.
  pick_bucket / schedule                   closed-form bucket sequences (llm_runner.c:143-245).
  generate                                 its recorded (phase, start, L) calls, padding, `last`
                                           and fed-back tokens equal schedule_calls on ragged
                                           prompts, bucket switches, 'max', running out of
                                           buckets and stop ids.
"""
