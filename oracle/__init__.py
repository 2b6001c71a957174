"""CPU oracle for the lite-vllm continuous-batching hot path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import, call or link anything under
oracle/, and only as the checker (or, for cpu_baseline, as the timed CPU
restatement of the reference algorithm).  The product package
(lite-vllm_amd/litevllm) never imports it and has no CPU fallback.

Modules (each function cites the reference file:line it restates; the
reference is lite-vllm 0.1.0, pure Python/torch):

  packing    ModelRunner.prepare_inputs      engine/model_runner.py:180-260
  scatter    KV scatter                      layers/attention.py:17-33, 79-84
  attention  Attention._decode_fast / _prefill layers/attention.py:91-151
  layers     RMSNorm, residual add, q/k norm + RoPE + cache write, SiLU gate
                                              models/llama.py:24-38,
                                              models/qwen3.py:75-84, 131-140,
                                              layers/rotary_emb.py:104-117
  model      Llama/Qwen3 decoder, greedy decoding, fp32, one sequence at a
             time plus a batched decode step   models/llama.py, models/qwen3.py
  sampler    Sampler.sample (greedy)          layers/sampler.py:60-84, 111-124
             temperature sampling: the build's fixed-order inverse-CDF
             definition, restated in C (sampler_ref.c) because the
             reference draws with torch.multinomial, which no vector pins.

How each function is pinned (checks live in tests/test_oracle_*.py):
  packing    hand-worked known-answer fixture (tests/golden/packing_kat.json),
             literal-loop restatement vs vectorised expansion, closed-form
             invariants (positions, slot // bs, slot % bs, cu_seqlens).
  scatter    round-trip gather returns the input; sentinel-filled untouched
             slots unchanged.
  attention  brute-force float64 loops on tiny shapes; torch SDPA (library
             routine) per sequence; ctx = 1 -> V[0]; equal keys -> mean(V);
             chunk of length 1 == decode; chunk at offset == rows of the
             full prefill.
  layers     rms_norm vs torch.nn.functional.rms_norm (library) and exact
             power-of-4 scale invariance; rope: position 0 is the identity,
             rotation keeps each pair's norm, scores depend only on the
             position difference, composition of two rotations; silu_mul vs
             x * sigmoid(x) and at 0; cache write round trip.
  model      incremental decode == full prefill; batched decode step ==
             per-sequence forward; RMSNorm vs F.rms_norm; RoPE position
             sensitivity (tests/test_oracle_model.py).
  sampler    greedy: the reference's KATs (tests/test_sampler.py:11-17,
             28-36) and first-index tie rule; temperature: exp2_det vs
             numpy exp2, chi-square of many draws vs softmax(x/T), agreement
             with a float64 inverse CDF away from bin edges, special cases
             (u = 0, tiny T -> argmax, one-hot logits, -inf entries never
             drawn).
"""
