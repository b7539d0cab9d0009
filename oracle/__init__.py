"""CPU oracle for the speculative verify/accept + paged-KV path.  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the checker (or, in the baseline leg, as the timed CPU path).  The product
(iitj_llm_coopt_amd) never imports it and has no CPU fallback.

Each function restates the reference algorithm (mohsinmubarak/iitj-llm-coopt, cited
file:line) in numpy / torch-CPU:
  oracle.codec     quantize / dequantize          engine/kv_tier_manager.py:21-41
  oracle.paged     slot mapping, KV write,        engine/block_manager.py:216-229,
                   paged causal GQA attention,    engine/model.py:186-207, :242-247,
                   tier swap, block migration     engine/kv_tier_manager.py:99, 119,
                                                  engine/block_manager.py:165-187
  oracle.accept    softmax, sample, verify         engine/spec_decode.py:12-49,
                   (explicit uniforms), batched    engine/engine.py:421-446
                   greedy accept
How each is pinned (reference known-answer tests, closed forms, brute force, library
routines) is stated in its module docstring and exercised by tests/test_oracle_*.py.
"""
