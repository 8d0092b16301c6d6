"""CPU oracle for the MI355X KV-cache hot path.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import anything from this package, as the checker or as
the timed CPU baseline; the product (llm-experiments_amd/) never does.

  kv_oracle     float64 numpy restatement of the cache layout, append,
                decode attention and causal (prefix-offset) prefill
  model_oracle  float64 numpy restatement of the reference model (forward,
                cached decode step, greedy and the reference's padded-window
                generate loop) and its float32 torch CPU forward (CPU baseline)
  c_oracle      ctypes binding of c/kv_attn_ref.c, an fp32 C restatement of
                the reference's decode-attention kernel (CPU baseline)
"""
