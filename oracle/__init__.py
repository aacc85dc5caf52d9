"""CPU oracle for the dl-inference operator plugin path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the checker (or the timed CPU baseline), never as the product path.

  oracle.ops     numpy float64 restatement of each reference operator (python/dli_ops/aot/
                 <op>/kernel.py + template.cc semantics), plus bf16 round-to-nearest-even.
  oracle.qwen2   Qwen2 decoder (prefill + greedy decode) in torch fp32 on the CPU with the
                 bf16 rounding points of the dli.graph.v1 graph.
"""
