"""CPU restatement of the reference's decode-hot-path arithmetic.

TEST INFRASTRUCTURE ONLY. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import anything under `oracle/`, and only as
the reference results or as the timed CPU baseline, never as the product path.

Modules:
  q4nx_oracle    tile format, dequantisation and GEMV (tools/q4nx.py, lm_head.py,
                 granite_gemv.py reference functions)
  decode_oracle  RMSNorm, RoPE, SwiGLU, GQA decode attention, fused groups and the
                 granite-shaped decode step composed from them
  cpu_oracle     ctypes binding to cpu_oracle.c, the threaded C restatement used for
                 large shapes and as the CPU baseline
"""
