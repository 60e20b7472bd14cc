"""CPU oracle for the quantized-linear hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain numpy, what the reference's numpy fallback computes for the
GPTQ int4/int8 dequant-matmul, the GGUF Q4_K dequant, the MoE expert MLP and the CPU decode
path. It exists to check the HIP library. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it, and only as the reference the GPU results are
compared with or as the timed CPU baseline; the product package (`webpytorch_amd`) never imports it and has no CPU fallback.

Modules and what pins each function (anything not listed as pinned says so in its docstring):
  gptq.py    -- GPTQ dequant / matmul / quantizer (`webtorch/_core.py:3782-3824, 4046-4072`)
  q4k.py     -- Q4_K super-block dequant (`webtorch/ggufload.py:116-130, 188-202`)
  moe.py     -- sparse MoE MLP (`webtorch/lm_engine.py:294-333`)
  decode.py  -- growing-cache CPU decode of a Qwen2-shaped model (`webtorch/llm.py:1619-1636`)
"""
