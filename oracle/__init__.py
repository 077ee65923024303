"""CPU oracle of the decode hot path — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's arithmetic (byteprof/optim/skinny.py, byteprof/quant/triton_int8.py,
byteprof/optim/mlstm_multistep.py) used to check the gfx950 kernels. Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import it, and only as the checker: no product code path calls it, and the
product raises when its HIP library is missing instead of falling back to anything here.

Modules:
  numerics  bf16 / fp16 rounding on float arrays (bit-exact round-to-nearest-even), error metrics
  skinny    fp64 matmul oracle, dequantize, the per-row int8 quantizer
  mlstm     the stabilised multi-step mLSTM recurrence in fp64 with the reference's io-dtype roundings, and the
            unstabilised closed form that pins it
  olmo      the OLMo-2 decode step (one token, static KV cache) with the roundings of transformers'
            Olmo2ForCausalLM in bf16, pinned against that model on the CPU

How each function is pinned (checked against something other than itself) is stated in its docstring; the tests
that do it are tests/test_oracle.py. Every function here is pinned; none is "parity unpinned", except where a
docstring says so.
"""
