"""byteprof_amd: the batch-1 decode hot path of byteprof (skinny weight-only matmul, fused int8 weight-only
product, fused multi-step mLSTM recurrence) as hand-written gfx950 (MI355X) HIP kernels behind a C ABI
(include/byteprof_amd.h, libbyteprof_amd.so), with Python modules that keep the reference's call signatures:

  byteprof_amd.optim.skinny         skinny_mm, get_cfg, dequantize        (byteprof/optim/skinny.py)
  byteprof_amd.optim.skinny_linear  SkinnyLinear                          (byteprof/optim/skinny_linear.py)
  byteprof_amd.quant.hip_int8       gemv_int8, quantize_rowwise_int8      (byteprof/quant/triton_int8.py)
  byteprof_amd.quant.integrate      Int8Linear, apply_quantization        (byteprof/quant/integrate.py)
  byteprof_amd.quant.select         olmo_should_quantize, ...             (byteprof/quant/select.py)
  byteprof_amd.quant.accounting     linear_bytes                          (byteprof/quant/accounting.py)
  byteprof_amd.optim.draft_fused    multistep_fw                          (byteprof/optim/draft_fused.py)
"""

__version__ = "0.1.0"
