"""gfx950 kernels of byteprof's decode loops: skinny matmul, its nn.Linear drop-in, the fused mLSTM multistep."""
