"""Weight-only int8 quantization on gfx950: quantizer, fused product, module swap, byte accounting."""
