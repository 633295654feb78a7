"""KV-cache operators (static per-tensor FP8 quantization on write, dequantization on gather)."""
