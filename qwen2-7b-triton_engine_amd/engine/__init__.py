"""Qwen2-7B-shaped decode harness on the W4A16 AWQ GEMM and the fp16 lm_head GEMV."""
