"""HIP kernel wrappers with the reference engine's qwen3/kernels/ interface."""
