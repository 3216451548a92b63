"""Benchmarks of the fused kernels against the unfused baseline and torch SDPA (the reference's
benchmarks/ folder, restated for MI355X)."""
