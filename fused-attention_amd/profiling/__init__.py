"""Performance-run tracking (rocprofv3) for the fused attention kernels."""
