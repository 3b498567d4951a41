"""Block-sparse decode kernels (HIP, gfx950; GPU only)."""
