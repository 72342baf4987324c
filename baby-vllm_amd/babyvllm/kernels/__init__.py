"""HIP kernels of the paged-KV hot path behind the reference's Python signatures."""
