"""Model definitions whose hot operations run on the babyvllm HIP kernels."""
