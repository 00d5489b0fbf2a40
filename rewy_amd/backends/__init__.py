"""Backward orchestration on the HIP kernels."""
