"""Paged KV pool (reference engine/runtime/paged_cache.py) backed by the HIP kernels."""
