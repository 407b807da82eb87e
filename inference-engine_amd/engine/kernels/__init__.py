"""HIP kernels of the paged-KV hot path, called through the C ABI of lib/libpaged_kv.so."""
