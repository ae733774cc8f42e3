"""MI355X-native paged-attention decode path of small-inference: the paged KV caches (bf16 and both INT8 formats)
with their begin / write / attend interface, the block manager whose indexing they share, and the kernel-level
functions, all backed by hand-written gfx950 HIP kernels in libsmallinf_hip.so (csrc/, include/smallinf_hip.h).

Module names follow the reference's engine/ package so its callers need no change: block_manager, paged_cache,
quant_cache, quant, attention, config; hip_decode and hip_quant replace triton_decode and triton_quant.
"""
