"""CPU oracle of the paged-attention decode path (TEST INFRASTRUCTURE ONLY).

Restates the reference's algorithm (Shivram08/small-inference, engine/quant.py, engine/block_manager.py,
engine/paged_cache.py, engine/attention.py, engine/quant_cache.py, engine/triton_decode.py) on the CPU:
quant_ref.c (plain C, the bit-exact INT8 quantizer) and paged_ref.py (numpy: indexing, metadata,
gather-then-attend, INT8 dequantize-then-attend, split merging; torch on the CPU for the timed baseline).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it, and only as the checker.
Nothing under small-inference_amd/ imports it.
"""
