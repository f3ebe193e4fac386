"""mashbox_amd — MI355X-native quantized linear for mashbox (GGUF Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K and int8 per-channel weights).

    mashbox_amd.kernels   mashbox's kernel-package surface (TYPES, repack_host, repack, matmul, dequant, plane_bytes,
                          kq_covers, picks_layer) on the hand-written gfx950 kernels of libmbq.so
    mashbox_amd.int8      the int8 per-output-channel linear(x, {"q", "s"})
    mashbox_amd.ops       mashbox's ops boundary for these weights (prepare, qmatmul, dequant, contract_check, ...)

libmbq.so is built in-tree by mashbox_amd.build; importing a module that needs it raises when it is missing.
"""
__version__ = "0.1.0"
