"""blackhole_runtime on MI355X: HIP kernels for gfx950 behind the reference runtime's API.

hex_moe.py   the HEX fused-MoE operator: HexTier, hex_moe, hex_moe_fused, hex_moe_dequant,
             dequant_all, align, direct, plan, default_config (and route_topk, hex_dequant)
vllm_hex.py  the "blackhole-hex" quantization method for vLLM (loaded as a vLLM plugin)
hex_check.py GPU check against an fp32 dequant + matmul reference, and per-layer timings
_lib.py      ctypes binding of libbh_hex.so (C ABI: include/bh_hex.h)
"""
