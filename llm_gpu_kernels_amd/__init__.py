"""MI355X-native (gfx950) MoE forward: routing, grouped expert GEMMs, combine.

The Python layer mirrors the reference's prepared operator API; all compute
runs in hand-written HIP kernels of ``_lib/libmoe_mi355x.so`` (C ABI in
``include/``).  Importing the package does not load the library; the first
prepare/quantise call does, and raises if it has not been built.
"""
from .moe import (FrozenMoEPolicy, GemmConfig, PreparedMoE, PreparedRoutedMoE, prepare_configured_moe,
                  prepare_cuda_moe, prepare_moe, prepare_ranked_moe_launcher, prepare_routed_moe,
                  prepare_w4_layout_moe, prepare_w4_moe)
from .attention import PreparedSegmentedGQA, prepare_cuda_gqa_compact, prepare_segmented_gqa
from .weight_quant import (PackedGateUp, RepackedGateUp, TiledGateUp, dequantize_tiled,
                           quantize_gate_up, repack_gate_up, restore_v1_layout, tile_gate_up)

__all__ = [
    "FrozenMoEPolicy", "GemmConfig", "PreparedMoE", "PreparedRoutedMoE", "prepare_configured_moe",
    "prepare_cuda_moe", "prepare_moe", "prepare_ranked_moe_launcher", "prepare_routed_moe",
    "prepare_w4_layout_moe", "prepare_w4_moe", "PackedGateUp", "RepackedGateUp", "TiledGateUp",
    "dequantize_tiled", "quantize_gate_up", "repack_gate_up", "restore_v1_layout", "tile_gate_up", "PreparedSegmentedGQA", "prepare_segmented_gqa",
    "prepare_cuda_gqa_compact",
]
