"""MI355X (gfx950) per-layer NF4/int4 LoRA training compute for SpillTune.

The hot path -- 4-bit dequant, fused dequant-GEMM forward and input gradient,
rank-r LoRA products, the decoder-layer elementwise kernels -- runs in the
hand-written HIP kernels of ``libspilltune_hip.so`` (C ABI in
``include/spilltune_hip.h``); this package is the Python host side that mirrors
the reference's projection / functional / recompute / session interfaces.
"""
__version__ = "0.1.0"
