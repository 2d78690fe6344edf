"""
lazylora_amd — LazyLoRA's routed-expert MXFP4 hot path, rebuilt for AMD Instinct MI355X.

    from lazylora_amd.native import kernel        # MXFP4Kernel: gemm / gemm_t / dequant / routed_*
    from lazylora_amd.experts import ExpertLayer  # one layer's packed experts, stacked in HBM
    from lazylora_amd.routed import RoutedExpertsFunction
    from lazylora_amd.router import KimiK3MoERouter  # gate GEMM + device top-k selection

The arithmetic runs in hand-written gfx950 HIP kernels behind a C ABI
(include/lazylora_mxfp4.h, built into lazylora_amd/liblazylora_mxfp4.so by lazylora_amd.build).
"""

__all__ = ["native", "experts", "routed", "router"]
