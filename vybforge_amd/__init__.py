"""vybforge_amd — MI355X-native fused dequant-matmul library (libvybdq) for VybForge's Infer path.

``vybforge_amd._lib`` binds the C-ABI (include/vybdq.h) with ctypes; ``vybforge_amd.ops``
mirrors the reference host's call surface (GGUF type-id dispatch of packed GEMV/GEMM,
the EXL3 expert path and the MoE block) on torch device tensors.
"""

__all__ = ["ops"]
