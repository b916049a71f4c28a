"""wisp_amd - the MI355X (gfx950) native side of the paged fused-MoE layer.

``csrc/`` holds the HIP kernels (routing, the GPU pager, page-in copy kernel,
decode GEMV and MFMA grouped expert GEMMs, block-FP8 experts, cross-layer
prefetch) and the C ABI declared in ``include/wisp_hip.h``; ``build`` compiles
them into the in-tree ``libwisp_hip.so`` and ``_lib`` binds it with ctypes.
The drop-in host layer that calls it lives under the reference's import path,
``wisp.integrations.vllm``.
"""
__version__ = "0.1.0"
__all__ = ["__version__"]
