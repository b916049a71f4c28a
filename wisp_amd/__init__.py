"""wisp_amd - paged fused-MoE layer for AMD Instinct MI355X (gfx950).

Expert weights live in pinned host memory; a fixed HBM scratch of ``cap``
slots per layer holds the experts the current tokens route to, managed by an
LRU pager that runs on the GPU.  Routing, paging decisions, page-in and the
expert GEMMs are HIP kernels in ``libwisp_hip.so`` (C ABI:
``include/wisp_hip.h``).
"""
__version__ = "0.1.0"
__all__ = ["__version__"]
