"""wisp - routing-aware expert paging for a paged fused-MoE layer, on MI355X.

The reference's package name and import surface
(``src/wisp/__init__.py``, ``src/wisp/integrations/vllm/__init__.py:37-39``)::

    from wisp.integrations.vllm import install_wisp_moe, is_installed
    install_wisp_moe()   # before the model is built

``wisp.integrations.vllm`` holds the host side of the path (the plug-in entry
point, ``WispMoEState``, the patched MoE methods, FP8 paging and the
cross-layer prefetch table).  Every call on the path goes through the HIP
library of ``wisp_amd`` (kernels and C ABI for gfx950); there is no CPU or
PyTorch fallback.
"""
__version__ = "0.1.0"
__all__ = ["__version__"]
