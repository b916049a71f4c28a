"""vLLM integration: ``install_wisp_moe()`` pages MoE experts from pinned host
memory into a small HBM scratch (``WISP_MODE``, ``WISP_CAP_EXPERTS``).

Same import surface as the reference's ``wisp.integrations.vllm``
(``src/wisp/integrations/vllm/__init__.py:37-39``)::

    from wisp.integrations.vllm import install_wisp_moe
    install_wisp_moe()   # before the model is built
"""
from .fused_moe import install_wisp_moe, is_installed
from .fused_moe_fp8 import install_wisp_fp8, is_fp8_installed

__all__ = ["install_wisp_moe", "is_installed", "install_wisp_fp8", "is_fp8_installed"]
