"""Entry point for vLLM's ``vllm.general_plugins`` group (reference
``src/wisp/integrations/vllm/plugin.py:47-97``).

vLLM calls plug-in entry points in every process it starts (engine parent,
engine core, workers) before the model is built; ``register`` is idempotent
and honours ``WISP_PLUGIN_DISABLE``.
"""
from __future__ import annotations

import logging
import os

logger = logging.getLogger(__name__)


def register() -> None:
    if os.environ.get("WISP_PLUGIN_DISABLE", "0").strip().lower() in ("1", "true", "yes", "on"):
        logger.info("wisp plugin: WISP_PLUGIN_DISABLE set - not patching")
        return
    try:
        from .fused_moe import install_wisp_moe, is_installed
    except ImportError as e:  # pragma: no cover - torch missing on this host
        logger.warning("wisp plugin: import failed (%s); plug-in not installed", e)
        return
    if is_installed():
        logger.debug("wisp plugin: already patched in this process")
        return
    install_wisp_moe()
    logger.info("wisp plugin: patched (WISP_MODE=%s WISP_CAP_EXPERTS=%s)",
                os.environ.get("WISP_MODE", "paged"), os.environ.get("WISP_CAP_EXPERTS", "auto"))
