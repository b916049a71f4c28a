"""WISP_MODE / WISP_CAP_EXPERTS resolution and the install surface
(reference fused_moe.py:76-118, 1245-1315; plugin.py:47-97)."""
import importlib
import logging

import pytest

fm = importlib.import_module("wisp.integrations.vllm.fused_moe")


@pytest.mark.parametrize("raw,want", [(None, "paged"), ("paged", "paged"), ("resident", "resident"),
                                      ("copy", "copy"), ("day1", "copy"), ("day2a", "resident"),
                                      ("day2b", "paged"), (" PAGED ", "paged")])
def test_resolve_mode(monkeypatch, raw, want):
    if raw is None:
        monkeypatch.delenv("WISP_MODE", raising=False)
    else:
        monkeypatch.setenv("WISP_MODE", raw)
    assert fm._resolve_mode() == want


def test_resolve_mode_unknown_warns(monkeypatch, caplog):
    monkeypatch.setenv("WISP_MODE", "bogus")
    with caplog.at_level(logging.WARNING):
        assert fm._resolve_mode() == "paged"
    assert "unrecognised" in caplog.text


@pytest.mark.parametrize("raw,E,want", [(None, 128, 24), (None, 8, 8), ("8", 128, 8),
                                        ("1", 128, 2), ("999", 128, 128), ("0", 8, 2),
                                        ("abc", 128, 128), ("-5", 16, 2)])
def test_resolve_cap(monkeypatch, raw, E, want):
    if raw is None:
        monkeypatch.delenv("WISP_CAP_EXPERTS", raising=False)
    else:
        monkeypatch.setenv("WISP_CAP_EXPERTS", raw)
    assert fm._resolve_cap_experts(E) == want


def test_install_is_idempotent_and_refreshes_config(monkeypatch):
    from wisp.integrations.vllm import layer
    cls = layer.UnquantizedFusedMoEMethod
    orig = (cls.create_weights, cls.process_weights_after_loading, cls.forward_cuda)
    try:
        first = fm.install_wisp_moe(mode="paged", cap_experts=8)
        assert fm.is_installed()
        assert fm.install_wisp_moe(mode="resident") is False
        assert fm._WISP_RUNTIME_CONFIG == {"mode": "resident", "cap_experts_override": None}
        assert cls.forward_cuda is fm._patched_forward_cuda
        assert first in (True, False)
    finally:
        cls.create_weights, cls.process_weights_after_loading, cls.forward_cuda = orig
        if hasattr(cls, "_wisp_patched"):
            delattr(cls, "_wisp_patched")


def test_plugin_register_honours_disable(monkeypatch):
    from wisp.integrations.vllm import plugin
    monkeypatch.setenv("WISP_PLUGIN_DISABLE", "1")
    plugin.register()
    assert not fm.is_installed()


def test_create_weights_rejects_bias():
    import torch
    from wisp.integrations.vllm.layer import FusedMoEConfig, UnquantizedFusedMoEMethod
    m = UnquantizedFusedMoEMethod(FusedMoEConfig(has_bias=True))
    with pytest.raises(NotImplementedError):
        fm._patched_create_weights(m, torch.nn.Module(), 4, 16, 8, torch.float32)


def test_create_weights_allocates_host_slab():
    import torch
    from wisp.integrations.vllm.layer import UnquantizedFusedMoEMethod
    layer = torch.nn.Module()
    fm._patched_create_weights(UnquantizedFusedMoEMethod(), layer, 4, 16, 8, torch.bfloat16)
    assert layer.w13_weight.shape == (4, 16, 16) and layer.w2_weight.shape == (4, 16, 8)
    assert layer.w13_weight.device.type == "cpu"
    # w2 of expert e follows its w13 in one slab: one copy per miss
    assert layer.w2_weight.data_ptr() - layer.w13_weight.data_ptr() == 16 * 16 * 2
    assert layer.w13_weight.stride(0) == layer.w2_weight.stride(0) == 3 * 8 * 16


def test_unsupported_call_arguments():
    with pytest.raises(NotImplementedError):
        fm._check_supported({"scoring_func": "sigmoid"})
    with pytest.raises(NotImplementedError):
        fm._check_supported({"use_grouped_topk": True})
    fm._check_supported({"scoring_func": "softmax", "topk_group": None})


# --- block-FP8 path (reference fused_moe_fp8.py:48-58, 362-390) -------------

f8m = importlib.import_module("wisp.integrations.vllm.fused_moe_fp8")


@pytest.mark.parametrize("raw,E,want", [(None, 128, 24), (None, 8, 8), ("8", 128, 8),
                                        ("2", 128, 8), ("2", 4, 8), ("999", 128, 128),
                                        ("abc", 128, 24), ("abc", 16, 16), ("-5", 16, 8)])
def test_resolve_cap_fp8(monkeypatch, raw, E, want):
    if raw is None:
        monkeypatch.delenv("WISP_CAP_EXPERTS", raising=False)
    else:
        monkeypatch.setenv("WISP_CAP_EXPERTS", raw)
    assert f8m._resolve_cap_experts(E) == want


def test_fp8_slab_layout_qwen3_shape():
    lay = f8m.Fp8SlabLayout(2048, 768, (128, 128))
    assert lay.s13_shape == (12, 16) and lay.s2_shape == (16, 6)
    assert lay.o_w2 == 2 * 768 * 2048 and lay.o_s13 == 3 * 768 * 2048
    assert lay.o_s2 == lay.o_s13 + 4 * 12 * 16 and lay.used == lay.o_s2 + 4 * 16 * 6
    assert lay.slab % 256 == 0 and lay.slab - lay.used < 256
    import torch
    buf = torch.zeros((3, lay.slab), dtype=torch.uint8)
    w13, w2, s13, s2 = lay.views(buf)
    assert w13.shape == (3, 1536, 2048) and w13.dtype == torch.float8_e4m3fn
    assert s2.shape == (3, 16, 6) and s2.dtype == torch.float32
    s2[1].fill_(2.0)
    raw = buf[1, lay.o_s2:lay.used].view(torch.float32)
    assert torch.equal(raw, torch.full((96,), 2.0))
    # DeepSeek-V3-shaped and block_n 64 layouts keep the scales 16-byte aligned
    for H, I, blk in ((7168, 2048, (128, 128)), (1024, 384, (64, 128))):
        lay = f8m.Fp8SlabLayout(H, I, blk)
        assert lay.o_s13 % 16 == 0 and lay.o_s2 % 4 == 0


def test_install_fp8_patches_standin_once():
    from wisp.integrations.vllm import layer
    cls = layer.Fp8MoEMethod
    names = ("create_weights", "process_weights_after_loading", "apply")
    orig = {n: cls.__dict__[n] for n in names}
    was = getattr(cls, f8m._PATCHED_FLAG, False)
    try:
        if was:
            for n in names:
                setattr(cls, n, getattr(cls, "_wisp_original_" + n))
            delattr(cls, f8m._PATCHED_FLAG)
        assert f8m.install_wisp_fp8() is True and f8m.is_fp8_installed()
        assert f8m.install_wisp_fp8() is False
        assert cls.apply is f8m._patched_apply
        assert cls._wisp_original_apply is (orig["apply"] if not was
                                           else getattr(cls, "_wisp_original_apply"))
    finally:
        for n, f in orig.items():
            setattr(cls, n, f)
        if was:
            setattr(cls, f8m._PATCHED_FLAG, True)
        elif hasattr(cls, f8m._PATCHED_FLAG):
            delattr(cls, f8m._PATCHED_FLAG)


def test_reference_import_path_and_entry_point():
    """Caller code written against the reference imports unchanged
    (src/wisp/integrations/vllm/__init__.py:37-39), and the vLLM plug-in
    entry point names the reference's module (pyproject.toml:35-36)."""
    import configparser
    import os
    import re

    from wisp.integrations.vllm import install_wisp_moe, is_installed
    from wisp.integrations.vllm.fused_moe import WispMoEState
    from wisp.integrations.vllm.plugin import register
    assert callable(install_wisp_moe) and callable(is_installed) and callable(register)
    assert WispMoEState.__module__ == "wisp.integrations.vllm.fused_moe"
    assert fm.__all__ == ["install_wisp_moe", "is_installed", "WispMoEState"]
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    with open(os.path.join(root, "pyproject.toml")) as f:
        text = f.read()
    block = re.search(r'\[project\.entry-points\."vllm\.general_plugins"\]\s*\n([^\[]*)', text)
    assert block, "no vllm.general_plugins entry point"
    cp = configparser.ConfigParser()
    cp.read_string("[ep]\n" + block.group(1))
    assert cp["ep"]["wisp"].strip('"') == "wisp.integrations.vllm.plugin:register"
