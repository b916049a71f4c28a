"""The plug-in surface end to end on the GPU: install_wisp_moe patches the
MoE method class and a vLLM-shaped layer built after it pages its experts."""
import pytest
import torch

from wisp_amd import workloads as W
from wisp.integrations.vllm import fused_moe as fm
from wisp.integrations.vllm import layer as L

pytestmark = pytest.mark.gpu


@pytest.fixture
def patched():
    cls = L.UnquantizedFusedMoEMethod
    orig = (cls.create_weights, cls.process_weights_after_loading, cls.forward_cuda)
    yield
    cls.create_weights, cls.process_weights_after_loading, cls.forward_cuda = orig
    if hasattr(cls, "_wisp_patched"):
        delattr(cls, "_wisp_patched")
    fm._LAYER_STATES.clear()
    fm._LAYER_BY_ID.clear()


def _layer(wl):
    sh = wl.shape
    m = L.FusedMoE(sh.experts, sh.top_k, sh.hidden, sh.inter, sh.dtype)
    w13, w2 = wl.views()
    m.load_weights(w13, w2)
    m.process_weights_after_loading()
    return m


@pytest.mark.parametrize("mode", ["paged", "resident", "copy"])
def test_patched_layer_matches_unpatched(patched, mode):
    wl = W.toy(steps=12, pin=True)
    base = _layer(wl)                     # unpatched: all experts on the GPU
    fm.install_wisp_moe(mode=mode, cap_experts=4)
    paged = _layer(wl)
    assert paged.w13_weight.numel() == 0  # placeholders, as in the reference
    if mode != "copy":
        assert paged._wisp_state.cap_experts == (4 if mode == "paged" else 16)
    for t in range(wl.steps):
        x, lg = wl.x[t].cuda(), wl.logits[t].cuda()
        a, b = base(x, lg), paged(x, lg)
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), t


def test_unsupported_kwargs_raise(patched):
    wl = W.toy(steps=1, pin=True)
    fm.install_wisp_moe(mode="paged", cap_experts=4)
    m = _layer(wl)
    with pytest.raises(NotImplementedError):
        m.quant_method.forward_cuda(m, wl.x[0].cuda(), False, 2, wl.logits[0].cuda(), True,
                                    scoring_func="sigmoid")
    with pytest.raises(NotImplementedError):
        m.quant_method.forward_cuda(m, wl.x[0].cuda(), False, 2, wl.logits[0].cuda(), True,
                                    expert_map=torch.arange(16, device="cuda"))
