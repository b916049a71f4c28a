"""vLLM-shaped MoE layers for hosts without vLLM.

``UnquantizedFusedMoEMethod`` here has the three methods the plug-in patches
(``create_weights``, ``process_weights_after_loading``, ``forward_cuda``)
with vLLM 0.11's signatures, and ``FusedMoE`` builds a layer the way vLLM's
``FusedMoE`` does: ``quant_method.create_weights`` at construction, the
loader writes ``w13_weight [E, 2I, H]`` / ``w2_weight [E, H, I]`` through
``param.data.copy_``, then ``process_weights_after_loading``, then calls go
through ``quant_method.forward_cuda``.  ``install_wisp_moe`` patches this
class when vLLM is absent, so the same layer call runs the paged path.

The unpatched ``forward_cuda`` keeps every expert on the GPU and runs the
same HIP routing and expert kernels with slot = expert id.

``Fp8MoEMethod`` / ``Fp8FusedMoE`` do the same for vLLM 0.11's block-quantised
FP8 MoE method (``create_weights``, ``process_weights_after_loading``,
``apply``; weights float8_e4m3fn with float32 ``*_weight_scale_inv`` block
scales), which ``install_wisp_fp8`` patches.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class FusedMoEConfig:
    has_bias: bool = False
    is_act_and_mul: bool = True


class UnquantizedFusedMoEMethod:
    def __init__(self, moe: FusedMoEConfig | None = None) -> None:
        self.moe = moe or FusedMoEConfig()
        self.topk_indices_dtype = None
        self.moe_quant_config = None

    def create_weights(self, layer: torch.nn.Module, num_experts: int, hidden_size: int,
                       intermediate_size_per_partition: int, params_dtype: torch.dtype,
                       **extra_weight_attrs) -> None:
        if self.moe.has_bias:
            raise NotImplementedError("expert biases are not supported")
        dev = torch.device("cuda", torch.cuda.current_device())
        I = intermediate_size_per_partition
        w13 = torch.nn.Parameter(torch.empty(num_experts, 2 * I, hidden_size, dtype=params_dtype,
                                             device=dev), requires_grad=False)
        w2 = torch.nn.Parameter(torch.empty(num_experts, hidden_size, I, dtype=params_dtype,
                                            device=dev), requires_grad=False)
        layer.register_parameter("w13_weight", w13)
        layer.register_parameter("w2_weight", w2)

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        return None

    def forward_cuda(self, layer: torch.nn.Module, x: torch.Tensor, use_grouped_topk: bool,
                     top_k: int, router_logits: torch.Tensor, renormalize: bool,
                     topk_group=None, num_expert_group=None, global_num_experts: int = -1,
                     expert_map=None, custom_routing_function=None, scoring_func: str = "softmax",
                     routed_scaling_factor: float = 1.0, e_score_correction_bias=None,
                     apply_router_weight_on_input: bool = False, activation: str = "silu",
                     enable_eplb: bool = False, expert_load_view=None,
                     logical_to_physical_map=None, logical_replica_count=None) -> torch.Tensor:
        from .fused_moe import _check_supported, _route_and_experts
        _check_supported(dict(use_grouped_topk=use_grouped_topk, topk_group=topk_group,
                              num_expert_group=num_expert_group,
                              custom_routing_function=custom_routing_function,
                              scoring_func=scoring_func,
                              routed_scaling_factor=routed_scaling_factor,
                              e_score_correction_bias=e_score_correction_bias,
                              apply_router_weight_on_input=apply_router_weight_on_input,
                              activation=activation, enable_eplb=enable_eplb))
        if expert_map is not None:
            raise NotImplementedError("expert_map (expert parallelism) is not supported")
        return _route_and_experts(x, router_logits, top_k, renormalize, layer.w13_weight,
                                  layer.w2_weight)


class FusedMoE(torch.nn.Module):
    """MoE block with vLLM ``FusedMoE``'s construction and call sequence."""

    def __init__(self, num_experts: int, top_k: int, hidden_size: int, intermediate_size: int,
                 params_dtype: torch.dtype = torch.bfloat16, renormalize: bool = True,
                 prefix: str = "") -> None:
        super().__init__()
        self.num_experts, self.top_k = num_experts, top_k
        self.hidden_size, self.intermediate_size = hidden_size, intermediate_size
        self.renormalize = renormalize
        self.prefix = prefix
        self.quant_method = UnquantizedFusedMoEMethod()
        self.quant_method.create_weights(self, num_experts, hidden_size, intermediate_size,
                                         params_dtype)

    def load_weights(self, w13: torch.Tensor, w2: torch.Tensor) -> None:
        """What the checkpoint loader does: copy into the registered params."""
        self.w13_weight.data.copy_(w13)
        self.w2_weight.data.copy_(w2)

    def process_weights_after_loading(self) -> None:
        self.quant_method.process_weights_after_loading(self)

    def forward(self, hidden_states: torch.Tensor, router_logits: torch.Tensor) -> torch.Tensor:
        return self.quant_method.forward_cuda(self, hidden_states, use_grouped_topk=False,
                                              top_k=self.top_k, router_logits=router_logits,
                                              renormalize=self.renormalize)


class Fp8MoEMethod:
    """vLLM's block-quantised FP8 MoE method: the parts the plug-in patches."""

    def __init__(self, weight_block_size=(128, 128), block_quant: bool = True) -> None:
        self.block_quant = block_quant
        self.weight_block_size = list(weight_block_size)
        self.topk_indices_dtype = None
        self.moe_quant_config = None
        self.rocm_aiter_moe_enabled = False

    def create_weights(self, layer: torch.nn.Module, num_experts: int, hidden_size: int,
                       intermediate_size_per_partition: int, params_dtype: torch.dtype,
                       **extra_weight_attrs) -> None:
        dev = torch.device("cuda", torch.cuda.current_device())
        I, H = intermediate_size_per_partition, hidden_size
        bn, bk = self.weight_block_size
        f8 = torch.float8_e4m3fn
        layer.orig_dtype = params_dtype
        layer.weight_block_size = self.weight_block_size
        for name, shape, dtype in (
                ("w13_weight", (num_experts, 2 * I, H), f8),
                ("w2_weight", (num_experts, H, I), f8),
                ("w13_weight_scale_inv", (num_experts, 2 * -(-I // bn), -(-H // bk)),
                 torch.float32),
                ("w2_weight_scale_inv", (num_experts, -(-H // bn), -(-I // bk)), torch.float32)):
            t = torch.zeros(shape, dtype=dtype, device=dev)
            if dtype == torch.float32:
                t.fill_(1.0)
            layer.register_parameter(name, torch.nn.Parameter(t, requires_grad=False))

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        return None

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, router_logits: torch.Tensor,
              top_k: int, renormalize: bool, use_grouped_topk: bool = False, topk_group=None,
              num_expert_group=None, global_num_experts: int = -1, expert_map=None,
              custom_routing_function=None, scoring_func: str = "softmax",
              routed_scaling_factor: float = 1.0, e_score_correction_bias=None,
              apply_router_weight_on_input: bool = False, activation: str = "silu",
              enable_eplb: bool = False, expert_load_view=None, logical_to_physical_map=None,
              logical_replica_count=None) -> torch.Tensor:
        from .fused_moe import _check_supported
        from .fused_moe_fp8 import route_and_experts_fp8
        _check_supported(dict(use_grouped_topk=use_grouped_topk, topk_group=topk_group,
                              num_expert_group=num_expert_group,
                              custom_routing_function=custom_routing_function,
                              scoring_func=scoring_func,
                              routed_scaling_factor=routed_scaling_factor,
                              e_score_correction_bias=e_score_correction_bias,
                              apply_router_weight_on_input=apply_router_weight_on_input,
                              activation=activation, enable_eplb=enable_eplb))
        if expert_map is not None:
            raise NotImplementedError("expert_map (expert parallelism) is not supported")
        return route_and_experts_fp8(x, router_logits, top_k, renormalize, layer.w13_weight,
                                     layer.w2_weight, layer.w13_weight_scale_inv,
                                     layer.w2_weight_scale_inv, tuple(self.weight_block_size))


class Fp8FusedMoE(torch.nn.Module):
    """Block-FP8 MoE block with vLLM ``FusedMoE``'s construction and call
    sequence (activations in ``params_dtype``, bfloat16)."""

    def __init__(self, num_experts: int, top_k: int, hidden_size: int, intermediate_size: int,
                 weight_block_size=(128, 128), params_dtype: torch.dtype = torch.bfloat16,
                 renormalize: bool = True, prefix: str = "") -> None:
        super().__init__()
        self.num_experts, self.top_k = num_experts, top_k
        self.hidden_size, self.intermediate_size = hidden_size, intermediate_size
        self.renormalize = renormalize
        self.prefix = prefix
        self.quant_method = Fp8MoEMethod(weight_block_size)
        self.quant_method.create_weights(self, num_experts, hidden_size, intermediate_size,
                                         params_dtype)

    def load_weights(self, w13: torch.Tensor, w2: torch.Tensor, s13: torch.Tensor,
                     s2: torch.Tensor) -> None:
        """What the checkpoint loader does: copy into the registered params."""
        self.w13_weight.data.copy_(w13)
        self.w2_weight.data.copy_(w2)
        self.w13_weight_scale_inv.data.copy_(s13)
        self.w2_weight_scale_inv.data.copy_(s2)

    def process_weights_after_loading(self) -> None:
        self.quant_method.process_weights_after_loading(self)

    def forward(self, hidden_states: torch.Tensor, router_logits: torch.Tensor) -> torch.Tensor:
        return self.quant_method.apply(self, hidden_states, router_logits, top_k=self.top_k,
                                       renormalize=self.renormalize)
