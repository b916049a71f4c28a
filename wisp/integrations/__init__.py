"""Framework integrations of the paged fused-MoE layer."""
