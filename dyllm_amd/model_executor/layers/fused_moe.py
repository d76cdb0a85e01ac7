"""MoE routing and grouped experts (dyllm/model_executor/layers/fused_moe.py) on the HIP
kernels: ``moe_gate`` (:375-408), ``moe_align_block_size`` (:37-85), ``fused_experts``
(:269-335, SiLU gating)."""
from ...ops import fused_experts, moe_align_block_size, moe_gate

__all__ = ["moe_gate", "moe_align_block_size", "fused_experts"]
