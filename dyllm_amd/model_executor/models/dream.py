"""Dream (Qwen2-shaped) bidirectional decoder (dyllm/model_executor/models/dream.py:26-236):
the LLaDA layer structure with q/k/v biases and grouped-query attention (e.g. 28 query heads
over 4 K/V heads). The attention kernels map query head h to K/V head h / (H / H_kv). Logits are
shifted by one position in the sampler (DreamSampler)."""
from __future__ import annotations

from .llada import LLaDADecoderLayer, LLaDAForDLM


class DreamDecoderLayer(LLaDADecoderLayer):
    pass


class DreamForDLM(LLaDAForDLM):
    layer_cls = DreamDecoderLayer

    def normalize_weight_name(self, name: str) -> str:
        return name        # the checkpoint already uses the module names (dream.py:218-219)
