"""Engine and model configuration (dyllm/config.py:10-63).

``Config(model, ...)`` keeps the reference's fields. ``model`` is either a local directory
holding a HuggingFace-style ``config.json`` (optionally ``*.safetensors`` weights and tokenizer
files), as in the reference, or the name of a shape preset from ``PRESETS`` (random-initialised
weights of that architecture; no checkpoint is needed). The model description is parsed into
``ModelConfig`` without executing any code from the directory (the reference calls
``AutoConfig.from_pretrained(..., trust_remote_code=True)``, config.py:40).
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, fields, replace
from typing import Optional


@dataclass
class ModelConfig:
    """Architecture fields the model classes read (llada.py:152-218, dream.py:147-213,
    lladamoe.py:56-62,190-310), under their HuggingFace names."""
    model_type: str = "llada"             # "llada" (dense or MoE) or "Dream"
    vocab_size: int = 126464
    hidden_size: int = 4096
    num_hidden_layers: int = 32
    num_attention_heads: int = 32
    num_key_value_heads: int = 32
    head_dim: int = 128
    intermediate_size: int = 12288
    max_position_embeddings: int = 4096
    rope_theta: float = 500000.0
    rms_norm_eps: float = 1e-5
    qkv_bias: bool = False
    qk_layernorm: bool = False
    tie_word_embeddings: bool = False
    mask_token_id: Optional[int] = 126336
    eos_token_id: Optional[int] = 126081
    num_experts: int = 0
    num_experts_per_tok: int = 0
    expert_intermediate_size: int = 0
    norm_topk_prob: bool = False

    @property
    def is_moe(self) -> bool:
        return self.num_experts > 0

    @classmethod
    def from_dict(cls, d: dict) -> "ModelConfig":
        """HuggingFace config.json -> ModelConfig. Accepts the LLaDA names (d_model, n_heads,
        n_kv_heads, n_layers, mlp_hidden_size, max_sequence_length, weight_tying, include_bias),
        the Dream/Qwen2 names and the LLaDA-MoE names."""
        g = d.get
        mt = g("model_type", "llada")
        hidden = g("hidden_size", g("d_model"))
        heads = g("num_attention_heads", g("n_heads"))
        if hidden is None or heads is None:
            raise ValueError("config.json lacks hidden_size/d_model or num_attention_heads/n_heads")
        kv = g("num_key_value_heads", g("n_kv_heads")) or heads
        inter = g("intermediate_size", g("mlp_hidden_size")) or 0
        eos = g("eos_token_id")
        if isinstance(eos, list):
            eos = eos[0]
        out = cls(
            model_type=mt,
            vocab_size=g("embedding_size") or g("vocab_size"),
            hidden_size=hidden,
            num_hidden_layers=g("num_hidden_layers", g("n_layers")),
            num_attention_heads=heads,
            num_key_value_heads=kv,
            head_dim=g("head_dim") or hidden // heads,
            intermediate_size=inter,
            max_position_embeddings=g("max_position_embeddings", g("max_sequence_length", 4096)),
            rope_theta=float(g("rope_theta", 10000.0)),
            rms_norm_eps=float(g("rms_norm_eps", 1e-5)),
            qkv_bias=bool(g("attention_bias", g("include_bias", mt == "Dream"))),
            qk_layernorm=bool(g("qk_layernorm", False)),
            tie_word_embeddings=bool(g("tie_word_embeddings", g("weight_tying", False))),
            mask_token_id=g("mask_token_id"),
            eos_token_id=eos,
            num_experts=int(g("num_experts", 0) or 0),
            num_experts_per_tok=int(g("num_experts_per_tok", 0) or 0),
            expert_intermediate_size=int(g("expert_intermediate_size", g("moe_intermediate_size", 0)) or 0),
            norm_topk_prob=bool(g("norm_topk_prob", False)),
        )
        return out


# Shape presets: the architectures of the reference's three model families (and small ones for
# tests). Weights are random-initialised; token ids are those of the public checkpoints.
PRESETS = {
    "llada-8b": ModelConfig(),
    "dream-7b": ModelConfig(model_type="Dream", vocab_size=152064, hidden_size=3584, num_hidden_layers=28,
                            num_attention_heads=28, num_key_value_heads=4, intermediate_size=18944,
                            max_position_embeddings=32768, rope_theta=1000000.0, rms_norm_eps=1e-6, qkv_bias=True,
                            mask_token_id=151666, eos_token_id=151643),
    "llada-moe-7b": ModelConfig(vocab_size=157184, hidden_size=2048, num_hidden_layers=16, num_attention_heads=16,
                                num_key_value_heads=16, intermediate_size=0, max_position_embeddings=8192,
                                rope_theta=50000.0, qk_layernorm=True, mask_token_id=156895, eos_token_id=156892,
                                num_experts=64, num_experts_per_tok=8, expert_intermediate_size=1024),
    "tiny-llada": ModelConfig(vocab_size=512, hidden_size=256, num_hidden_layers=2, num_attention_heads=2,
                              num_key_value_heads=2, intermediate_size=512, max_position_embeddings=2048,
                              mask_token_id=511, eos_token_id=510),
    "tiny-dream": ModelConfig(model_type="Dream", vocab_size=512, hidden_size=512, num_hidden_layers=2,
                              num_attention_heads=4, num_key_value_heads=2, intermediate_size=768,
                              max_position_embeddings=2048, rope_theta=1000000.0, rms_norm_eps=1e-6, qkv_bias=True,
                              mask_token_id=511, eos_token_id=510),
    "tiny-llada-moe": ModelConfig(vocab_size=512, hidden_size=256, num_hidden_layers=2, num_attention_heads=2,
                                  num_key_value_heads=2, intermediate_size=0, max_position_embeddings=2048,
                                  qk_layernorm=True, mask_token_id=511, eos_token_id=510, num_experts=8,
                                  num_experts_per_tok=2, expert_intermediate_size=256),
}


def load_model_config(model: str) -> ModelConfig:
    if model in PRESETS:
        return replace(PRESETS[model])
    path = os.path.join(model, "config.json")
    if not os.path.isfile(path):
        raise ValueError(f"{model!r} is neither a shape preset ({sorted(PRESETS)}) nor a directory with config.json")
    with open(path) as f:
        return ModelConfig.from_dict(json.load(f))


@dataclass
class Config:
    model: str
    max_num_batched_tokens: int = 65536
    max_num_seqs: int = 16
    max_model_len: int = 4096
    gpu_memory_utilization: float = 0.9
    tensor_parallel_size: int = 1
    expert_parallel_size: int = 1
    enforce_eager: bool = False
    hf_config: Optional[ModelConfig] = None
    eos: int = -1
    mask_id: int = -1
    num_full_steps: int = 8
    threshold: float = 0.99
    dist_port: Optional[int] = None
    dtype: str = "bfloat16"
    seed: int = 0                      # random-initialisation seed when no weights are loaded
    # Sparse-step cadence: after `refresh_period` processed steps, a step queries only the response
    # rows (Q-pruned) except every `refresh_period`-th, which queries all rows (model_runner.py:211,
    # where the period is the constant 4).
    refresh_period: int = 4
    # Overrides the checkpoint's max_position_embeddings (the RoPE table length and the cap on
    # max_model_len, config.py:51-58) for contexts longer than the checkpoint was trained on.
    max_position_embeddings: Optional[int] = None

    def __post_init__(self):
        if self.tensor_parallel_size != 1 or self.expert_parallel_size != 1:
            raise ValueError("this build runs one process on one GPU: tensor_parallel_size and "
                             "expert_parallel_size must be 1")
        if self.dtype != "bfloat16":
            raise ValueError("the HIP kernels compute in bfloat16 only")
        if self.hf_config is None:
            self.hf_config = load_model_config(self.model)
        if self.refresh_period < 1:
            raise ValueError("refresh_period must be at least 1")
        if self.max_position_embeddings is not None:
            if self.max_position_embeddings < 1:
                raise ValueError("max_position_embeddings must be positive")
            self.hf_config = replace(self.hf_config, max_position_embeddings=int(self.max_position_embeddings))
        self.mask_id = self.hf_config.mask_token_id
        if self.hf_config.eos_token_id is not None:
            self.eos = self.hf_config.eos_token_id
        self.max_model_len = min(self.max_model_len, self.hf_config.max_position_embeddings)
        if self.max_num_batched_tokens < self.max_model_len:
            raise ValueError("max_num_batched_tokens must be at least max_model_len")

    @property
    def model_dir(self) -> Optional[str]:
        return self.model if os.path.isdir(self.model) else None


CONFIG_FIELDS = {f.name for f in fields(Config)}
