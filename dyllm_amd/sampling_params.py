"""Per-request decoding parameters (dyllm/sampling_params.py:4-24, the fields the mask-based
models read; the DiffusionGemma-only fields are accepted and ignored)."""
from dataclasses import dataclass
from typing import Optional


@dataclass
class SamplingParams:
    temperature: float = 1.0
    max_new_tokens: int = 256
    steps: int = 64
    num_full_steps: int = 16
    block_size: int = 32
    ignore_eos: bool = False
    algorithm: str = "confidence"
    top_p: Optional[float] = None
    top_k: Optional[int] = None
    confidence_threshold: Optional[float] = None
    input_len: Optional[int] = None
    entropy_bound: Optional[float] = None
    t_max: Optional[float] = None
    t_min: Optional[float] = None
    max_denoising_steps: Optional[int] = None
    convergence_threshold: Optional[float] = None
    stability_threshold: Optional[int] = None
    mask_id: Optional[int] = None
