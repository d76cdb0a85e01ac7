"""Model families (dyllm/model_executor/models/__init__.py, dyllm/engine/model_runner.py:53-76)."""
from .dream import DreamForDLM
from .llada import LLaDAForDLM
from .lladamoe import LLaDAMoEForDLM

__all__ = ["LLaDAForDLM", "LLaDAMoEForDLM", "DreamForDLM", "model_class"]


def model_class(cfg):
    if cfg.model_type == "Dream":
        return DreamForDLM
    if cfg.model_type == "llada":
        return LLaDAMoEForDLM if cfg.is_moe else LLaDAForDLM
    raise ValueError(f"Unsupported model type: {cfg.model_type}")
