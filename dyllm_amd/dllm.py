"""Public entry point (dyllm/dllm.py:1-4): ``dLLM(model, threshold=...).generate(prompts, params)``."""
from .engine.llm_engine import DLLMEngine


class dLLM(DLLMEngine):
    pass
