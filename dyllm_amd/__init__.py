"""MI355X-native (gfx950) DyLLM saliency hot path.

Public API mirrors the reference: ``dLLM(model, threshold=..., tensor_parallel_size=1)``
with ``.generate(prompts, SamplingParams)``; the per-layer hot path runs on hand-written
HIP kernels reached through the C ABI in ``libdyllm_hip.so``.
"""

__all__ = ["dLLM", "SamplingParams"]


def __getattr__(name):
    if name == "dLLM":
        from .dllm import dLLM

        return dLLM
    if name == "SamplingParams":
        from .sampling_params import SamplingParams

        return SamplingParams
    raise AttributeError(name)
