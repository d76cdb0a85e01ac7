from .parallel_state import tensor_parallel_cosine_mask

__all__ = ["tensor_parallel_cosine_mask"]
