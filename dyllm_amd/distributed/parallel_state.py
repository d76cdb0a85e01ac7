"""The decisive tau test (dyllm/distributed/parallel_state.py:52-66).

One GPU: no all-reduce; the three additive fp32 statistics of each row are turned into the
salient decision on the device. With tensor parallelism the only exchange would be a
SUM all-reduce of these [T, 3] statistics before this call."""
from .. import ops


def tensor_parallel_cosine_mask(stats, threshold):
    """``stats[..., 0:3]`` = dot and the two squared norms; returns cos < threshold."""
    return ops.tensor_parallel_cosine_mask(stats.contiguous(), threshold)
