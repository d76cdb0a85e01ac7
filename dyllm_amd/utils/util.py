"""Row gather helper (dyllm/utils/util.py:19-36) on the HIP row-copy kernel."""
from .. import ops


def gather_rows_2D(x, row_idx):
    """x: [L, D], row_idx: [K] -> [K, D]."""
    return ops.gather_rows_2D(x.contiguous(), row_idx)
