"""Running / finished sequence bookkeeping (dyllm/utils/metadata.py:6-28)."""
from dataclasses import dataclass, field
from typing import List, Optional

import torch


@dataclass
class MetaData:
    running_seqs: List[int] = field(default_factory=list)
    running_seqs_tensor: Optional[torch.Tensor] = None
    finished_seqs: List[int] = field(default_factory=list)


_METADATA = MetaData()


def get_metadata() -> MetaData:
    return _METADATA


def reset_metadata():
    global _METADATA
    _METADATA = MetaData()
